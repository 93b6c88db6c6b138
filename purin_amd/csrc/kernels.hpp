// Batched shared-matrix Chambolle--Pock kernels for CDNA4 (gfx950).
//
// Layout and tiling (see common.hpp): per-sample vectors are batch-minor with
// leading dimension Bp; a 256-thread block is 4 wavefronts; blockIdx.x picks a
// batch tile of 64*S samples (S = 16 bytes / sizeof(T)), so when the number of
// tiles is a multiple of 8 every tile stays on one XCD and its gathered vector
// stays in that XCD's L2.  blockIdx.y walks rows (or columns) of K; the entries
// of the row/column a wave processes are wave-uniform scalar loads, and the
// batch columns are read with 16-byte-per-lane coalesced loads.
//
// The passes of one CP iteration (reference
// src/purin/solvers/chambolle_pock/kernels.py:91-150 and 153-175):
//   row pass   d+ = P(d + sigma (K ybar - r))          (K: row-scaled kept rows)
//   col pass   y+ = clip(a y - delta K^T d+ + delta yhat, lo, hi);
//              ybar+ = y+ + theta (y+ - y)             (+ column diagnostics)
//   res pass   max |K y+ - r| rows, r.d+ and finite(d+) (diagnostics)
//   decide     per-sample stop test and freeze          (kernels.py:260-278)
#pragma once

#include "common.hpp"

namespace purin {

template <typename T>
struct Mat {
  int m, n, me;
  const int32_t* __restrict__ rptr;
  const int32_t* __restrict__ ridx;
  const T* __restrict__ rval;
  const int32_t* __restrict__ cptr;
  const int32_t* __restrict__ cidx;
  const T* __restrict__ cval;
  // Per-sample coefficients (parameter-dependent rows, the reference's
  // values (B, m, w), src/purin/linalg/sparse/operators.py:515, 528): entry k
  // of sample b at rvb[k * vbp + b] (CSR order) / cvb[k * vbp + b] (CSC
  // order).  nullptr: the coefficients rval / cval are shared by the batch.
  const T* __restrict__ rvb;
  const T* __restrict__ cvb;
  int64_t vbp;
};

// Coefficient of CSR entry k (CSC entry k) for the S samples from b0.
template <typename T>
__device__ __forceinline__ typename Lane<T>::V row_coef(const Mat<T>& K, int k, int64_t b0) {
  return K.rvb ? vload(K.rvb + (size_t)k * K.vbp + b0) : vsplat<T>(K.rval[k]);
}
template <typename T>
__device__ __forceinline__ typename Lane<T>::V col_coef(const Mat<T>& K, int k, int64_t b0) {
  return K.cvb ? vload(K.cvb + (size_t)k * K.vbp + b0) : vsplat<T>(K.cval[k]);
}

template <typename T>
struct Iter {
  Mat<T> K;
  int64_t Bp;
  const T* __restrict__ tgt;  // n x Bp
  T* Y;                       // n x Bp
  T* YB;                      // n x Bp
  T* D;                       // m x Bp
  const T* __restrict__ R;    // m x Bp (scaled kept rhs)
  const T* __restrict__ LO;   // n x Bp, or n when shared
  const T* __restrict__ HI;
  int shared_bounds;
  const int32_t* done;        // Bp, or nullptr
  T sigma, a, delta, theta;
  // diagonal steps (kernels.py:76-88): per-row sigma and per-column a, delta
  // replace the scalars when set
  const T* __restrict__ sig_r;  // m or nullptr
  const T* __restrict__ a_c;    // n or nullptr
  const T* __restrict__ d_c;    // n or nullptr
  // per-sample steps (per-sample coefficients: each sample has its own norm
  // bound and accelerated schedule): [Bp] arrays, or with diagonal steps
  // [m][Bp] (sigma) and [n][Bp] (a, delta); nullptr when shared
  const T* __restrict__ sig_b;
  const T* __restrict__ a_b;
  const T* __restrict__ d_b;
  const T* __restrict__ th_b;
  const T* __restrict__ sig_rb;
  const T* __restrict__ a_cb;
  const T* __restrict__ d_cb;
  // general diagonal QP (diagonal_qp.py, kernels.py:68-73, 153-175): objective
  // 0.5 q y^2 + c y with per-sample q, c [n][Bp] replacing q = 1, c = -yhat;
  // the prox coefficients a = 1/(1 + tau q), delta = tau a and the offset
  // -delta c are formed from tau per sample [Bp] or per variable [n][Bp]
  const T* __restrict__ Q;
  const T* __restrict__ Cc;
  const T* __restrict__ tau_b;
  const T* __restrict__ tau_cb;
  // per-sample accelerated schedule: the column pass writes the next
  // iteration's tau, sigma, a, delta, theta ([5][Bp] at sch_next) from this
  // iteration's; gamma = min q per sample ([Bp]; nullptr: 1)
  T* sch_next;
  const T* __restrict__ gam;
  // dense adapter policy (chambolle_pock/dense.py:85-106): factored prox
  // a ((y - tau K^T d) - tau c) (kernels.py:140-142), no freezing of accepted
  // samples (freeze_converged=False: every sample keeps iterating and
  // counting until all are done) and no stationarity in the stop test
  int factored, nofreeze, nostat;
  // without freezing the loop must stop at the iteration where the last
  // sample is accepted (kernels.py:238-240); the passes and the stop test
  // return at once when *stop (the accepted count) has reached nstop
  const int32_t* stop;
  int64_t nstop;
  // K ybar by linearity (lin != 0): ybar = y + theta (y - y_prev)
  // (kernels.py:149) gives K~ybar = (1 + thp) K~y - thp K~y_prev, with thp the
  // previous iteration's theta (0 at the first, where ybar = y).  The row pass
  // takes K~y from a gather of Y (row pass template LIN 1, which stores it at
  // KYo) or from the previous residual pass (LIN 2, no gathers; the residual
  // pass stores K~y+ at KYo); ybar itself is not kept (YB is not written).
  const T* __restrict__ KYc;  // m x Bp: K~y of the current y (LIN 2)
  const T* __restrict__ KYp;  // m x Bp: K~y of the previous y (read when thp != 0)
  T* KYo;                     // m x Bp: K~y stored by the row pass (LIN 1) / residual pass
  T* TK;                      // n x Bp or nullptr: K~^T d stored by the final pass (MODE 2)
  const int32_t* __restrict__ kyrow;  // with KYo: the residual pass stores row i at
                                      // KYo + kyrow[i] * Bp (its full-row position)
  T thp;
  int lin;
  T* colpart;                 // [5][ncb][Bp]: primal, dual, stat, bound, finite
  T* rowpart;                 // [3][nrb][Bp]: residual max, r.d, finite
  int ncb, nrb;
};

// The accelerated update after an iteration (kernels.py:279-283) for one
// sample: nu = 1/sqrt(1 + gamma tau); tau <- nu tau; sigma <- sigma / nu;
// theta <- nu; and the prox coefficients a = 1/(1 + tau), delta = tau a of
// q = 1 for the new tau.  Every product and quotient is rounded.
template <typename T>
__device__ __forceinline__ void sched_next(T gamma, T tau, T sig, T* out, int64_t Bp, int64_t b) {
#pragma clang fp contract(off)
  const T one = T(1);
  const T nu = one / (T)__builtin_sqrt(one + gamma * tau);
  const T nt = nu * tau;
  const T a = one / (one + nt);
  out[b] = nt;
  out[Bp + b] = sig / nu;
  out[2 * Bp + b] = a;
  out[3 * Bp + b] = nt * a;
  out[4 * Bp + b] = nu;
}

// Step sizes of row i / column j for the S samples from b0 (shared scalar,
// diagonal, per-sample or per-sample diagonal).
template <typename T>
__device__ __forceinline__ typename Lane<T>::V step_sigma(const Iter<T>& A, int i, int64_t b0) {
  if (A.sig_rb) return vload(A.sig_rb + (size_t)i * A.Bp + b0);
  if (A.sig_b) return vload(A.sig_b + b0);
  return vsplat<T>(A.sig_r ? A.sig_r[i] : A.sigma);
}
template <typename T>
__device__ __forceinline__ typename Lane<T>::V step_a(const Iter<T>& A, int j, int64_t b0) {
  if (A.a_cb) return vload(A.a_cb + (size_t)j * A.Bp + b0);
  if (A.a_b) return vload(A.a_b + b0);
  return vsplat<T>(A.a_c ? A.a_c[j] : A.a);
}
template <typename T>
__device__ __forceinline__ typename Lane<T>::V step_delta(const Iter<T>& A, int j, int64_t b0) {
  if (A.d_cb) return vload(A.d_cb + (size_t)j * A.Bp + b0);
  if (A.d_b) return vload(A.d_b + b0);
  return vsplat<T>(A.d_c ? A.d_c[j] : A.delta);
}
template <typename T>
__device__ __forceinline__ typename Lane<T>::V step_theta(const Iter<T>& A, int64_t b0) {
  return A.th_b ? vload(A.th_b + b0) : vsplat<T>(A.theta);
}

// ---------------------------------------------------------------------------
// row pass: d <- P(d + sigma (K ybar - r)) for samples not yet done
// ---------------------------------------------------------------------------
template <typename T, bool MASKED, int LIN = 0>
__global__ __launch_bounds__(kBlock) void k_row_pass(Iter<T> A) {
  if (A.stop && *A.stop >= A.nstop) return;
  using V = typename Lane<T>::V;
  constexpr int S = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int64_t tile;
  int blk0;
  tile_block(tile, blk0);
  const int64_t b0 = (tile * kWave + lane) * S;
  V keep = vsplat<T>(T(0));
  if (MASKED) {
#pragma unroll
    for (int s = 0; s < S; ++s) keep[s] = A.done[b0 + s] ? T(1) : T(0);
  }
  for (int rb = blk0; rb * 4 < A.K.m; rb += gridDim.y) {
    const int i = rb * 4 + wave;
    if (i >= A.K.m) continue;
    const size_t roff = (size_t)i * A.Bp + b0;
    V acc = vsplat<T>(T(0));
    if (LIN == 2) {
      acc = vload(A.KYc + roff);
    } else {
      const int s0 = A.K.rptr[i], s1 = A.K.rptr[i + 1];
      const T* src = LIN ? A.Y : A.YB;
      // unrolled: four independent gathers in flight per wave (rows are short)
#pragma unroll 4
      for (int k = s0; k < s1; ++k) {
        const V x = vload(src + (size_t)A.K.ridx[k] * A.Bp + b0);
        acc += row_coef(A.K, k, b0) * x;
      }
      if (LIN == 1) vstore(A.KYo + roff, acc);
    }
    if (LIN && A.thp != T(0)) acc = (T(1) + A.thp) * acc - A.thp * vload(A.KYp + roff);
    T* dp = A.D + roff;
    const V d = vload(dp);
    const V r = vload(A.R + roff);
    V p = d + step_sigma(A, i, b0) * (acc - r);
    if (i >= A.K.me) {
#pragma unroll
      for (int s = 0; s < S; ++s) p[s] = maxp(p[s], T(0));
    }
    if (MASKED) {
#pragma unroll
      for (int s = 0; s < S; ++s) p[s] = keep[s] != T(0) ? d[s] : p[s];
    }
    vstore(dp, p);
  }
}

// ---------------------------------------------------------------------------
// column pass.  MODE 0: fixed-iteration update; 1: masked update + diagnostic
// partials of (y+, d+); 2: no update, diagnostics of the current (y, d).
// ---------------------------------------------------------------------------
// NT: the per-column streams (y, yhat or q and c, per-sample bounds, and the
// stores of y and ybar) are nontemporal, for problems whose per-iteration
// vectors exceed the caches: the gathered rows of d+ then keep L2 and MALL.
template <typename T, int MODE, int CPW, bool NT = false>
__global__ __launch_bounds__(kBlock) void k_col_pass(Iter<T> A) {
  if (MODE != 2 && A.stop && *A.stop >= A.nstop) return;
  using V = typename Lane<T>::V;
  constexpr int S = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int64_t tile;
  int blk0;
  tile_block(tile, blk0);
  const int64_t b0 = (tile * kWave + lane) * S;
  const T half = T(0.5), zero = T(0);
  // the per-sample schedule advances for every sample (done or not), once per
  // tile: wavefront 0 of the tile's first column block
  if (MODE != 2 && A.sch_next && blk0 == 0 && wave == 0) {
#pragma unroll
    for (int s = 0; s < S; ++s)
      sched_next(A.gam ? A.gam[b0 + s] : T(1), A.tau_b[b0 + s], A.sig_b[b0 + s], A.sch_next,
                 A.Bp, b0 + s);
  }
  V keep = vsplat<T>(T(0));
  if (MODE == 1) {
#pragma unroll
    for (int s = 0; s < S; ++s) keep[s] = A.done[b0 + s] ? T(1) : T(0);
  }
  V primal = vsplat<T>(zero), dualo = vsplat<T>(zero), stat = vsplat<T>(zero),
    bnd = vsplat<T>(zero), fin = vsplat<T>(T(1));
  for (int cb = blk0; cb * 4 * CPW < A.K.n; cb += gridDim.y) {
    for (int c = 0; c < CPW; ++c) {
      const int j = (cb * 4 + wave) * CPW + c;
      if (j >= A.K.n) break;
      const int s0 = A.K.cptr[j], s1 = A.K.cptr[j + 1];
      V t = vsplat<T>(zero);
      for (int k = s0; k < s1; ++k) {
        const V dd = vload(A.D + (size_t)A.K.cidx[k] * A.Bp + b0);
        t += col_coef(A.K, k, b0) * dd;
      }
      const size_t off = (size_t)j * A.Bp + b0;
      const V y = vload_s<NT>(A.Y + off);
      V tg, qv, cv;  // projection: yhat; general QP: q and c
      if (A.Q) {
        qv = vload_s<NT>(A.Q + off);
        cv = vload_s<NT>(A.Cc + off);
      } else {
        tg = vload_s<NT>(A.tgt + off);
      }
      V lo, hi;
      if (A.shared_bounds) {
        lo = vsplat<T>(A.LO[j]);
        hi = vsplat<T>(A.HI[j]);
      } else {
        lo = vload_s<NT>(A.LO + off);
        hi = vload_s<NT>(A.HI + off);
      }
      V yn;
      if (MODE == 2) {
        yn = y;
        if (A.TK) vstore(A.TK + off, t);  // for the multiplier recovery (post.hpp)
      } else {
        V sv;
        if (A.Q) {
          const V tau = A.tau_cb ? vload(A.tau_cb + off) : vload(A.tau_b + b0);
#pragma unroll
          for (int s = 0; s < S; ++s) {
            const T aj = T(1) / (T(1) + tau[s] * qv[s]);
            if (A.factored) {
              sv[s] = aj * ((y[s] - tau[s] * t[s]) - tau[s] * cv[s]);
            } else {
              const T dj = tau[s] * aj;
              const T oj = -dj * cv[s];
              sv[s] = aj * y[s] - dj * t[s] + oj;
            }
          }
        } else {
          const V aj = step_a(A, j, b0), dj = step_delta(A, j, b0);
          sv = aj * y - dj * t + dj * tg;
        }
#pragma unroll
        for (int s = 0; s < S; ++s) yn[s] = clipp(sv[s], lo[s], hi[s]);
        V yb = yn + step_theta(A, b0) * (yn - y);
        if (MODE == 1) {
          const V yo = y;
          const V ybo = A.lin ? yo : vload(A.YB + off);
#pragma unroll
          for (int s = 0; s < S; ++s) {
            if (keep[s] != zero && !A.nofreeze) {
              yn[s] = yo[s];  // frozen sample: keep state (its diagnostics are unused)
              yb[s] = ybo[s];
            }
          }
        }
        vstore_s<NT>(A.Y + off, yn);
        if (!A.lin) vstore_s<NT>(A.YB + off, yb);  // with lin the row pass forms K ybar
      }
      if (MODE != 0 && A.Q) {
        // diagnostics (kernels.py:158-174, 272-274) with general q, c
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const T yv = yn[s], q = qv[s], c = cv[s];
          primal[s] += half * q * yv * yv + c * yv;
          const T tf = c + t[s];
          const T mz = q > T(1e-12) ? clipp(-tf / q, lo[s], hi[s]) : (tf >= zero ? lo[s] : hi[s]);
          dualo[s] += half * q * (mz * mz) + tf * mz;
          const T g = yv - clipp(yv - ((q * yv + c) + t[s]), lo[s], hi[s]);
          stat[s] = maxp(stat[s], absv(g));
          bnd[s] = maxp(bnd[s], maxp(maxp(lo[s] - yv, zero), maxp(yv - hi[s], zero)));
          if (!finite(yv)) fin[s] = zero;
        }
      } else if (MODE != 0) {
        // diagnostics (kernels.py:158-174, 272-274) with q = 1, c = -yhat
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const T yv = yn[s], c = -tg[s];
          primal[s] += half * yv * yv + c * yv;
          const T tf = c + t[s];
          const T mz = clipp(-tf, lo[s], hi[s]);
          dualo[s] += half * mz * mz + tf * mz;
          const T g = yv - clipp(yv - ((yv + c) + t[s]), lo[s], hi[s]);
          stat[s] = maxp(stat[s], absv(g));
          bnd[s] = maxp(bnd[s], maxp(maxp(lo[s] - yv, zero), maxp(yv - hi[s], zero)));
          if (!finite(yv)) fin[s] = zero;
        }
      }
    }
    if (MODE != 0) {
      __shared__ T buf[kBlock * S];
      const V p0 = block_combine<T>(primal, buf, OpAdd());
      const V p1 = block_combine<T>(dualo, buf, OpAdd());
      const V p2 = block_combine<T>(stat, buf, OpMax());
      const V p3 = block_combine<T>(bnd, buf, OpMax());
      const V p4 = block_combine<T>(fin, buf, OpMin());
      if (wave == 0) {
        const size_t plane = (size_t)A.ncb * A.Bp;
        T* base = A.colpart + (size_t)cb * A.Bp + b0;
        vstore(base, p0);
        vstore(base + plane, p1);
        vstore(base + 2 * plane, p2);
        vstore(base + 3 * plane, p3);
        vstore(base + 4 * plane, p4);
      }
      primal = dualo = stat = bnd = vsplat<T>(zero);
      fin = vsplat<T>(T(1));
    }
  }
}

// ---------------------------------------------------------------------------
// Column pass of the fixed-iteration loop with a quarter wavefront per column:
// a batch tile is 16 lanes x S samples (32 in fp64), so the slice of d+ that a
// tile's columns gather, m x 16 S values, is a quarter of k_col_pass's.  With
// 8 such tiles (or a multiple of 8), each XCD walks one tile's columns at a
// time (tile_block), and where the wide tile's slice exceeds an XCD's 4 MB L2
// while the narrow one fits, the gathers hit L2 instead of re-reading d+ from
// beyond it.  The streams (y, yhat, bounds, y and ybar stores) are 256-byte
// runs per quarter wavefront.  Same arithmetic, in the same order, as
// k_col_pass<MODE 0> (bit-identical results); the plain projection only (no
// QP terms, no per-sample schedule advance).
// ---------------------------------------------------------------------------
template <typename T, bool NT, int P = 16>
__global__ __launch_bounds__(kBlock) void k_col_pass_q(Iter<T> A) {
  if (A.stop && *A.stop >= A.nstop) return;
  using V = typename Lane<T>::V;
  constexpr int S = Lane<T>::S;
  constexpr int CW = kWave / P;  // columns per wavefront
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int64_t tile;
  int blk0;
  tile_block(tile, blk0);
  const int64_t b0 = (tile * P + lane % P) * S;
  const int q = lane / P;
  for (int cb = blk0; cb * 4 * CW < A.K.n; cb += gridDim.y) {
    const int j = (cb * 4 + wave) * CW + q;
    if (j >= A.K.n) break;
    const int s0 = A.K.cptr[j], s1 = A.K.cptr[j + 1];
    V t = vsplat<T>(T(0));
    for (int k = s0; k < s1; ++k) {
      const V dd = vload(A.D + (size_t)A.K.cidx[k] * A.Bp + b0);
      t += col_coef(A.K, k, b0) * dd;
    }
    const size_t off = (size_t)j * A.Bp + b0;
    const V y = vload_s<NT>(A.Y + off);
    const V tg = vload_s<NT>(A.tgt + off);
    V lo, hi;
    if (A.shared_bounds) {
      lo = vsplat<T>(A.LO[j]);
      hi = vsplat<T>(A.HI[j]);
    } else {
      lo = vload_s<NT>(A.LO + off);
      hi = vload_s<NT>(A.HI + off);
    }
    const V aj = step_a(A, j, b0), dj = step_delta(A, j, b0);
    const V sv = aj * y - dj * t + dj * tg;
    V yn;
#pragma unroll
    for (int s = 0; s < S; ++s) yn[s] = clipp(sv[s], lo[s], hi[s]);
    const V yb = yn + step_theta(A, b0) * (yn - y);
    vstore_s<NT>(A.Y + off, yn);
    if (!A.lin) vstore_s<NT>(A.YB + off, yb);
  }
}

// ---------------------------------------------------------------------------
// residual pass: per kept row r = K y - rhs -> |r| (eq) / max(r,0) (ineq);
// r.d and finite(d) for the dual objective and the finiteness test.
// ---------------------------------------------------------------------------
template <typename T, int RPW>
__global__ __launch_bounds__(kBlock) void k_res_pass(Iter<T> A) {
  if (A.stop && *A.stop >= A.nstop) return;
  using V = typename Lane<T>::V;
  constexpr int S = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int64_t tile;
  int blk0;
  tile_block(tile, blk0);
  const int64_t b0 = (tile * kWave + lane) * S;
  const T zero = T(0);
  for (int rb = blk0; rb * 4 * RPW < A.K.m; rb += gridDim.y) {
    V res = vsplat<T>(zero), rd = vsplat<T>(zero), fin = vsplat<T>(T(1));
    for (int c = 0; c < RPW; ++c) {
      const int i = (rb * 4 + wave) * RPW + c;
      if (i >= A.K.m) break;
      const int s0 = A.K.rptr[i], s1 = A.K.rptr[i + 1];
      V acc = vsplat<T>(zero);
#pragma unroll 4
      for (int k = s0; k < s1; ++k)
        acc += row_coef(A.K, k, b0) * vload(A.Y + (size_t)A.K.ridx[k] * A.Bp + b0);
      const size_t off = (size_t)i * A.Bp + b0;
      if (A.KYo)  // K~y+ for the next row pass (lin), or for the multiplier recovery
        vstore(A.KYo + (A.kyrow ? (size_t)A.kyrow[i] * A.Bp + b0 : off), acc);
      const V r = vload(A.R + off);
      const V d = vload(A.D + off);
      const V e = acc - r;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const T v = i < A.K.me ? absv(e[s]) : maxp(e[s], zero);
        res[s] = maxp(res[s], v);
        rd[s] += r[s] * d[s];
        if (!finite(d[s])) fin[s] = zero;
      }
    }
    __shared__ T buf[kBlock * S];
    const V p0 = block_combine<T>(res, buf, OpMax());
    const V p1 = block_combine<T>(rd, buf, OpAdd());
    const V p2 = block_combine<T>(fin, buf, OpMin());
    if (wave == 0) {
      const size_t plane = (size_t)A.nrb * A.Bp;
      T* base = A.rowpart + (size_t)rb * A.Bp + b0;
      vstore(base, p0);
      vstore(base + plane, p1);
      vstore(base + 2 * plane, p2);
    }
  }
}

// Per-sample reduction of the partials, the stop test and the freeze
// (kernels.py:260-278) or, when FINAL, the final convergence verdict
// (kernels.py:291-305).  A block of kDecideGroups x 64 threads owns 64
// samples: group g reduces the column chunks c = g, g + G, ... and the row
// chunks likewise, in increasing order; the groups then combine in LDS in
// group order.  Grid: Bp / 64 blocks.
//
// PRE (small batches, few blocks): a first pass of (Bp / 64) x kDecideSplit
// blocks folds, per sample, the chunks c = y, y + P, y + 2P, ... (y =
// blockIdx.y, P = gridDim.y) the same way and writes the P partials in the
// chunk-partial layout ([5][P][Bp] column totals, then [3][P][Bp] row totals
// at ``pre``); the decision pass then folds those P chunks.
constexpr int kDecideGroups = 16;
constexpr int kDecideSplit = 16;

template <typename T, bool FINAL, bool PRE = false>
__global__ __launch_bounds__(64 * kDecideGroups) void k_decide(
    Iter<T> A, int64_t batch, T tol_scalar, const T* __restrict__ tolv, int32_t* done,
    int32_t* count, int32_t* ndone, const int32_t* feasible, T* out_res, T* out_gap,
    int32_t* out_conv, int32_t* out_fin, T* pre = nullptr) {
  if (!FINAL && A.stop && *A.stop >= A.nstop) return;
  constexpr int G = kDecideGroups;
  __shared__ T buf[G][64];
  const int lane = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int64_t b = (int64_t)blockIdx.x * 64 + lane;  // < Bp by the grid
  const T zero = T(0);
  const size_t cplane = (size_t)A.ncb * A.Bp, rplane = (size_t)A.nrb * A.Bp;
  // this block's chunk subsequence: chunk c0 + cs * c for c < nc (nr for rows)
  const int cs = PRE ? (int)gridDim.y : 1, c0 = PRE ? (int)blockIdx.y : 0;
  const int nc = PRE ? (A.ncb > c0 ? (A.ncb - c0 + cs - 1) / cs : 0) : A.ncb;
  const int nr = PRE ? (A.nrb > c0 ? (A.nrb - c0 + cs - 1) / cs : 0) : A.nrb;
  T q[8] = {zero, zero, zero, zero, T(1), zero, zero, T(1)};  // primal, dual, stat, bnd, fin, res, rd, fin_d
  // Chunks c = g, g + G, ... in increasing order.  The loads of U chunks are
  // issued before they are folded in (a chain of dependent waits otherwise:
  // a small batch has few lanes and many chunks per lane); the order of the
  // folds is unchanged.
  constexpr int U = 8;
  int c = g;
  for (; c + (U - 1) * G < nc; c += U * G) {
    T v[5][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const T* p = A.colpart + (size_t)(c0 + cs * (c + u * G)) * A.Bp + b;
#pragma unroll
      for (int k = 0; k < 5; ++k) v[k][u] = p[k * cplane];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      q[0] += v[0][u];
      q[1] += v[1][u];
      q[2] = maxp(q[2], v[2][u]);
      q[3] = maxp(q[3], v[3][u]);
      if (v[4][u] == zero) q[4] = zero;
    }
  }
  for (; c < nc; c += G) {
    const T* p = A.colpart + (size_t)(c0 + cs * c) * A.Bp + b;
    q[0] += p[0];
    q[1] += p[cplane];
    q[2] = maxp(q[2], p[2 * cplane]);
    q[3] = maxp(q[3], p[3 * cplane]);
    if (p[4 * cplane] == zero) q[4] = zero;
  }
  int r = g;
  for (; r + (U - 1) * G < nr; r += U * G) {
    T v[3][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const T* p = A.rowpart + (size_t)(c0 + cs * (r + u * G)) * A.Bp + b;
#pragma unroll
      for (int k = 0; k < 3; ++k) v[k][u] = p[k * rplane];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      q[5] = maxp(q[5], v[0][u]);
      q[6] += v[1][u];
      if (v[2][u] == zero) q[7] = zero;
    }
  }
  for (; r < nr; r += G) {
    const T* p = A.rowpart + (size_t)(c0 + cs * r) * A.Bp + b;
    q[5] = maxp(q[5], p[0]);
    q[6] += p[rplane];
    if (p[2 * rplane] == zero) q[7] = zero;
  }
  // combine the groups in order 0, 1, ..., G-1 (sum for 0, 1, 6; max for 2, 3, 5; and for 4, 7)
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    buf[g][lane] = q[k];
    __syncthreads();
    if (g == 0) {
      T v = buf[0][lane];
      for (int h = 1; h < G; ++h) {
        const T o = buf[h][lane];
        if (k == 0 || k == 1 || k == 6) v += o;
        else if (k == 2 || k == 3 || k == 5) v = maxp(v, o);
        else v = (v != zero && o != zero) ? T(1) : zero;
      }
      q[k] = v;
    }
    __syncthreads();
  }
  if (PRE) {
    if (g == 0) {
      const size_t P = gridDim.y, Bp = (size_t)A.Bp, y = blockIdx.y;
#pragma unroll
      for (int k = 0; k < 5; ++k) pre[((size_t)k * P + y) * Bp + b] = q[k];
#pragma unroll
      for (int k = 0; k < 3; ++k) pre[((size_t)(5 + k) * P + y) * Bp + b] = q[5 + k];
    }
    return;
  }
  if (g != 0 || b >= batch) return;
  if (!FINAL && done[b]) {
    if (A.nofreeze) count[b] += 1;  // accepted samples keep iterating (and counting)
    return;
  }
  const T tol = tolv ? tolv[b] : tol_scalar;
  const T primal = q[0], dualo = q[1], stat = q[2], bnd = q[3], res = q[5], rd = q[6];
  const bool fin = q[4] != zero, fin_d = q[7] != zero;
  const T dual_obj = dualo - rd;
  const T gap = maxp(primal - dual_obj, zero) /
                maxp(T(1), maxp(absv(primal), absv(dual_obj)));
  const T residual = maxp(res, bnd);
  if (!FINAL) {
    count[b] += 1;
    const bool ok = fin && fin_d && finite(gap) && residual <= tol && gap <= tol &&
                    (A.nostat || stat <= tol);
    if (ok) {
      done[b] = 1;
      atomicAdd(ndone, 1);
    }
  } else {
    const bool f = fin && fin_d && finite(gap) && finite(residual);
    const bool conv = f && residual <= tol && gap <= tol && (A.nostat || stat <= tol) &&
                      (feasible == nullptr || feasible[b] != 0);
    out_res[b] = A.nostat ? residual : maxp(residual, stat);
    out_gap[b] = gap;
    out_conv[b] = conv ? 1 : 0;
    out_fin[b] = f ? 1 : 0;
  }
}

// ---------------------------------------------------------------------------
// layout conversion
// ---------------------------------------------------------------------------
// dst[c * Bp + b] = src[b * ld + c] (times/divided by colmul[c]); zero padding
// for b >= B.  mode: 0 copy, 1 multiply, 2 divide.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_to_minor(const T* __restrict__ src, int64_t B,
                                                      int64_t C, int64_t ld, T* __restrict__ dst,
                                                      int64_t Bp, const T* __restrict__ colmul,
                                                      int mode) {
  __shared__ T tile[64][65];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t c0 = (int64_t)blockIdx.x * 64, b0 = (int64_t)blockIdx.y * 64;
  const int64_t c = c0 + tx;
  // the thread's 16 loads are issued together (unrolled; unguarded in a tile
  // inside the batch and the columns)
  T v[16];
  if (b0 + 64 <= B && c0 + 64 <= C) {
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = src[(b0 + ty + 4 * k) * ld + c];
    if (mode != 0) {
      const T f = colmul[c];
#pragma unroll
      for (int k = 0; k < 16; ++k) v[k] = mode == 1 ? v[k] * f : v[k] / f;
    }
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int64_t b = b0 + ty + 4 * k;
      v[k] = T(0);
      if (b < B && c < C) {
        v[k] = src[b * ld + c];
        if (mode == 1) v[k] = v[k] * colmul[c];
        else if (mode == 2) v[k] = v[k] / colmul[c];
      }
    }
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) tile[ty + 4 * k][tx] = v[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int r = ty + 4 * k;
    const int64_t cc = c0 + r, b = b0 + tx;
    if (cc < C && b < Bp) dst[cc * Bp + b] = tile[tx][r];
  }
}

// dst[b * ld + c] = src[c * Bp + b] (times/divided by colmul[c]) for b < B.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_to_major(const T* __restrict__ src, int64_t Bp,
                                                      int64_t C, T* __restrict__ dst, int64_t B,
                                                      int64_t ld, const T* __restrict__ colmul,
                                                      int mode) {
  __shared__ T tile[64][65];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t c0 = (int64_t)blockIdx.x * 64, b0 = (int64_t)blockIdx.y * 64;
  const int64_t b = b0 + tx;
  // the thread's 16 loads are issued together (unrolled; unguarded in a tile
  // inside the batch and the columns)
  T v[16];
  if (b0 + 64 <= B && c0 + 64 <= C) {
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = src[(c0 + ty + 4 * k) * Bp + b];
    if (mode != 0) {
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const T f = colmul[c0 + ty + 4 * k];
        v[k] = mode == 1 ? v[k] * f : v[k] / f;
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int64_t c = c0 + ty + 4 * k;
      v[k] = T(0);
      if (c < C && b < B) {
        v[k] = src[c * Bp + b];
        if (mode == 1) v[k] = v[k] * colmul[c];
        else if (mode == 2) v[k] = v[k] / colmul[c];
      }
    }
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) tile[ty + 4 * k][tx] = v[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int64_t bb = b0 + ty + 4 * k, c = c0 + tx;
    if (bb < B && c < C) dst[bb * ld + c] = tile[tx][ty + 4 * k];
  }
}

template <typename T>
__global__ void k_fill(T* p, int64_t count, T v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

// Kept-row data from the full rows: R[i] = RF[kept[i]] * scale_i and
// D[i] = MF[kept[i]] / scale_i (bounds.py:230-239).
template <typename T>
__global__ void k_prep_rows(int m, int64_t Bp, const int32_t* __restrict__ kept,
                            const T* __restrict__ scale, const T* __restrict__ scale_b,
                            const T* __restrict__ RF, const T* __restrict__ MF,
                            T* __restrict__ R, T* __restrict__ D) {
  const int64_t total = (int64_t)m * Bp;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / Bp, b = e - i * Bp;
    const int64_t src = (int64_t)kept[i] * Bp + b;
    const T sc = scale_b ? scale_b[e] : scale[i];  // per-sample scales: [m][Bp]
    R[e] = RF[src] * sc;
    if (D) D[e] = MF ? MF[src] / sc : T(0);
  }
}

// Variable bounds from singleton inequality rows (bounds.py:193-209).
// ``cols`` samples per variable: Bp (per-sample) or 1 (shared bounds, sample 0).
template <typename T>
__global__ void k_prep_bounds(int n, int64_t Bp, int64_t cols, const int32_t* __restrict__ bptr,
                              const int32_t* __restrict__ brow, const T* __restrict__ bcoef,
                              const T* __restrict__ bcoef_b, const T* __restrict__ RF,
                              T* __restrict__ LO, T* __restrict__ HI, int32_t* feasible,
                              int64_t batch) {
  const int64_t total = (int64_t)n * cols;
  const T inf = __builtin_inf();
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t j = e / cols, b = e - j * cols;
    T lo = -inf, hi = inf;
    bool ok = true;
    for (int k = bptr[j]; k < bptr[j + 1]; ++k) {
      const T c = bcoef_b ? bcoef_b[(int64_t)k * Bp + b] : bcoef[k];  // per-sample: [nb][Bp]
      const T rr = RF[(int64_t)brow[k] * Bp + b];
      const T th = rr / (c != T(0) ? c : T(1));
      if (c < T(0)) lo = maxp(lo, th);
      if (c > T(0)) hi = minp(hi, th);
      if (!(c != T(0) || rr >= T(0))) ok = false;
    }
    if (!(lo <= hi)) ok = false;
    LO[e] = lo;
    HI[e] = hi;
    if (!ok) {
      if (cols == 1) {
        for (int64_t s = 0; s < batch; ++s) feasible[s] = 0;
      } else if (b < batch) {
        feasible[b] = 0;
      }
    }
  }
}

// Plain products for the first-kernel entry point: out = K x (rows) or K^T x
// (columns), one row/column per wave.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_spmv_rows(Mat<T> K, int64_t Bp, const T* __restrict__ X,
                                                       T* __restrict__ out) {
#pragma clang fp contract(off)  // rounded products, the oracle's and the host's order
  using V = typename Lane<T>::V;
  constexpr int S = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b0 = ((int64_t)blockIdx.x * kWave + lane) * S;
  for (int rb = blockIdx.y; rb * 4 < K.m; rb += gridDim.y) {
    const int i = rb * 4 + wave;
    if (i >= K.m) continue;
    V acc = vsplat<T>(T(0));
    for (int k = K.rptr[i]; k < K.rptr[i + 1]; ++k)
      acc += row_coef(K, k, b0) * vload(X + (size_t)K.ridx[k] * Bp + b0);
    vstore(out + (size_t)i * Bp + b0, acc);
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_spmv_cols(Mat<T> K, int64_t Bp, const T* __restrict__ X,
                                                       T* __restrict__ out) {
#pragma clang fp contract(off)  // rounded products, the oracle's and the host's order
  using V = typename Lane<T>::V;
  constexpr int S = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b0 = ((int64_t)blockIdx.x * kWave + lane) * S;
  for (int cb = blockIdx.y; cb * 4 < K.n; cb += gridDim.y) {
    const int j = cb * 4 + wave;
    if (j >= K.n) continue;
    V acc = vsplat<T>(T(0));
    for (int k = K.cptr[j]; k < K.cptr[j + 1]; ++k)
      acc += col_coef(K, k, b0) * vload(X + (size_t)K.cidx[k] * Bp + b0);
    vstore(out + (size_t)j * Bp + b0, acc);
  }
}

template <typename T>
__global__ void k_write_header(int64_t* hdr, int64_t batch, int64_t Bp, int64_t kind,
                               int64_t shared, int64_t dtype, int64_t n, int64_t m, int64_t M) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    hdr[0] = 0x5055524e43503031LL;
    hdr[1] = batch;
    hdr[2] = Bp;
    hdr[3] = kind;
    hdr[4] = shared;
    hdr[5] = dtype;
    hdr[6] = n;
    hdr[7] = m;
    hdr[8] = M;
  }
}

template <typename T>
__global__ void k_finish_solve(int64_t batch, const int32_t* __restrict__ count,
                               const T* __restrict__ ores, const T* __restrict__ ogap,
                               const int32_t* __restrict__ oconv, int32_t* iterations, T* residual,
                               T* gap, uint8_t* converged) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  if (iterations) iterations[b] = count[b];
  if (residual) residual[b] = ores[b];
  if (gap) gap[b] = ogap[b];
  if (converged) converged[b] = oconv[b] ? 1 : 0;
}

// *snap = *src (one word): the accepted count at the start of an iteration
static __global__ void k_snap(const int32_t* __restrict__ src, int32_t* snap) {
  if (threadIdx.x == 0) *snap = *src;
}

template <typename T>
__global__ void k_init_flags(int64_t batch, int64_t Bp, int32_t* done, int32_t* count,
                             int32_t* feasible, const uint8_t* __restrict__ feas_in,
                             int32_t* ndone) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b == 0) *ndone = 0;
  if (b >= Bp) return;
  done[b] = b < batch ? 0 : 1;
  count[b] = 0;
  feasible[b] = b < batch ? (feas_in ? (feas_in[b] ? 1 : 0) : 1) : 0;
}

}  // namespace purin
