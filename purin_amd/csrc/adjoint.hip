// Implicit VJP through the CP fixed point on the device.
//
// Reference: custom_vjp ``bwd`` (src/purin/solvers/chambolle_pock/bounds.py:80-165)
// and _batched_restarted_gmres
// (src/purin/solvers/primal_dual_interior_point/operators.py:792-1125).
//
// The state z = (y, d, ybar) of width W = 2n + m is stored batch-minor with
// rows [0,n) = y, [n,n+m) = d, [n+m,2n+m) = ybar.  One cp_step (theta = 1,
// fixed-step prox from the power-iteration steps) is linearised once at the
// saved state into masks C (clip, per variable) and D (dual projection, per
// row); its transpose Jacobian is then one K u (row pass) and one K^T w
// (column pass):
//   G = gy + 2 gb,  u = C G,  w = D (gd - delta K u),
//   pullback(gy, gd, gb) = (a u - gb, w, sigma K^T w),
//   g_rhs = -sigma w, g_target = delta u, g_lower = Clo G, g_upper = Chi G.
// GMRES solves (I - J^T) lambda = [cot_y * converged, 0, 0] with the
// reference's restart cycles, two-pass classical Gram--Schmidt, Givens
// rotations, per-sample active masks and candidate acceptance.  The basis is
// kept raw (vectors Z with an upper-triangular map to the orthonormal ones,
// see k_gm_tri), so each Arnoldi step makes two passes over it: a read-only
// dot pass and one update-and-dot pass that writes the next raw vector.  The
// per-sample scalars (chunk sums, triangular products, Givens rotations,
// back-substitution) run on the device.

#include <algorithm>
#include <cmath>
#include <vector>

#include "forward.hpp"
#include "kernels.hpp"
#include "plan.hpp"
#include "persample.hpp"

namespace purin {

constexpr int kChunk = 64;        // rows per Gram--Schmidt block
constexpr int kRowsPerThread = kChunk / 4;
constexpr int kMaxRestart = 128;    // restart cap (Hessenberg workspace grows as restart^2)
constexpr int kStepCheck = 8;       // Arnoldi steps between host reads of the active count

template <typename T>
struct Adj {
  Mat<T> K;  // scaled kept rows
  int64_t Bp;
  int n, m;
  T a, delta, sigma;
  // diagonal steps (bounds.py:83-86): per-column a, delta and per-row sigma
  // replace the scalars when set.  The VJP's delta K u and sigma K^T w then
  // read K (delta . u) and K^T (sigma . w): U and Wv hold the scaled vectors.
  const T* a_c;    // n or nullptr
  const T* d_c;    // n or nullptr
  const T* sig_r;  // m or nullptr
  // per-sample steps (per-sample coefficients): [Bp] scalars per sample, or
  // with diagonal steps [n][Bp] / [m][Bp]; nullptr when shared
  const T* a_b;
  const T* d_b;
  const T* sig_b;
  const T* a_cb;
  const T* d_cb;
  const T* sig_rb;
  int dg;        // 1: U and Wv hold delta . u and sigma . w (any non-scalar step)
  // general diagonal QP (diagonal_qp.py:131-219): q, c [n][Bp]; the prox
  // a = 1/(1 + tau q), delta = tau a is formed from tau per sample (tau_b) or
  // per variable (tau_cb); Spre keeps the pre-clip value for the q gradient
  const T* Q;
  const T* Cc;
  const T* tau_b;
  const T* tau_cb;
  T* Spre;
  int factored;  // the dense adapter's prox arithmetic a ((y - tau t) - tau c)
  const T* vsc;  // [Bp] per-sample scale of the operator's input, or nullptr
  int64_t ldv;   // row stride of the operator's input and output (Bp, or a basis slot's)
  const T* Cm;   // n x Bp
  const T* Dm;   // m x Bp
  T* U;          // n x Bp scratch (u)
  T* Wv;         // m x Bp scratch (w)
};

// Steps of column j / row i for sample b (shared, diagonal, per-sample or
// per-sample diagonal).
template <typename T>
__device__ __forceinline__ T adj_tau(const Adj<T>& S, int64_t j, int64_t b) {
  return S.tau_cb ? S.tau_cb[j * S.Bp + b] : S.tau_b[b];
}
template <typename T>
__device__ __forceinline__ T adj_a(const Adj<T>& S, int64_t j, int64_t b) {
  if (S.Q) return T(1) / (T(1) + adj_tau(S, j, b) * S.Q[j * S.Bp + b]);
  if (S.a_cb) return S.a_cb[j * S.Bp + b];
  if (S.a_b) return S.a_b[b];
  return S.a_c ? S.a_c[j] : S.a;
}
template <typename T>
__device__ __forceinline__ T adj_d(const Adj<T>& S, int64_t j, int64_t b) {
  if (S.Q) return adj_tau(S, j, b) * adj_a(S, j, b);
  if (S.d_cb) return S.d_cb[j * S.Bp + b];
  if (S.d_b) return S.d_b[b];
  return S.d_c ? S.d_c[j] : S.delta;
}
template <typename T>
__device__ __forceinline__ T adj_sig(const Adj<T>& S, int64_t i, int64_t b) {
  if (S.sig_rb) return S.sig_rb[i * S.Bp + b];
  if (S.sig_b) return S.sig_b[b];
  return S.sig_r ? S.sig_r[i] : S.sigma;
}

// sigma of row i for the S samples from b0 (adj_sig as one vector: the
// per-sample arrays hold a lane's samples contiguously)
template <typename T>
__device__ __forceinline__ typename Lane<T>::V adj_sig_v(const Adj<T>& S, int64_t i, int64_t b0) {
  if (S.sig_rb) return vload(S.sig_rb + (size_t)i * S.Bp + b0);
  if (S.sig_b) return vload(S.sig_b + b0);
  return vsplat<T>(S.sig_r ? S.sig_r[i] : S.sigma);
}

// d/dx of max(x, y) and min(x, y) with JAX's balanced tie rule.
template <typename T>
__device__ __forceinline__ T dmax_dx(T x, T y) {
  const T ans = maxp(x, y);
  return x == ans ? (y == ans ? T(0.5) : T(1)) : T(0);
}
template <typename T>
__device__ __forceinline__ T dmin_dx(T x, T y) {
  const T ans = minp(x, y);
  return x == ans ? (y == ans ? T(0.5) : T(1)) : T(0);
}

// ---------------------------------------------------------------------------
// linearisation at z = (y, d, y): D mask and d+ (rows), then C/Clo/Chi (cols)
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kBlock) void k_lin_rows(Adj<T> S, const T* __restrict__ Y,
                                                     const T* __restrict__ Dd,
                                                     const T* __restrict__ R, T* Dm, T* dplus) {
  using V = typename Lane<T>::V;
  constexpr int Sn = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b0 = ((int64_t)blockIdx.x * kWave + lane) * Sn;
  for (int rb = blockIdx.y; rb * 4 < S.m; rb += gridDim.y) {
    const int i = rb * 4 + wave;
    if (i >= S.m) continue;
    V acc = vsplat<T>(T(0));
    for (int k = S.K.rptr[i]; k < S.K.rptr[i + 1]; ++k)
      acc += row_coef(S.K, k, b0) * vload(Y + (size_t)S.K.ridx[k] * S.Bp + b0);
    const size_t off = (size_t)i * S.Bp + b0;
    const V sg = adj_sig_v(S, i, b0);
    const V p = vload(Dd + off) + sg * (acc - vload(R + off));
    V dm, dp;
#pragma unroll
    for (int s = 0; s < Sn; ++s) {
      if (i < S.K.me) {
        dm[s] = T(1);
        dp[s] = p[s];
      } else {
        dm[s] = dmax_dx(p[s], T(0));
        dp[s] = maxp(p[s], T(0));
      }
    }
    vstore(Dm + off, dm);
    vstore(dplus + off, dp);
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_lin_cols(Adj<T> S, const T* __restrict__ Y,
                                                     const T* __restrict__ tgt,
                                                     const T* __restrict__ LO,
                                                     const T* __restrict__ HI, int shared_bounds,
                                                     const T* __restrict__ dplus, T* Cm, T* Clo,
                                                     T* Chi) {
  using V = typename Lane<T>::V;
  constexpr int Sn = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b0 = ((int64_t)blockIdx.x * kWave + lane) * Sn;
  for (int cb = blockIdx.y; cb * 4 < S.n; cb += gridDim.y) {
    const int j = cb * 4 + wave;
    if (j >= S.n) continue;
    V t = vsplat<T>(T(0));
    for (int k = S.K.cptr[j]; k < S.K.cptr[j + 1]; ++k)
      t += col_coef(S.K, k, b0) * vload(dplus + (size_t)S.K.cidx[k] * S.Bp + b0);
    const size_t off = (size_t)j * S.Bp + b0;
    const V y = vload(Y + off);
    V aj, dj;
#pragma unroll
    for (int q = 0; q < Sn; ++q) {
      aj[q] = adj_a(S, j, b0 + q);
      dj[q] = adj_d(S, j, b0 + q);
    }
    V s;
    if (S.Q) {  // offset -delta c (kernels.py:68-73), or the factored form (140-142)
      const V cv = vload(S.Cc + off);
#pragma unroll
      for (int q = 0; q < Sn; ++q) {
        if (S.factored) {
          const T tau = adj_tau(S, j, b0 + q);
          s[q] = aj[q] * ((y[q] - tau * t[q]) - tau * cv[q]);
        } else {
          s[q] = aj[q] * y[q] - dj[q] * t[q] + (-dj[q] * cv[q]);
        }
      }
      vstore(S.Spre + off, s);
    } else {
      s = aj * y - dj * t + dj * vload(tgt + off);
    }
    V lo, hi;
    if (shared_bounds) {
      lo = vsplat<T>(LO[j]);
      hi = vsplat<T>(HI[j]);
    } else {
      lo = vload(LO + off);
      hi = vload(HI + off);
    }
    V c, cl, ch;
#pragma unroll
    for (int q = 0; q < Sn; ++q) {
      // clip = minimum(maximum(s, lo), hi)
      const T m1 = maxp(s[q], lo[q]);
      const T dm1 = dmin_dx(m1, hi[q]);
      c[q] = dm1 * dmax_dx(s[q], lo[q]);
      cl[q] = dm1 * dmax_dx(lo[q], s[q]);
      ch[q] = dmin_dx(hi[q], m1);
    }
    vstore(Cm + off, c);
    vstore(Clo + off, cl);
    vstore(Chi + off, ch);
  }
}

// ---------------------------------------------------------------------------
// operator out = v - pullback(v) in three passes; v and out are W x Bp.  The
// input, the masks and the output are streamed nontemporally, so that the
// prefix rows the last Gram--Schmidt pass read stay in the MALL for the next
// dot pass (which starts on them); u and w, gathered, stay cacheable.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kBlock) void k_op_cols1(Adj<T> S, const T* __restrict__ v,
                                                     T* __restrict__ out) {
  using V = typename Lane<T>::V;
  constexpr int Sn = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b0 = ((int64_t)blockIdx.x * kWave + lane) * Sn;
  const V sc = S.vsc ? vload(S.vsc + b0) : vsplat<T>(T(1));
  for (int cb = blockIdx.y; cb * 4 < S.n; cb += gridDim.y) {
    const int j = cb * 4 + wave;
    if (j >= S.n) continue;
    const size_t off = (size_t)j * S.Bp + b0;
    const size_t voff = (size_t)j * S.ldv + b0;
    const size_t boff = (size_t)(S.n + S.m + j) * S.ldv + b0;
    V gy = vload_once(v + voff), gb = vload_once(v + boff);
    if (S.vsc) {
      gy = gy * sc;
      gb = gb * sc;
    }
    const V u = vload_once(S.Cm + off) * (gy + T(2) * gb);
    if (S.dg) {
      V du, o;
#pragma unroll
      for (int s = 0; s < Sn; ++s) {
        du[s] = adj_d(S, j, b0 + s) * u[s];
        o[s] = gy[s] - (adj_a(S, j, b0 + s) * u[s] - gb[s]);
      }
      vstore(S.U + off, du);
      vstore_once(out + voff, o);
    } else {
      vstore(S.U + off, u);
      vstore_once(out + voff, gy - (S.a * u - gb));
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_op_rows(Adj<T> S, const T* __restrict__ v,
                                                    T* __restrict__ out) {
  using V = typename Lane<T>::V;
  constexpr int Sn = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b0 = ((int64_t)blockIdx.x * kWave + lane) * Sn;
  for (int rb = blockIdx.y; rb * 4 < S.m; rb += gridDim.y) {
    const int i = rb * 4 + wave;
    if (i >= S.m) continue;
    V acc = vsplat<T>(T(0));
#pragma unroll 4
    for (int k = S.K.rptr[i]; k < S.K.rptr[i + 1]; ++k)
      acc += row_coef(S.K, k, b0) * vload(S.U + (size_t)S.K.ridx[k] * S.Bp + b0);
    const size_t off = (size_t)i * S.Bp + b0;
    const size_t voff = (size_t)(S.n + i) * S.ldv + b0;
    V gd = vload_once(v + voff);
    if (S.vsc) gd = gd * vload(S.vsc + b0);
    if (S.dg) {
      const V w = vload_once(S.Dm + off) * (gd - acc);
      const V sg = adj_sig_v(S, i, b0);
      vstore(S.Wv + off, sg * w);
      vstore_once(out + voff, gd - w);
    } else {
      const V w = vload_once(S.Dm + off) * (gd - S.delta * acc);
      vstore(S.Wv + off, w);
      vstore_once(out + voff, gd - w);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_op_cols2(Adj<T> S, const T* __restrict__ v,
                                                     T* __restrict__ out) {
  using V = typename Lane<T>::V;
  constexpr int Sn = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b0 = ((int64_t)blockIdx.x * kWave + lane) * Sn;
  for (int cb = blockIdx.y; cb * 4 < S.n; cb += gridDim.y) {
    const int j = cb * 4 + wave;
    if (j >= S.n) continue;
    V acc = vsplat<T>(T(0));
#pragma unroll 4
    for (int k = S.K.cptr[j]; k < S.K.cptr[j + 1]; ++k)
      acc += col_coef(S.K, k, b0) * vload(S.Wv + (size_t)S.K.cidx[k] * S.Bp + b0);
    const size_t off = (size_t)(S.n + S.m + j) * S.ldv + b0;
    V gb = vload_once(v + off);
    if (S.vsc) gb = gb * vload(S.vsc + b0);
    if (S.dg)
      vstore_once(out + off, gb - acc);
    else
      vstore_once(out + off, gb - S.sigma * acc);
  }
}

// ---------------------------------------------------------------------------
// batched reductions over the W rows of a state vector
// ---------------------------------------------------------------------------
// MODE 0: part[i][c][b] = sum_rows V_i x                       (dots)
// MODE 1: x <- x - sum_i h_i V_i;  part[i][c][b] = sum V_i x   (update + dots)
// MODE 2: x <- x - sum_i h_i V_i;  part[0] = sum x^2, part[1] = finite(x)
// MODE 3: part[0] = sum x^2                                    (norm)
// MODE 4: part[0] = max |x|                                    (inf-norm)
// MODE 5: MODE 1, and part[nv] = sum x^2
template <typename T, int MODE>
__global__ __launch_bounds__(kBlock) void k_gs(const T* __restrict__ basis, int64_t vstride,
                                               int nv, T* x, const T* __restrict__ h,
                                               int64_t W, int64_t Bp, T* part, int nchunk,
                                               int64_t ld) {
  using V = typename Lane<T>::V;
  constexpr int Sn = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t b0 = ((int64_t)blockIdx.x * kWave + lane) * Sn;
  const int c = blockIdx.y;
  const int64_t r0 = (int64_t)c * kChunk + wave * kRowsPerThread;
  __shared__ T buf[kBlock * Sn];
  V xr[kRowsPerThread];
#pragma unroll
  for (int r = 0; r < kRowsPerThread; ++r)
    xr[r] = (r0 + r < W) ? vload(x + (size_t)(r0 + r) * ld + b0) : vsplat<T>(T(0));
  if (MODE == 1 || MODE == 2 || MODE == 5) {
    for (int i = 0; i < nv; ++i) {
      const V hi = vload(h + (size_t)i * Bp + b0);
      const T* vi = basis + (size_t)i * vstride;
#pragma unroll
      for (int r = 0; r < kRowsPerThread; ++r)
        if (r0 + r < W) xr[r] = xr[r] - hi * vload(vi + (size_t)(r0 + r) * ld + b0);
    }
#pragma unroll
    for (int r = 0; r < kRowsPerThread; ++r)
      if (r0 + r < W) vstore(x + (size_t)(r0 + r) * ld + b0, xr[r]);
  }
  const size_t plane = (size_t)nchunk * Bp;
  if (MODE == 0 || MODE == 1 || MODE == 5) {
    for (int i = 0; i < nv; ++i) {
      const T* vi = basis + (size_t)i * vstride;
      V acc = vsplat<T>(T(0));
#pragma unroll
      for (int r = 0; r < kRowsPerThread; ++r)
        if (r0 + r < W) acc += vload(vi + (size_t)(r0 + r) * ld + b0) * xr[r];
      const V tot = block_combine<T>(acc, buf, OpAdd());
      if (wave == 0) vstore(part + (size_t)i * plane + (size_t)c * Bp + b0, tot);
    }
    if (MODE == 5) {
      V acc = vsplat<T>(T(0));
#pragma unroll
      for (int r = 0; r < kRowsPerThread; ++r) acc += xr[r] * xr[r];
      const V tot = block_combine<T>(acc, buf, OpAdd());
      if (wave == 0) vstore(part + (size_t)nv * plane + (size_t)c * Bp + b0, tot);
    }
  } else if (MODE == 2 || MODE == 3) {
    V acc = vsplat<T>(T(0)), fin = vsplat<T>(T(1));
#pragma unroll
    for (int r = 0; r < kRowsPerThread; ++r) {
      acc += xr[r] * xr[r];
#pragma unroll
      for (int s = 0; s < Sn; ++s)
        if (!finite(xr[r][s])) fin[s] = T(0);
    }
    const V tot = block_combine<T>(acc, buf, OpAdd());
    const V f = block_combine<T>(fin, buf, OpMin());
    if (wave == 0) {
      vstore(part + (size_t)c * Bp + b0, tot);
      if (MODE == 2) vstore(part + plane + (size_t)c * Bp + b0, f);
    }
  } else {
    V acc = vsplat<T>(T(0));
#pragma unroll
    for (int r = 0; r < kRowsPerThread; ++r)
#pragma unroll
      for (int s = 0; s < Sn; ++s) acc[s] = maxp(acc[s], absv(xr[r][s]));
    const V tot = block_combine<T>(acc, buf, OpMax());
    if (wave == 0) vstore(part + (size_t)c * Bp + b0, tot);
  }
}

// out[i][b] = reduce_c part[i][c][b] in chunk order; op 0 = sum, 1 = max, 2 = min
template <typename T>
__global__ void k_reduce(const T* __restrict__ part, int nv, int nchunk, int64_t Bp, T* out,
                         int op) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (int64_t)nv * Bp) return;
  const int64_t i = e / Bp, b = e - i * Bp;
  const T* p = part + (size_t)i * nchunk * Bp + b;
  T acc = p[0];
  for (int c = 1; c < nchunk; ++c) {
    const T v = p[(size_t)c * Bp];
    acc = op == 0 ? acc + v : (op == 1 ? maxp(acc, v) : minp(acc, v));
  }
  out[e] = acc;
}

// ---------------------------------------------------------------------------
// The dot pass part_i = V_i . x for a short prefix (nv <= NV <= 8), split by
// rows: a block of 4 wavefronts owns one batch tile (64 lanes x 16 bytes of
// samples) and a contiguous range of ``rpb`` rows, and each wavefront walks a
// quarter of it.  Per row a lane loads x and the prefix vectors' entries of the
// same row (coalesced 1 KB wavefront accesses, nv of them in flight per row).
// The dot products accumulate in registers and are combined across the 4
// wavefronts once, at the end (wave 0 + 1 + 2 + 3), into part[i][chunk][b].
// ---------------------------------------------------------------------------
template <typename T, int NV>
__global__ __launch_bounds__(kBlock) void k_gs_dots_rows(const T* __restrict__ basis,
                                                         int64_t vstride, int nv,
                                                         const T* __restrict__ x, int64_t W,
                                                         int64_t Bp, T* part, int nchunk,
                                                         int64_t rpb, int64_t ld) {
  using V = typename Lane<T>::V;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b0 = ((int64_t)blockIdx.x * kWave + lane) * Lane<T>::S;
  const int c = blockIdx.y;
  __shared__ V cb[3][kWave];
  const int64_t rpw = (rpb + 3) / 4;
  const int64_t r_begin = (int64_t)c * rpb + wave * rpw;
  const int64_t r_end = std::min<int64_t>(W, std::min<int64_t>((int64_t)(c + 1) * rpb, r_begin + rpw));
  V acc[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) acc[i] = V(T(0));
  for (int64_t r = r_begin; r < r_end; ++r) {
    const size_t off = (size_t)r * ld + b0;
    const V xr = vload(x + off);
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (i < nv) acc[i] += vload(basis + (size_t)i * vstride + off) * xr;
  }
  const size_t plane = (size_t)nchunk * Bp;
  const size_t pout = (size_t)c * Bp + b0;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (i >= nv) continue;
    V v = acc[i];
    if (wave > 0) cb[wave - 1][lane] = v;
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int w = 0; w < 3; ++w) v += cb[w][lane];
      vstore(part + (size_t)i * plane + pout, v);
    }
    __syncthreads();
  }
}

// The first Gram--Schmidt pass, part_i = V_i . x, with the prefix vectors split
// across the block's 4 wavefronts: wavefront w owns V_i for i = w, w+4, ... and
// walks all rows of the block's chunk, loading x itself (the four loads of a
// row hit L2 together).  Each wavefront writes the partial sums of its own
// vectors, so there is no cross-wavefront combine; every load is a coalesced
// 1 KB wavefront access.
template <typename T, int NV>
__global__ __launch_bounds__(kBlock) void k_gs_dots(const T* __restrict__ basis, int64_t vstride,
                                                    int nv, const T* __restrict__ x, int64_t W,
                                                    int64_t Bp, T* part, int nchunk, int64_t rpb, int64_t ld) {
  using V = typename Lane<T>::V;
  constexpr int Sn = Lane<T>::S;
  constexpr int NW = NV / 4;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b0 = ((int64_t)blockIdx.x * kWave + lane) * Sn;
  const int c = blockIdx.y;
  // every load is issued unconditionally (a vector index past the prefix is
  // clamped to the last vector, an L2 hit) so all NW loads of a row are in
  // flight together; the accumulation is masked instead
  const T* vp[NW];
  bool own[NW];
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    own[j] = wave + 4 * j < nv;
    vp[j] = basis + (size_t)std::min(wave + 4 * j, nv - 1) * vstride;
  }
  V acc[NW];
#pragma unroll
  for (int j = 0; j < NW; ++j) acc[j] = vsplat<T>(T(0));
  const int64_t r_begin = (int64_t)c * rpb;
  const int64_t r_end = std::min<int64_t>(W, r_begin + rpb);
  // rows last to first: the update-and-dot pass that follows walks the same
  // chunks first to last, so it starts on the rows read last here, which the
  // MALL still holds
  for (int64_t r = r_end - 1; r >= r_begin; --r) {
    const size_t off = (size_t)r * ld + b0;
    const V xr = vload(x + off);
    V v[NW];
#pragma unroll
    for (int j = 0; j < NW; ++j) v[j] = vload(vp[j] + off);
    __builtin_amdgcn_sched_barrier(0);  // issue all loads of the row before any FMA
#pragma unroll
    for (int j = 0; j < NW; ++j)
      if (own[j]) acc[j] += v[j] * xr;
  }
  const size_t plane = (size_t)nchunk * Bp;
#pragma unroll
  for (int j = 0; j < NW; ++j)
    if (own[j]) vstore(part + (size_t)(wave + 4 * j) * plane + (size_t)c * Bp + b0, acc[j]);
}

// The second Gram--Schmidt pass (x <- x - sum_i h_i V_i, then part_i = V_i . x
// for i < nv and part_nv = x . x)
// with the prefix vectors split across the block's 4 wavefronts instead of
// the rows: wavefront w holds V_i for i = w, w+4, ... of two rows at a time
// (at most NV/4 per wavefront, so registers stay low), forms its share of
// sum_i h_i V_i, and the 4 shares meet in LDS (one barrier per 2 rows, double
// buffered).  Every wavefront then has the updated rows and dots them with
// the prefix entries it already holds: V is read from HBM once.  Each
// wavefront owns the dot products of its own vectors, so the partials need no
// cross-wavefront combine.  Shares are summed in wavefront order 0+1+2+3.
template <typename T, int NV>
__global__ __launch_bounds__(kBlock) void k_gs_update_dots(const T* __restrict__ basis,
                                                           int64_t vstride, int nv, T* x,
                                                           const T* __restrict__ h, int64_t W,
                                                           int64_t Bp, T* part, int nchunk,
                                                           int64_t rpb, int64_t ld) {
  using V = typename Lane<T>::V;
  constexpr int Sn = Lane<T>::S;
  constexpr int NW = NV / 4;  // vectors per wavefront
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b0 = ((int64_t)blockIdx.x * kWave + lane) * Sn;
  const int c = blockIdx.y;
  __shared__ V share[2][4][2][kWave];
  V hw[NW], acc[NW], nrm = vsplat<T>(T(0));
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    const int i = wave + 4 * j;
    hw[j] = i < nv ? vload(h + (size_t)i * Bp + b0) : vsplat<T>(T(0));
    acc[j] = vsplat<T>(T(0));
  }
  const int64_t r_begin = (int64_t)c * rpb;
  const int64_t r_end = std::min<int64_t>(W, r_begin + rpb);
  int g = 0;
  for (int64_t r = r_begin; r < r_end; r += 2, ++g) {
    const bool two = r + 1 < r_end;
    const size_t off0 = (size_t)r * ld + b0, off1 = off0 + (size_t)ld;
    const V x0 = vload(x + off0);
    const V x1 = two ? vload(x + off1) : vsplat<T>(T(0));
    V v0[NW], v1[NW];
    V p0 = vsplat<T>(T(0)), p1 = vsplat<T>(T(0));
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      const int i = wave + 4 * j;
      v0[j] = vsplat<T>(T(0));
      v1[j] = vsplat<T>(T(0));
      if (i < nv) {
        v0[j] = vload(basis + (size_t)i * vstride + off0);
        if (two) v1[j] = vload(basis + (size_t)i * vstride + off1);
      }
      p0 += hw[j] * v0[j];
      p1 += hw[j] * v1[j];
    }
    share[g & 1][wave][0][lane] = p0;
    share[g & 1][wave][1][lane] = p1;
    __syncthreads();
    const V s0 = ((share[g & 1][0][0][lane] + share[g & 1][1][0][lane]) + share[g & 1][2][0][lane]) +
                 share[g & 1][3][0][lane];
    const V s1 = ((share[g & 1][0][1][lane] + share[g & 1][1][1][lane]) + share[g & 1][2][1][lane]) +
                 share[g & 1][3][1][lane];
    const V y0 = x0 - s0, y1 = x1 - s1;
    if (wave == 0) {
      vstore(x + off0, y0);
      nrm += y0 * y0;
      if (two) {
        vstore(x + off1, y1);
        nrm += y1 * y1;
      }
    }
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      acc[j] += v0[j] * y0;
      acc[j] += v1[j] * y1;
    }
  }
  const size_t plane = (size_t)nchunk * Bp;
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    const int i = wave + 4 * j;
    if (i < nv) vstore(part + (size_t)i * plane + (size_t)c * Bp + b0, acc[j]);
  }
  if (wave == 0) vstore(part + (size_t)nv * plane + (size_t)c * Bp + b0, nrm);
}

// elementwise helpers on W x Bp vectors
template <typename T>
__global__ void k_axpby(int64_t total, T* out, const T* __restrict__ a, const T* __restrict__ b,
                        T beta) {  // out = a + beta * b
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x)
    out[e] = a[e] + beta * b[e];
}

// V0 = r / max(beta, eps) per sample
template <typename T>
__global__ void k_scale_cols(int64_t total, int64_t Bp, T* out, int64_t ldo,
                             const T* __restrict__ in, const T* __restrict__ scale) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = e / Bp, b = e - row * Bp;
    out[row * ldo + b] = in[e] * scale[b];
  }
}

// x += sum_{i < row_steps[b]} coeff_i V_i, with V_i at basis + i * vstride and
// row stride ld
template <typename T>
__global__ void k_correction(int64_t total, int64_t Bp, T* x, const T* __restrict__ basis,
                             int64_t vstride, int64_t ld, const T* __restrict__ coeff,
                             const int32_t* __restrict__ steps) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = e / Bp, b = e - row * Bp;
    const int k = steps[b];
    if (k == 0) continue;
    const T* vr = basis + row * ld + b;
    T acc = T(0);
    for (int i = 0; i < k; ++i) acc += coeff[(size_t)i * Bp + b] * vr[(size_t)i * vstride];
    x[e] = x[e] + acc;
  }
}

// ---------------------------------------------------------------------------
// per-sample GMRES scalars (operators.py:820-821, 873-917, 996-1091)
// ---------------------------------------------------------------------------
template <typename T>
struct Gm {
  int64_t batch, Bp;
  int restart;
  T* thr;        // threshold
  T* rinf;       // residual_inf
  int32_t* cyc;  // cycle_active
  int32_t* act;  // active
  int32_t* steps;
  T* scale;
  T* H;          // [(restart+1)][restart][Bp]: H[i][j] of sample b at (i*restart + j)*Bp + b
  T* cs;         // [restart][Bp]
  T* sn;
  T* g;          // [(restart+1)][Bp]
  T* coeff;      // [restart][Bp] (back-substitution output)
  int32_t* counter;  // [0] active count at a cycle's start, [1] unconverged count
  int32_t* stepcnt;  // [restart+1]: samples active at the start of Arnoldi step s
  // raw-basis map (k_gm_tri): v_j = sum_{i<=j} Z_i Tm[i][j]
  T* Tm;   // [(restart+1)][(restart+1)][Bp], upper triangular
  T* Hu;   // [(restart+1)][restart][Bp]: the unrotated Hessenberg matrix
  T* U2;   // [restart+1][Bp]: g2 / nu of the last step
  T* G1;   // [restart+1][Bp]: V^T y of the current step
  T* Q1;   // [restart+1][Bp]: Tm G1, the first projection's coefficients on Z
  T* Cg;   // [restart+1][Bp]: the lagged correction c of the current step
  T* Wc;   // [restart][Bp]: Tm coeff, the cycle's correction on Z
  int32_t* total;  // [Bp]: Arnoldi steps over all cycles (operators.py:1092-1097)
};

template <typename T>
__global__ void k_gm_thresholds(Gm<T> G, const T* __restrict__ rhs_inf, T tol, T atol) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= G.Bp) return;
  G.thr[b] = maxp(atol, tol * rhs_inf[b]);
  G.rinf[b] = rhs_inf[b];  // x0 = 0: rhs - matvec(0) = rhs
}

template <typename T>
__global__ void k_gm_count_unconverged(Gm<T> G) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b < G.batch && G.rinf[b] > G.thr[b]) atomicAdd(&G.counter[1], 1);
}

template <typename T>
__global__ void k_gm_cycle_init(Gm<T> G, const T* __restrict__ beta2) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= G.Bp) return;
  const int R = G.restart;
  const T eps = T(1e-30);
  const T beta = __builtin_sqrt(beta2[b]);
  G.scale[b] = T(1) / maxp(beta, eps);
  const int c = (b < G.batch && G.rinf[b] > G.thr[b]) ? 1 : 0;
  G.cyc[b] = c;
  G.act[b] = c;
  G.steps[b] = 0;
  for (int i = 0; i < R; ++i) {
    G.cs[(size_t)i * G.Bp + b] = T(0);
    G.sn[(size_t)i * G.Bp + b] = T(0);
  }
  for (int i = 0; i <= R; ++i) G.g[(size_t)i * G.Bp + b] = i == 0 ? beta : T(0);
  for (int i = 0; i < (R + 1) * R; ++i) G.H[(size_t)i * G.Bp + b] = T(0);
  G.Tm[b] = T(1);  // Z_0 = r / beta is stored normalised
  if (c) atomicAdd(&G.stepcnt[0], 1);
}

// One Arnoldi step's per-sample algebra on the raw basis (operators.py:834-871,
// 996-1081).
//
// Basis slot i holds a raw vector Z_i.  The orthonormal Arnoldi vectors are
// v_j = sum_{i<=j} Z_i Tm[i][j], with Tm upper triangular: Z_0 = v_0, and
// Z_{j+1} is the image of step j after one projection, so the off-diagonal
// entries of Tm are of the order of the rounding error.  Step ``it`` applies
// the operator to Z_it Tm[it][it], giving y, and then runs
//   pass A   p = Z^T y                                  (reads the prefix)
//   MODE 1   g1 = Tm^T p (= V^T y),  q1 = Tm g1         (V g1 = Z q1)
//   pass B   y1 = y - Z q1 stored as Z_{it+1},  p2 = Z^T y1,  |y1|^2
//   MODE 2   g2 = Tm^T p2 (= V^T y1), the Hessenberg column, the Givens
//            step, and column it+1 of Tm: v_{it+1} = (y1 - V g2) / nu.
// This is the reference's two-pass classical Gram--Schmidt: the image is
// projected on the prefix twice, each time with dot products taken against
// the vector being corrected.  The second subtraction is carried by Tm
// instead of a third pass over the basis, and the operator reads the raw
// vector, so
//  * Z_it Tm[it][it] = v_it + V u with u = g2 / nu of step it - 1, and
//    A V = V Hu (Hu: the unrotated Hessenberg matrix), give
//    A v_it = y - V c with c = Hu[0..it][0..it-1] u;
//  * the column is h = g1 + g2 - c, and h[it+1] = |y1 - V g2| =
//    sqrt(|y1|^2 - |g2|^2), as y1 - V g2 is orthogonal to V;
//  * the rotations, the stop test (residual estimate, finiteness, happy
//    breakdown at 1e-14) and the masking by the step's active flag are the
//    reference's.  Tm's new column is zero for a sample inactive at the
//    step's start, as the reference keeps a zero basis vector there.
// A block of 16 wavefronts owns kTriS = 16 samples: lane l of a wavefront
// serves sample l mod 16 as worker 4 w + l / 16 (64 workers per sample).  The
// chunk sums split each plane's chunks into 4 interleaved quarters summed in
// chunk order and combined as (q0 + q1) + (q2 + q3); the workers then split
// the outputs of the triangular products, and one lane per sample runs the
// Givens step from LDS.  LDS (dynamic, (5R + 4) * kTriS elements): the reduced
// planes P[R+2], the coefficients Gv[R+1], the Hessenberg column Col[R+1] and
// the rotations Cs[R], Sn[R], each over the block's samples.
constexpr int kTriS = 16;

template <typename T, int MODE>
__global__ __launch_bounds__(1024) void k_gm_tri(Gm<T> G, int it, const T* __restrict__ part,
                                                 int nchunk) {
  extern __shared__ __align__(16) unsigned char tri_raw[];
  const int R = G.restart, R1 = R + 1;
  T* P = reinterpret_cast<T*>(tri_raw);  // [R + 2][kTriS]
  T* Gv = P + (size_t)(R + 2) * kTriS;   // [R + 1][kTriS]
  T* Col = Gv + (size_t)(R + 1) * kTriS; // [R + 1][kTriS]
  T* Cs = Col + (size_t)(R + 1) * kTriS; // [R][kTriS]
  T* Sn = Cs + (size_t)R * kTriS;        // [R][kTriS]
  __shared__ T s_inv[kTriS];
  __shared__ int s_keep[kTriS];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sl = lane & (kTriS - 1), q = lane >> 4;
  const int worker = wave * 4 + q;
  const int64_t Bp = G.Bp;
  const int64_t b = (int64_t)blockIdx.x * kTriS + sl;
  const int nv = it + 1;
  const int planes = MODE == 1 ? nv : nv + 1;
  const size_t plane = (size_t)nchunk * Bp;
  for (int i = wave; i < planes; i += 16) {
    const T* pp = part + (size_t)i * plane + b;
    T acc = T(0);
#pragma unroll 8
    for (int c = q; c < nchunk; c += 4) acc += pp[(size_t)c * Bp];
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    if (q == 0) P[i * kTriS + sl] = acc;
  }
  __syncthreads();
  const T* Tm = G.Tm + b;
  const size_t tcol = (size_t)Bp, trow = (size_t)R1 * Bp;  // Tm[i][j] at i * trow + j * tcol
  const int active = MODE == 2 ? G.act[b] : 0;
  for (int j = worker; j < nv; j += 64) {
    T acc = T(0);
#pragma unroll 8
    for (int i = 0; i <= j; ++i) acc += Tm[i * trow + j * tcol] * P[i * kTriS + sl];
    Gv[j * kTriS + sl] = acc;
    if (MODE == 1) {
      G.G1[(size_t)j * Bp + b] = acc;
    } else {
      // c_j = sum_k Hu[j][k] u_k, k in [max(j - 1, 0), it - 1] (Hu is upper Hessenberg)
      T cj = T(0);
#pragma unroll 8
      for (int k = j > 0 ? j - 1 : 0; k < it; ++k)
        cj += G.Hu[((size_t)j * R + k) * Bp + b] * G.U2[(size_t)k * Bp + b];
      const T col = (G.G1[(size_t)j * Bp + b] + acc) - cj;
      Col[j * kTriS + sl] = col;
      if (active) G.Hu[((size_t)j * R + it) * Bp + b] = col;
    }
  }
  if (MODE == 2) {
    for (int j = worker; j < it; j += 64) {
      Cs[j * kTriS + sl] = G.cs[(size_t)j * Bp + b];
      Sn[j * kTriS + sl] = G.sn[(size_t)j * Bp + b];
    }
  }
  __syncthreads();
  if (MODE == 1) {
    for (int i = worker; i < nv; i += 64) {
      T acc = T(0);
#pragma unroll 8
      for (int j = i; j < nv; ++j) acc += Tm[i * trow + j * tcol] * Gv[j * kTriS + sl];
      G.Q1[(size_t)i * Bp + b] = acc;
    }
    return;
  }
  if (worker == 0) {
    const T eps = T(1e-30), brk = T(1e-14);
    T ss = T(0);
    for (int j = 0; j < nv; ++j) ss += Gv[j * kTriS + sl] * Gv[j * kTriS + sl];
    const T n1 = P[nv * kTriS + sl];
    const T d2 = n1 - ss;
    const T next_norm = d2 < T(0) ? T(0) : __builtin_sqrt(d2);  // NaN stays NaN
    T carry = Col[sl];
    for (int ri = 0; ri < it; ++ri) {
      const T c = Cs[ri * kTriS + sl], s = Sn[ri * kTriS + sl];
      const T f = carry, sc = Col[(ri + 1) * kTriS + sl];
      if (active) G.H[((size_t)ri * R + it) * Bp + b] = c * f + s * sc;
      carry = -s * f + c * sc;
    }
    const T diag = carry, sub = next_norm;
    const T rnorm = hypotv(diag, sub);
    const T safe = maxp(rnorm, eps);
    const T nc = rnorm > eps ? diag / safe : T(1);
    const T ns = rnorm > eps ? sub / safe : T(0);
    const T pc = G.g[(size_t)it * Bp + b], pn = G.g[(size_t)(it + 1) * Bp + b];
    const T rc = nc * pc + ns * pn;
    const T rn = -ns * pc + nc * pn;
    const T inv = T(1) / maxp(next_norm, eps);
    if (active) {
      G.Hu[((size_t)(it + 1) * R + it) * Bp + b] = next_norm;
      G.cs[(size_t)it * Bp + b] = nc;
      G.sn[(size_t)it * Bp + b] = ns;
      G.H[((size_t)it * R + it) * Bp + b] = rnorm;
      G.H[((size_t)(it + 1) * R + it) * Bp + b] = T(0);
      G.g[(size_t)it * Bp + b] = rc;
      G.g[(size_t)(it + 1) * Bp + b] = rn;
      G.steps[b] = it + 1;
    }
    const T est = absv(rn);
    // |y1|^2 is finite exactly when y1, and hence (y1 - V g2) / nu, is
    const bool finite_ok = finite(est) && finite(rnorm) && finite(n1);
    const bool happy = next_norm <= brk;
    const int still = (active && finite_ok && !happy && est > G.thr[b]) ? 1 : 0;
    G.act[b] = still;
    G.Tm[(size_t)(it + 1) * trow + (size_t)(it + 1) * tcol + b] = active ? inv : T(0);
    s_inv[sl] = inv;
    s_keep[sl] = active;
    if (still && b < G.batch) atomicAdd(&G.stepcnt[it + 1], 1);
  }
  __syncthreads();
  // column it + 1 of Tm: v_{it+1} = (Z_{it+1} - Z Tm g2) / nu, and u = g2 / nu
  const T inv = s_inv[sl];
  const bool keep = s_keep[sl] != 0;
  for (int i = worker; i < nv; i += 64) {
    T acc = T(0);
#pragma unroll 8
    for (int j = i; j < nv; ++j) acc += Tm[i * trow + j * tcol] * Gv[j * kTriS + sl];
    G.Tm[(size_t)i * trow + (size_t)(it + 1) * tcol + b] = keep ? -(acc * inv) : T(0);
    G.U2[(size_t)i * Bp + b] = keep ? Gv[i * kTriS + sl] * inv : T(0);
  }
}

// The cycle's correction on the raw basis: x += sum_{j < steps} coeff_j v_j =
// sum_i Z_i Wc_i with Wc_i = sum_{i <= j < steps} Tm[i][j] coeff_j.
template <typename T>
__global__ void k_gm_tcoef(Gm<T> G) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int i = blockIdx.y;
  if (b >= G.Bp) return;
  const int steps = G.steps[b];
  const size_t trow = (size_t)(G.restart + 1) * G.Bp;
  T acc = T(0);
#pragma unroll 8
  for (int j = i; j < steps; ++j) acc += G.Tm[i * trow + (size_t)j * G.Bp + b] * G.coeff[(size_t)j * G.Bp + b];
  G.Wc[(size_t)i * G.Bp + b] = acc;
}

// Back substitution (operators.py:902-917), one thread per sample in blocks of
// 64; the partial solution stays in LDS (restart x 64 entries, dynamic), and
// the zero entries of the trailing sum (columns at or left of the row and
// beyond the sample's steps) are skipped.
template <typename T>
__global__ __launch_bounds__(64) void k_gm_backsub(Gm<T> G) {
  extern __shared__ __align__(16) unsigned char bs_raw[];
  T* val = reinterpret_cast<T*>(bs_raw);  // [restart][64]
  const int t = threadIdx.x;
  const int64_t b = (int64_t)blockIdx.x * 64 + t;
  if (b >= G.Bp) return;
  const int R = G.restart;
  const int64_t Bp = G.Bp;
  const T eps = T(1e-30);
  const int steps = G.steps[b];
  for (int row = R - 1; row >= 0; --row) {
    T v = T(0);
    if (row < steps) {
      T trailing = T(0);
#pragma unroll 8
      for (int c = row + 1; c < steps; ++c)
        trailing += G.H[((size_t)row * R + c) * Bp + b] * val[c * 64 + t];
      const T num = G.g[(size_t)row * Bp + b] - trailing;
      const T d = G.H[((size_t)row * R + row) * Bp + b];
      const T safe = absv(d) > eps ? d : T(1);
      v = num / safe;
    }
    val[row * 64 + t] = v;
    G.coeff[(size_t)row * Bp + b] = v;
  }
}

template <typename T>
__global__ void k_gm_cycle_end(Gm<T> G, const T* __restrict__ cand_inf) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= G.Bp) return;
  if (G.cyc[b]) G.rinf[b] = cand_inf[b];
  G.total[b] += G.steps[b];  // total_row_iterations + row_steps (0 when inactive)
}

// info / valid (operators.py:1119-1122, bounds.py:148-153) and the masked
// cotangent weight for the final pullback.
template <typename T>
__global__ void k_gm_finish(Gm<T> G, const T* __restrict__ xfin, const int32_t* __restrict__ conv,
                            T adjoint_tol, int force, T* lam_w, uint8_t* valid, int32_t* info,
                            T* residual) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= G.Bp) return;
  const bool fin = xfin[b] != T(0) && finite(G.rinf[b]);
  const int code = !fin ? 2 : (G.rinf[b] <= G.thr[b] ? 0 : 1);
  const bool eligible = b < G.batch && (force || conv[b] != 0);
  const bool ok = eligible && fin && (code == 0 || G.rinf[b] <= adjoint_tol);
  lam_w[b] = ok ? T(1) : T(0);
  if (b < G.batch) {
    if (valid) valid[b] = ok ? 1 : 0;
    if (info) info[b] = code;
    if (residual) residual[b] = G.rinf[b];
  }
}

// rhs g = [cot_y * eligible, 0, 0]; cot arrives batch-minor in ``cot``
// With cotd (the general QP's dual cotangent, diagonal_qp.py:197-200), the
// rows n..n+m of g are cotd * eligible.
template <typename T>
__global__ void k_gm_rhs(int64_t n, int64_t m, int64_t W, int64_t Bp, int64_t batch,
                         const T* __restrict__ cot, const T* __restrict__ cotd,
                         const int32_t* __restrict__ conv, int force, T* g) {
  const int64_t total = W * Bp;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = e / Bp, b = e - row * Bp;
    const bool elig = b < batch && (force || conv[b] != 0);
    T v = T(0);
    if (row < n)
      v = cot[e];
    else if (cotd && row < n + m)
      v = cotd[e - n * Bp];
    g[e] = elig ? v : T(0);
  }
}

// Final pullback of lambda (masked by lam_w): outputs in internal layout, with
// non-finite values replaced by zero (bounds.py:154-165).
// General QP: gt receives g_c = -delta u and gq g_q = -tau a u s, with s the
// pre-clip value (d s / d q = -tau a s for a = 1/(1 + tau q), delta = tau a).
template <typename T>
__global__ void k_final_u(Adj<T> S, const T* __restrict__ lam, const T* __restrict__ lam_w,
                          const T* __restrict__ Clo, const T* __restrict__ Chi, T* gt, T* glo,
                          T* ghi, T* gq) {
  const int64_t total = (int64_t)S.n * S.Bp;
  const int64_t boff = (int64_t)(S.n + S.m) * S.Bp;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = e % S.Bp;
    const T w = lam_w[b];
    const T gy = w != T(0) ? lam[e] : T(0), gb = w != T(0) ? lam[boff + e] : T(0);
    const T G = gy + T(2) * gb;
    const T u = S.Cm[e] * G;
    const T a = adj_d(S, e / S.Bp, b) * u, l = Clo[e] * G, h = Chi[e] * G;
    S.U[e] = S.dg ? a : u;
    if (S.Q) {
      const int64_t j = e / S.Bp;
      if (gq) {
        const T g = -(adj_tau(S, j, b) * adj_a(S, j, b) * u * S.Spre[e]);
        gq[e] = finite(g) ? g : T(0);
      }
      gt[e] = finite(a) ? -a : T(0);
    } else {
      gt[e] = finite(a) ? a : T(0);
    }
    glo[e] = finite(l) ? l : T(0);
    ghi[e] = finite(h) ? h : T(0);
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_final_w(Adj<T> S, const T* __restrict__ lam,
                                                    const T* __restrict__ lam_w, T* gr,
                                                    T* sw) {
  using V = typename Lane<T>::V;
  constexpr int Sn = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b0 = ((int64_t)blockIdx.x * kWave + lane) * Sn;
  for (int rb = blockIdx.y; rb * 4 < S.m; rb += gridDim.y) {
    const int i = rb * 4 + wave;
    if (i >= S.m) continue;
    V acc = vsplat<T>(T(0));
    for (int k = S.K.rptr[i]; k < S.K.rptr[i + 1]; ++k)
      acc += row_coef(S.K, k, b0) * vload(S.U + (size_t)S.K.ridx[k] * S.Bp + b0);
    const size_t off = (size_t)i * S.Bp + b0;
    const V gd = vload(lam + (size_t)(S.n + i) * S.Bp + b0);
    const V sg = adj_sig_v(S, i, b0);
    V out, swv;
#pragma unroll
    for (int s = 0; s < Sn; ++s) {
      const T lw = lam_w[b0 + s];
      const T w = S.dg ? S.Dm[off + s] * ((lw != T(0) ? gd[s] : T(0)) - acc[s])
                       : S.Dm[off + s] * ((lw != T(0) ? gd[s] : T(0)) - S.delta * acc[s]);
      const T r = sg[s] * w;
      swv[s] = r;
      out[s] = finite(r) ? -r : T(0);
    }
    vstore(gr + off, out);
    if (sw) vstore(sw + off, swv);
  }
}

// Gradient w.r.t. the coefficients of the kept rows, per sample, in the
// caller's entry order (per-sample coefficients).  The pullback of the scaled
// entry K~_ij = s_i K_ij is g~_ij = (sigma w)_i ybar_j - d+_i (delta u)_j
// (the VJP of cp_step, bounds.py:109-141), cleaned of non-finite values
// (bounds.py:155).  The row scale s_i = 1/||K_i|| (bounds.py:210-214) and the
// scaled rhs r~_i = s_i r_i chain it to the original entries:
//   g_ij = s_i g~_ij - s_i^3 K_ij (sum_j' g~_ij' K_ij' + g_r~_i r_i),
// the second term only when row scaling is on and ||K_i|| > 1e-30.
// One kept row per wavefront; sw = sigma . w, U = delta . u.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_gvals_rows(
    Mat<T> K, int64_t Bp, const T* __restrict__ sw, const T* __restrict__ Y,
    const T* __restrict__ U, const T* __restrict__ dplus, const T* __restrict__ gr,
    const T* __restrict__ RVo, const T* __restrict__ SC, const T* __restrict__ RF,
    const int32_t* __restrict__ kept, int row_scaling, const int32_t* __restrict__ kcsr,
    T* __restrict__ GVF) {
  using V = typename Lane<T>::V;
  constexpr int Sn = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b0 = ((int64_t)blockIdx.x * kWave + lane) * Sn;
  const T zero = T(0);
  for (int rb = blockIdx.y; rb * 4 < K.m; rb += gridDim.y) {
    const int i = rb * 4 + wave;
    if (i >= K.m) continue;
    const size_t off = (size_t)i * Bp + b0;
    const V swi = vload(sw + off), dpi = vload(dplus + off);
    V gsc = vsplat<T>(zero), sq = vsplat<T>(zero);
    const int s0 = K.rptr[i], s1 = K.rptr[i + 1];
    for (int k = s0; k < s1; ++k) {
      const size_t jo = (size_t)K.ridx[k] * Bp + b0;
      const V g = swi * vload(Y + jo) - dpi * vload(U + jo);
      const V ko = vload(RVo + (size_t)k * Bp + b0);
#pragma unroll
      for (int s = 0; s < Sn; ++s) gsc[s] += (finite(g[s]) ? g[s] : zero) * ko[s];
      sq += ko * ko;
    }
    const V sc = vload(SC + off);
    gsc += vload(gr + off) * vload(RF + (size_t)kept[i] * Bp + b0);
    V c3;
#pragma unroll
    for (int s = 0; s < Sn; ++s)
      c3[s] = (row_scaling && __builtin_sqrt(sq[s]) > T(1e-30)) ? sc[s] * sc[s] * sc[s] * gsc[s]
                                                               : zero;
    for (int k = s0; k < s1; ++k) {
      const size_t jo = (size_t)K.ridx[k] * Bp + b0;
      const V g = swi * vload(Y + jo) - dpi * vload(U + jo);
      const V ko = vload(RVo + (size_t)k * Bp + b0);
      V out;
#pragma unroll
      for (int s = 0; s < Sn; ++s) out[s] = sc[s] * (finite(g[s]) ? g[s] : zero) - c3[s] * ko[s];
      vstore(GVF + (size_t)kcsr[k] * Bp + b0, out);
    }
  }
}

// g_rhs in the full row space for project(): kept rows g_r * scale, bound
// rows through their threshold (ties at a bound split evenly).  With
// per-sample coefficients (scale_b, bcoef_b) the scales and bound
// coefficients are per sample, and the gradient of a bound row's coefficient,
// -g_threshold * rhs / c^2 = -g_rhs * threshold, goes to GVF[bpos[k]].
template <typename T>
__global__ void k_grhs_full(int m, int n, int64_t Bp, const int32_t* __restrict__ kept,
                            const T* __restrict__ scale, const T* __restrict__ scale_b,
                            const T* __restrict__ gr, const int32_t* __restrict__ bptr,
                            const int32_t* __restrict__ brow, const T* __restrict__ bcoef,
                            const T* __restrict__ bcoef_b, const T* __restrict__ RF,
                            const T* __restrict__ LO, const T* __restrict__ HI, int shared_bounds,
                            const T* __restrict__ glo, const T* __restrict__ ghi, T* out,
                            const int32_t* __restrict__ bpos, T* GVF) {
  const int64_t total_rows = out ? (int64_t)m * Bp : 0;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total_rows;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / Bp, b = e - i * Bp;
    out[(int64_t)kept[i] * Bp + b] = gr[e] * (scale_b ? scale_b[e] : scale[i]);
  }
  const int64_t total_cols = (int64_t)n * Bp;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total_cols;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t j = e / Bp, b = e - j * Bp;
    const T lo = shared_bounds ? LO[j] : LO[e];
    const T hi = shared_bounds ? HI[j] : HI[e];
    const int k0 = bptr[j], k1 = bptr[j + 1];
    T nlo = T(0), nhi = T(0);
    for (int k = k0; k < k1; ++k) {
      const T c = bcoef_b ? bcoef_b[(int64_t)k * Bp + b] : bcoef[k];
      const T th = RF[(int64_t)brow[k] * Bp + b] / (c != T(0) ? c : T(1));
      if (c < T(0) && th == lo) nlo += T(1);
      if (c > T(0) && th == hi) nhi += T(1);
    }
    for (int k = k0; k < k1; ++k) {
      const T c = bcoef_b ? bcoef_b[(int64_t)k * Bp + b] : bcoef[k];
      const T th = RF[(int64_t)brow[k] * Bp + b] / (c != T(0) ? c : T(1));
      T gthr = T(0);
      if (c < T(0) && th == lo) gthr += glo[e] / maxp(nlo, T(1));
      if (c > T(0) && th == hi) gthr += ghi[e] / maxp(nhi, T(1));
      const T v = c != T(0) ? gthr / c : gthr;
      if (out) out[(int64_t)brow[k] * Bp + b] = finite(v) ? v : T(0);
      if (GVF) {
        const T gc = c != T(0) ? -v * th : T(0);
        GVF[(int64_t)bpos[k] * Bp + b] = finite(gc) ? gc : T(0);
      }
    }
  }
}

template <typename T>
__global__ void k_copy_i32(int64_t count, const int32_t* __restrict__ src, int32_t* dst) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < count) dst[e] = src[e];
}

static size_t al(size_t x) { return (x + 255) & ~size_t(255); }

// ---------------------------------------------------------------------------
// BiCGSTAB over the whole batch as one vector (the dense layer's
// fixed_point_pullback, src/purin/autodiff/fixed_point.py:8-40, with
// jax.scipy.sparse.linalg.bicgstab of jax 0.6.2: van der Vorst's BiCGSTAB,
// rho = alpha = omega = 1 and rhat = p = q = r0 initially, the early exit
// when |s|^2 < atol2, breakdown codes -10 (rho = 0) and -11 (alpha or
// omega = 0), atol2 = max(tol^2 |b|^2, atol^2)).  Dot products over all
// W x Bp entries (padding is zero) in a fixed two-level order; the scalars
// live in the device array sc[].
// ---------------------------------------------------------------------------
constexpr int kBiBlocks = 1024;
enum BiSlot { kBS = 0, kAtol2, kRho, kAlpha, kOmega, kRho_, kAlpha_, kOmega_, kBeta, kSS, kTS,
              kTT, kRQ, kRS, kK, kSlots };

template <typename T>
__global__ __launch_bounds__(256) void k_bi_dot(const T* __restrict__ x, const T* __restrict__ y,
                                                int64_t total, T* part) {
  __shared__ T buf[256];
  T acc = T(0);
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x)
    acc += x[e] * y[e];
  buf[threadIdx.x] = acc;
  __syncthreads();
  for (int h = 128; h > 0; h >>= 1) {
    if ((int)threadIdx.x < h) buf[threadIdx.x] += buf[threadIdx.x + h];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = buf[0];
}

template <typename T>
__global__ __launch_bounds__(256) void k_bi_sum(const T* __restrict__ part, int np, T* sc,
                                                int slot) {
  __shared__ T buf[256];
  T acc = T(0);
  for (int i = threadIdx.x; i < np; i += blockDim.x) acc += part[i];
  buf[threadIdx.x] = acc;
  __syncthreads();
  for (int h = 128; h > 0; h >>= 1) {
    if ((int)threadIdx.x < h) buf[threadIdx.x] += buf[threadIdx.x + h];
    __syncthreads();
  }
  if (threadIdx.x == 0) sc[slot] = buf[0];
}

// op: 0 start (atol2, rho = alpha = omega = 1, k = 0), 1 beta, 2 alpha_, 3 omega_,
// 4 the iteration's end (k, and rho/alpha/omega <- the new values)
template <typename T>
__global__ void k_bi_scalar(T* sc, int op, T tol, T atol) {
  if (threadIdx.x != 0) return;
  const T one = T(1);
  if (op == 0) {
    sc[kAtol2] = maxp(tol * tol * sc[kBS], atol * atol);
    sc[kRho] = sc[kAlpha] = sc[kOmega] = one;
    sc[kK] = T(0);
  } else if (op == 1) {
    sc[kBeta] = sc[kRho_] / sc[kRho] * sc[kAlpha] / sc[kOmega];
  } else if (op == 2) {
    sc[kAlpha_] = sc[kRho_] / sc[kRQ];
  } else if (op == 3) {
    sc[kOmega_] = sc[kTS] / sc[kTT];
  } else {
    T k = (sc[kOmega_] == T(0) || sc[kAlpha_] == T(0)) ? T(-11) : sc[kK] + one;
    if (sc[kRho_] == T(0)) k = T(-10);
    sc[kK] = k;
    sc[kRho] = sc[kRho_];
    sc[kAlpha] = sc[kAlpha_];
    sc[kOmega] = sc[kOmega_];
  }
}

// mode 0: p = r + beta (p - omega q); 1: s = r - alpha_ q;
// 2: x, r update with the early exit
template <typename T>
__global__ void k_bi_vec(int mode, int64_t total, const T* __restrict__ sc, T* x, T* r, T* p,
                         const T* __restrict__ q, T* s, const T* __restrict__ t) {
  const T beta = sc[kBeta], omega = sc[kOmega], alpha_ = sc[kAlpha_], omega_ = sc[kOmega_];
  const bool early = sc[kSS] < sc[kAtol2];
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    if (mode == 0) {
      p[e] = r[e] + beta * (p[e] - omega * q[e]);
    } else if (mode == 1) {
      s[e] = r[e] - alpha_ * q[e];
    } else if (early) {
      x[e] = x[e] + alpha_ * p[e];
      r[e] = s[e];
    } else {
      x[e] = x[e] + (alpha_ * p[e] + omega_ * s[e]);
      r[e] = s[e] - omega_ * t[e];
    }
  }
}

template <typename T>
__global__ void k_fill_weights(int64_t batch, int64_t Bp, T* w) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b < Bp) w[b] = b < batch ? T(1) : T(0);
}

// Inputs and extra outputs of the general diagonal QP's VJP (diagonal_qp.py:131-219).
template <typename T>
struct QPAdjArgs {
  const T* q;         // (B, n)
  const T* c;         // (B, n)
  const T* cot_dual;  // (B, M) cotangent of the multipliers, or nullptr
  T* g_q;             // (B, n) or nullptr
  int dense;          // the dense layer's backward (dense_implicit.py:198-209):
                      // BiCGSTAB over the batch, frozen prox (no q gradient),
                      // no convergence masking
};

// ``size_only``: compute the workspace bytes of this call into *size_only and
// return, touching neither the device nor the plan (purin_cp_workspace_bytes).
template <typename T>
static int adjoint_impl(purin_cp_plan* p, hipStream_t st, int64_t batch, const void* saved,
                        const T* cot_y, const purin_cp_adjoint_options& o, T* g_target, T* g_rhs,
                        T* g_lower, T* g_upper, uint8_t* valid, int32_t* info, T* gres,
                        const T* values = nullptr, T* g_values = nullptr,
                        bool per_sample = false, const QPAdjArgs<T>* qa = nullptr,
                        int64_t* size_only = nullptr) {
  if (!size_only && (!saved || !cot_y))
    return set_error(PURIN_CP_ERR_ARG, "NULL saved state or cotangent");
  if (!size_only && per_sample && !qa && p->nnz_full && !values)
    return set_error(PURIN_CP_ERR_ARG, "NULL values");
  if (!size_only && qa && (!qa->q || !qa->c)) return set_error(PURIN_CP_ERR_ARG, "NULL q or c");
  if (batch < 1) return set_error(PURIN_CP_ERR_ARG, "batch must be positive");
  if (o.restart < 1 || o.max_iterations < 1)
    return set_error(PURIN_CP_ERR_ARG, "linear iteration limits must be positive");
  if (o.tolerance <= 0.0 || o.atol < 0.0) return set_error(PURIN_CP_ERR_ARG, "linear tolerances are invalid");
  const Layout L = make_layout(p, batch);
  const int64_t Bp = L.Bp, n = p->n, m = p->m, M = p->M;
  const int64_t W = 2 * n + m;
  // the dense layer's BiCGSTAB keeps its five work vectors in the basis slots
  const int restart = (qa && qa->dense)
                          ? 5
                          : (int)std::min<int64_t>({(int64_t)o.restart, (int64_t)o.max_iterations, W});
  if (restart > kMaxRestart) return set_error(PURIN_CP_ERR_UNSUPPORTED, "restart above 128");
  static_assert((kMaxRestart + 2) * 4 <= kPinnedBytes, "per-step counts must fit the pinned buffer");
  const bool dense = qa && qa->dense;
  // workspace
  const int nchunk = (int)((W + kChunk - 1) / kChunk);
  // Gram--Schmidt passes: about 1024 blocks of 4 wavefronts over the batch tiles
  const int64_t TS0 = (int64_t)kWave * Lane<T>::S;
  const int64_t tiles0 = Bp / TS0;
  // at most 8 resident blocks of 4 wavefronts per CU: the partial sums need at
  // most that many chunks per batch tile
  int cus = 0;
  PURIN_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, p->device));
  const int nchunk2 = (int)std::max<int64_t>(
      1, std::min<int64_t>(((int64_t)8 * cus + tiles0 - 1) / tiles0, (W + 3) / 4));
  const size_t es = sizeof(T);
  const size_t vec = (size_t)W * Bp * es;
  size_t o_ = 0;
  auto take = [&](size_t bytes) { size_t r = o_; o_ = al(o_ + bytes); return r; };
  const size_t oV = take(vec * (restart + 1)), oX = take(vec), oG = take(vec), oRr = take(vec),
               oT1 = take(vec), oCm = take(n * Bp * es), oClo = take(n * Bp * es),
               oChi = take(n * Bp * es), oDm = take(m * Bp * es), oDp = take(m * Bp * es),
               oU = take(n * Bp * es), oWv = take(m * Bp * es),
               oPart = take((size_t)(restart + 1) * std::max(nchunk, nchunk2) * Bp * es),
               oS1 = take(Bp * es), oS2 = take(Bp * es), oThr = take(Bp * es), oRinf = take(Bp * es),
               oCyc = take(Bp * 4), oAct = take(Bp * 4), oSteps = take(Bp * 4),
               oScale = take(Bp * es), oHess = take((size_t)Bp * (restart + 1) * restart * es),
               oCs = take((size_t)restart * Bp * es), oSn = take((size_t)restart * Bp * es),
               oGv = take((size_t)(restart + 1) * Bp * es), oCoef = take((size_t)restart * Bp * es),
               oCnt = take(256), oStepCnt = take((size_t)(restart + 2) * 4), oLw = take(Bp * es), oGt = take(n * Bp * es),
               oGlo = take(n * Bp * es), oGhi = take(n * Bp * es), oGr = take(m * Bp * es),
               oGF = take((size_t)M * Bp * es),
               oTm = take((size_t)(restart + 1) * (restart + 1) * Bp * es),
               oHu = take((size_t)(restart + 1) * restart * Bp * es),
               oU2 = take((size_t)(restart + 1) * Bp * es), oG1 = take((size_t)(restart + 1) * Bp * es),
               oQ1 = take((size_t)(restart + 1) * Bp * es), oCg = take((size_t)(restart + 1) * Bp * es),
               oWc = take((size_t)restart * Bp * es), oTot = take(Bp * 4);
  // per-sample coefficients: the forward's per-sample arrays are rebuilt from
  // values in a region laid out like the forward workspace, plus sigma . w and
  // the coefficient gradient in entry order
  const Layout Lv = per_sample ? make_layout(p, batch, true) : Layout{};
  const size_t oPS = per_sample ? take(Lv.ws_end) : 0;
  const size_t oSw = per_sample ? take(m * Bp * es) : 0;
  const size_t oGV = per_sample ? take((size_t)p->nnz_full * Bp * es) : 0;
  const size_t oBi = (qa && qa->dense) ? take((size_t)(kBiBlocks + kSlots) * es) : 0;
  const size_t oSp = qa ? take(n * Bp * es) : 0;    // pre-clip values (q gradient)
  const size_t oGq = qa ? take(n * Bp * es) : 0;    // g_q
  const size_t oCd = (qa && qa->cot_dual) ? take((size_t)std::max<int64_t>(M, 1) * Bp * es) : 0;
  const size_t oCds = (qa && qa->cot_dual) ? take((size_t)std::max<int64_t>(m, 1) * Bp * es) : 0;
  if (size_only) {
    *size_only = (int64_t)o_;
    return PURIN_CP_OK;
  }
  // the adjoint reads the saved header and its per-step counts through stream
  // synchronisations: not under capture
  {
    bool cap = false;
    if (int rc = stream_capturing(st, &cap)) return rc;
    if (cap)
      return set_error(PURIN_CP_ERR_ARG,
                       "the adjoint reads device-side counters (stream synchronisations): "
                       "not under stream capture");
  }
  const bool own_ws = o.workspace == nullptr;
  if (own_ws) {  // the last-call steps live in the plan's adjoint workspace, which may grow below
    std::lock_guard<std::mutex> lock(p->mu);
    p->adj_steps = nullptr;
    p->adj_steps_batch = 0;
  }
  // header written by the forward call
  int64_t hdr[9];
  PURIN_HIP(hipMemcpyAsync(hdr, saved, sizeof(hdr), hipMemcpyDeviceToHost, st));
  PURIN_HIP(hipStreamSynchronize(st));
  if (hdr[0] != kSavedMagic || hdr[1] != batch || hdr[2] != Bp || hdr[5] != p->dtype ||
      hdr[6] != n || hdr[7] != m)
    return set_error(PURIN_CP_ERR_ARG, "saved state does not belong to this plan and batch");
  const int kind = (int)hdr[3];
  const int shared = (int)hdr[4];
  if (dense ? kind != 4 : (qa ? kind != 3 : kind >= 3))
    return set_error(PURIN_CP_ERR_ARG,
                     dense ? "saved state is not from purin_cp_dense_solve"
                           : (qa ? "saved state is not from purin_cp_qp_solve"
                                 : "saved state is from purin_cp_qp_solve or purin_cp_dense_solve: "
                                   "use purin_cp_qp_adjoint or purin_cp_dense_adjoint"));
  if (!qa && per_sample != (kind == 2))
    return set_error(PURIN_CP_ERR_ARG, per_sample
                                           ? "saved state is not from purin_cp_project_values"
                                           : "saved state is from purin_cp_project_values: use "
                                             "purin_cp_adjoint_values");
  const char* sv = (const char*)saved;
  const T* Tt = (const T*)(sv + L.Tt);
  const T* Y = (const T*)(sv + L.Y);
  const T* Dd = (const T*)(sv + L.D);
  const T* R = (const T*)(sv + L.R);
  const T* LO = (const T*)(sv + L.LO);
  const T* HI = (const T*)(sv + L.HI);
  const T* RF = (const T*)(sv + L.RF);
  const int32_t* conv = (const int32_t*)(sv + L.conv);
  const T* metric = (kind == 1 || kind == 2) ? (const T*)p->metric : nullptr;

  int err = PURIN_CP_OK;
  char* ws = (char*)workspace(p, o_, st, &err, true, o.workspace, o.workspace_bytes);
  if (!ws) return err;
  HostWords hw(p);  // this call's host words for the counter reads
  T* Vb = (T*)(ws + oV);
  // GMRES basis: slot i, row r, sample b at r * zld + i * zs + b (the rows of all
  // slots interleaved, so a pass over the prefix reads one contiguous run per
  // row); the dense BiCGSTAB keeps contiguous vectors of vstride elements
  const int64_t vstride = W * Bp;
  const int64_t zs = Bp, zld = (int64_t)(restart + 1) * Bp;
  T* X = (T*)(ws + oX);
  T* Gr = (T*)(ws + oG);
  T* Rr = (T*)(ws + oRr);
  T* T1 = (T*)(ws + oT1);
  T* part = (T*)(ws + oPart);
  T* S1 = (T*)(ws + oS1);
  T* S2 = (T*)(ws + oS2);
  Gm<T> G{batch, Bp, restart, (T*)(ws + oThr), (T*)(ws + oRinf), (int32_t*)(ws + oCyc),
          (int32_t*)(ws + oAct), (int32_t*)(ws + oSteps),
          (T*)(ws + oScale), (T*)(ws + oHess), (T*)(ws + oCs), (T*)(ws + oSn), (T*)(ws + oGv),
          (T*)(ws + oCoef), (int32_t*)(ws + oCnt), (int32_t*)(ws + oStepCnt),
          (T*)(ws + oTm), (T*)(ws + oHu), (T*)(ws + oU2), (T*)(ws + oG1), (T*)(ws + oQ1),
          (T*)(ws + oCg), (T*)(ws + oWc), (int32_t*)(ws + oTot)};

  Adj<T> S{};
  S.K = kept_matrix<T>(p, true);
  S.Bp = Bp;
  S.ldv = Bp;
  S.n = (int)n;
  S.m = (int)m;
  const T tau = (T)p->tau_adj;
  S.sigma = (T)p->sigma_adj;
  S.a = T(1) / (T(1) + tau);
  S.delta = tau * S.a;
  PerSample<T> PS{};
  if (qa) {
    // the QP's q, c and per-sample steps: diagonal steps, or tau = s/(max q + L),
    // sigma = s/L with L from the norm bound or the power iteration
    // (diagonal_qp.py:137-160)
    char* wq = ws + oPS;
    T* QQ = (T*)(wq + Lv.QQ);
    T* QC = (T*)(wq + Lv.QC);
    T* qmax = (T*)(wq + Lv.QS);
    to_minor<T>(st, qa->q, batch, n, n, QQ, Bp, nullptr, 0);
    to_minor<T>(st, qa->c, batch, n, n, QC, Bp, nullptr, 0);
    k_qp_stats<T><<<(unsigned)(Bp / 64), 1024, 0, st>>>(n, Bp, batch, QQ, LO, HI, qmax,
                                                              qmax + Bp, nullptr);
    if (int rc = prepare_values<T>(p, st, batch, Lv, wq, values, T(1), kQPAdjoint, qmax,
                                   qmax + Bp, &PS))
      return rc;
    if (PS.RVs) {  // the plan's own coefficients: one shared copy of the scaled entries
      S.K.rval = PS.RVs;
      S.K.cval = PS.CVs;
    } else {
      S.K.rvb = PS.RV;
      S.K.cvb = PS.CV;
      S.K.vbp = Bp;
    }
    S.Q = QQ;
    S.Cc = QC;
    S.Spre = (T*)(ws + oSp);
    S.factored = qa->dense;
    if (p->diag) {
      S.tau_cb = PS.tau_cb;
      S.sig_rb = PS.sig_rb;
    } else {
      S.tau_b = PS.tau_b;
      S.sig_b = PS.sig_b;
    }
    S.dg = 1;
  } else if (per_sample) {
    // per-sample scaled entries and the adjoint's per-sample steps: the
    // power-iteration L of each sample's matrix (bounds.py:88-101) or its
    // diagonal steps (bounds.py:83-86)
    if (int rc = prepare_values<T>(p, st, batch, Lv, ws + oPS, values, T(1), kProjectAdjoint,
                                   nullptr, nullptr, &PS))
      return rc;
    S.K.rvb = PS.RV;
    S.K.cvb = PS.CV;
    S.K.vbp = Bp;
    if (p->diag) {
      S.a_cb = PS.a_cb;
      S.d_cb = PS.d_cb;
      S.sig_rb = PS.sig_rb;
    } else {
      S.a_b = PS.a_b;
      S.d_b = PS.d_b;
      S.sig_b = PS.sig_b;
    }
    S.dg = 1;
  } else if (p->diag) {  // the forward's diagonal steps (bounds.py:83-86)
    S.a_c = (const T*)p->diag_a;
    S.d_c = (const T*)p->diag_d;
    S.sig_r = (const T*)p->diag_sig;
    S.dg = 1;
  }
  S.Cm = (const T*)(ws + oCm);
  S.Dm = (const T*)(ws + oDm);
  S.U = (T*)(ws + oU);
  S.Wv = (T*)(ws + oWv);

  constexpr int64_t TS = tile_samples<T>();
  const dim3 grow = tile_grid(Bp, TS, (m + 3) / 4), gcol = tile_grid(Bp, TS, (n + 3) / 4);
  const dim3 ggs((unsigned)(Bp / TS), (unsigned)nchunk);
  const unsigned eb = 2048, sb = (unsigned)((Bp + 255) / 256);
  const int64_t total = W * Bp;

  // linearisation (bounds.py:109-129)
  if (m) k_lin_rows<T><<<grow, kBlock, 0, st>>>(S, Y, Dd, R, (T*)(ws + oDm), (T*)(ws + oDp));
  k_lin_cols<T><<<gcol, kBlock, 0, st>>>(S, Y, Tt, LO, HI, shared, (const T*)(ws + oDp),
                                          (T*)(ws + oCm), (T*)(ws + oClo), (T*)(ws + oChi));
  // out = A (vsc . v), vsc a per-sample scale or nullptr
  auto op = [&](const T* v, T* out, const T* vsc, int64_t ldv) {
    S.vsc = vsc;
    S.ldv = ldv;
    k_op_cols1<T><<<gcol, kBlock, 0, st>>>(S, v, out);
    if (m) k_op_rows<T><<<grow, kBlock, 0, st>>>(S, v, out);
    k_op_cols2<T><<<gcol, kBlock, 0, st>>>(S, v, out);
    S.vsc = nullptr;
    S.ldv = Bp;
  };
  auto reduce = [&](int mode_nv, T* out, int opk) {
    k_reduce<T><<<(unsigned)((mode_nv * Bp + 255) / 256), 256, 0, st>>>(part, mode_nv, nchunk, Bp,
                                                                         out, opk);
  };
  auto read_counter = [&](int idx, int32_t* val) -> int {
    PURIN_HIP(hipMemcpyAsync(hw.get(), G.counter, 2 * sizeof(int32_t), hipMemcpyDeviceToHost, st));
    PURIN_HIP(hipStreamSynchronize(st));
    *val = hw.get()[idx];
    return PURIN_CP_OK;
  };
  // active counts at the start of Arnoldi steps [0, upto] of the current cycle
  auto read_stepcnt = [&](int upto, std::vector<int32_t>& out) -> int {
    out.resize(upto + 1);
    PURIN_HIP(hipMemcpyAsync(hw.get(), G.stepcnt, (upto + 1) * sizeof(int32_t),
                             hipMemcpyDeviceToHost, st));
    PURIN_HIP(hipStreamSynchronize(st));
    for (int i = 0; i <= upto; ++i) out[i] = hw.get()[i];
    return PURIN_CP_OK;
  };
  auto zero_counters = [&]() { k_fill<int32_t><<<1, 64, 0, st>>>(G.counter, 2, 0); };
  // one round of resident blocks per pass: the chunk count per batch tile is the
  // kernel's resident block count over the tiles (so no partial second round)
  int last_nchunk = 1;
  auto resident_chunks = [&](auto kern, int64_t* chunks) -> int {
    int per_cu = 0;
    PURIN_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kBlock, 0));
    *chunks = std::max<int64_t>(
        1, std::min<int64_t>({(int64_t)std::max(per_cu, 1) * cus / tiles0, (W + 3) / 4,
                              (int64_t)nchunk2}));
    return PURIN_CP_OK;
  };
  // the update-and-dot pass: two blocks per CU over the batch tiles (as fast
  // as more, and fewer chunk partials for the per-sample reduction)
  auto launch_gs = [&](auto kern, int nv, T* img, const T* h) -> int {
    const int64_t chunks = std::max<int64_t>(
        1, std::min<int64_t>({(int64_t)2 * cus / tiles0, (W + 3) / 4, (int64_t)nchunk2}));
    const int64_t rpb = (W + chunks - 1) / chunks;
    last_nchunk = (int)chunks;
    kern<<<dim3((unsigned)tiles0, (unsigned)chunks), kBlock, 0, st>>>(Vb, zs, nv, img, h, W, Bp,
                                                                    part, (int)chunks, rpb, zld);
    return PURIN_CP_OK;
  };
  auto launch_rows = [&](auto kern, int nv, const T* img) -> int {
    int64_t chunks = 1;
    if (int rc = resident_chunks(kern, &chunks)) return rc;
    const int64_t rpb = (W + chunks - 1) / chunks;
    last_nchunk = (int)chunks;
    kern<<<dim3((unsigned)tiles0, (unsigned)chunks), kBlock, 0, st>>>(Vb, zs, nv, img, W, Bp,
                                                                    part, (int)chunks, rpb, zld);
    return PURIN_CP_OK;
  };
  // the dot pass: two blocks per CU over the batch tiles, the same chunks as
  // the update-and-dot pass (launch_gs), so that pass B begins each chunk on
  // the rows this pass read last (k_gs_dots walks its chunk backwards)
  auto launch_dots = [&](auto kern, int nv, const T* img) -> int {
    const int64_t per_cu = 2;
    const int64_t chunks = std::max<int64_t>(
        1, std::min<int64_t>({per_cu * cus / tiles0, (W + 3) / 4, (int64_t)nchunk2}));
    const int64_t rpb = (W + chunks - 1) / chunks;
    last_nchunk = (int)chunks;
    kern<<<dim3((unsigned)tiles0, (unsigned)chunks), kBlock, 0, st>>>(Vb, zs, nv, img, W, Bp,
                                                                    part, (int)chunks, rpb, zld);
    return PURIN_CP_OK;
  };
  // pass A (mode 0): part_i = Z_i . y; pass B (mode 1): y <- y - sum_i h_i Z_i,
  // part_i = Z_i . y, part_nv = y . y
  auto gs_pass = [&](int mode, int nv, T* img, const T* h) -> int {
    const int bucket = nv <= 8 ? 8 : (nv <= 16 ? 16 : (nv <= 24 ? 24 : 32));
    if (mode == 0) {
      // up to 8 vectors the row-split pass is faster: the vector-split one
      // re-reads x once per wavefront, which dominates for a short prefix
      if (bucket == 8) return launch_rows(k_gs_dots_rows<T, 8>, nv, img);
      if (bucket == 16) return launch_dots(k_gs_dots<T, 16>, nv, img);
      if (bucket == 24) return launch_dots(k_gs_dots<T, 24>, nv, img);
      return launch_dots(k_gs_dots<T, 32>, nv, img);
    }
    if (bucket == 8) return launch_gs(k_gs_update_dots<T, 8>, nv, img, h);
    if (bucket == 16) return launch_gs(k_gs_update_dots<T, 16>, nv, img, h);
    if (bucket == 24) return launch_gs(k_gs_update_dots<T, 24>, nv, img, h);
    return launch_gs(k_gs_update_dots<T, 32>, nv, img, h);
  };

  // rhs g = [cot * eligible, 0, 0] (cotangent divided by sqrt(D) for a metric)
  to_minor<T>(st, cot_y, batch, n, n, T1, Bp, metric, metric ? 2 : 0);
  // the QP's dual cotangent w.r.t. the scaled dual: cot_dual * scale (the
  // returned multipliers are dual * scale, diagonal_qp.py:274)
  T* cotd = nullptr;
  if (qa && qa->cot_dual && m) {
    T* CD = (T*)(ws + oCd);
    cotd = (T*)(ws + oCds);
    to_minor<T>(st, qa->cot_dual, batch, M, M, CD, Bp, nullptr, 0);
    k_prep_rows<T><<<2048, 256, 0, st>>>((int)m, Bp, p->dkept, (const T*)p->dscale, PS.SC, CD,
                                         nullptr, cotd, nullptr);
  }
  k_gm_rhs<T><<<eb, 256, 0, st>>>(n, m, W, Bp, batch, T1, cotd, conv,
                                  dense ? 1 : o.force_eligible, Gr);
  T* lam_w = (T*)(ws + oLw);
  purin_cp_adjoint_stats stats{};
  if (dense) {
    // BiCGSTAB on (I - J^T) v = g over the whole batch (fixed_point.py:8-40)
    T* bpart = (T*)(ws + oBi);
    T* bsc = bpart + kBiBlocks;
    T* RH = Vb;
    T* Pv = Vb + vstride;
    T* Qv = Vb + 2 * vstride;
    T* Sv = Vb + 3 * vstride;
    T* Tv = Vb + 4 * vstride;
    auto dot = [&](const T* x, const T* y, int slot) {
      k_bi_dot<T><<<kBiBlocks, 256, 0, st>>>(x, y, total, bpart);
      k_bi_sum<T><<<1, 256, 0, st>>>(bpart, kBiBlocks, bsc, slot);
    };
    auto bi_vec = [&](int mode) {
      k_bi_vec<T><<<eb, 256, 0, st>>>(mode, total, bsc, X, Rr, Pv, Qv, Sv, Tv);
    };
    dot(Gr, Gr, kBS);
    k_bi_scalar<T><<<1, 64, 0, st>>>(bsc, 0, (T)o.tolerance, (T)o.atol);
    k_fill<T><<<eb, 256, 0, st>>>(X, total, T(0));
    // r0 = b - A(0) = b; rhat = p = q = r0
    for (T* dst : {Rr, RH, Pv, Qv})
      PURIN_HIP(hipMemcpyAsync(dst, Gr, vec, hipMemcpyDeviceToDevice, st));
    int64_t iters = 0;
    T* host = (T*)hw.get();
    for (;;) {
      dot(Rr, Rr, kRS);
      PURIN_HIP(hipMemcpyAsync(host, bsc, kSlots * sizeof(T), hipMemcpyDeviceToHost, st));
      PURIN_HIP(hipStreamSynchronize(st));
      const T rs = host[kRS], atol2 = host[kAtol2], kk = host[kK];
      if (!(rs > atol2 && kk < (T)o.max_iterations && kk >= T(0))) break;
      dot(RH, Rr, kRho_);
      k_bi_scalar<T><<<1, 64, 0, st>>>(bsc, 1, T(0), T(0));
      bi_vec(0);
      op(Pv, Qv, nullptr, Bp);
      dot(RH, Qv, kRQ);
      k_bi_scalar<T><<<1, 64, 0, st>>>(bsc, 2, T(0), T(0));
      bi_vec(1);
      dot(Sv, Sv, kSS);
      op(Sv, Tv, nullptr, Bp);
      dot(Tv, Sv, kTS);
      dot(Tv, Tv, kTT);
      k_bi_scalar<T><<<1, 64, 0, st>>>(bsc, 3, T(0), T(0));
      bi_vec(2);
      k_bi_scalar<T><<<1, 64, 0, st>>>(bsc, 4, T(0), T(0));
      ++iters;
    }
    stats.arnoldi_steps = iters;
    stats.cycles = (int32_t)host[kK];  // iterations, or -10 / -11 at breakdown
    k_fill_weights<T><<<sb, 256, 0, st>>>(batch, Bp, lam_w);
    if (o.arnoldi_iterations)
      k_fill<int32_t><<<sb, 256, 0, st>>>(o.arnoldi_iterations, batch, (int32_t)iters);
  } else {
  // threshold = max(atol, tol * max|g|) and residual_inf = max|g - A 0| = max|g|
  k_gs<T, 4><<<ggs, kBlock, 0, st>>>(nullptr, 0, 0, Gr, nullptr, W, Bp, part, nchunk, Bp);
  reduce(1, S1, 1);
  k_gm_thresholds<T><<<sb, 256, 0, st>>>(G, S1, (T)o.tolerance, (T)o.atol);
  k_fill<T><<<eb, 256, 0, st>>>(X, total, T(0));
  PURIN_HIP(hipMemcpyAsync(Rr, Gr, vec, hipMemcpyDeviceToDevice, st));  // r = g - A(0)

  const dim3 tri_grid((unsigned)(Bp / kTriS));
  const size_t tri_lds = (size_t)(5 * restart + 4) * kTriS * es;
  if (int rc = raise_lds_cap((const void*)k_gm_tri<T, 1>, tri_lds)) return rc;
  if (int rc = raise_lds_cap((const void*)k_gm_tri<T, 2>, tri_lds)) return rc;
  int64_t completed = 0;
  k_fill<int32_t><<<sb, 256, 0, st>>>(G.total, Bp, 0);
  while (completed < o.max_iterations) {
    zero_counters();
    k_gm_count_unconverged<T><<<sb, 256, 0, st>>>(G);
    int32_t unconverged = 0;
    if (int rc = read_counter(1, &unconverged)) return rc;
    if (unconverged == 0) break;
    const int cycle_limit = (int)std::min<int64_t>(restart, o.max_iterations - completed);
    ++stats.cycles;
    // beta = ||r||, V0 = r / max(beta, eps)
    k_gs<T, 3><<<ggs, kBlock, 0, st>>>(nullptr, 0, 0, Rr, nullptr, W, Bp, part, nchunk, Bp);
    reduce(1, S1, 0);
    k_fill<int32_t><<<1, 256, 0, st>>>(G.stepcnt, restart + 2, 0);
    k_gm_cycle_init<T><<<sb, 256, 0, st>>>(G, S1);
    k_scale_cols<T><<<eb, 256, 0, st>>>(total, Bp, Vb, zld, Rr, G.scale);
    // Arnoldi steps.  The reference loop runs step s while s < cycle_limit and
    // some sample is active at its start (operators.py:943-1082); a step with
    // no active sample changes no state here (every update is masked by the
    // active flags), so the host reads the per-step active counts only every
    // kStepCheck steps and at the end, and takes the first empty step as the
    // cycle's length.
    int launched = 0;
    std::vector<int32_t> cnt;
    while (launched < cycle_limit) {
      const int chunk_end = std::min(cycle_limit, launched + kStepCheck);
      if (int rc = read_stepcnt(launched, cnt)) return rc;
      if (cnt[launched] == 0) break;
      for (int it = launched; it < chunk_end; ++it) {
        // slot it holds Z_it; y = A (Z_it Tm[it][it]) goes to slot it + 1, where
        // pass B turns it into Z_{it+1}
        T* zk = Vb + (size_t)it * zs;
        T* img = Vb + (size_t)(it + 1) * zs;
        const int nv = it + 1;
        op(zk, img, G.Tm + ((size_t)it * (restart + 1) + it) * Bp, zld);
        int nch = nchunk;
        if (nv <= 32) {
          if (int rc = gs_pass(0, nv, img, nullptr)) return rc;
          nch = last_nchunk;
        } else {
          k_gs<T, 0><<<ggs, kBlock, 0, st>>>(Vb, zs, nv, img, nullptr, W, Bp, part, nchunk, zld);
        }
        k_gm_tri<T, 1><<<tri_grid, 1024, tri_lds, st>>>(G, it, part, nch);
        nch = nchunk;
        if (nv <= 32) {
          if (int rc = gs_pass(1, nv, img, G.Q1)) return rc;
          nch = last_nchunk;
        } else {
          k_gs<T, 5><<<ggs, kBlock, 0, st>>>(Vb, zs, nv, img, G.Q1, W, Bp, part, nchunk, zld);
        }
        k_gm_tri<T, 2><<<tri_grid, 1024, tri_lds, st>>>(G, it, part, nch);
      }
      launched = chunk_end;
    }
    int it = launched;
    if (int rc = read_stepcnt(launched, cnt)) return rc;
    for (int s2 = 0; s2 < launched; ++s2)
      if (cnt[s2] == 0) {
        it = s2;
        break;
      }
    k_gm_backsub<T><<<(unsigned)(Bp / 64), 64, (size_t)restart * 64 * sizeof(T), st>>>(G);
    k_gm_tcoef<T><<<dim3((unsigned)((Bp + 255) / 256), (unsigned)restart), 256, 0, st>>>(G);
    k_correction<T><<<eb, 256, 0, st>>>(total, Bp, X, Vb, zs, zld, G.Wc, G.steps);
    // candidate residual r = g - A x (operators.py:1084-1091)
    op(X, T1, nullptr, Bp);
    k_axpby<T><<<eb, 256, 0, st>>>(total, Rr, Gr, T1, T(-1));
    k_gs<T, 4><<<ggs, kBlock, 0, st>>>(nullptr, 0, 0, Rr, nullptr, W, Bp, part, nchunk, Bp);
    reduce(1, S1, 1);
    k_gm_cycle_end<T><<<sb, 256, 0, st>>>(G, S1);
    completed += it;
    stats.arnoldi_steps += it;
  }
  if (o.arnoldi_iterations)
    PURIN_HIP(hipMemcpyAsync(o.arnoldi_iterations, G.total, (size_t)batch * sizeof(int32_t),
                             hipMemcpyDeviceToDevice, st));
  if (own_ws) {  // read by purin_cp_last_adjoint_iterations until the next such call
    std::lock_guard<std::mutex> lock(p->mu);
    p->adj_steps = G.total;
    p->adj_steps_batch = batch;
  }
  // finiteness of the solution, info, valid (operators.py:1119-1122, bounds.py:148-153)
  k_gs<T, 2><<<ggs, kBlock, 0, st>>>(nullptr, 0, 0, X, nullptr, W, Bp, part, nchunk, Bp);
  k_reduce<T><<<sb, 256, 0, st>>>(part + (size_t)nchunk * Bp, 1, nchunk, Bp, S2, 2);
  k_gm_finish<T><<<sb, 256, 0, st>>>(G, S2, conv, (T)o.adjoint_tolerance, o.force_eligible,
                                     lam_w, valid, info, gres);
  }
  // final pullback of the masked lambda
  T* gt = (T*)(ws + oGt);
  T* glo = (T*)(ws + oGlo);
  T* ghi = (T*)(ws + oGhi);
  T* gr = (T*)(ws + oGr);
  T* gq = (qa && !dense) ? (T*)(ws + oGq) : nullptr;  // the dense layer's prox is frozen
  k_final_u<T><<<eb, 256, 0, st>>>(S, X, lam_w, (const T*)(ws + oClo), (const T*)(ws + oChi), gt,
                                   glo, ghi, gq);
  if (qa && qa->g_q) {
    if (gq)
      to_major<T>(st, gq, Bp, n, qa->g_q, batch, n, nullptr, 0);
    else
      k_fill<T><<<eb, 256, 0, st>>>(qa->g_q, batch * n, T(0));
  }
  T* sw = per_sample ? (T*)(ws + oSw) : nullptr;
  if (m) k_final_w<T><<<grow, kBlock, 0, st>>>(S, X, lam_w, gr, sw);
  if (g_target) to_major<T>(st, gt, Bp, n, g_target, batch, n, metric, metric ? 1 : 0);
  if (kind >= 1) {
    T* GF = (g_rhs && M) ? (T*)(ws + oGF) : nullptr;
    T* GV = (per_sample && g_values && p->nnz_full) ? (T*)(ws + oGV) : nullptr;
    if (GV && m)
      k_gvals_rows<T><<<grow, kBlock, 0, st>>>(S.K, Bp, sw, Y, S.U, (const T*)(ws + oDp), gr,
                                              PS.RVo, PS.SC, RF, p->dkept,
                                              qa ? 0 : p->opts.row_scaling, p->ps_kcsr, GV);
    if (GF || (GV && !p->bound.empty()))
      k_grhs_full<T><<<eb, 256, 0, st>>>((int)m, (int)n, Bp, p->dkept, (const T*)p->dscale,
                                         per_sample ? PS.SC : nullptr, gr, p->bptr, p->brow,
                                         (const T*)p->dbcoef, per_sample ? PS.BC : nullptr, RF,
                                         LO, HI, shared, glo, ghi, GF, p->ps_bpos, GV);
    if (GF) to_major<T>(st, GF, Bp, M, g_rhs, batch, M, nullptr, 0);
    if (GV) to_major<T>(st, GV, Bp, p->nnz_full, g_values, batch, p->nnz_full, nullptr, 0);
  } else {
    if (g_rhs && m) to_major<T>(st, gr, Bp, m, g_rhs, batch, m, nullptr, 0);
  }
  if (g_lower) to_major<T>(st, glo, Bp, n, g_lower, batch, n, nullptr, 0);
  if (g_upper) to_major<T>(st, ghi, Bp, n, g_upper, batch, n, nullptr, 0);
  PURIN_HIP(hipGetLastError());
  {
    std::lock_guard<std::mutex> lock(p->mu);
    p->adjoint_stats = stats;
  }
  return PURIN_CP_OK;
}

template <typename T>
static int adjoint_bytes_t(const purin_cp_plan* cp, int32_t entry, int64_t batch,
                           const purin_cp_adjoint_options& o, int64_t* bytes) {
  purin_cp_plan* p = const_cast<purin_cp_plan*>(cp);  // size_only touches nothing
  const T dummy = T(0);
  // the largest variant of each entry: a dual cotangent for the QP adjoints
  const QPAdjArgs<T> qa{&dummy, &dummy, &dummy, nullptr, entry == PURIN_CP_ENTRY_DENSE_ADJOINT};
  const bool per_sample = entry != PURIN_CP_ENTRY_ADJOINT;
  const bool qp = entry == PURIN_CP_ENTRY_QP_ADJOINT || entry == PURIN_CP_ENTRY_DENSE_ADJOINT;
  return adjoint_impl<T>(p, nullptr, batch, nullptr, nullptr, o, nullptr, nullptr, nullptr,
                         nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, per_sample,
                         qp ? &qa : nullptr, bytes);
}

int adjoint_workspace_bytes(const purin_cp_plan* p, int32_t entry, int64_t batch,
                            const purin_cp_adjoint_options& o, int64_t* bytes) {
  return p->dtype == PURIN_CP_F64 ? adjoint_bytes_t<double>(p, entry, batch, o, bytes)
                                  : adjoint_bytes_t<float>(p, entry, batch, o, bytes);
}

}  // namespace purin

using namespace purin;

extern "C" int purin_cp_dense_adjoint(purin_cp_plan* p, void* stream, int64_t batch,
                                      const void* saved, const void* q, const void* c,
                                      const void* values, const void* cot_y,
                                      const void* cot_dual, const purin_cp_adjoint_options* opts,
                                      void* g_q, void* g_c, void* g_values, void* g_rhs,
                                      void* g_lower, void* g_upper) {
  if (!p) return set_error(PURIN_CP_ERR_ARG, "NULL plan");
  purin_cp_adjoint_options o;
  purin_cp_default_adjoint_options(&o);
  if (opts) o = *opts;
  hipStream_t st = (hipStream_t)stream;
  if (p->dtype == PURIN_CP_F64) {
    const QPAdjArgs<double> qa{(const double*)q, (const double*)c, (const double*)cot_dual,
                               (double*)g_q, 1};
    return adjoint_impl<double>(p, st, batch, saved, (const double*)cot_y, o, (double*)g_c,
                                (double*)g_rhs, (double*)g_lower, (double*)g_upper, nullptr,
                                nullptr, nullptr, (const double*)values, (double*)g_values, true,
                                &qa);
  }
  const QPAdjArgs<float> qa{(const float*)q, (const float*)c, (const float*)cot_dual,
                            (float*)g_q, 1};
  return adjoint_impl<float>(p, st, batch, saved, (const float*)cot_y, o, (float*)g_c,
                             (float*)g_rhs, (float*)g_lower, (float*)g_upper, nullptr, nullptr,
                             nullptr, (const float*)values, (float*)g_values, true, &qa);
}

extern "C" int purin_cp_qp_adjoint(purin_cp_plan* p, void* stream, int64_t batch,
                                   const void* saved, const void* q, const void* c,
                                   const void* values, const void* cot_y, const void* cot_dual,
                                   const purin_cp_adjoint_options* opts, void* g_q, void* g_c,
                                   void* g_values, void* g_rhs, void* g_lower, void* g_upper,
                                   uint8_t* valid, int32_t* info, void* gmres_residual) {
  if (!p) return set_error(PURIN_CP_ERR_ARG, "NULL plan");
  purin_cp_adjoint_options o;
  purin_cp_default_adjoint_options(&o);
  if (opts) o = *opts;
  hipStream_t st = (hipStream_t)stream;
  if (p->dtype == PURIN_CP_F64) {
    const QPAdjArgs<double> qa{(const double*)q, (const double*)c, (const double*)cot_dual,
                               (double*)g_q, 0};
    return adjoint_impl<double>(p, st, batch, saved, (const double*)cot_y, o, (double*)g_c,
                                (double*)g_rhs, (double*)g_lower, (double*)g_upper, valid, info,
                                (double*)gmres_residual, (const double*)values,
                                (double*)g_values, true, &qa);
  }
  const QPAdjArgs<float> qa{(const float*)q, (const float*)c, (const float*)cot_dual,
                            (float*)g_q, 0};
  return adjoint_impl<float>(p, st, batch, saved, (const float*)cot_y, o, (float*)g_c,
                             (float*)g_rhs, (float*)g_lower, (float*)g_upper, valid, info,
                             (float*)gmres_residual, (const float*)values, (float*)g_values, true,
                             &qa);
}

extern "C" int purin_cp_adjoint_values(purin_cp_plan* p, void* stream, int64_t batch,
                                       const void* saved, const void* values, const void* cot_y,
                                       const purin_cp_adjoint_options* opts, void* g_target,
                                       void* g_rhs, void* g_values, uint8_t* valid, int32_t* info,
                                       void* gmres_residual) {
  if (!p) return set_error(PURIN_CP_ERR_ARG, "NULL plan");
  purin_cp_adjoint_options o;
  purin_cp_default_adjoint_options(&o);
  if (opts) o = *opts;
  hipStream_t st = (hipStream_t)stream;
  if (p->dtype == PURIN_CP_F64)
    return adjoint_impl<double>(p, st, batch, saved, (const double*)cot_y, o, (double*)g_target,
                                (double*)g_rhs, nullptr, nullptr, valid, info,
                                (double*)gmres_residual, (const double*)values,
                                (double*)g_values, true);
  return adjoint_impl<float>(p, st, batch, saved, (const float*)cot_y, o, (float*)g_target,
                             (float*)g_rhs, nullptr, nullptr, valid, info, (float*)gmres_residual,
                             (const float*)values, (float*)g_values, true);
}

extern "C" int purin_cp_adjoint(purin_cp_plan* p, void* stream, int64_t batch, const void* saved,
                                const void* target, const void* rhs, const void* cot_y,
                                const purin_cp_adjoint_options* opts, void* g_target, void* g_rhs,
                                void* g_lower, void* g_upper, uint8_t* valid, int32_t* info,
                                void* gmres_residual) {
  (void)target;  // the saved state holds the forward's inputs
  (void)rhs;
  if (!p) return set_error(PURIN_CP_ERR_ARG, "NULL plan");
  purin_cp_adjoint_options o;
  purin_cp_default_adjoint_options(&o);
  if (opts) o = *opts;
  hipStream_t st = (hipStream_t)stream;
  if (p->dtype == PURIN_CP_F64)
    return adjoint_impl<double>(p, st, batch, saved, (const double*)cot_y, o, (double*)g_target,
                                (double*)g_rhs, (double*)g_lower, (double*)g_upper, valid, info,
                                (double*)gmres_residual);
  return adjoint_impl<float>(p, st, batch, saved, (const float*)cot_y, o, (float*)g_target,
                             (float*)g_rhs, (float*)g_lower, (float*)g_upper, valid, info,
                             (float*)gmres_residual);
}
