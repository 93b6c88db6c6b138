// Per-sample coefficients: every sample has its own constraint values (the
// reference's values (B, m_tot, w) from jax.vmap(_numeric_one), bounds.py:192,
// when coefficients depend on parameters).  The sparsity structure is the
// plan's; the values arrive per call and are laid out batch-minor, entry k of
// sample b at [k * Bp + b], in CSR order (row pass) and CSC order (column
// pass).  These kernels prepare what the shared-coefficient plan computes on
// the host once: row scales, scaled values, norm bounds, step sizes and the
// tolerance, each per sample (bounds.py:193-236, kernels.py:209-227).
#pragma once

#include "common.hpp"
#include "kernels.hpp"
#include "plan.hpp"

namespace purin {

// dst[k * Bp + b] = src[map[k] * Bp + b]
template <typename T>
__global__ void k_gather_entries(const T* __restrict__ src, int64_t Bp,
                                 const int32_t* __restrict__ map, int64_t K, T* __restrict__ dst) {
  const int64_t total = K * Bp;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t k = e / Bp, b = e - k * Bp;
    dst[e] = src[(int64_t)map[k] * Bp + b];
  }
}

// dst[k * Bp + b] = src[k] for b < batch, 0 for the padding
template <typename T>
__global__ void k_bcast_entries(const T* __restrict__ src, int64_t K, int64_t Bp, int64_t batch,
                                T* __restrict__ dst) {
  const int64_t total = K * Bp;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t k = e / Bp, b = e - k * Bp;
    dst[e] = b < batch ? src[k] : T(0);
  }
}

// Per kept row (one row per wavefront, lanes over samples): the row norm and
// scale (bounds.py:210-214; 1 without row scaling or for an empty row), the
// scaled values RV = RVo * scale, the absolute row sum of RV (the norm bound,
// kernels.py:214-220; with diagonal steps sigma_i = safety / rowsum_i,
// kernels.py:76-88).  Per block: the max row sum and min scale of its rows,
// into part[0][rb][b] and part[1][rb][b].
template <typename T>
__global__ __launch_bounds__(kBlock) void k_ps_rows(int m, int64_t Bp, const int32_t* __restrict__ rptr,
                                                    const T* __restrict__ RVo, int row_scaling,
                                                    T safety, T* __restrict__ SC, T* __restrict__ RV,
                                                    T* __restrict__ sig_rb, T* __restrict__ part,
                                                    int nrb) {
#pragma clang fp contract(off)
  using V = typename Lane<T>::V;
  constexpr int S = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b0 = ((int64_t)blockIdx.x * kWave + lane) * S;
  const T zero = T(0), one = T(1);
  for (int rb = blockIdx.y; rb < nrb; rb += gridDim.y) {
    V rmax = vsplat<T>(zero), smin = vsplat<T>(one);
    for (int c = 0; c < kRowsPerWaveEarly; ++c) {
      const int i = (rb * 4 + wave) * kRowsPerWaveEarly + c;
      if (i >= m) break;
      const int s0 = rptr[i], s1 = rptr[i + 1];
      V sq = vsplat<T>(zero);
      for (int k = s0; k < s1; ++k) {
        const V v = vload(RVo + (size_t)k * Bp + b0);
        sq += v * v;
      }
      V sc = vsplat<T>(one);
      if (row_scaling) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const T norm = __builtin_sqrt(sq[s]);
          sc[s] = norm > zero ? one / maxp(norm, T(1e-30)) : one;
        }
      }
      vstore(SC + (size_t)i * Bp + b0, sc);
      V rs = vsplat<T>(zero);
      for (int k = s0; k < s1; ++k) {
        const V v = vload(RVo + (size_t)k * Bp + b0) * sc;
        vstore(RV + (size_t)k * Bp + b0, v);
#pragma unroll
        for (int s = 0; s < S; ++s) rs[s] += absv(v[s]);
      }
      if (sig_rb) {
        V sg;
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const T r = rs[s] > zero ? maxp(rs[s], T(1e-12)) : one;
          sg[s] = safety / r;
        }
        vstore(sig_rb + (size_t)i * Bp + b0, sg);
      }
#pragma unroll
      for (int s = 0; s < S; ++s) {
        rmax[s] = maxp(rmax[s], rs[s]);
        smin[s] = minp(smin[s], sc[s]);
      }
    }
    __shared__ T buf[kBlock * S];
    const V p0 = block_combine<T>(rmax, buf, OpMax());
    const V p1 = block_combine<T>(smin, buf, OpMin());
    if (wave == 0) {
      vstore(part + (size_t)rb * Bp + b0, p0);
      vstore(part + (size_t)(nrb + rb) * Bp + b0, p1);
    }
  }
}

// Per column (one column per wavefront): scaled values in CSC order
// CV = CVo * scale[row] (the same products as RV), the absolute column sum
// (norm bound; with diagonal steps tau_j = safety / colsum_j and the prox
// coefficients a_j = 1/(1 + tau_j), delta_j = tau_j a_j), and per block the max
// column sum into part[cb][b].
template <typename T>
__global__ __launch_bounds__(kBlock) void k_ps_cols(int n, int64_t Bp, const int32_t* __restrict__ cptr,
                                                    const int32_t* __restrict__ cidx,
                                                    const T* __restrict__ CVo, const T* __restrict__ SC,
                                                    T safety, T* __restrict__ CV, T* __restrict__ a_cb,
                                                    T* __restrict__ d_cb, T* __restrict__ tau_cb,
                                                    T* __restrict__ part, int ncb) {
#pragma clang fp contract(off)
  using V = typename Lane<T>::V;
  constexpr int S = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b0 = ((int64_t)blockIdx.x * kWave + lane) * S;
  const T zero = T(0), one = T(1);
  for (int cb = blockIdx.y; cb < ncb; cb += gridDim.y) {
    V cmax = vsplat<T>(zero);
    for (int c = 0; c < kRowsPerWaveEarly; ++c) {
      const int j = (cb * 4 + wave) * kRowsPerWaveEarly + c;
      if (j >= n) break;
      V cs = vsplat<T>(zero);
      for (int k = cptr[j]; k < cptr[j + 1]; ++k) {
        const V v = vload(CVo + (size_t)k * Bp + b0) * vload(SC + (size_t)cidx[k] * Bp + b0);
        vstore(CV + (size_t)k * Bp + b0, v);
#pragma unroll
        for (int s = 0; s < S; ++s) cs[s] += absv(v[s]);
      }
      if (a_cb || tau_cb) {
        V av, dv, tv;
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const T c2 = cs[s] > zero ? maxp(cs[s], T(1e-12)) : one;
          const T tau = safety / c2;
          tv[s] = tau;
          av[s] = one / (one + tau);
          dv[s] = tau * av[s];
        }
        if (a_cb) {
          vstore(a_cb + (size_t)j * Bp + b0, av);
          vstore(d_cb + (size_t)j * Bp + b0, dv);
        }
        if (tau_cb) vstore(tau_cb + (size_t)j * Bp + b0, tv);
      }
#pragma unroll
      for (int s = 0; s < S; ++s) cmax[s] = maxp(cmax[s], cs[s]);
    }
    __shared__ T buf[kBlock * S];
    const V p0 = block_combine<T>(cmax, buf, OpMax());
    if (wave == 0) vstore(part + (size_t)cb * Bp + b0, p0);
  }
}

// Per-sample steps (one thread per sample; kernels.py:209-227):
// L = max(sqrt(max rowsum * max colsum), 1e-12) from the block partials (or
// the power-iteration estimate Lpi when given), sigma = s/L,
// tau = s/L (accelerated and min q > 0) or s/(max q + L), a = 1/(1 + tau),
// delta = tau a (the prox of q = 1), theta = 1; the tolerance
// tol * min(1, min_i scale_i) (bounds.py:233-236).  qmax / qmin: per-sample
// max and min of a general diagonal q, or nullptr for q = 1.
template <typename T>
__global__ void k_ps_steps(int64_t Bp, const T* __restrict__ rpart, int nrb,
                           const T* __restrict__ cpart, int ncb, const T* __restrict__ Lpi,
                           T safety, int accelerated, T tol, const T* __restrict__ qmax,
                           const T* __restrict__ qmin, T* tau_b, T* sig_b, T* a_b, T* d_b,
                           T* th_b, T* tol_b) {
#pragma clang fp contract(off)
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= Bp) return;
  const T zero = T(0), one = T(1);
  T rmax = zero, cmax = zero, smin = one;
  for (int r = 0; r < nrb; ++r) {
    rmax = maxp(rmax, rpart[(size_t)r * Bp + b]);
    smin = minp(smin, rpart[(size_t)(nrb + r) * Bp + b]);
  }
  for (int c = 0; c < ncb; ++c) cmax = maxp(cmax, cpart[(size_t)c * Bp + b]);
  const T norm = Lpi ? Lpi[b] : (T)__builtin_sqrt(rmax * cmax);
  const T L = maxp(norm, T(1e-12));
  const T sigma = safety / L;
  const T qhi = qmax ? qmax[b] : one, qlo = qmin ? qmin[b] : one;
  const T tau = (accelerated && qlo > T(0)) ? safety / L : safety / (qhi + L);
  tau_b[b] = tau;
  sig_b[b] = sigma;
  a_b[b] = one / (one + tau);
  d_b[b] = tau * a_b[b];
  th_b[b] = one;
  tol_b[b] = tol * minp(one, smin);
}

// Per-sample sums over the rows of two vectors (batch-minor, R rows), one
// thread per sample adding in row order with every product rounded (no fused
// multiply-add), the order the oracle's norm estimate and the plan's host
// power iteration use: xy[b] = sum_r x[r][b] y[r][b], yy[b] = sum_r y[r][b]^2.
// Adjacent threads read adjacent samples, so every load is coalesced.
template <typename T>
__global__ __launch_bounds__(256) void k_ps_dots(int64_t R, int64_t Bp, const T* __restrict__ x,
                                                 const T* __restrict__ y, T* xy, T* yy) {
#pragma clang fp contract(off)
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= Bp) return;
  T s1 = T(0), s2 = T(0);
  for (int64_t r = 0; r < R; ++r) {
    const T yv = y[r * Bp + b];
    if (x) s1 = s1 + x[r * Bp + b] * yv;
    s2 = s2 + yv * yv;
  }
  if (xy) xy[b] = s1;
  yy[b] = s2;
}

// x[r][b] = y[r][b] / (sqrt(yy[b]) + eps)
template <typename T>
__global__ void k_ps_normalize(int64_t R, int64_t Bp, const T* __restrict__ y,
                               const T* __restrict__ yy, T eps, T* __restrict__ x) {
#pragma clang fp contract(off)
  const int64_t total = R * Bp;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = e % Bp;
    x[e] = y[e] / ((T)__builtin_sqrt(yy[b]) + eps);
  }
}

// x[j][b] = start value of column j (the same start vector for every sample)
template <typename T>
__global__ void k_ps_start(int64_t n, int64_t Bp, const T* __restrict__ start, T* __restrict__ x) {
  const int64_t total = n * Bp;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x)
    x[e] = start[e / Bp];
}

// Per sample of a general diagonal QP: max_j q, min_j q, and valid =
// all(q > 0) & all(lower <= upper) (diagonal_qp.py:120-123) into feas[b] for
// b < batch (0 beyond).  Grid Bp / 64 blocks of 1024 threads.
template <typename T>
__global__ __launch_bounds__(1024) void k_qp_stats(int64_t n, int64_t Bp, int64_t batch,
                                                  const T* __restrict__ Q,
                                                  const T* __restrict__ LO,
                                                  const T* __restrict__ HI, T* qmax, T* qmin,
                                                  int32_t* feas) {
  // a block owns 64 samples (one per lane); its 16 wavefronts take the columns
  // j = w, w + 16, ... and meet in LDS (max, min and the AND do not depend on
  // the order in which they combine)
  __shared__ T s_hi[16][64], s_lo[16][64];
  __shared__ int s_ok[16][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t b = (int64_t)blockIdx.x * 64 + lane;
  T hi = Q[b], lo = Q[b];
  bool ok = true;
  for (int64_t j = w; j < n; j += 16) {
    const T q = Q[j * Bp + b];
    hi = maxp(hi, q);
    lo = minp(lo, q);
    ok = ok && q > T(0) && LO[j * Bp + b] <= HI[j * Bp + b];
  }
  s_hi[w][lane] = hi;
  s_lo[w][lane] = lo;
  s_ok[w][lane] = ok ? 1 : 0;
  __syncthreads();
  if (w == 0) {
    for (int k = 1; k < 16; ++k) {
      hi = maxp(hi, s_hi[k][lane]);
      lo = minp(lo, s_lo[k][lane]);
      ok = ok && s_ok[k][lane] != 0;
    }
    qmax[b] = hi;
    qmin[b] = lo;
    if (feas) feas[b] = (b < batch && ok) ? 1 : 0;
  }
}

// L[b] = sqrt(max(eig[b], 0)) + eps
template <typename T>
__global__ void k_ps_norm_final(int64_t Bp, const T* __restrict__ eig, T eps, T* L) {
#pragma clang fp contract(off)
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b < Bp) L[b] = (T)__builtin_sqrt(maxp(eig[b], T(0))) + eps;
}

}  // namespace purin
