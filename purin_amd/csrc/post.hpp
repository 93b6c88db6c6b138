// Post-processing of a projection on the device: dual unscaling and placement,
// bound-multiplier recovery, original-unit residuals, slacks and status codes.
// Reference: src/purin/solvers/chambolle_pock/bounds.py:247-317.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace purin {

template <typename T>
struct Post {
  Mat<T> K;                      // kept rows, ORIGINAL coefficients
  int64_t Bp, me, mi;
  const T* __restrict__ scale;   // m
  const T* __restrict__ scale_b; // per-sample coefficients: [m][Bp] scales, else nullptr
  const int32_t* __restrict__ kept;
  const int32_t* __restrict__ bptr;
  const int32_t* __restrict__ brow;
  const T* __restrict__ bcoef;
  const T* __restrict__ bcoef_b; // per-sample coefficients: [nb][Bp], else nullptr
  // general diagonal QP (diagonal_qp.py:276-319): q, c [n][Bp]; stationarity
  // is max |y - clip(y - (q y + c + K^T dual), lo, hi)| and there are no bound rows
  const T* __restrict__ Q;
  const T* __restrict__ Cc;
  const T* __restrict__ tgt;     // n x Bp
  // n x Bp or nullptr: K~^T d of the final diagnostics pass (k_col_pass MODE 2),
  // the same sum K^T (d * scale) with the scale folded into the coefficients
  const T* __restrict__ TK;
  // with KY set: K~y of the final diagnostics pass, stored at each kept row's
  // full-row position of DF (read there before the multiplier overwrites it)
  bool KY;
  const T* __restrict__ Y;       // n x Bp
  const T* __restrict__ D;       // m x Bp (scaled duals)
  const T* __restrict__ RF;      // M x Bp (original rhs)
  const T* __restrict__ LO;
  const T* __restrict__ HI;
  int shared_bounds;
  T* DF;                         // M x Bp multipliers
  T* SL;                         // mi x Bp slacks
  T* rowpart;                    // [2][nrb][Bp]: residual max, finite(dual)
  T* colpart;                    // [3][ncb][Bp]: residual max (bound rows), stationarity, finite
  int nrb, ncb;
};

// Row scale of kept row i / coefficient of bound row k for the S samples from b0.
template <typename T>
__device__ __forceinline__ typename Lane<T>::V post_scale(const Post<T>& P, int i, int64_t b0) {
  return P.scale_b ? vload(P.scale_b + (size_t)i * P.Bp + b0) : vsplat<T>(P.scale[i]);
}
template <typename T>
__device__ __forceinline__ typename Lane<T>::V post_bcoef(const Post<T>& P, int k, int64_t b0) {
  return P.bcoef_b ? vload(P.bcoef_b + (size_t)k * P.Bp + b0) : vsplat<T>(P.bcoef[k]);
}

// Right-hand side of bound row ``row`` for the S samples from b0: with shared
// bounds the caller promises every sample's bound rows are equal and only
// sample 0 is read (include/purin_cp.h, shared_bounds).
template <typename T>
__device__ __forceinline__ typename Lane<T>::V post_bound_rhs(const Post<T>& P, int64_t row,
                                                              int64_t b0) {
  const T* r = P.RF + (size_t)row * P.Bp;
  return P.shared_bounds ? vsplat<T>(r[0]) : vload(r + b0);
}

// Kept rows: multiplier = d * scale (bounds.py:247), r = K y - rhs (285-289),
// slack = max(-r, 0) for inequality rows (311).
template <typename T, int RPW>
__global__ __launch_bounds__(kBlock) void k_post_rows(Post<T> P) {
  using V = typename Lane<T>::V;
  constexpr int S = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int64_t tile;
  int blk0;
  tile_block(tile, blk0);
  const int64_t b0 = (tile * kWave + lane) * S;
  const T zero = T(0);
  for (int rb = blk0; rb * 4 * RPW < P.K.m; rb += gridDim.y) {
    V res = vsplat<T>(zero), fin = vsplat<T>(T(1));
    for (int c = 0; c < RPW; ++c) {
      const int i = (rb * 4 + wave) * RPW + c;
      if (i >= P.K.m) break;
      const int64_t row = P.kept[i];
      V acc = vsplat<T>(zero);
      if (P.KY) {  // K y = K~y / scale
        acc = vload(P.DF + (size_t)row * P.Bp + b0) / post_scale(P, i, b0);
      } else {
        const int s0 = P.K.rptr[i], s1 = P.K.rptr[i + 1];
        for (int k = s0; k < s1; ++k)
          acc += row_coef(P.K, k, b0) * vload(P.Y + (size_t)P.K.ridx[k] * P.Bp + b0);
      }
      const V d = vload(P.D + (size_t)i * P.Bp + b0);
      const V full = d * post_scale(P, i, b0);
      vstore(P.DF + (size_t)row * P.Bp + b0, full);
      const V r = acc - vload(P.RF + (size_t)row * P.Bp + b0);
      if (row < P.me) {
#pragma unroll
        for (int s = 0; s < S; ++s) res[s] = maxp(res[s], absv(r[s]));
      } else {
        V sl;
#pragma unroll
        for (int s = 0; s < S; ++s) {
          res[s] = maxp(res[s], maxp(r[s], zero));
          sl[s] = maxp(-r[s], zero);
        }
        vstore(P.SL + (size_t)(row - P.me) * P.Bp + b0, sl);
      }
#pragma unroll
      for (int s = 0; s < S; ++s)
        if (!finite(full[s])) fin[s] = zero;
    }
    __shared__ T buf[kBlock * S];
    const V p0 = block_combine<T>(res, buf, OpMax());
    const V p1 = block_combine<T>(fin, buf, OpMin());
    if (wave == 0) {
      T* base = P.rowpart + (size_t)rb * P.Bp + b0;
      vstore(base, p0);
      vstore(base + (size_t)P.nrb * P.Bp, p1);
    }
  }
}

// Variables: base stationarity y - yhat + K_kept^T dual (bounds.py:248-249),
// bound multipliers split among tied rows (252-284), bound-row residuals and
// slacks (285-289, 311), full stationarity (290).
template <typename T, int CPW>
__global__ __launch_bounds__(kBlock) void k_post_cols(Post<T> P) {
  using V = typename Lane<T>::V;
  constexpr int S = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int64_t tile;
  int blk0;
  tile_block(tile, blk0);
  const int64_t b0 = (tile * kWave + lane) * S;
  const T zero = T(0), one = T(1);
  for (int cb = blk0; cb * 4 * CPW < P.K.n; cb += gridDim.y) {
    V res = vsplat<T>(zero), stat = vsplat<T>(zero), fin = vsplat<T>(one);
    for (int c = 0; c < CPW; ++c) {
      const int j = (cb * 4 + wave) * CPW + c;
      if (j >= P.K.n) break;
      const size_t off = (size_t)j * P.Bp + b0;
      V tk = vsplat<T>(zero);
      if (P.TK) {
        tk = vload(P.TK + off);
      } else {
        const int s0 = P.K.cptr[j], s1 = P.K.cptr[j + 1];
        for (int k = s0; k < s1; ++k) {
          const int i = P.K.cidx[k];
          tk += col_coef(P.K, k, b0) * (vload(P.D + (size_t)i * P.Bp + b0) * post_scale(P, i, b0));
        }
      }
      const V y = vload(P.Y + off);
      V lo, hi;
      if (P.shared_bounds) {
        lo = vsplat<T>(P.LO[j]);
        hi = vsplat<T>(P.HI[j]);
      } else {
        lo = vload(P.LO + off);
        hi = vload(P.HI + off);
      }
      if (P.Q) {
        const V q = vload(P.Q + off), cc = vload(P.Cc + off);
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const T g = y[s] - clipp(y[s] - ((q[s] * y[s] + cc[s]) + tk[s]), lo[s], hi[s]);
          stat[s] = maxp(stat[s], absv(g));
          if (!finite(y[s])) fin[s] = zero;
        }
        continue;
      }
      const V dy = y - vload(P.tgt + off);
      const V base = dy + tk;
      const int k0 = P.bptr[j], k1 = P.bptr[j + 1];
      V lc = vsplat<T>(zero), uc = vsplat<T>(zero);
      for (int k = k0; k < k1; ++k) {
        const V cfv = post_bcoef(P, k, b0);
        const V rr = post_bound_rhs(P, P.brow[k], b0);
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const T cf = cfv[s];
          const T th = rr[s] / (cf != zero ? cf : one);
          lc[s] += (cf < zero && th == lo[s] && y[s] == lo[s]) ? one : zero;
          uc[s] += (cf > zero && th == hi[s] && y[s] == hi[s]) ? one : zero;
        }
      }
      V tfull = tk;
      for (int k = k0; k < k1; ++k) {
        const V cfv = post_bcoef(P, k, b0);
        const int64_t row = P.brow[k];
        const V rr = post_bound_rhs(P, row, b0);
        V bd, sl;
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const T cf = cfv[s];
          const T th = rr[s] / (cf != zero ? cf : one);
          const bool il = cf < zero && th == lo[s] && y[s] == lo[s];
          const bool iu = cf > zero && th == hi[s] && y[s] == hi[s];
          T v = il ? maxp(base[s], zero) / maxp(lc[s], one) : zero;
          v = v + (iu ? maxp(-base[s], zero) / maxp(uc[s], one) : zero);
          v = v / (cf != zero ? absv(cf) : one);
          bd[s] = v;
          tfull[s] += cf * v;
          const T r = cf * y[s] - rr[s];
          res[s] = maxp(res[s], maxp(r, zero));
          sl[s] = maxp(-r, zero);
          if (!finite(v)) fin[s] = zero;
        }
        vstore(P.DF + (size_t)row * P.Bp + b0, bd);
        vstore(P.SL + (size_t)(row - P.me) * P.Bp + b0, sl);
      }
#pragma unroll
      for (int s = 0; s < S; ++s) {
        stat[s] = maxp(stat[s], absv(dy[s] + tfull[s]));
        if (!finite(y[s])) fin[s] = zero;
      }
    }
    __shared__ T buf[kBlock * S];
    const V p0 = block_combine<T>(res, buf, OpMax());
    const V p1 = block_combine<T>(stat, buf, OpMax());
    const V p2 = block_combine<T>(fin, buf, OpMin());
    if (wave == 0) {
      const size_t plane = (size_t)P.ncb * P.Bp;
      T* base = P.colpart + (size_t)cb * P.Bp + b0;
      vstore(base, p0);
      vstore(base + plane, p1);
      vstore(base + 2 * plane, p2);
    }
  }
}

// Per-sample verdict (bounds.py:285-305).  A block of kDecideGroups x 64
// threads owns 64 samples: group g takes the row and column chunks c = g,
// g + G, ...; the groups combine in LDS (max and "and": order-independent).
// Grid: Bp / 64 blocks.
template <typename T>
__global__ __launch_bounds__(64 * kDecideGroups) void k_post_final(
    Post<T> P, int64_t batch, T tol_cfg, T residual_factor, const int32_t* __restrict__ cp_conv,
    const T* __restrict__ cp_gap, const int32_t* __restrict__ count, int32_t* status,
    int32_t* iterations, T* residual_out, uint8_t* finite_out, uint8_t* eligible_out) {
  constexpr int G = kDecideGroups;
  __shared__ T buf[G][64];
  const int lane = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int64_t b = (int64_t)blockIdx.x * 64 + lane;  // < Bp by the grid
  const T zero = T(0);
  T q[3] = {zero, zero, T(1)};  // residual, stationarity, finite
  for (int r = g; r < P.nrb; r += G) {
    const T* p = P.rowpart + (size_t)r * P.Bp + b;
    q[0] = maxp(q[0], p[0]);
    if (p[(size_t)P.nrb * P.Bp] == zero) q[2] = zero;
  }
  const size_t plane = (size_t)P.ncb * P.Bp;
  for (int c = g; c < P.ncb; c += G) {
    const T* p = P.colpart + (size_t)c * P.Bp + b;
    q[0] = maxp(q[0], p[0]);
    q[1] = maxp(q[1], p[plane]);
    if (p[2 * plane] == zero) q[2] = zero;
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    buf[g][lane] = q[k];
    __syncthreads();
    if (g == 0) {
      T v = buf[0][lane];
      for (int h = 1; h < G; ++h) {
        const T o = buf[h][lane];
        v = k < 2 ? maxp(v, o) : ((v != zero && o != zero) ? T(1) : zero);
      }
      q[k] = v;
    }
    __syncthreads();
  }
  if (g != 0 || b >= batch) return;
  const T res = q[0], stat = q[1];
  const bool fin = q[2] != zero;
  const T residual = maxp(res, stat);
  // the QP's finiteness omits the gap (diagonal_qp.py:291-295)
  const bool f = fin && finite(residual) && (P.Q || finite(cp_gap[b]));
  const bool conv = f && cp_conv[b] != 0 && residual <= tol_cfg;
  if (status) status[b] = conv ? 0 : (f ? 1 : 3);
  if (iterations) iterations[b] = count[b];
  if (residual_out) residual_out[b] = residual * residual_factor;
  if (finite_out) finite_out[b] = f ? 1 : 0;
  if (eligible_out) eligible_out[b] = conv ? 1 : 0;
}

}  // namespace purin
