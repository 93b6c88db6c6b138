// Resident fixed-iteration CP kernel: one workgroup keeps a tile of BT samples
// on chip for every iteration of the solve.
//
// Per workgroup (1024 threads = 16 wavefronts):
//   LDS      two regions, samples interleaved so a gather reads BT consecutive
//            values with one 16-byte load:
//              Gy[(n+1) * BT]  ybar, read by the row pass, written by the column pass
//              Gd[(m+1) * BT]  d+,   read by the column pass, written by the row pass
//            Entry n of Gy and entry m of Gd stay zero: padding entries of the
//            sliced-ELL matrix point there, so the gather loops have no branches.
//   VGPRs    y of the thread's columns and d of its rows, for the BT samples.
//   streamed the tile's yhat and scaled rhs in slot order (coalesced; they stay in
//            L2/MALL across iterations) and the matrix in 64-lane sliced ELL.
// Rows and columns are assigned to (slot, thread) in decreasing-degree order so
// the lanes of a wavefront walk rows/columns of (almost) equal length.
//
// One iteration (reference src/purin/solvers/chambolle_pock/kernels.py:91-150):
//   row pass   d <- P(d + sigma (K ybar - r)); Gd <- d          (reads Gy only)
//   barrier
//   col pass   y+ = clip(a y - delta K^T d+ + delta yhat, lo, hi);
//              Gy <- y+ + theta (y+ - y); y <- y+                (reads Gd only)
//   barrier
// Only the fixed-iteration mode runs here; the per-sample stop test uses the
// streaming passes (kernels.hpp).
#pragma once

#include "common.hpp"

namespace purin {

template <typename T>
struct Res {
  int n, m, me;
  int64_t Bp;
  const int32_t* __restrict__ rowmap;  // [SL * NT]
  const int32_t* __restrict__ colmap;  // [SL * NT]
  const int32_t* __restrict__ rslice;  // per 64-slot slice {offset, width}
  const int32_t* __restrict__ cslice;
  const int32_t* __restrict__ ridx;    // padding points at column n (zero slot)
  const T* __restrict__ rval;
  const int32_t* __restrict__ cidx;    // padding points at row m (zero slot)
  const T* __restrict__ cval;
  const T* __restrict__ Ts;   // [tiles][SL*NT][BT] targets in slot order
  const T* __restrict__ Rs;   // [tiles][SL*NT][BT] scaled rhs in slot order
  const T* __restrict__ D0s;  // [tiles][SL*NT][BT] initial duals in slot order
  const T* __restrict__ Ls;   // shared: [SL*NT]; else [tiles][SL*NT][BT]
  const T* __restrict__ Hs;
  int shared_bounds;
  const T* __restrict__ sched;  // [iters][4] = sigma, a, delta, theta
  int64_t iters;
  T* Y;  // n x Bp
  T* D;  // m x Bp
};

template <typename T, int BT>
struct Pack;
template <>
struct Pack<double, 2> {
  typedef double V __attribute__((ext_vector_type(2)));
};
template <>
struct Pack<float, 4> {
  typedef float V __attribute__((ext_vector_type(4)));
};

// sum_q val[q] * G[idx[q]] over one sliced-ELL slice, 4 entries per step with
// the index/value loads of a step issued before its LDS gathers.
template <typename T, int BT>
__device__ __forceinline__ typename Pack<T, BT>::V slice_dot(const int32_t* __restrict__ idx,
                                                             const T* __restrict__ val,
                                                             const typename Pack<T, BT>::V* G,
                                                             int off, int width, int lane) {
  using V = typename Pack<T, BT>::V;
  V acc = V(T(0));
  int q = 0;
  for (; q + 4 <= width; q += 4) {
    int j[4];
    T v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      j[u] = idx[off + (q + u) * 64 + lane];
      v[u] = val[off + (q + u) * 64 + lane];
    }
    V x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = G[j[u]];
#pragma unroll
    for (int u = 0; u < 4; ++u) acc += v[u] * x[u];
  }
  for (; q < width; ++q) {
    const int jj = idx[off + q * 64 + lane];
    const T vv = val[off + q * 64 + lane];
    acc += vv * G[jj];
  }
  return acc;
}

template <typename T, int BT, int SL, bool SB>
__global__ __launch_bounds__(1024) void k_resident(Res<T> A) {
  constexpr int NT = 1024;
  using V = typename Pack<T, BT>::V;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  V* Gy = reinterpret_cast<V*>(smem_raw);
  V* Gd = Gy + (A.n + 1);
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int64_t tile = blockIdx.x;
  const V vzero = V(T(0));

  int ri[SL], cj[SL];
#pragma unroll
  for (int r = 0; r < SL; ++r) ri[r] = A.rowmap[r * NT + t];
#pragma unroll
  for (int c = 0; c < SL; ++c) cj[c] = A.colmap[c * NT + t];

  const V* Ts = reinterpret_cast<const V*>(A.Ts) + tile * (int64_t)(SL * NT);
  const V* Rs = reinterpret_cast<const V*>(A.Rs) + tile * (int64_t)(SL * NT);
  const V* D0 = reinterpret_cast<const V*>(A.D0s) + tile * (int64_t)(SL * NT);
  V y[SL], d[SL];
#pragma unroll
  for (int c = 0; c < SL; ++c) {
    y[c] = cj[c] >= 0 ? Ts[c * NT + t] : vzero;
    if (cj[c] >= 0) Gy[cj[c]] = y[c];  // ybar0 = y0 = yhat
  }
#pragma unroll
  for (int r = 0; r < SL; ++r) {
    d[r] = ri[r] >= 0 ? D0[r * NT + t] : vzero;
    if (ri[r] >= 0) Gd[ri[r]] = vzero;
  }
  if (t == 0) {
    Gy[A.n] = vzero;
    Gd[A.m] = vzero;
  }
  __syncthreads();

  for (int64_t it = 0; it < A.iters; ++it) {
    const T sigma = A.sched[4 * it], a = A.sched[4 * it + 1];
    const T delta = A.sched[4 * it + 2], theta = A.sched[4 * it + 3];
    // ---- row pass (reads Gy, writes Gd) ---------------------------------------
#pragma unroll
    for (int r = 0; r < SL; ++r) {
      if (ri[r] < 0) continue;
      const int z = r * (NT / 64) + wave;
      const V acc = slice_dot<T, BT>(A.ridx, A.rval, Gy, A.rslice[2 * z], A.rslice[2 * z + 1],
                                     lane);
      const V rr = Rs[r * NT + t];
      V p = d[r] + sigma * (acc - rr);
      if (ri[r] >= A.me) {
#pragma unroll
        for (int s = 0; s < BT; ++s) p[s] = maxp(p[s], T(0));
      }
      d[r] = p;
      Gd[ri[r]] = p;
    }
    __syncthreads();
    // ---- column pass (reads Gd, writes Gy) --------------------------------------
#pragma unroll
    for (int c = 0; c < SL; ++c) {
      if (cj[c] < 0) continue;
      const int z = c * (NT / 64) + wave;
      const V tt = slice_dot<T, BT>(A.cidx, A.cval, Gd, A.cslice[2 * z], A.cslice[2 * z + 1],
                                    lane);
      const V tg = Ts[c * NT + t];
      V lo, hi;
      if (SB) {
        lo = V(A.Ls[c * NT + t]);
        hi = V(A.Hs[c * NT + t]);
      } else {
        lo = reinterpret_cast<const V*>(A.Ls)[tile * (int64_t)(SL * NT) + c * NT + t];
        hi = reinterpret_cast<const V*>(A.Hs)[tile * (int64_t)(SL * NT) + c * NT + t];
      }
      const V sv = a * y[c] - delta * tt + delta * tg;
      V yn;
#pragma unroll
      for (int s = 0; s < BT; ++s) yn[s] = clipp(sv[s], lo[s], hi[s]);
      Gy[cj[c]] = yn + theta * (yn - y[c]);
      y[c] = yn;
    }
    __syncthreads();
  }
  // ---- hand the state to the batch-minor layout ---------------------------------
  const int64_t b0 = tile * BT;
#pragma unroll
  for (int c = 0; c < SL; ++c)
    if (cj[c] >= 0)
#pragma unroll
      for (int s = 0; s < BT; ++s) A.Y[(int64_t)cj[c] * A.Bp + b0 + s] = y[c][s];
#pragma unroll
  for (int r = 0; r < SL; ++r)
    if (ri[r] >= 0)
#pragma unroll
      for (int s = 0; s < BT; ++s) A.D[(int64_t)ri[r] * A.Bp + b0 + s] = d[r][s];
}

// dst[(tile*K + k)*BT + s] = src[map[k]*Bp + tile*BT + s] (0 for empty slots)
template <typename T, int BT>
__global__ void k_res_gather(const T* __restrict__ src, int64_t Bp, const int32_t* __restrict__ map,
                             int K, int64_t tiles, T* __restrict__ dst) {
  const int64_t total = tiles * K * BT;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int s = (int)(e % BT);
    const int64_t rest = e / BT;
    const int k = (int)(rest % K);
    const int64_t tile = rest / K;
    const int32_t j = map[k];
    dst[e] = j >= 0 ? src[(int64_t)j * Bp + tile * BT + s] : T(0);
  }
}

template <typename T>
__global__ void k_res_gather_shared(const T* __restrict__ src, const int32_t* __restrict__ map,
                                    int K, T* __restrict__ dst) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k < K) dst[k] = map[k] >= 0 ? src[map[k]] : T(0);
}

}  // namespace purin
