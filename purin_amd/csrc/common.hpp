// Shared device helpers for the CDNA4 (gfx950) Chambolle--Pock kernels.
//
// Internal layout: every per-sample vector is stored batch-minor, element e of
// sample b at [e * Bp + b], with Bp the batch rounded up to whole wavefront
// tiles.  A wavefront lane owns S consecutive samples (16 bytes: 2 doubles or
// 4 floats), so one wave moves 1 KiB per load and the matrix entries the wave
// walks (a row or a column of K) are wave-uniform scalar loads.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstddef>
#include <cstdint>

namespace purin {

constexpr int kWave = 64;
constexpr int kBlock = 256;  // 4 wavefronts
// ints per wavefront of the resident kernels' wave table: first chunk; the
// chunk counts of the row slots and of the column slots (4 x u8 each); the
// slots' entries in their last chunk, rows and columns (4 x u8 each); the row
// and column section chunk counts; flags: bit 0 (1) when the first row slot
// spans two or more chunks, bit 1 (2) when the first column slot does
constexpr int kResWtab = 8;

// Batch tile and first row / column block of a block of a (tiles x blocks)
// grid.  Blocks are dealt to the 8 XCDs round-robin in launch order (x
// fastest).  With more than 8 batch tiles (a multiple of 8), an XCD's
// consecutive blocks walk one tile's row / column blocks before the next
// tile's, so the few tiles an XCD holds at once keep their gathered vectors in
// its L2; otherwise blockIdx.x is the tile (every tile stays on one XCD).
__device__ __forceinline__ void tile_block(int64_t& tile, int& blk) {
  const unsigned X = gridDim.x, Y = gridDim.y;
  if (X > 8 && (X & 7u) == 0) {
    const unsigned L = blockIdx.y * X + blockIdx.x;
    const unsigned j = L >> 3;
    tile = (int64_t)((L & 7u) + 8u * (j / Y));
    blk = (int)(j % Y);
  } else {
    tile = blockIdx.x;
    blk = (int)blockIdx.y;
  }
}

template <typename T>
struct Lane;
template <>
struct Lane<double> {
  static constexpr int S = 2;
  typedef double V __attribute__((ext_vector_type(2)));
};
template <>
struct Lane<float> {
  static constexpr int S = 4;
  typedef float V __attribute__((ext_vector_type(4)));
};

// Samples per wavefront tile and per block tile.
template <typename T>
constexpr int tile_samples() {
  return kWave * Lane<T>::S;
}

inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

template <typename T>
__device__ __forceinline__ typename Lane<T>::V vload(const T* p) {
  return *reinterpret_cast<const typename Lane<T>::V*>(p);
}
// Load of a value read once: marked nontemporal so it does not displace gathered
// vectors from L2.
template <typename T>
__device__ __forceinline__ typename Lane<T>::V vload_once(const T* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const typename Lane<T>::V*>(p));
}
template <typename T>
__device__ __forceinline__ void vstore(T* p, typename Lane<T>::V v) {
  *reinterpret_cast<typename Lane<T>::V*>(p) = v;
}
// Store of a value not read again by this kernel: nontemporal, like vload_once.
template <typename T>
__device__ __forceinline__ void vstore_once(T* p, typename Lane<T>::V v) {
  __builtin_nontemporal_store(v, reinterpret_cast<typename Lane<T>::V*>(p));
}
// A load or store of a streamed vector: nontemporal when NT.
template <bool NT, typename T>
__device__ __forceinline__ typename Lane<T>::V vload_s(const T* p) {
  if constexpr (NT) return vload_once(p);
  else return vload(p);
}
template <bool NT, typename T>
__device__ __forceinline__ void vstore_s(T* p, typename Lane<T>::V v) {
  if constexpr (NT) vstore_once(p, v);
  else vstore(p, v);
}
template <typename T>
__device__ __forceinline__ typename Lane<T>::V vsplat(T x) {
  typename Lane<T>::V v;
#pragma unroll
  for (int s = 0; s < Lane<T>::S; ++s) v[s] = x;
  return v;
}

// NaN-propagating max/min (jnp.maximum / jnp.minimum semantics).
template <typename T>
__device__ __forceinline__ T maxp(T x, T y) {
  return (x != x) ? x : ((y != y) ? y : (x > y ? x : y));
}
template <typename T>
__device__ __forceinline__ T minp(T x, T y) {
  return (x != x) ? x : ((y != y) ? y : (x < y ? x : y));
}
// jnp.clip(x, lo, hi) == minimum(maximum(x, lo), hi)
template <typename T>
__device__ __forceinline__ T clipp(T x, T lo, T hi) {
  return minp(maxp(x, lo), hi);
}
__device__ __forceinline__ double hypotv(double x, double y) { return ::hypot(x, y); }
__device__ __forceinline__ float hypotv(float x, float y) { return ::hypotf(x, y); }
__device__ __forceinline__ double absv(double x) { return __builtin_fabs(x); }
__device__ __forceinline__ float absv(float x) { return __builtin_fabsf(x); }
template <typename T>
__device__ __forceinline__ bool finite(T x) {
  return __builtin_isfinite(x);
}

// Block-wide (4 waves) combine of one value per lane-sample, in wave order.
// ``buf`` holds kBlock*S elements of LDS.  Returns the combined value in
// wave 0's lanes (other waves' return values are unspecified).
template <typename T, typename Op>
__device__ __forceinline__ typename Lane<T>::V block_combine(typename Lane<T>::V v, T* buf,
                                                             Op op) {
  constexpr int S = Lane<T>::S;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int s = 0; s < S; ++s) buf[(wave * kWave + lane) * S + s] = v[s];
  __syncthreads();
  typename Lane<T>::V out = v;
  if (wave == 0) {
#pragma unroll
    for (int w = 1; w < 4; ++w) {
#pragma unroll
      for (int s = 0; s < S; ++s) out[s] = op(out[s], buf[(w * kWave + lane) * S + s]);
    }
  }
  __syncthreads();
  return out;
}

struct OpAdd {
  template <typename T>
  __device__ T operator()(T a, T b) const { return a + b; }
};
struct OpMax {
  template <typename T>
  __device__ T operator()(T a, T b) const { return maxp(a, b); }
};
struct OpMin {
  template <typename T>
  __device__ T operator()(T a, T b) const { return minp(a, b); }
};

}  // namespace purin
