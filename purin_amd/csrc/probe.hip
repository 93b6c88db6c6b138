// Ceiling probes for the resident CP kernel's roofline (libpurin_probe.so).
//
// The resident kernel (resident.hpp) keeps each tile's iterate in LDS and
// registers, so HBM does not bound it: every iteration each workgroup reads
// the shared matrix as per-wavefront chunk streams from L2 and gathers the
// iterate from LDS.  These kernels measure what MI355X delivers for those two
// access patterns alone, with the same launch shape (1024-thread workgroups,
// one per tile, the kernel's dynamic LDS to give the same occupancy):
//   k_probe_stream  per-wavefront linear chunk streams, 3 x 16-byte loads per
//                   lane per 3072-byte chunk, SGPR base + lane offset, U chunks
//                   in flight, the same stream re-read by every workgroup (so
//                   it is served by L2, like the matrix);
//   k_probe_lds     ds_read_b128 at lane-contiguous (conflict-free) addresses,
//                   U reads in flight.
// Measurement only: no counterpart in the reference.  bench.py times them
// beside the kernel and reports the kernel's stream and LDS rates as fractions
// of the best rates these reach.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/purin_probe.h"

namespace {

typedef uint32_t U4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ U4 gload16(uint64_t wave_base, uint32_t off) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)wave_base);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(wave_base >> 32));
  const __attribute__((address_space(1))) unsigned char* base =
      (const __attribute__((address_space(1))) unsigned char*)(((uint64_t)hi << 32) | lo);
  return *reinterpret_cast<const __attribute__((address_space(1))) U4*>(base + off);
}

template <int U>
__global__ __launch_bounds__(1024) void k_probe_stream(const unsigned char* __restrict__ buf,
                                                       uint32_t wave_chunks, int iters,
                                                       uint32_t* __restrict__ sink) {
  extern __shared__ unsigned char lds_pin[];  // sized by the launch: occupancy only
  constexpr uint32_t CB = 3072u;
  const uint32_t lane16 = (threadIdx.x & 63u) * 16u;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const uint64_t wbase = (uint64_t)(uintptr_t)buf + (uint64_t)wave * wave_chunks * CB;
  U4 acc = {0u, 0u, 0u, 0u};
  for (int it = 0; it < iters; ++it) {
    for (uint32_t c = 0; c < wave_chunks; c += U) {
      U4 v[U][3];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint64_t cb = wbase + (uint64_t)(c + u) * CB;
        v[u][0] = gload16(cb, lane16);
        v[u][1] = gload16(cb, 1024u + lane16);
        v[u][2] = gload16(cb, 2048u + lane16);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2];
    }
  }
  // a per-lane vector store that the loads' results feed (never taken for the
  // probe's zero-filled buffers), so the loads are not removed
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9E3779B9u) sink[threadIdx.x] = acc.x;
}

template <int U>
__global__ __launch_bounds__(1024) void k_probe_lds(int iters, uint32_t span_mask,
                                                    uint32_t* __restrict__ sink) {
  extern __shared__ __align__(16) unsigned char lds[];
  const uint32_t t = threadIdx.x;
  U4* l4 = reinterpret_cast<U4*>(lds);
  for (uint32_t i = t; i * 16u <= span_mask; i += 1024u) l4[i] = U4{i, i ^ 1u, i ^ 2u, i ^ 3u};
  __syncthreads();
  U4 acc = {0u, 0u, 0u, 0u};
  uint32_t a = t * 16u;
  for (int it = 0; it < iters; ++it) {
    U4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = l4[((a + (uint32_t)u * 16384u) & span_mask) >> 4];
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
    a += 1024u;  // stays lane-contiguous: a wave reads 64 consecutive 16-byte entries
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9E3779B9u) sink[t] = acc.x;
}

}  // namespace

extern "C" {

int purin_probe_stream(void* stream, const void* buf, int64_t buf_bytes, int64_t wave_chunks,
                       int32_t iters, int32_t groups, int32_t lds_bytes, int32_t unroll,
                       int32_t reps, void* sink, int64_t sink_bytes, double* ms_per_launch) {
  if (!buf || !sink || !ms_per_launch || wave_chunks < 1 || iters < 1 || groups < 1 ||
      reps < 1 || lds_bytes < 0 || lds_bytes > 160 * 1024 || sink_bytes < 4096)
    return 1;
  if (unroll < 1 || wave_chunks % unroll != 0 || wave_chunks > (int64_t)1 << 20) return 1;
  // 16 wavefronts, each reading its own wave_chunks chunks of 3072 bytes
  if (16 * wave_chunks * 3072 > buf_bytes) return 1;
  hipStream_t st = (hipStream_t)stream;
  void (*kern)(const unsigned char*, uint32_t, int, uint32_t*) = nullptr;
  switch (unroll) {
    case 1: kern = k_probe_stream<1>; break;
    case 2: kern = k_probe_stream<2>; break;
    case 4: kern = k_probe_stream<4>; break;
    default: return 1;
  }
  if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                          lds_bytes) != hipSuccess)
    return 2;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 2;
  hipError_t e = hipEventRecord(e0, st);
  for (int r = 0; r < reps && e == hipSuccess; ++r) {
    kern<<<dim3((unsigned)groups), dim3(1024), (size_t)lds_bytes, st>>>(
        (const unsigned char*)buf, (uint32_t)wave_chunks, iters, (uint32_t*)sink);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipEventRecord(e1, st);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (e != hipSuccess) return 2;
  *ms_per_launch = (double)ms / reps;
  return 0;
}

int purin_probe_lds(void* stream, int32_t iters, int32_t groups, int32_t lds_bytes,
                    int32_t unroll, int32_t reps, void* sink, int64_t sink_bytes,
                    double* ms_per_launch) {
  if (!sink || !ms_per_launch || iters < 1 || groups < 1 || reps < 1 ||
      lds_bytes < 65536 || lds_bytes > 160 * 1024 || sink_bytes < 4096)
    return 1;
  hipStream_t st = (hipStream_t)stream;
  void (*kern)(int, uint32_t, uint32_t*) = nullptr;
  switch (unroll) {
    case 1: kern = k_probe_lds<1>; break;
    case 2: kern = k_probe_lds<2>; break;
    case 4: kern = k_probe_lds<4>; break;
    case 8: kern = k_probe_lds<8>; break;
    default: return 1;
  }
  if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                          lds_bytes) != hipSuccess)
    return 2;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 2;
  hipError_t e = hipEventRecord(e0, st);
  for (int r = 0; r < reps && e == hipSuccess; ++r) {
    // a 64 KiB span (4096 entries): within every launch's LDS (>= 64 KiB)
    kern<<<dim3((unsigned)groups), dim3(1024), (size_t)lds_bytes, st>>>(iters, 0xFFFFu,
                                                                        (uint32_t*)sink);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipEventRecord(e1, st);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (e != hipSuccess) return 2;
  *ms_per_launch = (double)ms / reps;
  return 0;
}

}  // extern "C"
