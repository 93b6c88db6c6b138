// Resident fixed-iteration CP kernel: one workgroup keeps a tile of BT samples
// on chip for every iteration of the solve.
//
// Per workgroup (1024 threads = 16 wavefronts), BT samples (2 fp64 / 4 fp32,
// 16 bytes) interleaved so that one gathered element is one ds_read_b128:
//   LDS      16-byte entries  Gy[0, n) | zero | Gd[0, m) | trash
//              Gy  ybar, read by the row pass, written by the column pass
//              Gd  d+,   read by the column pass, written by the row pass
//              zero stays 0: padding entries of the matrix stream point there
//              trash takes the stores of lanes that own no row / column
//   VGPRs    per thread and slot: y of its columns, the targets yhat and the
//            scaled right-hand sides, for the BT samples (loaded once)
//   stream   the shared matrix, read every iteration from L2: one linear
//            stream of chunks per wavefront (row slots, column slots, then a
//            copy of the first chunk), a chunk being 4 entries per lane stored
//            as {LDS byte address of the gathered element, coefficient}.  The
//            slots of a pass are packed back to back (a slot may begin and end
//            inside a chunk; only each pass's end is padded to a whole chunk).
//            The loads are raw buffer loads (the stream in a buffer resource,
//            the chunk's offset scalar, the lane's vector), and the
//            next chunk is always in flight while the current one is gathered,
//            across slot, pass and iteration boundaries.
// Rows and columns are assigned to (slot, thread) in decreasing-degree order
// so the lanes of a wavefront walk rows / columns of (almost) equal length.
//
// One iteration (reference src/purin/solvers/chambolle_pock/kernels.py:91-150):
//   row pass   d <- P(d + sigma (K ybar - r)); Gd <- d      (reads Gy and own Gd)
//   barrier
//   col pass   y+ = clip(a y - delta K^T d+ + delta yhat, lo, hi);
//              Gy <- y+ + theta (y+ - y); y <- y+            (reads Gd only)
//   barrier
// The arithmetic (operand order, fused multiply-adds) is that of the
// streaming passes in kernels.hpp; each row's and column's sum runs in the
// order the plan scheduled its gathers (for LDS classes), so the two paths
// agree to rounding.  k_resident runs the fixed-iteration mode;
// k_resident_early (below) adds the per-sample stop test.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace purin {

constexpr int kResChunk = 4;      // matrix entries per lane in one stream chunk
constexpr int kResWaves = 16;     // wavefronts of a resident workgroup

// One workgroup per CU, four wavefronts per SIMD, up to 128 VGPRs each.  (With
// one row and one column slot per thread the 8-sample fp32 tile's two LDS
// planes, 64 KB, would let two workgroups share a CU at 64 VGPRs per
// wavefront; the kernels then spill 164-180 bytes per lane and run 3x slower
// at config 4: 157 against 51 ms per 500-iteration launch.)

template <typename T>
struct ResVec;
template <>
struct ResVec<double> {
  static constexpr int BT = 2;
  typedef double V __attribute__((ext_vector_type(2)));
};
template <>
struct ResVec<float> {
  static constexpr int BT = 4;
  typedef float V __attribute__((ext_vector_type(4)));
};

// NB samples of a tile: one 16-byte LDS entry per gathered element (NB = 16 /
// sizeof(T)), or, for fp32 tiles of 8 samples, two 16-byte entries in two
// planes kResPlane bytes apart.  The second plane's read takes the first's
// address plus an immediate offset, so the matrix stream (plane-0 addresses),
// the LDS placement and its bank-class schedule serve both planes unchanged.
// Two planes are used where one row and one column slot per thread hold the
// problem (n, m <= 1024): the plane stride is then a constant that fits the
// instruction's offset field, and the registers have room for 8 samples.
template <typename T, int NB>
struct ResV;
template <>
struct ResV<double, 2> {
  typedef double V __attribute__((ext_vector_type(2)));
};
template <>
struct ResV<float, 4> {
  typedef float V __attribute__((ext_vector_type(4)));
};
template <>
struct ResV<float, 8> {
  typedef float V __attribute__((ext_vector_type(8)));
};
constexpr uint32_t kResPlane = (1024u + 1u + 1024u + 1u) * 16u;  // 32,800 B

// Bytes of one chunk of one wavefront: the offsets block (64 lanes x 4 u32 LDS
// byte addresses), then the coefficient blocks (64 lanes x 16 bytes each; 2
// for fp64, 1 for fp32).
template <typename T>
constexpr uint32_t res_chunk_bytes() {
  return 64u * 16u + 64u * kResChunk * (uint32_t)sizeof(T);
}

template <typename T>
struct Res {
  int n, m, me;
  int64_t Bp;
  int Kr, Kc;                          // slot-ordered strides: SLR*1024, SLC*1024
  const int32_t* __restrict__ rowmap;  // [Kr] kept row of each (slot, thread) or -1
  const int32_t* __restrict__ colmap;  // [Kc] column of each (slot, thread) or -1
  // [Kr] / [Kc] LDS entry (16-byte units) of each slot's row / column, or -1:
  // the plan places the entries so that a quarter wavefront's accesses spread
  // over the 16 entry classes (the stream's gather addresses use the same map)
  const int32_t* __restrict__ rowent;
  const int32_t* __restrict__ colent;
  const unsigned char* __restrict__ stream;  // the chunks
  const int32_t* __restrict__ wtab;    // [16][kResWtab]: first chunk; per row slot
                                       // and per column slot (4 x u8 each) its
                                       // chunks and the entries of its last chunk
  const T* __restrict__ Ts;   // [tiles][Kc][BT] targets in slot order
  const T* __restrict__ Rs;   // [tiles][Kr][BT] scaled rhs in slot order
  const T* __restrict__ D0s;  // [tiles][Kr][BT] initial duals in slot order
  const T* __restrict__ Ls;   // shared: [Kc]; else [tiles][Kc][BT]
  const T* __restrict__ Hs;
  const T* __restrict__ sched;  // [iters][4] = sigma, a, delta, theta
  int64_t iters;
  T* Y;  // n x Bp
  T* D;  // m x Bp
  // early-stop kernel only: the per-sample stop test and its outputs
  int64_t batch;
  T tol;                       // tolerance, or per sample from tolv [Bp] when set
  const T* __restrict__ tolv;
  int32_t* done;               // [Bp] accepted (1) or not (0)
  int32_t* count;              // [Bp] iterations committed
  // diagonal QP (k_resident with QP): Ts holds c; q and y0 in slot order; the
  // per-sample steps of iteration 0, [5][Bp] = tau, sigma, a, delta, theta
  // (only tau, sigma and, when accelerated, theta are read); gamma = min q
  // per sample for the accelerated update, or nullptr (fixed steps, theta 1)
  const T* __restrict__ Qs;
  const T* __restrict__ Y0s;
  const T* __restrict__ step0;
  const T* __restrict__ gam;
  int accel;  // per-sample steps (QP, per-sample coefficients): the accelerated update runs
  // per-sample coefficients (k_resident with VALS): each tile's coefficient
  // stream, [tiles][cs_tile] vectors of the tile's samples ([chunk][4][64] per
  // tile, the plan's stream order); the steps are per sample as for the QP,
  // with gamma 1 and the prox a, delta of q = 1 from step0's rows 2 and 3
  const T* __restrict__ Cs;
  int64_t cs_tile;
  // per-sample bounds (k_resident): the leading column slots whose bounds the
  // kernel holds in LDS after the image (the launch's LDS includes them)
  int lb_slots;
};

// One chunk of a wavefront's stream in registers: the lane's 4 LDS addresses
// and coefficients, shared by the tile's samples (CV = T), or per sample (CV =
// the tile's vector type, from the per-tile coefficient stream of per-sample
// coefficients).
template <typename T, typename CV = T>
struct Chunk {
  uint32_t o[kResChunk];
  CV v[kResChunk];
};

// LDS accesses by absolute byte address: the kernel declares no static LDS, so
// its dynamic LDS starts at address 0 and the stream's offsets are addresses.
template <typename V>
__device__ __forceinline__ V lds_read(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) V*>(addr);
}
template <typename V>
__device__ __forceinline__ void lds_write(uint32_t addr, V v) {
  *reinterpret_cast<__attribute__((address_space(3))) V*>(addr) = v;
}

// One gathered element (an entry of Gy, Gd, the zero or the trash entry) at its
// plane-0 address: 16 bytes, or 32 bytes split over the two planes.
template <typename V>
__device__ __forceinline__ V ent_read(uint32_t addr) {
  if constexpr (sizeof(V) == 32) {
    typedef float F4 __attribute__((ext_vector_type(4)));
    typedef const __attribute__((address_space(3))) F4* P4;
    const P4 p = reinterpret_cast<P4>(addr);
    const F4 lo = p[0], hi = p[kResPlane / 16];
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  } else {
    return lds_read<V>(addr);
  }
}
template <typename V>
__device__ __forceinline__ void ent_write(uint32_t addr, V v) {
  if constexpr (sizeof(V) == 32) {
    typedef float F4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) F4* P4;
    const P4 p = reinterpret_cast<P4>(addr);
    p[0] = __builtin_shufflevector(v, v, 0, 1, 2, 3);
    p[kResPlane / 16] = __builtin_shufflevector(v, v, 4, 5, 6, 7);
  } else {
    lds_write<V>(addr, v);
  }
}

// A tile vector in LDS as 16-byte granules ``stride`` bytes apart (one granule,
// or two for a 32-byte vector): the per-sample bounds held on chip, laid out
// so that consecutive lanes read consecutive granules (no bank conflicts).
template <typename V>
__device__ __forceinline__ V lds_read_split(uint32_t addr, uint32_t stride) {
  if constexpr (sizeof(V) == 32) {
    typedef float F4 __attribute__((ext_vector_type(4)));
    const F4 lo = lds_read<F4>(addr), hi = lds_read<F4>(addr + stride);
    return __builtin_bit_cast(V, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  } else {
    return lds_read<V>(addr);
  }
}
template <typename V>
__device__ __forceinline__ void lds_write_split(uint32_t addr, uint32_t stride, V v) {
  if constexpr (sizeof(V) == 32) {
    typedef float F4 __attribute__((ext_vector_type(4)));
    typedef float F8 __attribute__((ext_vector_type(8)));
    const F8 f = __builtin_bit_cast(F8, v);
    lds_write<F4>(addr, __builtin_shufflevector(f, f, 0, 1, 2, 3));
    lds_write<F4>(addr + stride, __builtin_shufflevector(f, f, 4, 5, 6, 7));
  } else {
    lds_write<V>(addr, v);
  }
}

// The chunk at byte ``cbyte`` of the stream (wave-uniform), loaded by each
// lane at its 16-byte offset.
// Per-sample coefficients (CV a vector): the offsets from the stream, the
// coefficients from ``cs``, the tile's coefficient stream, [chunk][4][64] CV.
template <typename T, typename CV = T>
__device__ __forceinline__ void load_chunk(Chunk<T, CV>& c, const unsigned char* __restrict__ stream,
                                           uint64_t cbyte, uint32_t lane16,
                                           const CV* __restrict__ cs = nullptr) {
  // raw buffer loads: the stream's base in a buffer resource (SGPRs, built
  // once per launch), the chunk's byte offset as the scalar offset and the
  // lane's 16 bytes as the vector offset, so a chunk costs no address
  // arithmetic beyond one scalar add per load (the stream is far below 2 GB)
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)stream, 0, 0x7fffffff, 0x00020000);
  const uint32_t cb = (uint32_t)cbyte;
  typedef uint32_t U4 __attribute__((ext_vector_type(4)));
  const U4 o = __builtin_amdgcn_raw_buffer_load_b128(rs, lane16, cb, 0);
  c.o[0] = o.x;
  c.o[1] = o.y;
  c.o[2] = o.z;
  c.o[3] = o.w;
  if constexpr (!std::is_same<CV, T>::value) {
    const uint64_t k = cbyte / res_chunk_bytes<T>();  // the chunk's index in the stream
    typedef const __attribute__((address_space(1))) CV* CVP;
    const CVP cp = (CVP)cs + (size_t)k * (4 * 64) + (lane16 >> 4);
#pragma unroll
    for (int u = 0; u < kResChunk; ++u) c.v[u] = cp[u * 64];
  } else if constexpr (sizeof(T) == 8) {
    typedef double D2 __attribute__((ext_vector_type(2)));
    const D2 x = __builtin_bit_cast(D2, __builtin_amdgcn_raw_buffer_load_b128(rs, lane16, cb + 1024u, 0));
    const D2 y = __builtin_bit_cast(D2, __builtin_amdgcn_raw_buffer_load_b128(rs, lane16, cb + 2048u, 0));
    c.v[0] = x.x;
    c.v[1] = x.y;
    c.v[2] = y.x;
    c.v[3] = y.y;
  } else {
    typedef float F4 __attribute__((ext_vector_type(4)));
    const F4 x = __builtin_bit_cast(F4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane16, cb + 1024u, 0));
    c.v[0] = x.x;
    c.v[1] = x.y;
    c.v[2] = x.z;
    c.v[3] = x.w;
  }
}

// acc <- fma(coefficient, gathered element, acc), per sample: the fused step of
// every sum over the stream.  Written as one intrinsic (not a product and a sum
// left to contraction), so no transformation can separate the product from its
// sum, e.g. hoist the products that the blocks of a split chunk share.
template <typename V, typename CV>
__device__ __forceinline__ void fma_acc(V& acc, CV c, V x) {
  if constexpr (std::is_same<CV, V>::value) {
    acc = __builtin_elementwise_fma(c, x, acc);
  } else {
    acc = __builtin_elementwise_fma(V(c), x, acc);
  }
}

// acc += sum over the chunk's 4 entries of coefficient * gathered element, in order
template <typename T, typename V, typename CV>
__device__ __forceinline__ void consume_chunk(const Chunk<T, CV>& c, V& acc) {
  V x[kResChunk];
#pragma unroll
  for (int u = 0; u < kResChunk; ++u) x[u] = ent_read<V>(c.o[u]);
#pragma unroll
  for (int u = 0; u < kResChunk; ++u) fma_acc(acc, c.v[u], x[u]);
}

// Entries [0, e) of the chunk to acc and entries [e, 4) to carry, in order:
// the chunk's last entries open the next slot (e is wave-uniform).
template <typename T, typename V, typename CV>
__device__ __forceinline__ void consume_split(const Chunk<T, CV>& c, int e, V& acc, V& carry) {
  V x[kResChunk];
#pragma unroll
  for (int u = 0; u < kResChunk; ++u) x[u] = ent_read<V>(c.o[u]);
  // one straight-line block per split point; the empty asm keeps the compiler
  // from merging the blocks into selects over both sums
  if (e == 1) {
    asm volatile("");
    fma_acc(acc, c.v[0], x[0]);
    fma_acc(carry, c.v[1], x[1]);
    fma_acc(carry, c.v[2], x[2]);
    fma_acc(carry, c.v[3], x[3]);
  } else if (e == 2) {
    asm volatile("");
    fma_acc(acc, c.v[0], x[0]);
    fma_acc(acc, c.v[1], x[1]);
    fma_acc(carry, c.v[2], x[2]);
    fma_acc(carry, c.v[3], x[3]);
  } else {
    asm volatile("");
    fma_acc(acc, c.v[0], x[0]);
    fma_acc(acc, c.v[1], x[1]);
    fma_acc(acc, c.v[2], x[2]);
    fma_acc(carry, c.v[3], x[3]);
  }
}

// A slot's last chunk: its own, or shared with the next slot (e < 4).
template <typename T, typename V, typename CV>
__device__ __forceinline__ void consume_last(const Chunk<T, CV>& c, int e, V& acc, V& carry) {
  if (e == kResChunk) {
    asm volatile("");
    consume_chunk(c, acc);
  } else {
    consume_split(c, e, acc, carry);
  }
}

// Sum over one slot.  The slots of a pass are packed: a slot may open inside
// the previous slot's last chunk (at most two slots share a chunk), and those
// head entries arrive summed in ``carry``, from the previous call, which
// consumed the shared chunk once.  The call then takes the slot's R entries
// from the next whole chunk on, and leaves in ``carry`` the head of the next
// slot when the slot's last chunk is shared (R and the split are
// wave-uniform: ``nch`` whole chunks, the last with ``e`` entries of the
// slot).  On entry b0 holds (or is loading) the slot's first whole
// chunk and ``pos`` indexes the next chunk of the wave's stream; on exit b0
// holds the chunk after the slot's last one.  The chunks are taken in pairs
// by a loop whose every pass issues the same loads (the next chunk into b1,
// then the one after into b0), so the compiler waits only for the chunk being
// consumed (the later chunk stays in flight); the last one or two chunks are
// taken after the loop, the last one whole or split.  ``pro`` (the first slot
// of a pass, spanning two or more chunks): b1 holds (or is loading) the
// slot's second chunk as well, loaded before the barrier that opened the pass
// so that the stream stays busy while the wavefronts wait there; the first
// two chunks are taken before the loop.  Summation order: the slot's entries
// in stream order, its head first.  SPLIT false: the pass has one slot, which
// owns every chunk it walks (no head, no split).
template <typename T, typename V, bool SPLIT, typename CV = T>
__device__ __forceinline__ V slot_sum(int nch, int e, V& carry, Chunk<T, CV>& b0,
                                      Chunk<T, CV>& b1, uint32_t& pos,
                                      const unsigned char* __restrict__ stream, uint32_t lane16,
                                      bool pro, const CV* __restrict__ cs = nullptr) {
  constexpr uint64_t CB = res_chunk_bytes<T>();
  if constexpr (!SPLIT) {
    // one slot per pass: it owns all its chunks (the pass's end is padded)
    V acc = V(T(0));
    int k = 0;
    if (pro) {  // nch >= 2
      consume_chunk(b0, acc);
      load_chunk(b0, stream, pos * CB, lane16, cs);
      ++pos;
      __builtin_amdgcn_sched_barrier(0);
      consume_chunk(b1, acc);
      k = 2;
    }
    for (; k + 1 < nch; k += 2) {
      load_chunk(b1, stream, pos * CB, lane16, cs);
      ++pos;
      __builtin_amdgcn_sched_barrier(0);
      consume_chunk(b0, acc);
      load_chunk(b0, stream, pos * CB, lane16, cs);
      ++pos;
      __builtin_amdgcn_sched_barrier(0);
      consume_chunk(b1, acc);
    }
    if (k < nch) {
      consume_chunk(b0, acc);
      load_chunk(b0, stream, pos * CB, lane16, cs);
      ++pos;
    }
    return acc;
  }
  V acc = carry;
  carry = V(T(0));
  int k = 0;
  if (pro) {  // nch >= 2, no head (the pass's first slot)
    consume_chunk(b0, acc);
    load_chunk(b0, stream, pos * CB, lane16, cs);
    ++pos;
    __builtin_amdgcn_sched_barrier(0);
    if (nch == 2) {
      consume_last(b1, e, acc, carry);
      return acc;
    }
    consume_chunk(b1, acc);
    k = 2;
  }
  for (; k + 2 < nch; k += 2) {
    load_chunk(b1, stream, pos * CB, lane16, cs);
    ++pos;
    // keep the load ahead of the consumption it overlaps (the scheduler would
    // otherwise sink it, leaving one chunk in flight)
    __builtin_amdgcn_sched_barrier(0);
    consume_chunk(b0, acc);
    load_chunk(b0, stream, pos * CB, lane16, cs);
    ++pos;
    __builtin_amdgcn_sched_barrier(0);
    consume_chunk(b1, acc);
  }
  if (k + 1 < nch) {
    load_chunk(b1, stream, pos * CB, lane16, cs);
    ++pos;
    __builtin_amdgcn_sched_barrier(0);
    consume_chunk(b0, acc);
    load_chunk(b0, stream, pos * CB, lane16, cs);
    ++pos;
    __builtin_amdgcn_sched_barrier(0);
    consume_last(b1, e, acc, carry);
  } else if (k < nch) {
    consume_last(b0, e, acc, carry);
    load_chunk(b0, stream, pos * CB, lane16, cs);
    ++pos;
  }
  return acc;
}

// Field k (8 bits) of a wave-table word of per-slot counts.
__device__ __forceinline__ int slot_field(uint32_t word, int k) {
  return (int)((word >> (8 * k)) & 255u);
}

// jnp.clip(x, lo, hi) for bounds that are not NaN: (x <= lo) is false for a
// NaN x, which therefore passes through, as minimum(maximum(x, lo), hi) does;
// ties and signed zeros resolve to the bound, as in clipp.
template <typename T>
__device__ __forceinline__ T clip_nonnan_bounds(T x, T lo, T hi) {
  const T r = x <= lo ? lo : x;
  return r >= hi ? hi : r;
}

// The resident kernels' clip for bounds that are not NaN and projection onto
// x >= 0.  fp32: gfx950's NaN-propagating v_maximum3_f32 / v_minimum3_f32
// (IEEE 754-2019 maximum and minimum), one instruction each where the
// compare-and-select forms take two per side; the values are jnp.clip's and
// jnp.maximum's, a NaN x passing through.  They differ from clipp / maxp
// only in the sign of a zero at a tie of +0 with -0 (these order -0 below
// +0).  fp64 (no such instruction): the compare-and-select forms.
template <typename T>
__device__ __forceinline__ T res_clip(T x, T lo, T hi) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_elementwise_minimum(__builtin_elementwise_maximum(x, lo), hi);
  } else {
    return clip_nonnan_bounds(x, lo, hi);
  }
}
template <typename T>
__device__ __forceinline__ T res_pos(T x) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_elementwise_maximum(x, T(0));
  } else {
    return maxp(x, T(0));
  }
}

// 1 / x for the QP prox's x = 1 + tau q, which lies in [1, 2) (q >= 0 and
// tau <= s / (max q + L) with s < 1, decreasing under the accelerated update,
// kernels.py:209-227): the hardware
// reciprocal estimate refined by two Newton-Raphson steps r <- r + r (1 - x r)
// (each with fused multiply-adds), within an ulp of the correctly rounded
// quotient, in 5 instructions where the IEEE division sequence takes about
// 10 (scale, estimate, refinement, fix-up).  Used by the fixed-iteration
// kernel only: the early-stop kernel keeps the streaming passes' division,
// so its stop decisions see the same prox.
template <typename T>
__device__ __forceinline__ T res_recip(T x) {
  T r;
  if constexpr (sizeof(T) == 8) {
    r = __builtin_amdgcn_rcp(x);
  } else {
    r = __builtin_amdgcn_rcpf(x);
  }
  T e = __builtin_elementwise_fma(-x, r, T(1));
  r = __builtin_elementwise_fma(r, e, r);
  e = __builtin_elementwise_fma(-x, r, T(1));
  return __builtin_elementwise_fma(r, e, r);
}

// A wave-uniform value kept in SGPRs (its lanes are equal: the first lane's).
template <typename T>
__device__ __forceinline__ T res_uniform(T x) {
  if constexpr (sizeof(T) == 8) {
    const uint64_t u = __builtin_bit_cast(uint64_t, x);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(u >> 32));
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  } else {
    return __builtin_bit_cast(T, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
  }
}

// The accelerated update of the diagonal QP's per-sample steps after an
// iteration (kernels.py:279-283, gamma = min q): nu = 1/sqrt(1 + gamma tau);
// tau <- nu tau; sigma <- sigma / nu; theta <- nu; every product and quotient
// rounded, as the streaming passes' sched_next forms them.  The steps are the
// same in every thread and stay in SGPRs.
template <typename T, int BT>
__device__ __forceinline__ void res_qp_schedule(const T (&gam)[BT], T (&tau)[BT], T (&sig)[BT],
                                                T (&th)[BT], T (&pa)[BT], T (&pd)[BT]) {
#pragma clang fp contract(off)
  const T one = T(1);
#pragma unroll
  for (int s = 0; s < BT; ++s) {
    const T nu = one / (T)__builtin_sqrt(one + gam[s] * tau[s]);
    const T nt = nu * tau[s];
    const T a = one / (one + nt);  // the prox of q = 1 (per-sample coefficients)
    tau[s] = res_uniform(nt);
    sig[s] = res_uniform(sig[s] / nu);
    th[s] = res_uniform(nu);
    pa[s] = res_uniform(a);
    pd[s] = res_uniform(nt * a);
  }
}

template <typename T, int SLR, int SLC, bool SB, int NB = ResVec<T>::BT, bool QP = false,
          bool VALS = false>
__global__ __launch_bounds__(1024) void k_resident(Res<T> A) {
  constexpr int NT = 1024;
  constexpr int BT = NB;
  using V = typename ResV<T, NB>::V;
  extern __shared__ __align__(16) unsigned char lds[];  // at LDS address 0 (no static LDS)
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int64_t tile = blockIdx.x;
  const uint32_t lane16 = (uint32_t)lane * 16u;
  const V vzero = V(T(0));
  const uint32_t trash_off = (uint32_t)(A.n + 1 + A.m) * 16u;

  const uint32_t first = (uint32_t)__builtin_amdgcn_readfirstlane(A.wtab[kResWtab * wave]);
  // per slot (8 bits each): whole chunks from the slot's first whole chunk on,
  // and the slot's entries in the last of them (4, or 1-3 when the next slot
  // opens inside it)
  const uint32_t rcnt = (uint32_t)__builtin_amdgcn_readfirstlane(A.wtab[kResWtab * wave + 1]);
  const uint32_t ccnt = (uint32_t)__builtin_amdgcn_readfirstlane(A.wtab[kResWtab * wave + 2]);
  const uint32_t rlast = (uint32_t)__builtin_amdgcn_readfirstlane(A.wtab[kResWtab * wave + 3]);
  const uint32_t clast = (uint32_t)__builtin_amdgcn_readfirstlane(A.wtab[kResWtab * wave + 4]);
  // bit 0 / bit 1: the first row / column slot spans two or more chunks, so
  // the pass's first two chunks are loaded before the barrier that opens it
  const uint32_t pro = (uint32_t)__builtin_amdgcn_readfirstlane(A.wtab[kResWtab * wave + 7]);

  const V* Ts = reinterpret_cast<const V*>(A.Ts) + tile * (int64_t)A.Kc;
  const V* Rs = reinterpret_cast<const V*>(A.Rs) + tile * (int64_t)A.Kr;
  const V* D0 = reinterpret_cast<const V*>(A.D0s) + tile * (int64_t)A.Kr;

  uint32_t soff_r[SLR], soff_c[SLC];
  // the targets (QP: c) stay in registers except in the variants with four
  // row and four column slots and per-sample bounds, which would spill them
  constexpr bool kHoldTarget = SB || SLR + SLC < 8;
  V y[SLC], tg[kHoldTarget ? SLC : 1], rr[SLR];
  // QP: q of the thread's columns.  QP and per-sample coefficients (VALS):
  // the tile's per-sample steps (the same in every thread): tau, sigma,
  // theta, the prox a, delta of q = 1 (VALS) of the current iteration, gamma
  constexpr bool kPS = QP || VALS;
  V qh[QP ? SLC : 1];
  T tau_s[BT], sig_s[BT], th_s[BT], gam_s[BT], pa_s[BT], pd_s[BT];
  if constexpr (kPS) {
    const int64_t bq = tile * BT;
#pragma unroll
    for (int s = 0; s < BT; ++s) {
      tau_s[s] = res_uniform(A.step0[bq + s]);
      sig_s[s] = res_uniform(A.step0[A.Bp + bq + s]);
      pa_s[s] = res_uniform(A.step0[2 * A.Bp + bq + s]);
      pd_s[s] = res_uniform(A.step0[3 * A.Bp + bq + s]);
      th_s[s] = res_uniform(A.accel ? A.step0[4 * A.Bp + bq + s] : T(1));
      gam_s[s] = res_uniform(A.gam ? A.gam[bq + s] : T(1));
    }
  }
  // per-sample coefficients: this tile's coefficient stream
  using CV = typename std::conditional<VALS, V, T>::type;
  const CV* cs = nullptr;
  if constexpr (VALS) cs = reinterpret_cast<const CV*>(A.Cs) + tile * A.cs_tile;
  uint32_t ineq = 0, nanb = 0;
  // shared bounds equal on every column of a wavefront's slots (box bounds,
  // e.g. [-1, 1]): its column pass then takes them from registers instead of
  // re-reading them from L2 every iteration.  The test is per wavefront (a
  // ballot; the kernel uses no LDS beyond its own dynamic layout).
  // The QP takes per-sample bounds; a box the same for every sample and
  // column of the wavefront's slots (e.g. [-1, 1]) is held the same way, with
  // the reference pair from the first lane's first column slot.
  T lo0 = A.Ls[0], hi0 = A.Hs[0];
  if constexpr (QP) {
    T rl = T(0), rh = T(0);
#pragma unroll
    for (int c = SLC - 1; c >= 0; --c) {  // ends on the first valid slot
      const int64_t e0 = (tile * (int64_t)A.Kc + c * NT + t) * BT;
      if (A.colmap[c * NT + t] >= 0) {
        rl = A.Ls[e0];
        rh = A.Hs[e0];
      }
    }
    lo0 = res_uniform(rl);
    hi0 = res_uniform(rh);
  }
  int same = (SB || QP) && lo0 == lo0 && hi0 == hi0;
#pragma unroll
  for (int c = 0; c < SLC; ++c) {
    const int j = A.colmap[c * NT + t];
#pragma unroll
    for (int s = 0; s < BT; ++s) {
      const int64_t e = SB ? (int64_t)(c * NT + t) : (tile * (int64_t)A.Kc + c * NT + t) * BT + s;
      if (A.Ls[e] != A.Ls[e] || A.Hs[e] != A.Hs[e] || A.Ls[e] > A.Hs[e]) nanb |= 1u << c;  // NaN or crossed bound
      if ((SB || QP) && j >= 0 && (A.Ls[e] != lo0 || A.Hs[e] != hi0)) same = 0;
    }
    soff_c[c] = j >= 0 ? (uint32_t)A.colent[c * NT + t] * 16u : trash_off;
    const V t0 = j >= 0 ? Ts[c * NT + t] : vzero;
    if constexpr (kHoldTarget) tg[c] = t0;
    if constexpr (QP) {  // y0 = ybar0: the caller's start or zero (diagonal_qp.py:257-262)
      qh[c] = j >= 0 ? reinterpret_cast<const V*>(A.Qs)[tile * (int64_t)A.Kc + c * NT + t] : vzero;
      y[c] = j >= 0 ? reinterpret_cast<const V*>(A.Y0s)[tile * (int64_t)A.Kc + c * NT + t] : vzero;
    } else {
      y[c] = t0;  // y0 = ybar0 = yhat (kernels.py:229-231)
    }
    ent_write<V>(soff_c[c], y[c]);
  }
#pragma unroll
  for (int r = 0; r < SLR; ++r) {
    const int i = A.rowmap[r * NT + t];
    soff_r[r] = i >= 0 ? (uint32_t)A.rowent[r * NT + t] * 16u : trash_off;
    rr[r] = i >= 0 ? Rs[r * NT + t] : vzero;
    if (i >= A.me) ineq |= 1u << r;  // kept rows: equalities first
    ent_write<V>(soff_r[r], i >= 0 ? D0[r * NT + t] : vzero);
  }
  if (t == 0) ent_write<V>((uint32_t)A.n * 16u, vzero);  // the zero slot
  const bool uni = __builtin_amdgcn_ballot_w64(same != 0) == ~0ull;  // all 64 lanes
  // per-sample bounds of the leading lb_slots column slots, held in LDS after
  // the image: slot c's lower bounds, then its upper bounds, each as 16-byte
  // granules of consecutive threads (two granule rows for a 32-byte vector).
  // Each thread reads back only what it wrote, so no barrier orders them.
  // Held on chip they leave the L2 to the other slots' bounds, which then
  // stay there instead of being re-read from beyond it every iteration.
  constexpr uint32_t VB = (uint32_t)sizeof(V);
  constexpr uint32_t GS = NT * 16u;  // bytes of one granule row
  const uint32_t lb_off = (VB == 32 ? 2u * kResPlane : trash_off + 16u) + (uint32_t)t * 16u;
  const int lbs = SB ? 0 : __builtin_amdgcn_readfirstlane(A.lb_slots);
  if constexpr (!SB) {
#pragma unroll
    for (int c = 0; c < SLC; ++c) {
      if (c < lbs) {
        const int64_t e = tile * (int64_t)A.Kc + c * NT + t;
        const uint32_t at = lb_off + (uint32_t)c * 2u * (VB / 16u) * GS;
        lds_write_split<V>(at, GS, reinterpret_cast<const V*>(A.Ls)[e]);
        lds_write_split<V>(at + (VB / 16u) * GS, GS, reinterpret_cast<const V*>(A.Hs)[e]);
      }
    }
  }
  __syncthreads();

  constexpr uint32_t CB = res_chunk_bytes<T>();
  Chunk<T, CV> b0, b1;
  load_chunk(b0, A.stream, (uint64_t)first * CB, lane16, cs);
  if (pro & 1u) load_chunk(b1, A.stream, (uint64_t)(first + 1) * CB, lane16, cs);

  // wave-uniform schedule scalars (QP, VALS: the per-sample steps in registers
  // instead), scalar loads through the constant address space.  Each
  // iteration's are loaded before the barrier that ends the previous one,
  // whose wait covers them, so no scalar load is outstanding in the passes
  // (one would make every wait on an LDS gather there wait for all of them)
  T sigma = T(0), a = T(0), delta = T(0), theta = T(0);
  auto load_sched = [&](int64_t i) {
    if constexpr (!kPS) {
      const __attribute__((address_space(4))) T* sc =
          (const __attribute__((address_space(4))) T*)(A.sched + 4 * i);
      sigma = sc[0];
      a = sc[1];
      delta = sc[2];
      theta = sc[3];
      asm volatile("" : "+s"(sigma), "+s"(a), "+s"(delta), "+s"(theta));
    }
  };
  load_sched(0);
  for (int64_t it = 0; it < A.iters; ++it) {
    uint32_t pos = first + 1 + (pro & 1u);
    V carry = vzero;  // the head of the next slot (a chunk shared by two slots)
    // the slot tables, opaque to the loop so that their fields are decoded at
    // each slot rather than held decoded in SGPRs across the iteration
    uint32_t rc = rcnt, rl = rlast, cc = ccnt, cl = clast;
    asm volatile("" : "+s"(rc), "+s"(rl), "+s"(cc), "+s"(cl));
    // ---- row pass (reads Gy and the thread's own Gd entries, writes Gd) -------
#pragma unroll
    for (int r = 0; r < SLR; ++r) {
      const V dold = ent_read<V>(soff_r[r]);
      const V acc = slot_sum<T, V, (SLR > 1), CV>(slot_field(rc, r), slot_field(rl, r), carry,
                                                  b0, b1, pos, A.stream, lane16,
                                                  r == 0 && (pro & 1u), cs);
      V p;
      if constexpr (kPS) {
        const V e = acc - rr[r];
#pragma unroll
        for (int s = 0; s < BT; ++s) p[s] = dold[s] + sig_s[s] * e[s];
      } else {
        p = dold + sigma * (acc - rr[r]);
      }
      if (ineq & (1u << r)) {
#pragma unroll
        for (int s = 0; s < BT; ++s) p[s] = res_pos(p[s]);
      }
      ent_write<V>(soff_r[r], p);
    }
    if (pro & 2u) {  // the column pass's second chunk (its first is in b0)
      load_chunk(b1, A.stream, (uint64_t)pos * CB, lane16, cs);
      ++pos;
    }
    __syncthreads();
    // ---- column pass (reads Gd, writes Gy) --------------------------------------
    carry = vzero;
#pragma unroll
    for (int c = 0; c < SLC; ++c) {
      // bounds are re-read each iteration (L2-resident when shared) rather
      // than held in registers: the opaque base keeps them inside the loop;
      // they are loaded before the gathers, which hide their latency
      typedef const __attribute__((address_space(1))) T* GP;
      typedef const __attribute__((address_space(1))) V* GV;
      GP lb = (GP)A.Ls;
      GP hb = (GP)A.Hs;
      asm volatile("" : "+s"(lb), "+s"(hb));
      V lo, hi;
      if ((SB || QP) && uni) {
        lo = V(lo0);
        hi = V(hi0);
      } else if (SB) {
        lo = V(lb[c * NT + t]);
        hi = V(hb[c * NT + t]);
      } else if (c < lbs) {
        const uint32_t at = lb_off + (uint32_t)c * 2u * (VB / 16u) * GS;
        lo = lds_read_split<V>(at, GS);
        hi = lds_read_split<V>(at + (VB / 16u) * GS, GS);
      } else {
        lo = ((GV)lb)[tile * (int64_t)A.Kc + c * NT + t];
        hi = ((GV)hb)[tile * (int64_t)A.Kc + c * NT + t];
      }
      V tgc;
      if constexpr (kHoldTarget) {
        tgc = tg[c];
      } else {  // re-read (L2) in the largest per-sample-bounds variant: registers
        typedef const __attribute__((address_space(1))) V* GVT;
        GVT tb = (GVT)A.Ts;
        asm volatile("" : "+s"(tb));
        tgc = tb[tile * (int64_t)A.Kc + c * NT + t];
      }
      const V tt = slot_sum<T, V, (SLC > 1), CV>(slot_field(cc, c), slot_field(cl, c), carry,
                                                 b0, b1, pos, A.stream, lane16,
                                                 c == 0 && (pro & 2u), cs);
      V sv;
      if constexpr (QP) {  // the general-q prox (kernels.py:68-73), as the streaming pass forms it
#pragma unroll
        for (int s = 0; s < BT; ++s) {
          const T aj = res_recip(T(1) + tau_s[s] * qh[c][s]);
          const T dj = tau_s[s] * aj;
          const T oj = -dj * tgc[s];
          sv[s] = aj * y[c][s] - dj * tt[s] + oj;
        }
      } else if constexpr (VALS) {  // per-sample a, delta of q = 1
#pragma unroll
        for (int s = 0; s < BT; ++s) sv[s] = pa_s[s] * y[c][s] - pd_s[s] * tt[s] + pd_s[s] * tgc[s];
      } else {
        sv = a * y[c] - delta * tt + delta * tgc;
      }
      V yn;
      if (nanb & (1u << c)) {  // a NaN or crossed bound on this lane: the exact NaN-propagating clip
#pragma unroll
        for (int s = 0; s < BT; ++s) yn[s] = clipp(sv[s], lo[s], hi[s]);
      } else {
#pragma unroll
        for (int s = 0; s < BT; ++s) yn[s] = res_clip(sv[s], lo[s], hi[s]);
      }
      if constexpr (kPS) {
        V yb;
#pragma unroll
        for (int s = 0; s < BT; ++s) yb[s] = yn[s] + th_s[s] * (yn[s] - y[c][s]);
        ent_write<V>(soff_c[c], yb);
      } else
        ent_write<V>(soff_c[c], yn + theta * (yn - y[c]));
      y[c] = yn;
    }
    if constexpr (kPS) {
      if (A.accel) res_qp_schedule<T, BT>(gam_s, tau_s, sig_s, th_s, pa_s, pd_s);
    }
    // the next row pass's second chunk (b0 holds the copy of its first)
    if (pro & 1u) load_chunk(b1, A.stream, (uint64_t)(first + 1) * CB, lane16, cs);
    if (it + 1 < A.iters) load_sched(it + 1);
    __syncthreads();
  }
  // ---- hand the state to the batch-minor layout ---------------------------------
  const int64_t b0s = tile * BT;
#pragma unroll
  for (int c = 0; c < SLC; ++c) {
    const int j = A.colmap[c * NT + t];
    if (j >= 0)
#pragma unroll
      for (int s = 0; s < BT; ++s) A.Y[(int64_t)j * A.Bp + b0s + s] = y[c][s];
  }
#pragma unroll
  for (int r = 0; r < SLR; ++r) {
    const int i = A.rowmap[r * NT + t];
    if (i >= 0) {
      const V d = ent_read<V>(soff_r[r]);
#pragma unroll
      for (int s = 0; s < BT; ++s) A.D[(int64_t)i * A.Bp + b0s + s] = d[s];
    }
  }
}

// ---------------------------------------------------------------------------
// Early-stop variant (freeze_converged and the stop test of kernels.py:228-290
// with check_stationarity, bounds.py:61-62).  The tile's samples stop
// independently: a sample accepted at iteration k keeps the state of
// iteration k (its later updates are masked and not counted), and the
// workgroup returns when all its samples are accepted or the iterations run
// out.  It walks the fixed kernel's chunk streams, two sweeps per iteration,
// with Gy holding the iterate y itself (not ybar):
//   row update    commit d+ where the sample is active: the candidate
//                   P(d + sigma (K ybar - r)) formed by the previous residual
//                   sweep, with K ybar = (1 + theta) K y - theta K y_prev
//                   (ybar = y + theta (y - y_prev), kernels.py:149; the first
//                   iteration's ybar is y): no gathers, no global loads
//   barrier
//   column pass   gathers Gd: y+ where active, Gy <- y+; the column
//                   diagnostics (primal and dual objective terms,
//                   stationarity and bound violation, kernels.py:153-175,
//                   272-274): the primal sum over 16-lane rows by DPP to
//                   LDS, the others kept per thread
//   barrier
//   residual      gathers Gy = y+: K y+, max |K y+ - r| (eq) /
//                   max(K y+ - r, 0) (ineq) and r . d+ (kernels.py:158-166)
//                   folded into the thread's dual terms and maxima, summed
//                   over 16-lane rows by DPP, to LDS; the next iteration's
//                   candidate duals
//   barrier
//   decision      wavefront s combines sample s's 64 partials of each total
//                   in one fixed order and applies the stop test
//                   (kernels.py:167-175, 260-278); the verdicts go through LDS
//   barrier
// The residual is exact; K ybar comes from the linear relation above, so the
// iterates differ from the fixed kernel's (which gathers ybar) by rounding.
// A non-finite y+ or d+ makes the primal or the dual sum non-finite, so the
// gap is not finite and the sample is not accepted (the finiteness flag of
// kernels.py:172).  On lanes whose bounds are neither NaN nor crossed
// (lo <= hi), y+ lies in [lo, hi] (bound violation 0) and the stationarity
// clip equals the dual term's; the other lanes take the full expressions.
// LDS: the fixed kernel's, then the partials [16 waves][4 rows][kResQ] and
// the BT verdicts, then K y of the first res_early_kyl(SLR, SLC) row slots.
constexpr int kResQ = 3;  // primal; dual objective (terms - r.d); max(stationarity, residual)

// LDS bytes of the early-stop kernel beyond the tile's image, for vectors of
// vb bytes (16, or 32 for two-plane tiles of nb = 8 samples): the partials
// [16 waves][4 rows][kResQ] and the verdicts (4 bytes per sample, 16-aligned).
constexpr uint32_t res_early_extra(uint32_t vb, uint32_t nb) {
  return 16u * 4u * kResQ * vb + ((4u * nb + 15u) / 16u) * 16u;
}
constexpr uint32_t kResEarlyExtra = res_early_extra(16u, 4u);  // one-plane tiles

// Row slots whose K y the early-stop kernel keeps in LDS instead of registers:
// as many as the largest LDS image of the (SLR, SLC) variant leaves room for
// beside the partials, in variants with five or more slots per thread (the
// smaller ones have registers to spare).  Measured at config 2's (3, 4): two
// slots, 14.9 -> 13.7 us per iteration (the registers they free remove most
// of the loop's spill traffic); one slot 14.1 us.
constexpr int res_early_kyl(int SLR, int SLC) {
  if (SLR + SLC < 5) return 0;
  const long image = (long)(SLR + SLC) * 1024 * 16 + 32;
  const long free_b = 160L * 1024 - image - (long)kResEarlyExtra;
  const long k = free_b / (1024L * 16);
  return (int)(k < 0 ? 0 : (k > SLR ? SLR : k));
}

// One DPP move of a 32- or 64-bit value (all lanes active, full row/bank masks).
template <int CTRL, typename T>
__device__ __forceinline__ T dpp_move(T v) {
  if constexpr (sizeof(T) == 8) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
    const uint32_t hi =
        (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  } else {
    return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF,
                                                             0xF, false));
  }
}

// max that ignores a NaN operand (v_max_f64 / v_max_f32): for maxima whose
// NaN cases the caller has already turned into an infinity or a non-finite sum
struct OpFMax {
  template <typename T>
  __device__ T operator()(T a, T b) const { return __builtin_fmax(a, b); }
};

// Combine the 16 lanes of each DPP row; lane 0 of the row holds
// ((q0 op q3) op (q2 op q1)) of its four quads q (each quad combined pairwise).
template <typename T, typename Op>
__device__ __forceinline__ T row16_combine(T v, Op op) {
  v = op(v, dpp_move<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = op(v, dpp_move<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = op(v, dpp_move<0x124>(v));  // row_ror:4
  v = op(v, dpp_move<0x128>(v));  // row_ror:8
  return v;
}

template <typename T>
__device__ __forceinline__ T read_lane(T v, int l) {
  if constexpr (sizeof(T) == 8) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  } else {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
  }
}

template <typename T, int SLR, int SLC, bool SB, int NB = ResVec<T>::BT, bool QP = false,
          bool VALS = false>
__global__ __launch_bounds__(1024) void k_resident_early(Res<T> A) {
  constexpr int NT = 1024;
  constexpr int BT = NB;
  using V = typename ResV<T, NB>::V;
  extern __shared__ __align__(16) unsigned char lds[];  // at LDS address 0 (no static LDS)
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int64_t tile = blockIdx.x;
  const uint32_t lane16 = (uint32_t)lane * 16u;
  const V vzero = V(T(0));
  const T zero = T(0), half = T(0.5), inf = T(__builtin_inf());
  const uint32_t trash_off = (uint32_t)(A.n + 1 + A.m) * 16u;
  // the partials after the image (after both planes of a two-plane tile)
  constexpr uint32_t VB = (uint32_t)sizeof(V);
  const uint32_t red_off = VB == 32 ? 2u * kResPlane : trash_off + 16u;
  const uint32_t dec_off = red_off + 16u * 4u * kResQ * VB;  // [BT] verdicts
  // per-sample bounds of the projection: the leading column slots' bounds are
  // held in LDS after the verdicts, in the room K y would take (k_resident's
  // layout), so K y stays in registers.  Only where four column slots'
  // bounds (4 MB per XCD) would crowd the L2 and the freed room takes a slot
  // of them (up to three row slots), or where K y is not in LDS anyway
  // (two-plane tiles); elsewhere the bounds stay in L2 and K y in LDS.
  constexpr bool kLB = !SB && !QP && !VALS && (VB == 32 || (SLC == 4 && SLR <= 3));
  constexpr int KYL = (VB == 32 || kLB) ? 0 : res_early_kyl(SLR, SLC);
  // [KYL][1024] K y of the first row slots, after the verdicts
  const uint32_t kyl_off = red_off + res_early_extra(VB, BT);
  constexpr uint32_t GS = NT * 16u;  // bytes of one granule row of held bounds
  const uint32_t lb_off = kyl_off + (uint32_t)t * 16u;
  const int lbs = kLB ? __builtin_amdgcn_readfirstlane(A.lb_slots) : 0;

  const uint32_t first = (uint32_t)__builtin_amdgcn_readfirstlane(A.wtab[kResWtab * wave]);
  // per slot (8 bits each): whole chunks from the slot's first whole chunk on,
  // and the slot's entries in the last of them (4, or 1-3 when the next slot
  // opens inside it)
  const uint32_t rcnt = (uint32_t)__builtin_amdgcn_readfirstlane(A.wtab[kResWtab * wave + 1]);
  const uint32_t ccnt = (uint32_t)__builtin_amdgcn_readfirstlane(A.wtab[kResWtab * wave + 2]);
  const uint32_t rlast = (uint32_t)__builtin_amdgcn_readfirstlane(A.wtab[kResWtab * wave + 3]);
  const uint32_t clast = (uint32_t)__builtin_amdgcn_readfirstlane(A.wtab[kResWtab * wave + 4]);
  // bit 0 / bit 1: the first row / column slot spans two or more chunks, so
  // a sweep's first two chunks are loaded before the barrier that opens it
  const uint32_t pro = (uint32_t)__builtin_amdgcn_readfirstlane(A.wtab[kResWtab * wave + 7]);

  const V* Rs = reinterpret_cast<const V*>(A.Rs) + tile * (int64_t)A.Kr;
  const V* D0 = reinterpret_cast<const V*>(A.D0s) + tile * (int64_t)A.Kr;

  // registers: per row slot K y of the current iterate (in LDS for the first
  // KYL slots) and, from the
  // residual sweep to the decision, the committed dual the sweep replaced in
  // Gd by the next candidate; the targets of the thread's columns and the
  // scaled right-hand sides of its rows, loaded once (re-reading them each
  // iteration from beyond L2 took 18.0 us per iteration at config 2's
  // shape, holding them 15.3 us with a few spilled values, the floor without
  // them 13.9 us).  y lives in Gy (each thread reads its own entries).
  // With four row slots per thread (m > 3072) the held values would spill
  // 116-228 bytes per lane, so those variants re-read them each iteration.
  constexpr bool kHold = SLR <= 3;
  uint32_t soff_r[SLR], soff_c[SLC];
  V ky[SLR], dk[SLR], tgh[kHold ? SLC : 1], rrh[kHold ? SLR : 1];
  // QP (as in k_resident): q of the thread's columns (Ts holds c).  QP and
  // per-sample coefficients (VALS): the tile's per-sample steps in SGPRs
  constexpr bool kPS = QP || VALS;
  V qh[QP ? SLC : 1];
  T tau_s[BT], sig_s[BT], th_s[BT], gam_s[BT], pa_s[BT], pd_s[BT];
  if constexpr (kPS) {
#pragma unroll
    for (int s = 0; s < BT; ++s) {
      const int64_t b = tile * BT + s;
      tau_s[s] = res_uniform(A.step0[b]);
      sig_s[s] = res_uniform(A.step0[A.Bp + b]);
      pa_s[s] = res_uniform(A.step0[2 * A.Bp + b]);
      pd_s[s] = res_uniform(A.step0[3 * A.Bp + b]);
      th_s[s] = res_uniform(A.accel ? A.step0[4 * A.Bp + b] : T(1));
      gam_s[s] = res_uniform(A.gam ? A.gam[b] : T(1));
    }
  }
  // per-sample coefficients: this tile's coefficient stream
  using CV = typename std::conditional<VALS, V, T>::type;
  const CV* cs = nullptr;
  if constexpr (VALS) cs = reinterpret_cast<const CV*>(A.Cs) + tile * A.cs_tile;
  typedef const __attribute__((address_space(1))) V* GV;
  uint32_t ineq = 0, nanb = 0, rvalid = 0, cvalid = 0;
  // shared bounds equal on every column of the wavefront's slots: taken from
  // registers in the loop (as in k_resident; a ballot, no LDS); for the QP's
  // per-sample bounds, one box for every column and sample of those slots
  T lo0 = A.Ls[0], hi0 = A.Hs[0];
  if constexpr (QP) {
    T rl = T(0), rh = T(0);
#pragma unroll
    for (int c = SLC - 1; c >= 0; --c) {  // ends on the first valid slot
      const int64_t e0 = (tile * (int64_t)A.Kc + c * NT + t) * BT;
      if (A.colmap[c * NT + t] >= 0) {
        rl = A.Ls[e0];
        rh = A.Hs[e0];
      }
    }
    lo0 = res_uniform(rl);
    hi0 = res_uniform(rh);
  }
  int same = (SB || QP) && lo0 == lo0 && hi0 == hi0;
#pragma unroll
  for (int c = 0; c < SLC; ++c) {
    const int j = A.colmap[c * NT + t];
#pragma unroll
    for (int s = 0; s < BT; ++s) {
      const int64_t e = SB ? (int64_t)(c * NT + t) : (tile * (int64_t)A.Kc + c * NT + t) * BT + s;
      // a NaN or crossed bound (written as the two NaN tests and lo > hi: the
      // single !(lo <= hi) made the per-sample-bounds variant spill 56 B more
      // per lane and run 24 % slower)
      if (A.Ls[e] != A.Ls[e] || A.Hs[e] != A.Hs[e] || A.Ls[e] > A.Hs[e]) nanb |= 1u << c;
      if ((SB || QP) && j >= 0 && (A.Ls[e] != lo0 || A.Hs[e] != hi0)) same = 0;
    }
    if (j >= 0) cvalid |= 1u << c;
    soff_c[c] = j >= 0 ? (uint32_t)A.colent[c * NT + t] * 16u : trash_off;
    // y0 = ybar0 = yhat (kernels.py:229-231), for the QP the caller's start or
    // zero (diagonal_qp.py:257-262); empty slots hold zeros
    const V t0 = reinterpret_cast<const V*>(A.Ts)[tile * (int64_t)A.Kc + c * NT + t];
    if constexpr (kHold) tgh[c] = t0;
    if constexpr (QP) {
      qh[c] = j >= 0 ? reinterpret_cast<const V*>(A.Qs)[tile * (int64_t)A.Kc + c * NT + t] : vzero;
      ent_write<V>(soff_c[c],
                   j >= 0 ? reinterpret_cast<const V*>(A.Y0s)[tile * (int64_t)A.Kc + c * NT + t]
                          : vzero);
    } else {
      ent_write<V>(soff_c[c], j >= 0 ? t0 : vzero);
    }
  }
#pragma unroll
  for (int r = 0; r < SLR; ++r) {
    const int i = A.rowmap[r * NT + t];
    if (i >= 0) rvalid |= 1u << r;
    soff_r[r] = i >= 0 ? (uint32_t)A.rowent[r * NT + t] * 16u : trash_off;
    if (i >= A.me) ineq |= 1u << r;  // kept rows: equalities first
    if constexpr (kHold) rrh[r] = Rs[r * NT + t];  // zero on empty slots
    ent_write<V>(soff_r[r], i >= 0 ? D0[r * NT + t] : vzero);
  }
  if (t == 0) ent_write<V>((uint32_t)A.n * 16u, vzero);  // the zero slot
  if constexpr (kLB) {  // each thread reads back only what it writes here
#pragma unroll
    for (int c = 0; c < SLC; ++c) {
      if (c < lbs) {
        const int64_t e = tile * (int64_t)A.Kc + c * NT + t;
        const uint32_t at = lb_off + (uint32_t)c * 2u * (VB / 16u) * GS;
        lds_write_split<V>(at, GS, reinterpret_cast<const V*>(A.Ls)[e]);
        lds_write_split<V>(at + (VB / 16u) * GS, GS, reinterpret_cast<const V*>(A.Hs)[e]);
      }
    }
  }
  const bool uni = __builtin_amdgcn_ballot_w64(same != 0) == ~0ull;  // all 64 lanes
  // samples of the tile: the padding samples beyond the batch never run
  const int64_t bs0 = tile * BT;
  uint32_t act = 0;
#pragma unroll
  for (int s = 0; s < BT; ++s)
    if (bs0 + s < A.batch) act |= 1u << s;
  int32_t cnt[BT];
#pragma unroll
  for (int s = 0; s < BT; ++s) cnt[s] = 0;
  const uint32_t red_at = red_off + (uint32_t)((wave * 4 + (lane >> 4)) * kResQ) * VB;
  const bool red_lead = (lane & 15) == 0;
  __syncthreads();

  constexpr uint32_t CB = res_chunk_bytes<T>();
  Chunk<T, CV> b0, b1;
  load_chunk(b0, A.stream, (uint64_t)first * CB, lane16, cs);
  if (pro & 1u) load_chunk(b1, A.stream, (uint64_t)(first + 1) * CB, lane16, cs);
  uint32_t pos = first + 1 + (pro & 1u);
  // K y0 (= K ybar0) by one row sweep, and the first candidate duals; b0 then
  // holds the first column chunk
  {
    const T sigma0 = kPS ? T(0) : A.sched[0];
    V carry = vzero;  // the head of the next slot (a chunk shared by two slots)
    const uint32_t rc = rcnt, rl = rlast;
#pragma unroll
    for (int r = 0; r < SLR; ++r) {
      const V rr = kHold ? rrh[kHold ? r : 0] : Rs[r * NT + t];
      const V k0 = slot_sum<T, V, (SLR > 1), CV>(slot_field(rc, r), slot_field(rl, r), carry,
                                                 b0, b1, pos, A.stream, lane16,
                                                 r == 0 && (pro & 1u), cs);
      if (r < KYL)
        ent_write<V>(kyl_off + (uint32_t)(r * NT + t) * 16u, k0);
      else
        ky[r] = k0;
      V p;
      if constexpr (kPS) {
        const V dd = ent_read<V>(soff_r[r]), e = k0 - rr;
#pragma unroll
        for (int s = 0; s < BT; ++s) p[s] = dd[s] + sig_s[s] * e[s];
      } else {
        p = ent_read<V>(soff_r[r]) + sigma0 * (k0 - rr);
      }
      if (ineq & (1u << r)) {
#pragma unroll
        for (int s = 0; s < BT; ++s) p[s] = res_pos(p[s]);
      }
      ent_write<V>(soff_r[r], p);  // the first iteration's d+ (every sample active)
    }
    if (pro & 2u) {  // the column pass's second chunk (its first is in b0)
      load_chunk(b1, A.stream, (uint64_t)pos * CB, lane16, cs);
      ++pos;
    }
  }
  __syncthreads();

  for (int64_t it = 0; it < A.iters && act != 0u; ++it) {
    T a = T(0), delta = T(0), theta = T(0);
    if constexpr (!kPS) {
      const __attribute__((address_space(4))) T* sc =
          (const __attribute__((address_space(4))) T*)(A.sched + 4 * it);
      a = sc[1];
      delta = sc[2];
      theta = sc[3];
    }
    // ---- column pass, masked, with the column diagnostics (Gd holds d+) ---------------
    V qp = vzero, qd = vzero, qc = vzero;
    V carry = vzero;  // the head of the next slot (a chunk shared by two slots)
    // the slot tables, opaque to the loop so that their fields are decoded at
    // each slot rather than held decoded in SGPRs across the iteration
    uint32_t rc = rcnt, rl = rlast, cc = ccnt, cl = clast;
    asm volatile("" : "+s"(rc), "+s"(rl), "+s"(cc), "+s"(cl));
#pragma unroll
    for (int c = 0; c < SLC; ++c) {
      typedef const __attribute__((address_space(1))) T* GP;
      GP lb = (GP)A.Ls;
      GP hb = (GP)A.Hs;
      V tg;
      if constexpr (kHold) {
        tg = tgh[kHold ? c : 0];
      } else {  // per tile, beyond L2: loaded ahead of the gathers that hide its latency
        GP tb = (GP)A.Ts;
        asm volatile("" : "+s"(tb));
        tg = ((GV)tb)[tile * (int64_t)A.Kc + c * NT + t];
      }
      const V tt = slot_sum<T, V, (SLC > 1), CV>(slot_field(cc, c), slot_field(cl, c), carry,
                                                 b0, b1, pos, A.stream, lane16,
                                                 c == 0 && (pro & 2u), cs);
      asm volatile("" : "+s"(lb), "+s"(hb));
      V lo, hi;
      if ((SB || QP) && uni) {
        lo = V(lo0);
        hi = V(hi0);
      } else if (SB) {
        lo = V(lb[c * NT + t]);
        hi = V(hb[c * NT + t]);
      } else if (kLB && c < lbs) {
        const uint32_t at = lb_off + (uint32_t)c * 2u * (VB / 16u) * GS;
        lo = lds_read_split<V>(at, GS);
        hi = lds_read_split<V>(at + (VB / 16u) * GS, GS);
      } else {
        lo = ((GV)lb)[tile * (int64_t)A.Kc + c * NT + t];
        hi = ((GV)hb)[tile * (int64_t)A.Kc + c * NT + t];
      }
      const V yo = ent_read<V>(soff_c[c]);
      V sv;
      if constexpr (QP) {  // the general-q prox (kernels.py:68-73), as in k_resident
#pragma unroll
        for (int s = 0; s < BT; ++s) {
          const T aj = T(1) / (T(1) + tau_s[s] * qh[c][s]);
          const T dj = tau_s[s] * aj;
          const T oj = -dj * tg[s];
          sv[s] = aj * yo[s] - dj * tt[s] + oj;
        }
      } else if constexpr (VALS) {  // per-sample a, delta of q = 1
#pragma unroll
        for (int s = 0; s < BT; ++s) sv[s] = pa_s[s] * yo[s] - pd_s[s] * tt[s] + pd_s[s] * tg[s];
      } else {
        sv = a * yo - delta * tt + delta * tg;
      }
      V yn;
      if (nanb & (1u << c)) {
#pragma unroll
        for (int s = 0; s < BT; ++s) yn[s] = clipp(sv[s], lo[s], hi[s]);
      } else {
#pragma unroll
        for (int s = 0; s < BT; ++s) yn[s] = res_clip(sv[s], lo[s], hi[s]);
      }
      if (act != (1u << BT) - 1u) {
#pragma unroll
        for (int s = 0; s < BT; ++s)
          if (!(act & (1u << s))) yn[s] = yo[s];  // a frozen sample keeps its state
      }
      if (QP && (cvalid & (1u << c))) {
        // diagnostics with general q, c (kernels.py:158-174, 272-274), the
        // streaming column pass's expressions; a non-finite stationarity term
        // counts as infinite, as in the NaN-bound branch below
#pragma unroll
        for (int s = 0; s < BT; ++s) {
          const T yv = yn[s], q = qh[QP ? c : 0][s], cq = tg[s];
          qp[s] += half * q * yv * yv + cq * yv;
          const T tf = cq + tt[s];
          const T mz = q > T(1e-12) ? clipp(-tf / q, lo[s], hi[s]) : (tf >= zero ? lo[s] : hi[s]);
          qd[s] += half * q * (mz * mz) + tf * mz;
          T g = maxp(absv(yv - clipp(yv - ((q * yv + cq) + tt[s]), lo[s], hi[s])),
                     maxp(maxp(lo[s] - yv, zero), maxp(yv - hi[s], zero)));
          if (!finite(g)) g = inf;
          qc[s] = __builtin_fmax(qc[s], g);
        }
      } else if (cvalid & (1u << c)) {  // diagnostics with q = 1, c = -yhat (kernels.py:158-174, 272-274)
        if (!(nanb & (1u << c))) {
          // Bounds neither NaN nor crossed (the usual lane): y+ is a clip to
          // [lo, hi], so its bound violation is 0 (with lo > hi it is lo - hi,
          // which keeps an infeasible sample running to max_iterations, so
          // such lanes take the full expressions below); y - (y + c + K^T d) = -c - K^T d, so the
          // stationarity clip is the dual term's clip m.  A non-finite y+
          // makes the primal sum non-finite, which the stop test rejects
          // through the gap (kernels.py:172's finiteness).
#pragma unroll
          for (int s = 0; s < BT; ++s) {
            const T yv = yn[s], cq = -tg[s];
            qp[s] += half * yv * yv + cq * yv;
            const T tf = cq + tt[s];
            const T mz = __builtin_fmin(__builtin_fmax(-tf, lo[s]), hi[s]);
            qd[s] += half * mz * mz + tf * mz;
            qc[s] = __builtin_fmax(qc[s], absv(yv - mz));
          }
        } else {  // a NaN or crossed bound on this lane: the reference's expressions, NaN-propagating
#pragma unroll
          for (int s = 0; s < BT; ++s) {
            const T yv = yn[s], cq = -tg[s];
            qp[s] += half * yv * yv + cq * yv;
            const T tf = cq + tt[s];
            const T mz = clipp(-tf, lo[s], hi[s]);
            qd[s] += half * mz * mz + tf * mz;
            const T xs = yv - ((yv + cq) + tt[s]);
            T g = maxp(absv(yv - clipp(xs, lo[s], hi[s])),
                       maxp(maxp(lo[s] - yv, zero), maxp(yv - hi[s], zero)));
            if (!finite(g)) g = inf;
            qc[s] = __builtin_fmax(qc[s], g);
          }
        }
      }
      ent_write<V>(soff_c[c], yn);  // Gy <- y+
    }
#pragma unroll
    for (int s = 0; s < BT; ++s) qp[s] = row16_combine(qp[s], OpAdd());
    if (red_lead) lds_write<V>(red_at, qp);
    // qd and qc stay in registers: the sweep folds its own terms into them
    // b0 holds the copy of the stream's first (row) chunk; its second chunk
    // goes into b1 before the barrier when the first row slot spans two
    if (pro & 1u) load_chunk(b1, A.stream, (uint64_t)(first + 1) * CB, lane16, cs);
    __syncthreads();
    // ---- residual sweep (gathers Gy = y+; own Gd entries = d+) ---------------------
    pos = first + 1 + (pro & 1u);
    // the next iteration's sigma (the candidates are formed only when it runs)
    const bool more = it + 1 < A.iters;
    const T sigma_n = (more && !kPS) ? A.sched[4 * (it + 1)] : zero;
    const T tp1 = T(1) + theta;
    // per-sample steps: this iteration's theta (of K ybar), then the steps of
    // the next one
    T thq[BT];
    if constexpr (kPS) {
#pragma unroll
      for (int s = 0; s < BT; ++s) thq[s] = th_s[s];
      if (A.accel) res_qp_schedule<T, BT>(gam_s, tau_s, sig_s, th_s, pa_s, pd_s);
    }
    // the slot-ordered rhs when not held: through an opaque base, so the loads
    // stay inside the loop
    GV rb = (GV)Rs;
    asm volatile("" : "+s"(rb));
    V qr = qd, qm = qc;  // the thread's dual terms and maxima of both passes
    carry = vzero;
#pragma unroll
    for (int r = 0; r < SLR; ++r) {
      const V rr = kHold ? rrh[kHold ? r : 0] : rb[r * NT + t];
      const V acc = slot_sum<T, V, (SLR > 1), CV>(slot_field(rc, r), slot_field(rl, r), carry,
                                                  b0, b1, pos, A.stream, lane16,
                                                  r == 0 && (pro & 1u), cs);
      const V d = ent_read<V>(soff_r[r]);
      if (rvalid & (1u << r)) {  // kernels.py:158-166
        // e = K y+ - r; equality rows |e|, inequality rows max(e, 0): max(e, w e)
        // with w = -1 / 0.  d * 0 is NaN for a non-finite d: it makes the
        // dual sum, and so the gap, non-finite (kernels.py:172's finiteness).
        const T w = (ineq & (1u << r)) ? zero : T(-1);
#pragma unroll
        for (int s = 0; s < BT; ++s) {
          const T e = acc[s] - rr[s];
          qm[s] = __builtin_fmax(qm[s], __builtin_fmax(e, w * e));
          qr[s] = (qr[s] - rr[s] * d[s]) - d[s] * zero;
        }
      }
      if (more) {
        // d+ of the next iteration from K ybar = (1 + theta) K y+ - theta K y, into
        // Gd where the sample is active (no thread gathers Gd in this sweep; the
        // next column pass does, after the barriers below).  The committed d+
        // stays in dk until the decision: a sample accepted now gets it back.
        const V kyo = r < KYL ? ent_read<V>(kyl_off + (uint32_t)(r * NT + t) * 16u) : ky[r];
        V p;
        if constexpr (kPS) {
#pragma unroll
          for (int s = 0; s < BT; ++s)
            p[s] = d[s] + sig_s[s] * (((T(1) + thq[s]) * acc[s] - thq[s] * kyo[s]) - rr[s]);
        } else {
          p = d + sigma_n * ((tp1 * acc - theta * kyo) - rr);
        }
        if (ineq & (1u << r)) {
#pragma unroll
          for (int s = 0; s < BT; ++s) p[s] = res_pos(p[s]);
        }
        if (act != (1u << BT) - 1u) {
#pragma unroll
          for (int s = 0; s < BT; ++s)
            if (!(act & (1u << s))) p[s] = d[s];  // a frozen sample keeps its dual
        }
        ent_write<V>(soff_r[r], p);
      }
      dk[r] = d;
      if (r < KYL)
        ent_write<V>(kyl_off + (uint32_t)(r * NT + t) * 16u, acc);
      else
        ky[r] = acc;
    }
    if (pro & 2u) {  // the next column pass's second chunk (its first is in b0)
      load_chunk(b1, A.stream, (uint64_t)pos * CB, lane16, cs);
      ++pos;
    }
#pragma unroll
    for (int s = 0; s < BT; ++s) qr[s] = row16_combine(qr[s], OpAdd());
    if (red_lead) lds_write<V>(red_at + VB, qr);
#pragma unroll
    for (int s = 0; s < BT; ++s) qm[s] = row16_combine(qm[s], OpFMax());
    if (red_lead) lds_write<V>(red_at + 2u * VB, qm);
    __syncthreads();
    // ---- the stop test of sample s, on wavefront s: lane l combines partial l
    // (wave l/4, DPP row l%4) in one fixed order; the verdicts go through LDS
    if (wave < BT) {
      const uint32_t pl = red_off + (uint32_t)(lane * kResQ) * VB;
      const V pp = lds_read<V>(pl), pd = lds_read<V>(pl + VB), pm = lds_read<V>(pl + 2u * VB);
      T vp = pp[0], vd = pd[0], vm = pm[0];
#pragma unroll
      for (int u = 1; u < BT; ++u)
        if (wave == u) {
          vp = pp[u];
          vd = pd[u];
          vm = pm[u];
        }
      const T xp = row16_combine(vp, OpAdd());
      const T xd = row16_combine(vd, OpAdd());
      const T xm = row16_combine(vm, OpFMax());
      const T primal =
          ((read_lane(xp, 0) + read_lane(xp, 16)) + read_lane(xp, 32)) + read_lane(xp, 48);
      const T dual_obj =
          ((read_lane(xd, 0) + read_lane(xd, 16)) + read_lane(xd, 32)) + read_lane(xd, 48);
      const T mx = __builtin_fmax(
          __builtin_fmax(__builtin_fmax(read_lane(xm, 0), read_lane(xm, 16)), read_lane(xm, 32)),
          read_lane(xm, 48));
      const int64_t b = bs0 + wave;
      const T tol = A.tolv ? (b < A.batch ? A.tolv[b] : T(0)) : A.tol;
      const T gap = maxp(primal - dual_obj, zero) / maxp(T(1), maxp(absv(primal), absv(dual_obj)));
      const bool ok = finite(gap) && mx <= tol && gap <= tol;
      if (lane == 0) lds_write<uint32_t>(dec_off + 4u * (uint32_t)wave, ok ? 1u : 0u);
    }
    __syncthreads();
    {
      uint32_t accept = 0;
#pragma unroll
      for (int s = 0; s < BT; ++s) {
        if (lds_read<uint32_t>(dec_off + 4u * (uint32_t)s) && (act & (1u << s))) accept |= 1u << s;
        if (act & (1u << s)) ++cnt[s];  // this iteration ran for the sample
      }
      accept = (uint32_t)__builtin_amdgcn_readfirstlane((int)accept);
      if (accept && more) {
        // accepted now: the sample keeps (y+, d+) of this iteration.  Its Gd
        // entries hold the candidate the sweep wrote; restore d+ (own entries).
        // The next column pass may gather either value for this sample only,
        // whose update and diagnostics are masked from here on, so no barrier
        // is needed before it.
#pragma unroll
        for (int r = 0; r < SLR; ++r) {
          V p = ent_read<V>(soff_r[r]);
#pragma unroll
          for (int s = 0; s < BT; ++s)
            if (accept & (1u << s)) p[s] = dk[r][s];
          ent_write<V>(soff_r[r], p);
        }
      }
      act = (uint32_t)__builtin_amdgcn_readfirstlane((int)(act & ~accept));
    }
    // b0 (and b1 when the first column slot spans two chunks) hold the first
    // column chunks again and pos follows them; the partials are rewritten
    // only after the next barrier
  }
  // ---- hand the state to the batch-minor layout ---------------------------------
#pragma unroll
  for (int c = 0; c < SLC; ++c) {
    const int j = A.colmap[c * NT + t];
    if (j >= 0) {
      const V yv = ent_read<V>(soff_c[c]);
#pragma unroll
      for (int s = 0; s < BT; ++s) A.Y[(int64_t)j * A.Bp + bs0 + s] = yv[s];
    }
  }
#pragma unroll
  for (int r = 0; r < SLR; ++r) {
    const int i = A.rowmap[r * NT + t];
    if (i >= 0) {
      const V d = ent_read<V>(soff_r[r]);
#pragma unroll
      for (int s = 0; s < BT; ++s) A.D[(int64_t)i * A.Bp + bs0 + s] = d[s];
    }
  }
#pragma unroll
  for (int s = 0; s < BT; ++s) {
    if (t == s) {
      A.count[bs0 + s] = cnt[s];
      A.done[bs0 + s] = (bs0 + s < A.batch && !(act & (1u << s))) ? 1 : 0;
    }
  }
}

// Per-sample coefficients in the plan's stream order: out[tile][k][u][lane]
// (BT values, the tile's samples) = the coefficient of stream entry (chunk k,
// lane, entry u): RV (kept CSR, [nnz][Bp]) for row sections, CV (kept CSC)
// for column sections, 0 for padding (srcmap: the plan's map, [chunk][lane][4]).
// One thread per (stream entry, tile), tiles fastest (the reads of one entry
// run along the batch).
template <typename T, int BT>
__global__ __launch_bounds__(256) void k_res_coef_stream(const int32_t* __restrict__ srcmap,
                                                         int64_t entries,
                                                         const T* __restrict__ RV,
                                                         const T* __restrict__ CV, int64_t Bp,
                                                         int64_t tiles, T* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= entries * tiles) return;
  const int64_t tile = gid % tiles, e = gid / tiles;
  const int64_t k = e >> 8;
  const int lane = (int)((e >> 2) & 63), u = (int)(e & 3);
  const int32_t src = srcmap[e];
  const int64_t o = (((tile * (entries >> 8) + k) * 4 + u) * 64 + lane) * BT;
  const int64_t b = tile * BT;
#pragma unroll
  for (int s = 0; s < BT; ++s) {
    T v = T(0);
    if (src >= 0)
      v = (src & kResSrcCol) ? CV[(int64_t)(src & ~kResSrcCol) * Bp + b + s]
                             : RV[(int64_t)src * Bp + b + s];
    out[o + s] = v;
  }
}

// dst[(tile*K + k)*BT + s] = src[map[k]*Bp + tile*BT + s] (0 for empty slots).
// A block moves 64 slots x 64 samples (64 / BT tiles) through LDS: it reads
// each slot's 64 samples as one contiguous run of the batch-minor source and
// writes each tile's 64 slots x BT values as one contiguous run.  Launch:
// grid (tiles / (64 / BT), K / 64), 256 threads; tiles and K are multiples of
// 64 (the padded batch and the slot counts are).
template <typename T, int BT>
__global__ __launch_bounds__(256) void k_res_gather(const T* __restrict__ src, int64_t Bp,
                                                    const int32_t* __restrict__ map, int K,
                                                    int64_t tiles, T* __restrict__ dst) {
  constexpr int TT = 64 / BT;  // tiles of the block
  __shared__ T buf[64][65];    // [slot][sample of the block]
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * TT;
  const int k0 = blockIdx.y * 64;
  const int64_t b = t0 * BT + tx;
  T v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int j = map[k0 + ty + 4 * i];
    v[i] = j >= 0 ? src[(int64_t)j * Bp + b] : T(0);
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) buf[ty + 4 * i][tx] = v[i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int e = threadIdx.x + 256 * i;  // (tile of the block, slot, sample): 64 * BT per tile
    const int tt = e / (64 * BT), rem = e % (64 * BT);
    const int kk = rem / BT, s = rem % BT;
    dst[((t0 + tt) * K + k0 + kk) * BT + s] = buf[kk][tt * BT + s];
  }
}

template <typename T>
__global__ void k_res_gather_shared(const T* __restrict__ src, const int32_t* __restrict__ map,
                                    int K, T* __restrict__ dst) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k < K) dst[k] = map[k] >= 0 ? src[map[k]] : T(0);
}

}  // namespace purin
