// Internal interface shared by the forward and adjoint drivers.
#pragma once

#include "kernels.hpp"
#include "plan.hpp"

namespace purin {

// Byte offsets of the saved-state region (filled by the forward, read by the
// adjoint) and of the plan workspace used by the forward.
struct Layout {
  int64_t Bp;
  int ncb, nrb;
  // saved region
  size_t hdr, Tt, Y, D, R, LO, HI, RF, conv, feas, saved_end;
  // forward workspace
  size_t YB, MF, DF, SL, colpart, rowpart, done, count, ndone, ores, ogap, ofin, X, Z;
  size_t RTs, RRs, RD0, RLs, RHs;  // resident path (slot-ordered inputs)
  size_t ws_end;
};

Layout make_layout(const purin_cp_plan* p, int64_t batch);

inline dim3 tile_grid(int64_t Bp, int64_t tile, int64_t blocks) {
  return dim3((unsigned)(Bp / tile), (unsigned)std::max<int64_t>(1, std::min<int64_t>(blocks, 65535)));
}

template <typename T>
inline Mat<T> kept_matrix(const purin_cp_plan* p, bool scaled) {
  Mat<T> K;
  K.m = (int)p->m;
  K.n = (int)p->n;
  K.me = (int)p->me;
  K.rptr = p->rptr;
  K.ridx = p->ridx;
  K.rval = (const T*)(scaled ? p->rval_s : p->rval_o);
  K.cptr = p->cptr;
  K.cidx = p->cidx;
  K.cval = (const T*)(scaled ? p->cval_s : p->cval_o);
  return K;
}

template <typename T>
inline void to_minor(hipStream_t st, const T* src, int64_t B, int64_t C, int64_t ld, T* dst, int64_t Bp,
              const T* colmul, int mode) {
  if (C == 0) return;
  dim3 grid((unsigned)((C + 63) / 64), (unsigned)(Bp / 64));
  k_to_minor<T><<<grid, kBlock, 0, st>>>(src, B, C, ld, dst, Bp, colmul, mode);
}

template <typename T>
inline void to_major(hipStream_t st, const T* src, int64_t Bp, int64_t C, T* dst, int64_t B, int64_t ld,
              const T* colmul, int mode) {
  if (C == 0 || B == 0) return;
  dim3 grid((unsigned)((C + 63) / 64), (unsigned)((B + 63) / 64));
  k_to_major<T><<<grid, kBlock, 0, st>>>(src, Bp, C, dst, B, ld, colmul, mode);
}

}  // namespace purin
