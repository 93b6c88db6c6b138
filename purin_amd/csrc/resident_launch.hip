// Launches of the resident (on-chip) CP kernels for one element type and one
// row-slot count.  The build compiles this file once per (type, row slots)
// pair, selected by PURIN_RES_F64 (1: double, 0: float) and PURIN_RES_SLR
// (1..4), so that the 128 kernel variants (4 column-slot counts, shared or
// per-sample bounds, fixed-iteration or early-stop, per pair) compile in
// parallel translation units.  forward.hip dispatches to them.

#include "plan.hpp"
#include "resident.hpp"

#ifndef PURIN_RES_F64
#error "compile with -DPURIN_RES_F64=0|1 -DPURIN_RES_SLR=1..4"
#endif

namespace purin {

// kind: 0 the projection, 1 the diagonal QP (per-sample bounds), 2
// per-sample coefficients, 3 the diagonal QP with per-sample coefficients
template <typename T, int SLR, int SLC, int NB>
static int launch_nb(const Res<T>& R, hipStream_t st, int64_t tiles, size_t lds, bool sb,
                     bool early, int kind) {
  if (((kind == 1 || kind == 3) && sb) || kind < 0 || kind > 3)
    return set_error(PURIN_CP_ERR_ARG, "resident kernel variant out of range");
  auto kern = kind == 1 ? (early ? k_resident_early<T, SLR, SLC, false, NB, true>
                                 : k_resident<T, SLR, SLC, false, NB, true>)
              : kind == 3 ? (early ? k_resident_early<T, SLR, SLC, false, NB, true, true>
                                   : k_resident<T, SLR, SLC, false, NB, true, true>)
              : kind == 2 ? (early ? (sb ? k_resident_early<T, SLR, SLC, true, NB, false, true>
                                         : k_resident_early<T, SLR, SLC, false, NB, false, true>)
                                   : (sb ? k_resident<T, SLR, SLC, true, NB, false, true>
                                         : k_resident<T, SLR, SLC, false, NB, false, true>))
              : early ? (sb ? k_resident_early<T, SLR, SLC, true, NB>
                            : k_resident_early<T, SLR, SLC, false, NB>)
                      : (sb ? k_resident<T, SLR, SLC, true, NB>
                            : k_resident<T, SLR, SLC, false, NB>);
  if (int rc = raise_lds_cap((const void*)kern, lds)) return rc;
  kern<<<dim3((unsigned)tiles), dim3(kResThreads), lds, st>>>(R);
  return PURIN_CP_OK;
}

// nb: samples per tile (resident.hpp, ResV); 8 only for fp32 with one row and
// one column slot per thread (two LDS planes)
template <typename T, int SLR, int SLC>
static int launch_one(const Res<T>& R, hipStream_t st, int64_t tiles, size_t lds, bool sb,
                      bool early, int nb, int kind) {
  constexpr int NB = sizeof(T) == 4 && SLR == 1 && SLC == 1 ? 8 : ResVec<T>::BT;
  if (nb != NB) return set_error(PURIN_CP_ERR_ARG, "resident tile size out of range");
  return launch_nb<T, SLR, SLC, NB>(R, st, tiles, lds, sb, early, kind);
}

template <typename T, int SLR>
int launch_resident_rows(const Res<T>& R, hipStream_t st, int64_t tiles, size_t lds, int slc,
                         bool sb, bool early, int nb, int kind) {
  switch (slc) {
    case 1: return launch_one<T, SLR, 1>(R, st, tiles, lds, sb, early, nb, kind);
    case 2: return launch_one<T, SLR, 2>(R, st, tiles, lds, sb, early, nb, kind);
    case 3: return launch_one<T, SLR, 3>(R, st, tiles, lds, sb, early, nb, kind);
    case 4: return launch_one<T, SLR, 4>(R, st, tiles, lds, sb, early, nb, kind);
    default: return set_error(PURIN_CP_ERR_ARG, "resident column slot count out of range");
  }
}

#if PURIN_RES_F64
template int launch_resident_rows<double, PURIN_RES_SLR>(const Res<double>&, hipStream_t, int64_t,
                                                         size_t, int, bool, bool, int, int);
#else
template int launch_resident_rows<float, PURIN_RES_SLR>(const Res<float>&, hipStream_t, int64_t,
                                                        size_t, int, bool, bool, int, int);
#endif

}  // namespace purin
