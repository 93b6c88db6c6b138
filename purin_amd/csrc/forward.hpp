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
  size_t YB, MF, DF, SL, colpart, rowpart, decpart, done, count, ndone, ores, ogap, ofin, X, Z;
  size_t RTs, RRs, RD0, RLs, RHs;  // resident path (slot-ordered inputs)
  size_t RQs, RY0;                 // resident diagonal QP: q and y0 in slot order
  size_t RCS;                      // resident per-sample coefficients: the tiles' coefficient streams
  // per-sample coefficients (values given per call): entry values in the
  // caller's order (VF), the kept CSR / CSC entries original (RVo, CVo) and
  // row-scaled (RV, CV), bound-row coefficients (BC), row scales (SC), steps
  size_t VF, RVo, CVo, RV, CV, BC, SC, SGR, ACB, DCB, STB, RPT, CPT, PX, PZ, PW, PD;
  size_t RVs, CVs;    // [nnz] the scaled CSR / CSC entries when every sample has the plan's
  size_t QQ, QC, QS;  // general QP: q, c (n x Bp) and per-sample max q, min q
  size_t ws_end;
};

// Optional parts of the forward workspace.
constexpr int kLayoutSpmm = 1;  // X, Z: purin_cp_spmm's batch-minor staging
constexpr int kLayoutWarm = 2;  // MF: warm-start multipliers / duals in batch-minor layout

Layout make_layout(const purin_cp_plan* p, int64_t batch, bool values = false, int extras = 0);

// Workspace bytes of an adjoint entry point (purin_cp_workspace_bytes; adjoint.hip):
// the largest over its optional arguments.
int adjoint_workspace_bytes(const purin_cp_plan* p, int32_t entry, int64_t batch,
                            const purin_cp_adjoint_options& o, int64_t* bytes);

// Per-sample coefficient arrays prepared for one call (see persample.hpp).
template <typename T>
struct PerSample {
  const T* RVo;   // [nnz][Bp] kept CSR entries, original
  const T* CVo;   // [nnz][Bp] kept CSC entries, original
  const T* RV;    // [nnz][Bp] row-scaled CSR
  const T* CV;    // [nnz][Bp] row-scaled CSC
  const T* RVs;   // [nnz] row-scaled CSR shared by every sample (the plan's own
  const T* CVs;   //   coefficients: sample 0's entries of RV / CV), or nullptr
  const T* BC;    // [nb][Bp] bound-row coefficients
  const T* SC;    // [m][Bp] row scales
  T* sig_rb;      // [m][Bp] diagonal sigma, or nullptr
  T* a_cb;        // [n][Bp] diagonal prox a, or nullptr
  T* d_cb;        // [n][Bp] diagonal prox delta, or nullptr
  T* tau_cb;      // [n][Bp] diagonal tau (general-q QP), or nullptr
  T* tau_b;       // [Bp] scalar steps (and schedule state) per sample
  T* sig_b;
  T* a_b;
  T* d_b;
  T* th_b;
  T* tol_b;       // [Bp] stop-test tolerance
};

// General diagonal QP objective (diagonal_qp.py): q, c [n][Bp] and the
// per-sample gamma = min q of the accelerated schedule (kernels.py:228, 279).
template <typename T>
struct QPRun {
  const T* Q;
  const T* Cc;
  const T* gamma;
  int dense;  // the dense adapter's policy (factored prox, no freezing, no stationarity)
};

// Which steps prepare_values computes.
enum ValuesMode {
  kProjectForward = 0,  // kernels.py:209-227 with q = 1 (norm bound or power iteration)
  kProjectAdjoint = 1,  // bounds.py:83-101: power-iteration L, tau = s/(1 + L)
  kQPForward = 2,       // kernels.py:209-227 with a general diagonal q
  kQPAdjoint = 3,       // diagonal_qp.py:137-160: norm bound or power L, tau = s/(max q + L)
};

// Gather and prepare the per-sample arrays from values (batch-major (B, nnz_full)
// in the plan's CSR entry order; nullptr: the plan's own values for every
// sample, plans that keep every row only).  qmax / qmin: per-sample extremes
// of a general q (QP modes).  forward.hip.
template <typename T>
int prepare_values(purin_cp_plan* p, hipStream_t st, int64_t batch, const Layout& L, char* ws,
                   const T* values, T tol, int mode, const T* qmax, const T* qmin,
                   PerSample<T>* ps);

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
  K.rvb = nullptr;
  K.cvb = nullptr;
  K.vbp = 0;
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
