// Forward drivers: purin_cp_spmm, purin_cp_solve, purin_cp_project.
//
// One CP iteration is two launches in fixed-iteration mode (row pass, column
// pass) and four with the per-sample stop test (row, column, residual,
// decide).  The per-iteration step scalars are the same for every sample
// (shared matrix => shared norm bound and shared tau/sigma/theta schedule,
// reference src/purin/solvers/chambolle_pock/kernels.py:209-227, 279-283), so
// the host computes them in the plan's precision and passes them as kernel
// arguments; nothing per-sample leaves the device inside the loop except the
// all-done counter, read every ``check_every`` iterations.

#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "plan.hpp"
#include "post.hpp"
#include "forward.hpp"
#include "resident.hpp"
#include "persample.hpp"

namespace purin {

static size_t al(size_t x) { return (x + 255) & ~size_t(255); }

Layout make_layout(const purin_cp_plan* p, int64_t batch, bool values, int extras) {
  Layout L{};
  const size_t es = elem_size(p);
  const int64_t Bp = padded_batch(p, batch);
  L.Bp = Bp;
  const size_t n = p->n, m = p->m, M = p->M, mi = p->mi;
  L.nrb = (int)((m + 4 * kRowsPerWaveEarly - 1) / (4 * kRowsPerWaveEarly));
  L.ncb = (int)((n + 4 * kRowsPerWaveEarly - 1) / (4 * kRowsPerWaveEarly));
  size_t o = 0;
  auto take = [&](size_t bytes) { size_t r = o; o = al(o + bytes); return r; };
  L.hdr = take(kSavedHeader);
  L.Tt = take(n * Bp * es);
  L.Y = take(n * Bp * es);
  L.D = take(m * Bp * es);
  L.R = take(m * Bp * es);
  L.LO = take(n * Bp * es);
  L.HI = take(n * Bp * es);
  L.RF = take(M * Bp * es);
  L.conv = take(Bp * 4);
  L.feas = take(Bp * 4);
  L.saved_end = o;
  o = 0;
  L.YB = take(n * Bp * es);
  L.MF = (extras & kLayoutWarm) ? take(M * Bp * es) : 0;
  L.DF = take(M * Bp * es);
  L.SL = take(mi * Bp * es);
  L.colpart = take((size_t)5 * std::max(L.ncb, 1) * Bp * es);
  L.rowpart = take((size_t)3 * std::max(L.nrb, 1) * Bp * es);
  L.decpart = take((size_t)8 * kDecideSplit * Bp * es);  // k_decide's split pre-pass
  L.done = take(Bp * 4);
  L.count = take(Bp * 4);
  L.ndone = take(256);
  L.ores = take(Bp * es);
  L.ogap = take(Bp * es);
  L.ofin = take(Bp * 4);
  if (extras & kLayoutSpmm) {  // spmm input / output staging
    L.X = take(std::max(n, m) * Bp * es);
    L.Z = take(std::max(n, m) * Bp * es);
  }
  if (p->res_ok) {  // resident path: slot-ordered copies of the per-sample inputs
    const size_t Kr = (size_t)p->res_mr * kResThreads, Kc = (size_t)p->res_mc * kResThreads;
    L.RTs = take(Kc * Bp * es);
    L.RRs = take(Kr * Bp * es);
    L.RD0 = take(Kr * Bp * es);
    L.RLs = take(Kc * Bp * es);
    L.RHs = take(Kc * Bp * es);
    if (values) {  // the diagonal QP and per-sample coefficients on the resident kernel
      L.RQs = take(Kc * Bp * es);
      L.RY0 = take(Kc * Bp * es);
      const size_t chunks = (size_t)p->res_stream_bytes /
                            (64 * 16 + 64 * 4 * (size_t)es);  // the plan's stream chunks
      L.RCS = take(chunks * 256 * Bp * es);
    }
  }
  if (values) {
    const size_t nnz = p->nnz, nb = p->bound.size();
    L.VF = take((size_t)p->nnz_full * Bp * es);
    L.RVo = take(nnz * Bp * es);
    L.CVo = take(nnz * Bp * es);
    L.RV = take(nnz * Bp * es);
    L.CV = take(nnz * Bp * es);
    L.RVs = take(std::max<size_t>(nnz, 1) * es);
    L.CVs = take(std::max<size_t>(nnz, 1) * es);
    L.BC = take(nb * Bp * es);
    L.SC = take(m * Bp * es);
    if (p->diag) {
      L.SGR = take(m * Bp * es);
      L.ACB = take(n * Bp * es);
      L.DCB = take(n * Bp * es);
    }
    // tau, sigma, a, delta, theta, tol, L, then the schedule's second buffer
    // (tau, sigma, a, delta, theta)
    L.STB = take((size_t)12 * Bp * es);
    L.RPT = take((size_t)2 * std::max(L.nrb, 1) * Bp * es);
    L.CPT = take((size_t)std::max(L.ncb, 1) * Bp * es);
    L.PX = take(n * Bp * es);  // power iteration vectors and dots
    L.PZ = take(std::max<size_t>(m, 1) * Bp * es);
    L.PW = take(n * Bp * es);
    L.PD = take((size_t)2 * Bp * es);
    L.QQ = take(n * Bp * es);
    L.QC = take(n * Bp * es);
    L.QS = take((size_t)2 * Bp * es);
  }
  L.ws_end = o;
  return L;
}

// Per-sample power iteration on K~^T K~ (kernels.py:52-65): every sample starts
// from the plan's normalised start vector; returns sqrt(max(eig, 0)) + eps in Lout.
template <typename T>
static void ps_power(const purin_cp_plan* p, hipStream_t st, const Layout& L, char* ws,
                     const Mat<T>& K, T* Lout) {
  const int64_t Bp = L.Bp, n = p->n, m = p->m;
  constexpr int64_t TS = tile_samples<T>();
  T* X = (T*)(ws + L.PX);
  T* Z = (T*)(ws + L.PZ);
  T* Wv = (T*)(ws + L.PW);
  T* eig = (T*)(ws + L.PD);
  T* ww = eig + Bp;
  const T eps = T(1e-12);
  k_ps_start<T><<<1024, 256, 0, st>>>(n, Bp, (const T*)p->ps_start, X);
  k_fill<T><<<8, 256, 0, st>>>(eig, Bp, T(0));
  for (int it = 0; it < p->opts.norm_iterations; ++it) {
    if (m) {
      k_spmv_rows<T><<<tile_grid(Bp, TS, (m + 3) / 4), kBlock, 0, st>>>(K, Bp, X, Z);
      k_spmv_cols<T><<<tile_grid(Bp, TS, (n + 3) / 4), kBlock, 0, st>>>(K, Bp, Z, Wv);
    } else {
      k_fill<T><<<1024, 256, 0, st>>>(Wv, n * Bp, T(0));
    }
    k_ps_dots<T><<<(unsigned)((Bp + 255) / 256), 256, 0, st>>>(n, Bp, X, Wv, eig, ww);
    k_ps_normalize<T><<<1024, 256, 0, st>>>(n, Bp, Wv, ww, eps, X);
  }
  k_ps_norm_final<T><<<(unsigned)((Bp + 255) / 256), 256, 0, st>>>(Bp, eig, eps, Lout);
}

// dst[k] = src[k][0]: sample 0's entry of each row of a [count][Bp] array
template <typename T>
__global__ void k_sample0(const T* __restrict__ src, int64_t Bp, int64_t count, T* dst) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (k < count) dst[k] = src[k * Bp];
}

template <typename T>
int prepare_values(purin_cp_plan* p, hipStream_t st, int64_t batch, const Layout& L, char* ws,
                   const T* values, T tol, int mode, const T* qmax, const T* qmin,
                   PerSample<T>* ps) {
  const bool adjoint = mode == kProjectAdjoint || mode == kQPAdjoint;
  const bool qp = mode == kQPForward || mode == kQPAdjoint;
  const int64_t Bp = L.Bp, n = p->n, m = p->m, nnz = p->nnz;
  const int64_t nb = (int64_t)p->bound.size();
  constexpr int64_t TS = tile_samples<T>();
  T* VF = (T*)(ws + L.VF);
  T* RVo = (T*)(ws + L.RVo);
  T* CVo = (T*)(ws + L.CVo);
  T* RV = (T*)(ws + L.RV);
  T* CV = (T*)(ws + L.CV);
  T* BC = (T*)(ws + L.BC);
  T* SC = (T*)(ws + L.SC);
  T* stb = (T*)(ws + L.STB);
  T* rpart = (T*)(ws + L.RPT);
  T* cpart = (T*)(ws + L.CPT);
  // padded samples (b >= batch) get zero coefficients (to_minor pads with 0)
  if (values) {
    to_minor<T>(st, values, batch, p->nnz_full, p->nnz_full, VF, Bp, nullptr, 0);
  } else {
    if (p->nnz != p->nnz_full)
      return set_error(PURIN_CP_ERR_ARG, "shared values need a plan that keeps every row");
    k_bcast_entries<T><<<2048, 256, 0, st>>>((const T*)p->rval_o, p->nnz_full, Bp, batch, VF);
  }
  if (nnz) {
    k_gather_entries<T><<<2048, 256, 0, st>>>(VF, Bp, p->ps_kcsr, nnz, RVo);
    k_gather_entries<T><<<2048, 256, 0, st>>>(VF, Bp, p->ps_kcsc, nnz, CVo);
  }
  if (nb) k_gather_entries<T><<<2048, 256, 0, st>>>(VF, Bp, p->ps_bpos, nb, BC);
  const bool diag = p->diag;
  const T safety = (T)p->opts.safety;
  ps->RVo = RVo;
  ps->CVo = CVo;
  ps->RV = RV;
  ps->CV = CV;
  ps->BC = BC;
  ps->SC = SC;
  ps->sig_rb = diag ? (T*)(ws + L.SGR) : nullptr;
  ps->a_cb = (diag && !qp) ? (T*)(ws + L.ACB) : nullptr;
  ps->d_cb = (diag && !qp) ? (T*)(ws + L.DCB) : nullptr;
  ps->tau_cb = (diag && qp) ? (T*)(ws + L.ACB) : nullptr;
  ps->tau_b = stb;
  ps->sig_b = stb + Bp;
  ps->a_b = stb + 2 * Bp;
  ps->d_b = stb + 3 * Bp;
  ps->th_b = stb + 4 * Bp;
  ps->tol_b = stb + 5 * Bp;
  T* Lpi = stb + 6 * Bp;
  if (m)
    k_ps_rows<T><<<tile_grid(Bp, TS, L.nrb), kBlock, 0, st>>>(
        (int)m, Bp, p->rptr, RVo, p->opts.row_scaling, safety, SC, RV, ps->sig_rb, rpart, L.nrb);
  k_ps_cols<T><<<tile_grid(Bp, TS, L.ncb), kBlock, 0, st>>>(
      (int)n, Bp, p->cptr, p->cidx, CVo, SC, safety, CV, ps->a_cb, ps->d_cb, ps->tau_cb, cpart,
      L.ncb);
  // the power iteration sets L for the projection's adjoint (bounds.py:88-101)
  // and wherever the norm bound is off (kernels.py:211-212, diagonal_qp.py:148-157)
  const bool power = !diag && (mode == kProjectAdjoint || !p->opts.norm_bound);
  if (power) {
    Mat<T> K = kept_matrix<T>(p, true);
    K.rvb = RV;
    K.cvb = CV;
    K.vbp = Bp;
    ps_power<T>(p, st, L, ws, K, Lpi);
  }
  k_ps_steps<T><<<(unsigned)((Bp + 255) / 256), 256, 0, st>>>(
      Bp, rpart, (int)(m ? L.nrb : 0), cpart, L.ncb, power ? Lpi : nullptr, safety,
      adjoint ? 0 : p->opts.accelerated, tol, qp ? qmax : nullptr, qp ? qmin : nullptr, ps->tau_b,
      ps->sig_b, ps->a_b, ps->d_b, ps->th_b, ps->tol_b);
  // with the plan's own coefficients every sample's scaled entries are the same
  // (the same broadcast values through the same per-sample arithmetic), so the
  // iterations can read one shared copy instead of B per-sample copies
  ps->RVs = ps->CVs = nullptr;
  if (!values && nnz) {
    T* RVs = (T*)(ws + L.RVs);
    T* CVs = (T*)(ws + L.CVs);
    const unsigned g = (unsigned)((nnz + 255) / 256);
    k_sample0<T><<<g, 256, 0, st>>>(RV, Bp, nnz, RVs);
    k_sample0<T><<<g, 256, 0, st>>>(CV, Bp, nnz, CVs);
    ps->RVs = RVs;
    ps->CVs = CVs;
  }
  PURIN_HIP(hipGetLastError());
  return PURIN_CP_OK;
}
template int prepare_values<double>(purin_cp_plan*, hipStream_t, int64_t, const Layout&, char*,
                                    const double*, double, int, const double*, const double*,
                                    PerSample<double>*);
template int prepare_values<float>(purin_cp_plan*, hipStream_t, int64_t, const Layout&, char*,
                                   const float*, float, int, const float*, const float*,
                                   PerSample<float>*);

// Samples per resident tile: 16 bytes of samples per gathered element, or 8
// fp32 samples in two LDS planes where one row and one column slot per thread
// hold the problem (resident.hpp, ResV): each tile's pass over the shared
// matrix stream then serves twice the samples.
int res_tile_samples(const purin_cp_plan* p) {
  if (p->dtype == PURIN_CP_F32 && p->res_mr == 1 && p->res_mc == 1) return 8;
  return p->dtype == PURIN_CP_F64 ? ResVec<double>::BT : ResVec<float>::BT;
}

// One translation unit per (element type, row slots): resident_launch.hip.
// kind: 0 the projection, 1 the diagonal QP, 2 per-sample coefficients, 3 the
// diagonal QP with per-sample coefficients
template <typename T, int SLR>
int launch_resident_rows(const Res<T>& R, hipStream_t st, int64_t tiles, size_t lds, int slc,
                         bool sb, bool early, int nb, int kind);

template <typename T>
static int launch_resident(const Res<T>& R, hipStream_t st, int64_t tiles, size_t lds, int slr,
                           int slc, bool sb, bool early, int nb, int kind) {
  switch (slr) {
    case 1: return launch_resident_rows<T, 1>(R, st, tiles, lds, slc, sb, early, nb, kind);
    case 2: return launch_resident_rows<T, 2>(R, st, tiles, lds, slc, sb, early, nb, kind);
    case 3: return launch_resident_rows<T, 3>(R, st, tiles, lds, slc, sb, early, nb, kind);
    case 4: return launch_resident_rows<T, 4>(R, st, tiles, lds, slc, sb, early, nb, kind);
    default: return set_error(PURIN_CP_ERR_ARG, "resident row slot count out of range");
  }
}

// LDS of the resident kernel (the early-stop one: with its partials), or 0
// when the problem does not fit on chip.
template <typename T>
static size_t resident_lds(const purin_cp_plan* p, bool early = false) {
  if (!p->res_ok) return 0;
  if (res_tile_samples(p) == 8)  // two planes of the largest one-slot image
    return (size_t)2 * kResPlane + (early ? res_early_extra(32u, 8u) : 0);
  // Gy (n) | zero | Gd (m) | trash, 16 bytes each
  const size_t lds = (size_t)(p->n + 1 + p->m + 1) * 16 +
                     (early ? kResEarlyExtra + (size_t)res_early_kyl(p->res_mr, p->res_mc) *
                                                   kResThreads * 16
                            : 0);
  return lds <= 160 * 1024 ? lds : 0;
}

// The CP loop on the resident kernel; fills Y and D like the passes (and, with
// early stop, the per-sample done flags and iteration counts).  qp (with ps):
// the diagonal QP, q and c per sample, y0 from Y, the per-sample steps of ps.
// ps alone: per-sample coefficients (ps's RV, CV laid out in the plan's stream
// order per tile) and per-sample steps.
template <typename T>
static int run_resident(purin_cp_plan* p, hipStream_t st, const Layout& L, char* sv, char* ws,
                        const purin_cp_solve_options& o, size_t lds, bool early = false,
                        int64_t batch = 0, T tol = T(0), const T* tolv = nullptr,
                        int32_t* done = nullptr, int32_t* count = nullptr, bool noalloc = false,
                        const QPRun<T>* qp = nullptr, const PerSample<T>* ps = nullptr) {
  const int BT = res_tile_samples(p);
  const int64_t Bp = L.Bp, tiles = Bp / BT;
  const int Kr = p->res_mr * kResThreads, Kc = p->res_mc * kResThreads;
  // the step schedule built with the plan covers kSchedCapacity iterations;
  // a longer call grows it stream-ordered (not in the no-allocation entry)
  if (noalloc && o.max_iterations > p->res_sched_len)
    return set_error(PURIN_CP_ERR_ARG,
                     "max_iterations exceeds the plan's step schedule (" +
                         std::to_string(p->res_sched_len) +
                         " iterations) in the no-allocation entry point");
  const void* sched = p->res_sched;  // per-sample steps (QP, coefficients) instead
  if (!ps)
    if (int rc = ensure_schedule(p, o.max_iterations, st, false, &sched)) return rc;
  Res<T> R{};
  R.n = (int)p->n;
  R.m = (int)p->m;
  R.me = (int)p->me;
  R.Bp = Bp;
  R.Kr = Kr;
  R.Kc = Kc;
  R.rowmap = p->res_rowmap;
  R.colmap = p->res_colmap;
  R.rowent = p->res_rowent;
  R.colent = p->res_colent;
  R.stream = p->res_stream;  // both kernels walk the same chunk streams
  R.wtab = p->res_wtab;
  R.batch = batch;
  R.tol = tol;
  R.tolv = tolv;
  R.done = done;
  R.count = count;
  T* Ts = (T*)(ws + L.RTs);
  T* Rs = (T*)(ws + L.RRs);
  T* D0s = (T*)(ws + L.RD0);
  T* Ls = (T*)(ws + L.RLs);
  T* Hs = (T*)(ws + L.RHs);
  // slot-ordered copies per tile (k_res_gather: 64 slots x 64 samples per block;
  // tiles and the slot counts are multiples of 64)
  const dim3 gc((unsigned)(tiles / (64 / BT)), (unsigned)(Kc / 64));
  const dim3 gr((unsigned)(tiles / (64 / BT)), (unsigned)(Kr / 64));
  auto gather = [&](dim3 g, const T* src, const int32_t* map, int K, T* dst) {
    if (BT == 8)
      k_res_gather<T, 8><<<g, 256, 0, st>>>(src, Bp, map, K, tiles, dst);
    else
      k_res_gather<T, ResVec<T>::BT><<<g, 256, 0, st>>>(src, Bp, map, K, tiles, dst);
  };
  if (qp) {  // c in the target's place, q, and the start y0
    T* Qs = (T*)(ws + L.RQs);
    T* Y0s = (T*)(ws + L.RY0);
    gather(gc, qp->Cc, p->res_colmap, Kc, Ts);
    gather(gc, qp->Q, p->res_colmap, Kc, Qs);
    gather(gc, (const T*)(sv + L.Y), p->res_colmap, Kc, Y0s);
    R.Qs = Qs;
    R.Y0s = Y0s;
    R.step0 = ps->tau_b;  // [5][Bp]: tau, sigma, a, delta, theta of iteration 0
    R.gam = p->opts.accelerated ? qp->gamma : nullptr;
    R.accel = p->opts.accelerated;
  } else {
    gather(gc, (const T*)(sv + L.Tt), p->res_colmap, Kc, Ts);
  }
  if (ps && !ps->RVs) {  // per-sample coefficients: each tile's stream of them
    const int64_t entries = p->res_stream_bytes / (int64_t)res_chunk_bytes<T>() * 256;
    T* CS = (T*)(ws + L.RCS);
    const int64_t threads = entries * tiles;
    const unsigned blocks = (unsigned)((threads + 255) / 256);
    if (BT == 8)
      k_res_coef_stream<T, 8><<<blocks, 256, 0, st>>>(p->res_srcmap, entries, ps->RV, ps->CV, Bp,
                                                      tiles, CS);
    else
      k_res_coef_stream<T, ResVec<T>::BT><<<blocks, 256, 0, st>>>(p->res_srcmap, entries, ps->RV,
                                                                  ps->CV, Bp, tiles, CS);
    R.Cs = CS;
    R.cs_tile = entries;
    if (!qp) {
      R.step0 = ps->tau_b;
      R.gam = nullptr;  // gamma = min q = 1
      R.accel = p->opts.accelerated;
    }
  }
  gather(gr, (const T*)(sv + L.R), p->res_rowmap, Kr, Rs);
  gather(gr, (const T*)(sv + L.D), p->res_rowmap, Kr, D0s);
  if (o.shared_bounds) {
    k_res_gather_shared<T><<<(Kc + 255) / 256, 256, 0, st>>>((const T*)(sv + L.LO), p->res_colmap, Kc, Ls);
    k_res_gather_shared<T><<<(Kc + 255) / 256, 256, 0, st>>>((const T*)(sv + L.HI), p->res_colmap, Kc, Hs);
  } else {
    gather(gc, (const T*)(sv + L.LO), p->res_colmap, Kc, Ls);
    gather(gc, (const T*)(sv + L.HI), p->res_colmap, Kc, Hs);
  }
  R.Ts = Ts;
  R.Rs = Rs;
  R.D0s = D0s;
  R.Ls = Ls;
  R.Hs = Hs;
  R.sched = (const T*)sched;
  R.iters = o.max_iterations;
  R.Y = (T*)(sv + L.Y);
  R.D = (T*)(sv + L.D);
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (o.timing) {
    PURIN_HIP(hipEventCreate(&e0));
    PURIN_HIP(hipEventCreate(&e1));
    PURIN_HIP(hipEventRecord(e0, st));
  }
  // per-sample bounds: the leading column slots' bounds held in the LDS the
  // image leaves free, so the rest stay in L2 (config 2 shape: one slot of
  // four).  The early-stop kernel does so for the projection with the plan's
  // coefficients where four column slots' bounds would crowd the L2 (up to
  // three row slots), in the room where it would otherwise keep K y of its
  // first row slots, and in two-plane tiles (the rule of k_resident_early).
  size_t lds_all = lds;
  const bool early_lb = !qp && !ps && (BT == 8 || (p->res_mc == 4 && p->res_mr <= 3));
  if (!o.shared_bounds && (!early || early_lb)) {
    if (early && BT != 8)
      lds_all -= (size_t)res_early_kyl(p->res_mr, p->res_mc) * kResThreads * 16;
    const size_t slot_lds = (size_t)2 * kResThreads * BT * sizeof(T);
    const size_t room = (size_t)160 * 1024 - lds_all;
    R.lb_slots = (int)std::min<size_t>((size_t)p->res_mc, room / slot_lds);
    lds_all += (size_t)R.lb_slots * slot_lds;
  }
  if (int rc = launch_resident<T>(R, st, tiles, lds_all, p->res_mr, p->res_mc,
                                  o.shared_bounds != 0, early, BT,
                                  qp ? (ps->RVs ? 1 : 3) : (ps ? 2 : 0)))
    return rc;
  PURIN_HIP(hipGetLastError());
  if (o.timing) {
    PURIN_HIP(hipEventRecord(e1, st));
    PURIN_HIP(hipEventSynchronize(e1));
    float ms = 0;
    PURIN_HIP(hipEventElapsedTime(&ms, e0, e1));
    purin_cp_timing t{};
    t.iterations = o.max_iterations;
    t.loop_ms = ms;
    t.resident = 1;
    record_timing(p, t);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
  }
  return PURIN_CP_OK;
}

// The CP loop on prepared internal arrays plus the final diagnostics.
template <typename T>
int run_iterations(purin_cp_plan* p, hipStream_t st, int64_t batch, const Layout& L, char* sv,
                   char* ws, const purin_cp_solve_options& o, T tol_scalar, const T* tolv,
                   const PerSample<T>* ps = nullptr, const QPRun<T>* qp = nullptr,
                   bool noalloc = false) {
  const int64_t Bp = L.Bp;
  constexpr int64_t TS = tile_samples<T>();
  Iter<T> A{};
  A.K = kept_matrix<T>(p, true);
  A.Bp = Bp;
  A.tgt = (const T*)(sv + L.Tt);
  A.Y = (T*)(sv + L.Y);
  A.YB = (T*)(ws + L.YB);
  A.D = (T*)(sv + L.D);
  A.R = (const T*)(sv + L.R);
  A.LO = (const T*)(sv + L.LO);
  A.HI = (const T*)(sv + L.HI);
  A.shared_bounds = o.shared_bounds;
  A.colpart = (T*)(ws + L.colpart);
  A.rowpart = (T*)(ws + L.rowpart);
  A.ncb = L.ncb;
  A.nrb = L.nrb;
  if (ps) {  // per-sample coefficients: per-sample matrix entries and steps
    if (ps->RVs) {  // the plan's own coefficients: one shared copy
      A.K.rval = ps->RVs;
      A.K.cval = ps->CVs;
    } else {
      A.K.rvb = ps->RV;
      A.K.cvb = ps->CV;
      A.K.vbp = Bp;
    }
    if (p->diag) {
      A.sig_rb = ps->sig_rb;
      A.a_cb = ps->a_cb;
      A.d_cb = ps->d_cb;
      A.tau_cb = ps->tau_cb;
    } else {
      A.sig_b = ps->sig_b;
      A.a_b = ps->a_b;
      A.d_b = ps->d_b;
      A.tau_b = ps->tau_b;
      if (p->opts.accelerated) A.th_b = ps->th_b;
    }
    tolv = ps->tol_b;
    if (qp) {  // general q, c: the column pass forms the prox from tau and q
      A.Q = qp->Q;
      A.Cc = qp->Cc;
      A.tgt = nullptr;
      A.factored = A.nofreeze = A.nostat = qp->dense;
    }
  } else if (p->diag) {  // diagonal steps (non-accelerated, so constant over the loop)
    A.sig_r = (const T*)p->diag_sig;
    A.a_c = (const T*)p->diag_a;
    A.d_c = (const T*)p->diag_d;
  }
  int32_t* done = (int32_t*)(ws + L.done);
  int32_t* count = (int32_t*)(ws + L.count);
  int32_t* ndone = (int32_t*)(ws + L.ndone);
  int32_t* snap = ndone + 1;  // accepted count at the start of the iteration (no freezing)
  const int m = A.K.m, n = A.K.n;
  const bool early = o.early_stop != 0;
  const size_t lds = resident_lds<T>(p, early);
  // the resident kernel takes one schedule of scalar steps for the whole tile,
  // or, for the diagonal QP, per-sample steps it advances itself
  const bool res_qp = qp && !qp->dense && ps && !o.shared_bounds;
  // per-sample coefficients: each tile streams its own
  const bool res_vals = !qp && ps && !ps->RVs;
  if (lds && !o.streaming && !p->diag && ((!ps && !qp) || res_qp || res_vals)) {
    if (int rc = run_resident<T>(p, st, L, sv, ws, o, lds, early, batch, tol_scalar, tolv, done,
                                 count, noalloc, res_qp ? qp : nullptr,
                                 (res_qp || res_vals) ? ps : nullptr))
      return rc;
    if (!early) {
      const int32_t cnt = (int32_t)o.max_iterations;
      k_fill<int32_t><<<(unsigned)((Bp + 255) / 256), 256, 0, st>>>(count, Bp, cnt);
    }
    A.done = nullptr;
    // free after the loop: the final passes leave K~^T d in the ybar buffer and
    // K~y at the kept rows' places of the multiplier buffer
    A.TK = A.YB;
    A.KYo = (T*)(ws + L.DF);
    A.kyrow = p->dkept;
    const dim3 gcolE0 = tile_grid(Bp, TS, L.ncb);
    const dim3 gres0 = tile_grid(Bp, TS, std::max(L.nrb, 1));
    const dim3 gdec0((unsigned)(Bp / 64));  // k_decide: 64 samples per block
    k_col_pass<T, 2, kRowsPerWaveEarly><<<gcolE0, kBlock, 0, st>>>(A);
    if (m) k_res_pass<T, kRowsPerWaveEarly><<<gres0, kBlock, 0, st>>>(A);
    k_decide<T, true><<<gdec0, 64 * kDecideGroups, 0, st>>>(A, batch, tol_scalar, tolv, done, count, ndone,
                                                (const int32_t*)(sv + L.feas), (T*)(ws + L.ores),
                                                (T*)(ws + L.ogap), (int32_t*)(sv + L.conv),
                                                (int32_t*)(ws + L.ofin));
    PURIN_HIP(hipGetLastError());
    return PURIN_CP_OK;
  }
  if (qp) {  // y0 is in Y already (the caller's or zero); ybar0 = y0 (kernels.py:229-231)
    PURIN_HIP(hipMemcpyAsync(A.YB, A.Y, (size_t)n * Bp * sizeof(T), hipMemcpyDeviceToDevice, st));
  } else {  // y0 = ybar0 = target (kernels.py:229-231, bounds.py:59)
    PURIN_HIP(hipMemcpyAsync(A.Y, A.tgt, (size_t)n * Bp * sizeof(T), hipMemcpyDeviceToDevice, st));
    PURIN_HIP(hipMemcpyAsync(A.YB, A.tgt, (size_t)n * Bp * sizeof(T), hipMemcpyDeviceToDevice, st));
  }
  const T* qgam = qp ? qp->gamma : nullptr;
  // per-sample accelerated schedule: two buffers of [5][Bp] (tau, sigma, a,
  // delta, theta); the passes read ``cur`` and the column pass writes the next
  // iteration's values into ``nxt``
  T* cur = nullptr;
  T* nxt = nullptr;
  auto set_steps = [&]() {
    A.tau_b = cur;
    A.sig_b = cur + Bp;
    A.a_b = cur + 2 * Bp;
    A.d_b = cur + 3 * Bp;
    A.th_b = cur + 4 * Bp;
    A.sch_next = nxt;
    A.gam = qgam;
  };
  if (ps && p->opts.accelerated && A.th_b) {
    cur = ps->tau_b;           // [5][Bp] from the steps prepared for iteration 0
    nxt = ps->tau_b + 7 * Bp;  // after tol and L
    set_steps();
  }

  const int check = o.check_every > 0 ? o.check_every : 32;
  const T one = T(1);
  T tau = (T)p->tau0, sigma = (T)p->sigma0, theta = one;
  const dim3 grow = tile_grid(Bp, TS, (m + 3) / 4);
  const dim3 gcol = tile_grid(Bp, TS, (n + 3) / 4);
  const dim3 gcolE = tile_grid(Bp, TS, L.ncb);
  // The fixed-iteration column pass takes a quarter wavefront per column
  // (k_col_pass_q: batch tiles of TS / 4 samples) where the slice of d+ a
  // wide tile gathers exceeds an XCD's L2 and the narrow tile's fits with
  // room for the streams, and the narrow tiles come in multiples of the 8 XCDs
  // (config 3: 10.2 MB -> 2.6 MB per tile).  The plain projection only.  Its
  // streams stay cached (no nontemporal hint): the row pass that follows
  // gathers the y it stores (config 3: column pass 59.2 us with the hint,
  // 51.0 us without; row pass 44.8 -> 42.0 us).
  const bool col_q = !A.Q && !A.sch_next && m > 0 &&
                     (double)m * TS * sizeof(T) > kL2Bytes &&
                     (double)m * (TS / 4) * sizeof(T) <= 0.625 * kL2Bytes &&
                     (Bp / (TS / 4)) % 8 == 0;
  const dim3 gcolq = tile_grid(Bp, TS / 4, (n + 15) / 16);
  const dim3 gres = tile_grid(Bp, TS, std::max(L.nrb, 1));
  const dim3 gdec((unsigned)(Bp / 64));  // k_decide: 64 samples per block
  // With fewer than 16 such blocks the per-sample stop test folds its chunk
  // partials in two passes: (Bp / 64) x kDecideSplit blocks each fold every
  // kDecideSplit-th chunk, then the decision folds those partials (config 3,
  // B = 256: 4 blocks folding 1250 column chunks each otherwise)
  const bool dec_split = Bp / 64 < 16;
  const dim3 gdecp((unsigned)(Bp / 64), (unsigned)kDecideSplit);
  T* const decpart = (T*)(ws + L.decpart);
  auto decide = [&]() {
    if (dec_split) {
      k_decide<T, false, true><<<gdecp, 64 * kDecideGroups, 0, st>>>(
          A, batch, tol_scalar, tolv, done, count, ndone, nullptr, nullptr, nullptr, nullptr,
          nullptr, decpart);
      Iter<T> A2 = A;
      A2.colpart = decpart;
      A2.ncb = kDecideSplit;
      A2.rowpart = decpart + (size_t)5 * kDecideSplit * Bp;
      A2.nrb = kDecideSplit;
      k_decide<T, false><<<gdec, 64 * kDecideGroups, 0, st>>>(A2, batch, tol_scalar, tolv, done,
                                                              count, ndone, nullptr, nullptr,
                                                              nullptr, nullptr, nullptr);
    } else {
      k_decide<T, false><<<gdec, 64 * kDecideGroups, 0, st>>>(A, batch, tol_scalar, tolv, done,
                                                              count, ndone, nullptr, nullptr,
                                                              nullptr, nullptr, nullptr);
    }
  };
  // K ybar by linearity (kernels.hpp, Iter::lin) where it moves fewer bytes:
  // with n > 2m the ybar stream the column pass writes (n per sample) outweighs
  // the two m-vectors of K y the row pass then reads and writes (fixed
  // iterations), and with the stop test the row pass needs no gathers at all
  // (the residual pass computes K y+).  Scalar schedule only (one theta for the
  // batch), not for the dense adapter's unfrozen loop.  The two K y buffers
  // take the ybar buffer's place (n x Bp >= 2 m x Bp).
  const bool lin = m > 0 && (int64_t)n > 2 * (int64_t)m && !A.th_b && !A.nofreeze;
  // The fixed-iteration (wide) column pass streams its per-column vectors past
  // the caches when one iteration's per-sample vectors (y, ybar, and yhat or q
  // and c; d, r) exceed the 256 MB MALL and it stores ybar, so that the
  // gathered rows of d+ stay cached (measured at config 3's shape with ybar
  // streamed: 4.6 % faster).  With K ybar from K y the row pass gathers the y
  // the column pass stores, and caching it wins (config 3, wide tiles: 822 ->
  // 869 projections/s without the hint).
  const bool col_nt = !lin &&
      (double)((A.Q ? 4 : 3) * (int64_t)n + 2 * (int64_t)m) * (double)Bp * sizeof(T) > kMallBytes;
  T* kyb[2] = {A.YB, A.YB + (size_t)m * Bp};
  T theta_prev = T(0);
  // optional event timing: events[3k] before the row pass, [3k+1] between the
  // passes, [3k+2] after the column pass (and the stop test) of iteration k
  const bool timing = o.timing != 0;
  std::vector<hipEvent_t> ev;
  if (timing) {
    ev.resize((size_t)3 * o.max_iterations);
    for (auto& e : ev) PURIN_HIP(hipEventCreate(&e));
  }
  std::vector<hipEvent_t> evd;  // after the column pass when the stop test runs
  if (timing && early) {
    evd.resize((size_t)o.max_iterations);
    for (auto& e : evd) PURIN_HIP(hipEventCreate(&e));
  }
  if (early) {  // the loop reads the device's all-done count every ``check`` iterations
    bool cap = false;
    if (int rc = stream_capturing(st, &cap)) return rc;
    if (cap)
      return set_error(PURIN_CP_ERR_ARG,
                       "early stop on the streaming passes reads a device flag (a stream "
                       "synchronisation): not under stream capture; capture fixed iterations "
                       "(early_stop = 0) or a problem the resident kernel takes");
  }
  HostWords host(p);
  int64_t it = 0;
  for (; it < o.max_iterations; ++it) {
    A.sigma = sigma;
    A.a = one / (one + tau);  // proximal_coefficients with q = 1 (kernels.py:68-73)
    A.delta = tau * A.a;
    A.theta = theta;
    if (timing) PURIN_HIP(hipEventRecord(ev[3 * it], st));
    if (lin) {  // this iteration's K y lands in kyb[it & 1]; kyb[(it + 1) & 1] holds the previous one
      A.lin = 1;
      A.thp = it == 0 ? T(0) : theta_prev;
      A.KYc = kyb[it & 1];
      A.KYp = kyb[(it + 1) & 1];
    }
    if (!early) {
      if (lin) {
        A.KYo = kyb[it & 1];
        k_row_pass<T, false, 1><<<grow, kBlock, 0, st>>>(A);
        A.KYo = nullptr;
      } else if (m) {
        k_row_pass<T, false><<<grow, kBlock, 0, st>>>(A);
      }
      if (timing) PURIN_HIP(hipEventRecord(ev[3 * it + 1], st));
      if (col_q)
        k_col_pass_q<T, false><<<gcolq, kBlock, 0, st>>>(A);
      else if (col_nt)
        k_col_pass<T, 0, kRowsPerWaveFixed, true><<<gcol, kBlock, 0, st>>>(A);
      else
        k_col_pass<T, 0, kRowsPerWaveFixed><<<gcol, kBlock, 0, st>>>(A);
    } else if (A.nofreeze) {
      // every sample iterates until the last is accepted; the kernels return
      // at once from the iteration after that (the host reads the count lazily)
      A.done = done;
      A.stop = snap;
      A.nstop = batch;
      k_snap<<<1, 64, 0, st>>>(ndone, snap);
      if (m) k_row_pass<T, false><<<grow, kBlock, 0, st>>>(A);
      if (timing) PURIN_HIP(hipEventRecord(ev[3 * it + 1], st));
      k_col_pass<T, 1, kRowsPerWaveEarly><<<gcolE, kBlock, 0, st>>>(A);
      if (timing) PURIN_HIP(hipEventRecord(evd[it], st));
      if (m) k_res_pass<T, kRowsPerWaveEarly><<<gres, kBlock, 0, st>>>(A);
      decide();
    } else {
      A.done = done;
      if (lin && it == 0) {  // K y0 (= K ybar0) by one gather of y0
        A.KYo = kyb[0];
        k_row_pass<T, true, 1><<<grow, kBlock, 0, st>>>(A);
        A.KYo = nullptr;
      } else if (lin) {  // K y from the previous residual pass: no gathers
        k_row_pass<T, true, 2><<<grow, kBlock, 0, st>>>(A);
      } else if (m) {
        k_row_pass<T, true><<<grow, kBlock, 0, st>>>(A);
      }
      if (timing) PURIN_HIP(hipEventRecord(ev[3 * it + 1], st));
      k_col_pass<T, 1, kRowsPerWaveEarly><<<gcolE, kBlock, 0, st>>>(A);
      if (timing) PURIN_HIP(hipEventRecord(evd[it], st));
      if (lin) A.KYo = kyb[(it + 1) & 1];  // K y+ for the next iteration's row pass
      if (m) k_res_pass<T, kRowsPerWaveEarly><<<gres, kBlock, 0, st>>>(A);
      A.KYo = nullptr;
      decide();
    }
    if (timing) PURIN_HIP(hipEventRecord(ev[3 * it + 2], st));
    theta_prev = theta;  // the theta of this iteration's ybar update
    if (p->opts.accelerated && A.th_b) {
      // the same update, per sample: the column pass wrote the next steps into
      // the other buffer; swap (kernels.py:279-283)
      std::swap(cur, nxt);
      set_steps();
    } else if (p->opts.accelerated) {  // kernels.py:279-283 with gamma = min q = 1
      const T nt = one / std::sqrt(one + tau);
      tau = nt * tau;
      sigma = sigma / nt;
      theta = nt;
    }
    if (early && ((it + 1) % check == 0)) {
      PURIN_HIP(hipMemcpyAsync(host.get(), ndone, sizeof(int32_t), hipMemcpyDeviceToHost, st));
      PURIN_HIP(hipStreamSynchronize(st));
      if (host.get()[0] >= batch) {
        ++it;
        break;
      }
    }
  }
  if (timing) {
    PURIN_HIP(hipStreamSynchronize(st));
    purin_cp_timing t{};
    t.iterations = it;
    for (int64_t k = 0; k < it; ++k) {
      float a = 0, b = 0, c = 0;
      PURIN_HIP(hipEventElapsedTime(&a, ev[3 * k], ev[3 * k + 1]));
      if (early) {
        PURIN_HIP(hipEventElapsedTime(&b, ev[3 * k + 1], evd[k]));
        PURIN_HIP(hipEventElapsedTime(&c, evd[k], ev[3 * k + 2]));
      } else {
        PURIN_HIP(hipEventElapsedTime(&b, ev[3 * k + 1], ev[3 * k + 2]));
      }
      t.row_ms += a;
      t.col_ms += b;
      t.diag_ms += c;
    }
    float total = 0;
    if (it > 0) PURIN_HIP(hipEventElapsedTime(&total, ev[0], ev[3 * (it - 1) + 2]));
    t.loop_ms = total;
    t.linear_kybar = lin ? 1 : 0;
    t.narrow_columns = col_q && !early ? 1 : 0;
    record_timing(p, t);
    for (auto& e : ev) (void)hipEventDestroy(e);
    for (auto& e : evd) (void)hipEventDestroy(e);
  }
  PURIN_HIP(hipGetLastError());
  if (!early) {
    const int32_t cnt = (int32_t)o.max_iterations;
    k_fill<int32_t><<<(unsigned)((Bp + 255) / 256), 256, 0, st>>>(count, Bp, cnt);
  }
  // final diagnostics on the returned state (kernels.py:291-305); the ybar /
  // K y buffers are free now: the final passes leave K~^T d there and K~y at
  // the kept rows' places of the multiplier buffer
  A.done = nullptr;
  A.stop = nullptr;
  A.TK = A.YB;
  A.KYo = (T*)(ws + L.DF);
  A.kyrow = p->dkept;
  k_col_pass<T, 2, kRowsPerWaveEarly><<<gcolE, kBlock, 0, st>>>(A);
  if (m) k_res_pass<T, kRowsPerWaveEarly><<<gres, kBlock, 0, st>>>(A);
  k_decide<T, true><<<gdec, 64 * kDecideGroups, 0, st>>>(A, batch, tol_scalar, tolv, done, count, ndone,
                                             (const int32_t*)(sv + L.feas), (T*)(ws + L.ores),
                                             (T*)(ws + L.ogap), (int32_t*)(sv + L.conv),
                                             (int32_t*)(ws + L.ofin));
  PURIN_HIP(hipGetLastError());
  return PURIN_CP_OK;
}

template <typename T>
static int check_layout_args(purin_cp_plan* p, int64_t batch) {
  if (!p) return set_error(PURIN_CP_ERR_ARG, "NULL plan");
  if ((p->dtype == PURIN_CP_F64) != (sizeof(T) == 8))
    return set_error(PURIN_CP_ERR_ARG, "dtype mismatch");
  if (batch < 1) return set_error(PURIN_CP_ERR_ARG, "batch_size and variable_size must be positive");
  return PURIN_CP_OK;
}

// Scratch of the no-allocation projection entry (purin_cp_project_noalloc):
// the plan workspace (and the saved state when the caller passes none) of one
// call, in a static device array that every GPU the library runs on holds
// until the process ends.  Host code never uses the array's name as an
// address: scratch_init_device() looks up each device's own copy once (with
// that device current) and keeps the pointer per device.
constexpr size_t kScratchBytes = (size_t)PURIN_CP_NOALLOC_SCRATCH_BYTES;
constexpr int kScratchDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kScratchDevices] = {};

int scratch_init_device(int device) {
  if (device < 0 || device >= kScratchDevices)
    return set_error(PURIN_CP_ERR_UNSUPPORTED, "device ordinal beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device]) return PURIN_CP_OK;
  int cur = -1;
  PURIN_HIP(hipGetDevice(&cur));
  if (cur != device) PURIN_HIP(hipSetDevice(device));
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (cur != device) (void)hipSetDevice(cur);
  if (e != hipSuccess) return hip_check(e, "hipGetSymbolAddress(scratch)");
  if (!ptr) return set_error(PURIN_CP_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
  g_scratch_ptr[device] = ptr;
  return PURIN_CP_OK;
}

// A call that would synchronise its stream -- timing (HIP events), or early
// stop on the streaming passes (the all-done flag read every check_every
// iterations) -- is refused on a stream under capture before it enqueues
// anything.  ``streaming_only``: the call cannot take the resident kernel
// (per-sample coefficients, the QP).
template <typename T>
static int check_capture(purin_cp_plan* p, hipStream_t st, const purin_cp_solve_options& o,
                         bool streaming_only) {
  const bool early = o.early_stop != 0;
  const bool resident = !streaming_only && resident_lds<T>(p, early) && !o.streaming && !p->diag;
  if (!o.timing && !(early && !resident)) return PURIN_CP_OK;
  bool cap = false;
  if (int rc = stream_capturing(st, &cap)) return rc;
  if (!cap) return PURIN_CP_OK;
  return set_error(PURIN_CP_ERR_ARG,
                   o.timing ? "timing synchronises the stream: not under stream capture"
                            : "early stop on the streaming passes reads a device flag (a stream "
                              "synchronisation): not under stream capture; capture fixed "
                              "iterations (early_stop = 0) or a problem the resident kernel takes");
}

// This call's buffers: the caller's workspace, the plan workspace (grown
// stream-ordered) or, for the no-allocation entry, the device's scratch array.
template <typename T>
static int prepare_buffers(purin_cp_plan* p, hipStream_t st, int64_t batch, void* saved,
                           Layout* L, char** sv, char** ws, bool values = false, int extras = 0,
                           bool noalloc = false, const purin_cp_solve_options* o = nullptr) {
  *L = make_layout(p, batch, values, extras);
  int err = PURIN_CP_OK;
  const size_t need = L->ws_end + (saved ? 0 : L->saved_end);
  char* base = nullptr;
  if (o && o->workspace) {  // the caller's: nothing is allocated, nothing of the plan's changes
    base = (char*)workspace(p, need, st, &err, false, o->workspace, o->workspace_bytes);
    if (!base) return err;
  } else if (noalloc) {
    int cur = -1;
    PURIN_HIP(hipGetDevice(&cur));
    if (cur != p->device)
      return set_error(PURIN_CP_ERR_ARG, "the plan was created on device " +
                                             std::to_string(p->device) +
                                             ", not the current device " + std::to_string(cur));
    if (need > kScratchBytes)
      return set_error(PURIN_CP_ERR_ARG,
                       "batch too large for the no-allocation entry point: the call needs " +
                           std::to_string(need) + " bytes of scratch, the maximum is " +
                           std::to_string(kScratchBytes));
    {
      std::lock_guard<std::mutex> lock(g_scratch_mu);
      base = (char*)g_scratch_ptr[p->device];
    }
    if (!base) return set_error(PURIN_CP_ERR_HIP, "no scratch address for this device");
  } else {
    base = (char*)workspace(p, need, st, &err);
    if (!base) return err;
  }
  *ws = base;
  *sv = saved ? (char*)saved : base + L->ws_end;
  return PURIN_CP_OK;
}

template <typename T>
static int spmm_impl(purin_cp_plan* p, hipStream_t st, int64_t batch, int transpose, int scaled,
                     const T* x, T* out) {
  int rc = check_layout_args<T>(p, batch);
  if (rc) return rc;
  if (!x || !out) return set_error(PURIN_CP_ERR_ARG, "NULL x/out");
  Layout L;
  char *sv, *ws;
  if ((rc = prepare_buffers<T>(p, st, batch, nullptr, &L, &sv, &ws, false, kLayoutSpmm)))
    return rc;
  const int64_t Bp = L.Bp;
  constexpr int64_t TS = tile_samples<T>();
  Mat<T> K = kept_matrix<T>(p, scaled != 0);
  T* X = (T*)(ws + L.X);
  T* Z = (T*)(ws + L.Z);
  const int64_t cin = transpose ? p->m : p->n, cout = transpose ? p->n : p->m;
  to_minor<T>(st, x, batch, cin, cin, X, Bp, nullptr, 0);
  if (!transpose) {
    if (p->m) k_spmv_rows<T><<<tile_grid(Bp, TS, (p->m + 3) / 4), kBlock, 0, st>>>(K, Bp, X, Z);
  } else {
    if (p->m == 0)
      k_fill<T><<<256, 256, 0, st>>>(Z, (int64_t)p->n * Bp, T(0));
    else
      k_spmv_cols<T><<<tile_grid(Bp, TS, (p->n + 3) / 4), kBlock, 0, st>>>(K, Bp, X, Z);
  }
  to_major<T>(st, Z, Bp, cout, out, batch, cout, nullptr, 0);
  PURIN_HIP(hipGetLastError());
  return PURIN_CP_OK;
}

template <typename T>
static void write_header(hipStream_t st, char* sv, int64_t batch, int64_t Bp, int kind,
                         int shared, const purin_cp_plan* p) {
  k_write_header<T><<<1, 64, 0, st>>>((int64_t*)sv, batch, Bp, kind, shared, p->dtype, p->n, p->m,
                                      p->M);
}

template <typename T>
static int solve_impl(purin_cp_plan* p, hipStream_t st, int64_t batch, const T* rhs,
                      const T* target, const T* dual0, const T* lower, const T* upper,
                      const T* tol, const uint8_t* feasible, const purin_cp_solve_options& o,
                      T* y, T* dual, int32_t* iterations, T* residual, T* gap,
                      uint8_t* converged, void* saved) {
  int rc = check_layout_args<T>(p, batch);
  if (rc) return rc;
  if (!target || !lower || !upper || (p->m && !rhs))
    return set_error(PURIN_CP_ERR_ARG, "NULL input array");
  if (o.max_iterations < 1) return set_error(PURIN_CP_ERR_ARG, "max_iterations must be a positive integer");
  if ((rc = check_capture<T>(p, st, o, false))) return rc;
  Layout L;
  char *sv, *ws;
  if ((rc = prepare_buffers<T>(p, st, batch, saved, &L, &sv, &ws, false, 0, false, &o))) return rc;
  const int64_t Bp = L.Bp, n = p->n, m = p->m;
  write_header<T>(st, sv, batch, Bp, 0, o.shared_bounds, p);
  to_minor<T>(st, target, batch, n, n, (T*)(sv + L.Tt), Bp, nullptr, 0);
  to_minor<T>(st, rhs, batch, m, m, (T*)(sv + L.R), Bp, nullptr, 0);
  if (dual0)
    to_minor<T>(st, dual0, batch, m, m, (T*)(sv + L.D), Bp, nullptr, 0);
  else if (m)
    k_fill<T><<<1024, 256, 0, st>>>((T*)(sv + L.D), m * Bp, T(0));
  if (o.shared_bounds) {
    PURIN_HIP(hipMemcpyAsync(sv + L.LO, lower, n * sizeof(T), hipMemcpyDeviceToDevice, st));
    PURIN_HIP(hipMemcpyAsync(sv + L.HI, upper, n * sizeof(T), hipMemcpyDeviceToDevice, st));
  } else {
    to_minor<T>(st, lower, batch, n, n, (T*)(sv + L.LO), Bp, nullptr, 0);
    to_minor<T>(st, upper, batch, n, n, (T*)(sv + L.HI), Bp, nullptr, 0);
  }
  k_init_flags<T><<<(unsigned)((Bp + 255) / 256), 256, 0, st>>>(
      batch, Bp, (int32_t*)(ws + L.done), (int32_t*)(ws + L.count), (int32_t*)(sv + L.feas),
      feasible, (int32_t*)(ws + L.ndone));
  // per-sample tolerance: pad to Bp in the ores scratch is not needed; the
  // decide kernels index tol[b] only for b < batch.
  if ((rc = run_iterations<T>(p, st, batch, L, sv, ws, o, (T)o.tolerance, tol))) return rc;
  if (y) to_major<T>(st, (const T*)(sv + L.Y), Bp, n, y, batch, n, nullptr, 0);
  if (dual) to_major<T>(st, (const T*)(sv + L.D), Bp, m, dual, batch, m, nullptr, 0);
  k_finish_solve<T><<<(unsigned)((batch + 255) / 256), 256, 0, st>>>(
      batch, (const int32_t*)(ws + L.count), (const T*)(ws + L.ores), (const T*)(ws + L.ogap),
      (const int32_t*)(sv + L.conv), iterations, residual, gap, converged);
  PURIN_HIP(hipGetLastError());
  return PURIN_CP_OK;
}

template <typename T>
static int project_impl(purin_cp_plan* p, hipStream_t st, int64_t batch, const T* target,
                        const T* rhs, const T* mult0, const purin_cp_solve_options& o, T* y,
                        T* mult, T* slacks, int32_t* status, int32_t* iterations, T* residual,
                        uint8_t* finite_out, uint8_t* eligible, void* saved,
                        const T* values = nullptr, bool per_sample = false, bool noalloc = false) {
  int rc = check_layout_args<T>(p, batch);
  if (rc) return rc;
  if (!target || (p->M && !rhs)) return set_error(PURIN_CP_ERR_ARG, "NULL input array");
  if (per_sample && p->nnz_full && !values) return set_error(PURIN_CP_ERR_ARG, "NULL values");
  if (per_sample && o.shared_bounds)
    return set_error(PURIN_CP_ERR_ARG, "shared_bounds needs shared coefficients");
  if (o.max_iterations < 1) return set_error(PURIN_CP_ERR_ARG, "max_iterations must be a positive integer");
  if (!(o.tolerance > 0.0) || !std::isfinite(o.tolerance))
    return set_error(PURIN_CP_ERR_ARG, "tolerance must be positive and finite");
  Layout L;
  char *sv, *ws;
  if (noalloc && o.timing)
    return set_error(PURIN_CP_ERR_ARG, "timing is not available in the no-allocation entry point");
  if (noalloc && p->res_ok && o.max_iterations > p->res_sched_len)
    return set_error(PURIN_CP_ERR_ARG,
                     "max_iterations exceeds the plan's step schedule (" +
                         std::to_string(p->res_sched_len) +
                         " iterations) in the no-allocation entry point");
  if ((rc = check_capture<T>(p, st, o, per_sample))) return rc;
  if ((rc = prepare_buffers<T>(p, st, batch, saved, &L, &sv, &ws, per_sample,
                               mult0 ? kLayoutWarm : 0, noalloc, &o)))
    return rc;
  const int64_t Bp = L.Bp, n = p->n, m = p->m, M = p->M;
  constexpr int64_t TS = tile_samples<T>();
  write_header<T>(st, sv, batch, Bp, per_sample ? 2 : 1, o.shared_bounds, p);
  const T* metric = (const T*)p->metric;
  // diagonal metric: targets scaled by sqrt(D) (metric.py:102-108), tolerance
  // divided and residual multiplied by max(1, sqrt(max D)) (metric.py:161-165)
  double factor = 1.0;
  if (metric)
    for (double s : p->metric_host) factor = std::max(factor, s);
  const double tol_cfg = o.tolerance / factor;
  to_minor<T>(st, target, batch, n, n, (T*)(sv + L.Tt), Bp, metric, metric ? 1 : 0);
  T* RF = (T*)(sv + L.RF);
  to_minor<T>(st, rhs, batch, M, M, RF, Bp, nullptr, 0);
  T* MF = nullptr;
  if (mult0) {
    MF = (T*)(ws + L.MF);
    to_minor<T>(st, mult0, batch, M, M, MF, Bp, nullptr, 0);
  }
  // per-sample coefficients: scales, scaled entries, steps and tolerances
  // tol * min(1, min_i scale_i) for every sample (bounds.py:192-236)
  PerSample<T> PS{};
  if (per_sample &&
      (rc = prepare_values<T>(p, st, batch, L, ws, values, (T)tol_cfg, kProjectForward, nullptr,
                              nullptr, &PS)))
    return rc;
  const PerSample<T>* ps = per_sample ? &PS : nullptr;
  if (m)
    k_prep_rows<T><<<2048, 256, 0, st>>>((int)m, Bp, p->dkept, (const T*)p->dscale,
                                         ps ? ps->SC : nullptr, RF, MF, (T*)(sv + L.R),
                                         (T*)(sv + L.D));
  k_init_flags<T><<<(unsigned)((Bp + 255) / 256), 256, 0, st>>>(
      batch, Bp, (int32_t*)(ws + L.done), (int32_t*)(ws + L.count), (int32_t*)(sv + L.feas),
      nullptr, (int32_t*)(ws + L.ndone));
  const int64_t cols = o.shared_bounds ? 1 : Bp;
  k_prep_bounds<T><<<2048, 256, 0, st>>>((int)n, Bp, cols, p->bptr, p->brow,
                                         (const T*)p->dbcoef, ps ? ps->BC : nullptr, RF,
                                         (T*)(sv + L.LO),
                                         (T*)(sv + L.HI), (int32_t*)(sv + L.feas), batch);
  // tolerance = tol * min(1, min_i scale_i) (bounds.py:233-236)
  const T tol_cp = (T)tol_cfg * std::min((T)1, (T)p->tol_factor);
  if ((rc = run_iterations<T>(p, st, batch, L, sv, ws, o, tol_cp, nullptr, ps, nullptr, noalloc)))
    return rc;
  // post-processing (bounds.py:247-317)
  Post<T> P{};
  P.K = kept_matrix<T>(p, false);
  if (ps) {
    P.K.rvb = ps->RVo;
    P.K.cvb = ps->CVo;
    P.K.vbp = Bp;
    P.scale_b = ps->SC;
    P.bcoef_b = ps->BC;
  }
  P.Bp = Bp;
  P.me = p->me;
  P.mi = p->mi;
  P.scale = (const T*)p->dscale;
  P.kept = p->dkept;
  P.bptr = p->bptr;
  P.brow = p->brow;
  P.bcoef = (const T*)p->dbcoef;
  P.tgt = (const T*)(sv + L.Tt);
  P.TK = (const T*)(ws + L.YB);  // K~^T d of the final diagnostics pass
  P.KY = true;                   // and its K~y, in DF
  P.Y = (const T*)(sv + L.Y);
  P.D = (const T*)(sv + L.D);
  P.RF = RF;
  P.LO = (const T*)(sv + L.LO);
  P.HI = (const T*)(sv + L.HI);
  P.shared_bounds = o.shared_bounds;
  P.DF = (T*)(ws + L.DF);
  P.SL = (T*)(ws + L.SL);
  P.rowpart = (T*)(ws + L.rowpart);
  P.colpart = (T*)(ws + L.colpart);
  P.nrb = L.nrb;
  P.ncb = L.ncb;
  if (m)
    k_post_rows<T, kRowsPerWaveEarly><<<tile_grid(Bp, TS, L.nrb), kBlock, 0, st>>>(P);
  k_post_cols<T, kRowsPerWaveEarly><<<tile_grid(Bp, TS, L.ncb), kBlock, 0, st>>>(P);
  k_post_final<T><<<(unsigned)(Bp / 64), 64 * kDecideGroups, 0, st>>>(
      P, batch, (T)tol_cfg, (T)factor, (const int32_t*)(sv + L.conv), (const T*)(ws + L.ogap),
      (const int32_t*)(ws + L.count), status, iterations, residual, finite_out, eligible);
  if (y) to_major<T>(st, (const T*)(sv + L.Y), Bp, n, y, batch, n, metric, metric ? 2 : 0);
  if (mult) to_major<T>(st, (const T*)(ws + L.DF), Bp, M, mult, batch, M, nullptr, 0);
  if (slacks) to_major<T>(st, (const T*)(ws + L.SL), Bp, p->mi, slacks, batch, p->mi, nullptr, 0);
  PURIN_HIP(hipGetLastError());
  return PURIN_CP_OK;
}

// General positive diagonal QP (PreparedDiagonalQP.solve, diagonal_qp.py:222-319):
// min 0.5 y'Qy + c'y over the plan's rows (every row kept) and bounds
// lower <= y <= upper, per-sample q, c, values, rhs and bounds.
template <typename T>
static int qp_solve_impl(purin_cp_plan* p, hipStream_t st, int64_t batch, const T* q, const T* c,
                         const T* values, const T* rhs, const T* lower, const T* upper,
                         const T* y0, const T* dual0, const purin_cp_solve_options& o, T* y,
                         T* mult, T* slacks, int32_t* status, int32_t* iterations, T* residual,
                         uint8_t* finite_out, uint8_t* converged_out, void* saved,
                         int dense = 0) {
  int rc = check_layout_args<T>(p, batch);
  if (rc) return rc;
  if (!q || !c || !lower || !upper || (p->M && !rhs))
    return set_error(PURIN_CP_ERR_ARG, "NULL input array");
  if (p->opts.bound_presolve)
    return set_error(PURIN_CP_ERR_ARG,
                     "the diagonal-QP entry needs a plan created with bound_presolve = 0");
  if (dense && (p->opts.row_scaling || p->opts.norm_bound || p->opts.diagonal_preconditioning))
    return set_error(PURIN_CP_ERR_ARG,
                     "the dense adapter needs a plan with row_scaling = 0, norm_bound = 0 and "
                     "diagonal_preconditioning = 0 (dense.py:85-106)");
  if (p->metric)
    return set_error(PURIN_CP_ERR_ARG, "QPData.q already defines the quadratic metric");
  if (o.max_iterations < 1) return set_error(PURIN_CP_ERR_ARG, "max_iterations must be a positive integer");
  if (!(o.tolerance > 0.0) || !std::isfinite(o.tolerance))
    return set_error(PURIN_CP_ERR_ARG, "tolerance must be positive and finite");
  if (o.shared_bounds) return set_error(PURIN_CP_ERR_ARG, "the diagonal QP takes per-sample bounds");
  if ((rc = check_capture<T>(p, st, o, true))) return rc;
  Layout L;
  char *sv, *ws;
  if ((rc = prepare_buffers<T>(p, st, batch, saved, &L, &sv, &ws, true, dual0 ? kLayoutWarm : 0,
                               false, &o)))
    return rc;
  const int64_t Bp = L.Bp, n = p->n, m = p->m, M = p->M;
  constexpr int64_t TS = tile_samples<T>();
  write_header<T>(st, sv, batch, Bp, dense ? 4 : 3, 0, p);
  T* QQ = (T*)(ws + L.QQ);
  T* QC = (T*)(ws + L.QC);
  T* qmax = (T*)(ws + L.QS);
  T* qmin = qmax + Bp;
  T* RF = (T*)(sv + L.RF);
  to_minor<T>(st, q, batch, n, n, QQ, Bp, nullptr, 0);
  to_minor<T>(st, c, batch, n, n, QC, Bp, nullptr, 0);
  to_minor<T>(st, lower, batch, n, n, (T*)(sv + L.LO), Bp, nullptr, 0);
  to_minor<T>(st, upper, batch, n, n, (T*)(sv + L.HI), Bp, nullptr, 0);
  to_minor<T>(st, rhs, batch, M, M, RF, Bp, nullptr, 0);
  if (y0)
    to_minor<T>(st, y0, batch, n, n, (T*)(sv + L.Y), Bp, nullptr, 0);
  else
    k_fill<T><<<1024, 256, 0, st>>>((T*)(sv + L.Y), n * Bp, T(0));
  T* MF = nullptr;
  if (dual0) {
    MF = (T*)(ws + L.MF);
    to_minor<T>(st, dual0, batch, M, M, MF, Bp, nullptr, 0);
  }
  k_init_flags<T><<<(unsigned)((Bp + 255) / 256), 256, 0, st>>>(
      batch, Bp, (int32_t*)(ws + L.done), (int32_t*)(ws + L.count), (int32_t*)(sv + L.feas),
      nullptr, (int32_t*)(ws + L.ndone));
  // valid = all(q > 0) & all(lower <= upper) ANDs into convergence (diagonal_qp.py:120-123)
  k_qp_stats<T><<<(unsigned)(Bp / 64), 1024, 0, st>>>(
      n, Bp, batch, QQ, (const T*)(sv + L.LO), (const T*)(sv + L.HI), qmax, qmin,
      (int32_t*)(sv + L.feas));
  PerSample<T> PS{};
  if ((rc = prepare_values<T>(p, st, batch, L, ws, values, (T)o.tolerance, kQPForward, qmax, qmin,
                              &PS)))
    return rc;
  // scaled rhs and initial dual / scale (diagonal_qp.py:257-273)
  if (m)
    k_prep_rows<T><<<2048, 256, 0, st>>>((int)m, Bp, p->dkept, (const T*)p->dscale, PS.SC, RF, MF,
                                         (T*)(sv + L.R), (T*)(sv + L.D));
  const QPRun<T> qr{QQ, QC, qmin, dense};
  if ((rc = run_iterations<T>(p, st, batch, L, sv, ws, o, (T)o.tolerance, nullptr, &PS, &qr)))
    return rc;
  // original-unit residual, status and slacks (diagonal_qp.py:276-319)
  Post<T> P{};
  P.K = kept_matrix<T>(p, false);
  P.K.rvb = PS.RVo;
  P.K.cvb = PS.CVo;
  P.K.vbp = Bp;
  P.scale_b = PS.SC;
  P.Q = QQ;
  P.Cc = QC;
  P.Bp = Bp;
  P.me = p->me;
  P.mi = p->mi;
  P.scale = (const T*)p->dscale;
  P.kept = p->dkept;
  P.bptr = p->bptr;
  P.brow = p->brow;
  P.bcoef = (const T*)p->dbcoef;
  P.Y = (const T*)(sv + L.Y);
  P.D = (const T*)(sv + L.D);
  P.RF = RF;
  P.LO = (const T*)(sv + L.LO);
  P.HI = (const T*)(sv + L.HI);
  P.DF = (T*)(ws + L.DF);
  P.SL = (T*)(ws + L.SL);
  P.rowpart = (T*)(ws + L.rowpart);
  P.colpart = (T*)(ws + L.colpart);
  P.nrb = L.nrb;
  P.ncb = L.ncb;
  if (m)
    k_post_rows<T, kRowsPerWaveEarly><<<tile_grid(Bp, TS, L.nrb), kBlock, 0, st>>>(P);
  k_post_cols<T, kRowsPerWaveEarly><<<tile_grid(Bp, TS, L.ncb), kBlock, 0, st>>>(P);
  k_post_final<T><<<(unsigned)(Bp / 64), 64 * kDecideGroups, 0, st>>>(
      P, batch, (T)o.tolerance, T(1), (const int32_t*)(sv + L.conv), (const T*)(ws + L.ogap),
      (const int32_t*)(ws + L.count), status, iterations, residual, finite_out, converged_out);
  if (y) to_major<T>(st, (const T*)(sv + L.Y), Bp, n, y, batch, n, nullptr, 0);
  if (mult) to_major<T>(st, (const T*)(ws + L.DF), Bp, M, mult, batch, M, nullptr, 0);
  if (slacks) to_major<T>(st, (const T*)(ws + L.SL), Bp, p->mi, slacks, batch, p->mi, nullptr, 0);
  PURIN_HIP(hipGetLastError());
  return PURIN_CP_OK;
}

}  // namespace purin

using namespace purin;

extern "C" {

int purin_cp_dense_solve(purin_cp_plan* p, void* stream, int64_t batch, const void* q,
                         const void* c, const void* values, const void* rhs, const void* lower,
                         const void* upper, const void* y0, const void* dual0,
                         const purin_cp_solve_options* opts, void* y, void* mult,
                         int32_t* iterations, void* saved) {
  if (!p) return set_error(PURIN_CP_ERR_ARG, "NULL plan");
  purin_cp_solve_options o;
  purin_cp_default_solve_options(&o);
  if (opts) o = *opts;
  hipStream_t st = (hipStream_t)stream;
  if (p->dtype == PURIN_CP_F64)
    return qp_solve_impl<double>(p, st, batch, (const double*)q, (const double*)c,
                                 (const double*)values, (const double*)rhs, (const double*)lower,
                                 (const double*)upper, (const double*)y0, (const double*)dual0, o,
                                 (double*)y, (double*)mult, nullptr, nullptr, iterations, nullptr,
                                 nullptr, nullptr, saved, 1);
  return qp_solve_impl<float>(p, st, batch, (const float*)q, (const float*)c, (const float*)values,
                              (const float*)rhs, (const float*)lower, (const float*)upper,
                              (const float*)y0, (const float*)dual0, o, (float*)y, (float*)mult,
                              nullptr, nullptr, iterations, nullptr, nullptr, nullptr, saved, 1);
}

int purin_cp_qp_solve(purin_cp_plan* p, void* stream, int64_t batch, const void* q, const void* c,
                      const void* values, const void* rhs, const void* lower, const void* upper,
                      const void* y0, const void* dual0, const purin_cp_solve_options* opts,
                      void* y, void* mult, void* slacks, int32_t* status, int32_t* iterations,
                      void* residual, uint8_t* finite_out, uint8_t* converged, void* saved) {
  if (!p) return set_error(PURIN_CP_ERR_ARG, "NULL plan");
  purin_cp_solve_options o;
  purin_cp_default_solve_options(&o);
  if (opts) o = *opts;
  hipStream_t st = (hipStream_t)stream;
  if (p->dtype == PURIN_CP_F64)
    return qp_solve_impl<double>(p, st, batch, (const double*)q, (const double*)c,
                                 (const double*)values, (const double*)rhs, (const double*)lower,
                                 (const double*)upper, (const double*)y0, (const double*)dual0, o,
                                 (double*)y, (double*)mult, (double*)slacks, status, iterations,
                                 (double*)residual, finite_out, converged, saved);
  return qp_solve_impl<float>(p, st, batch, (const float*)q, (const float*)c, (const float*)values,
                              (const float*)rhs, (const float*)lower, (const float*)upper,
                              (const float*)y0, (const float*)dual0, o, (float*)y, (float*)mult,
                              (float*)slacks, status, iterations, (float*)residual, finite_out,
                              converged, saved);
}


int64_t purin_cp_workspace_bytes(const purin_cp_plan* p, int32_t entry, int64_t batch,
                                 const purin_cp_adjoint_options* aopts) {
  if (!p) return set_error(PURIN_CP_ERR_ARG, "NULL plan"), -1;
  if (batch < 1) return set_error(PURIN_CP_ERR_ARG, "batch must be positive"), -1;
  auto forward = [&](bool values, int extras) -> int64_t {
    const Layout L = make_layout(p, batch, values, extras);
    return (int64_t)(L.ws_end + L.saved_end);  // saved == NULL puts the state in the workspace
  };
  switch (entry) {
    case PURIN_CP_ENTRY_SPMM: return forward(false, kLayoutSpmm);
    case PURIN_CP_ENTRY_SOLVE: return forward(false, 0);
    case PURIN_CP_ENTRY_PROJECT: return forward(false, kLayoutWarm);
    case PURIN_CP_ENTRY_PROJECT_VALUES:
    case PURIN_CP_ENTRY_QP_SOLVE:
    case PURIN_CP_ENTRY_DENSE_SOLVE: return forward(true, kLayoutWarm);
    case PURIN_CP_ENTRY_ADJOINT:
    case PURIN_CP_ENTRY_ADJOINT_VALUES:
    case PURIN_CP_ENTRY_QP_ADJOINT:
    case PURIN_CP_ENTRY_DENSE_ADJOINT: {
      purin_cp_adjoint_options o;
      purin_cp_default_adjoint_options(&o);
      if (aopts) o = *aopts;
      int64_t bytes = -1;
      if (adjoint_workspace_bytes(p, entry, batch, o, &bytes) != PURIN_CP_OK) return -1;
      return bytes;
    }
    default:
      return set_error(PURIN_CP_ERR_ARG, "unknown entry point " + std::to_string(entry)), -1;
  }
}

int64_t purin_cp_saved_bytes(const purin_cp_plan* p, int64_t batch) {
  if (!p || batch < 1) return -1;
  return (int64_t)make_layout(p, batch).saved_end;
}

int purin_cp_spmm(purin_cp_plan* p, void* stream, int64_t batch, int32_t transpose,
                  int32_t scaled, const void* x, void* out) {
  if (!p) return set_error(PURIN_CP_ERR_ARG, "NULL plan");
  hipStream_t st = (hipStream_t)stream;
  if (p->dtype == PURIN_CP_F64)
    return spmm_impl<double>(p, st, batch, transpose, scaled, (const double*)x, (double*)out);
  return spmm_impl<float>(p, st, batch, transpose, scaled, (const float*)x, (float*)out);
}

int purin_cp_solve(purin_cp_plan* p, void* stream, int64_t batch, const void* rhs,
                   const void* target, const void* dual0, const void* lower, const void* upper,
                   const void* tol, const uint8_t* feasible, const purin_cp_solve_options* opts,
                   void* y, void* dual, int32_t* iterations, void* residual, void* gap,
                   uint8_t* converged, void* saved) {
  if (!p) return set_error(PURIN_CP_ERR_ARG, "NULL plan");
  purin_cp_solve_options o;
  purin_cp_default_solve_options(&o);
  if (opts) o = *opts;
  hipStream_t st = (hipStream_t)stream;
  if (p->dtype == PURIN_CP_F64)
    return solve_impl<double>(p, st, batch, (const double*)rhs, (const double*)target,
                              (const double*)dual0, (const double*)lower, (const double*)upper,
                              (const double*)tol, feasible, o, (double*)y, (double*)dual,
                              iterations, (double*)residual, (double*)gap, converged, saved);
  return solve_impl<float>(p, st, batch, (const float*)rhs, (const float*)target,
                           (const float*)dual0, (const float*)lower, (const float*)upper,
                           (const float*)tol, feasible, o, (float*)y, (float*)dual, iterations,
                           (float*)residual, (float*)gap, converged, saved);
}

int purin_cp_project(purin_cp_plan* p, void* stream, int64_t batch, const void* target,
                     const void* rhs, const void* mult0, const purin_cp_solve_options* opts,
                     void* y, void* mult, void* slacks, int32_t* status, int32_t* iterations,
                     void* residual, uint8_t* finite_out, uint8_t* eligible, void* saved) {
  if (!p) return set_error(PURIN_CP_ERR_ARG, "NULL plan");
  purin_cp_solve_options o;
  purin_cp_default_solve_options(&o);
  if (opts) o = *opts;
  hipStream_t st = (hipStream_t)stream;
  if (p->dtype == PURIN_CP_F64)
    return project_impl<double>(p, st, batch, (const double*)target, (const double*)rhs,
                                (const double*)mult0, o, (double*)y, (double*)mult,
                                (double*)slacks, status, iterations, (double*)residual,
                                finite_out, eligible, saved);
  return project_impl<float>(p, st, batch, (const float*)target, (const float*)rhs,
                             (const float*)mult0, o, (float*)y, (float*)mult, (float*)slacks,
                             status, iterations, (float*)residual, finite_out, eligible, saved);
}

int purin_cp_project_noalloc(purin_cp_plan* p, void* stream, int64_t batch, const void* target,
                             const void* rhs, const void* mult0,
                             const purin_cp_solve_options* opts, void* y, void* mult,
                             void* slacks, int32_t* status, int32_t* iterations, void* residual,
                             uint8_t* finite_out, uint8_t* eligible, void* saved) {
  if (!p) return set_error(PURIN_CP_ERR_ARG, "NULL plan");
  purin_cp_solve_options o;
  purin_cp_default_solve_options(&o);
  if (opts) o = *opts;
  hipStream_t st = (hipStream_t)stream;
  if (p->dtype == PURIN_CP_F64)
    return project_impl<double>(p, st, batch, (const double*)target, (const double*)rhs,
                                (const double*)mult0, o, (double*)y, (double*)mult,
                                (double*)slacks, status, iterations, (double*)residual,
                                finite_out, eligible, saved, nullptr, false, true);
  return project_impl<float>(p, st, batch, (const float*)target, (const float*)rhs,
                             (const float*)mult0, o, (float*)y, (float*)mult, (float*)slacks,
                             status, iterations, (float*)residual, finite_out, eligible, saved,
                             nullptr, false, true);
}

int purin_cp_project_values(purin_cp_plan* p, void* stream, int64_t batch, const void* values,
                            const void* target, const void* rhs, const void* mult0,
                            const purin_cp_solve_options* opts, void* y, void* mult,
                            void* slacks, int32_t* status, int32_t* iterations, void* residual,
                            uint8_t* finite_out, uint8_t* eligible, void* saved) {
  if (!p) return set_error(PURIN_CP_ERR_ARG, "NULL plan");
  purin_cp_solve_options o;
  purin_cp_default_solve_options(&o);
  if (opts) o = *opts;
  hipStream_t st = (hipStream_t)stream;
  if (p->dtype == PURIN_CP_F64)
    return project_impl<double>(p, st, batch, (const double*)target, (const double*)rhs,
                                (const double*)mult0, o, (double*)y, (double*)mult,
                                (double*)slacks, status, iterations, (double*)residual,
                                finite_out, eligible, saved, (const double*)values, true);
  return project_impl<float>(p, st, batch, (const float*)target, (const float*)rhs,
                             (const float*)mult0, o, (float*)y, (float*)mult, (float*)slacks,
                             status, iterations, (float*)residual, finite_out, eligible, saved,
                             (const float*)values, true);
}

}  // extern "C"
