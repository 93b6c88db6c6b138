// Plan object behind the opaque purin_cp_plan handle.
#pragma once

#include <atomic>
#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/purin_cp.h"
#include "common.hpp"

// Kernel tiling constants shared by the host drivers and the kernels.
namespace purin {
constexpr int kRowsPerWaveFixed = 1;  // fixed-iteration passes: one row per wave
constexpr int kRowsPerWaveEarly = 8;  // diagnostic passes: 8 rows/columns per wave
constexpr int kSavedHeader = 256;     // bytes of the saved-state header
constexpr int64_t kSavedMagic = 0x5055524e43503031LL;  // "PURNCP01"
constexpr int kResThreads = 1024;   // threads of a resident workgroup
constexpr int kResMaxSlots = 4;     // rows / columns per thread (n, m <= 4096)
constexpr int32_t kResSrcCol = 1 << 30;  // stream-entry map: a column section's (CSC) entry
constexpr double kMallBytes = 256.0 * 1024 * 1024;  // MI355X Infinity Cache (MALL)
constexpr double kL2Bytes = 4.0 * 1024 * 1024;      // L2 of one MI355X XCD
constexpr int kPinnedBytes = 4096;  // host-pinned flag words of one call: counters, per-step counts
constexpr int kPinnedSlots = 16;    // calls that may read device flags at once through pinned memory
// Iterations of the step schedule built with the plan (the schedule of k
// iterations is a prefix of any longer one, so calls up to this count read it
// as it is; longer calls extend it stream-ordered).
constexpr int64_t kSchedCapacity = int64_t(1) << 16;
}  // namespace purin

struct purin_cp_plan {
  int32_t dtype = PURIN_CP_F64;
  int64_t n = 0, me = 0, mi = 0, M = 0;
  purin_cp_options opts{};

  // host-side structure
  std::vector<int64_t> kept;       // kept row -> original row
  std::vector<double> scale;       // per kept row, rounded to dtype
  std::vector<int64_t> bound;      // bound rows (original index), grouped by variable
  std::vector<int32_t> bvar;       // variable of each bound row
  std::vector<double> bcoef;       // coefficient of each bound row
  int64_t m = 0;                   // kept rows
  int64_t nnz = 0;                 // nonzeros of the kept rows
  double L = 0, tau0 = 0, sigma0 = 0;
  double Ladj = 0, tau_adj = 0, sigma_adj = 0;
  double tol_factor = 1;

  // device copies (element type = dtype for the value arrays)
  int32_t* rptr = nullptr;  // CSR of kept rows
  int32_t* ridx = nullptr;
  void* rval_s = nullptr;   // scaled coefficients
  void* rval_o = nullptr;   // original coefficients
  int32_t* cptr = nullptr;  // CSC of kept rows (increasing row per column)
  int32_t* cidx = nullptr;  // kept-row index
  void* cval_s = nullptr;
  void* cval_o = nullptr;
  void* dscale = nullptr;   // m
  int32_t* dkept = nullptr; // m: original row
  int32_t* bptr = nullptr;  // n+1: bound rows per variable
  int32_t* brow = nullptr;  // original row of each bound row
  void* dbcoef = nullptr;   // coefficient of each bound row
  void* metric = nullptr;   // sqrt(D) (n) or nullptr
  // per-sample coefficients: positions in the caller's CSR entry order of
  // each kept CSR entry, each kept CSC entry and each bound row's entry
  int64_t nnz_full = 0;
  int32_t* ps_kcsr = nullptr;
  int32_t* ps_kcsc = nullptr;
  int32_t* ps_bpos = nullptr;
  void* ps_start = nullptr;  // n: normalised power-iteration start vector
  // diagonal preconditioning (non-accelerated): per-row sigma (m), per-column
  // prox coefficients a and delta (n); nullptr when the steps are scalars
  bool diag = false;
  void* diag_sig = nullptr;
  void* diag_a = nullptr;
  void* diag_d = nullptr;
  std::vector<double> metric_host;

  // plan-owned workspace (grown on demand)
  void* ws = nullptr;
  size_t ws_bytes = 0;
  void* aws = nullptr;        // adjoint workspace
  size_t aws_bytes = 0;
  int32_t* pinned = nullptr;  // host-pinned flag words: kPinnedSlots slots of kPinnedBytes
  std::atomic<uint32_t> pinned_busy{0};  // bit s: slot s is held by a call (HostWords)

  // resident (on-chip) iteration schedule: degree-sorted rows/columns, one
  // thread per (slot, row) and (slot, column); built when n and m fit
  // kResMaxSlots * kResThreads and the tile's vectors fit in LDS
  bool res_ok = false;
  int32_t res_mr = 0, res_mc = 0;    // row / column slots per thread (1..kResMaxSlots)
  int32_t* res_rowmap = nullptr;     // Kr = mr * threads: kept row of each slot or -1
  int32_t* res_colmap = nullptr;     // Kc = mc * threads: column of each slot or -1
  int32_t* res_rowent = nullptr;     // Kr: LDS entry (16-byte units) of each row slot's d, or -1
  int32_t* res_colent = nullptr;     // Kc: LDS entry of each column slot's ybar / y, or -1
  unsigned char* res_stream = nullptr;  // per-wavefront chunk streams of the matrix
  int32_t* res_srcmap = nullptr;     // per stream entry: kept CSR / CSC (| kResSrcCol) entry, or -1
  int32_t* res_wtab = nullptr;       // [16][kResWtab] first chunk, slot widths, section chunks, flags
  int64_t res_stream_bytes = 0;
  int64_t res_iter_bytes = 0;        // matrix-stream bytes a workgroup reads per iteration
  int64_t res_iter_bytes_e = 0;      // the same for the early-stop kernel
  void* res_sched = nullptr;         // per-iteration (sigma, a, delta, theta)
  int64_t res_sched_len = 0;         // iterations the schedule holds
  std::vector<void*> sched_staging;  // pinned host copies of grown schedules (freed with the plan)
  std::vector<void*> sched_retired;  // replaced schedules: kernels on other streams may still
                                     // read them, so they are freed with the plan
  hipStream_t upload = nullptr;      // the plan's own stream for schedule uploads
  std::mutex mu;                     // guards the schedule, timing, adjoint stats and steps

  int device = 0;             // the device the plan was created on (its buffers live there)

  std::vector<void*> owned;   // device allocations freed with the plan
  purin_cp_timing timing{};   // last timed call
  purin_cp_adjoint_stats adjoint_stats{};  // last adjoint call
  int32_t* adj_steps = nullptr;  // per-sample Arnoldi steps of the last GMRES adjoint (in aws)
  int64_t adj_steps_batch = 0;
};

namespace purin {
// thread-local error message helpers (plan.hip)
int set_error(int code, const std::string& msg);
int hip_check(hipError_t e, const char* what);
int64_t padded_batch(const purin_cp_plan* p, int64_t batch);
size_t elem_size(const purin_cp_plan* p);
// The plan-owned workspace (adjoint: the adjoint's), grown stream-ordered on
// ``stream``; or the caller's ``caller`` (``caller_bytes``), checked for size and
// alignment.  Calls on the plan's workspace must be ordered; a stream under
// capture cannot grow it.
void* workspace(purin_cp_plan* p, size_t bytes, hipStream_t stream, int* err, bool adjoint = false,
                void* caller = nullptr, int64_t caller_bytes = 0);
// Make the resident step schedule hold at least ``iters`` iterations and return
// the buffer this call reads (*sched): built on the host and uploaded at plan
// creation (at_create), or extended once by a longer call, which uploads the
// new schedule on the plan's own stream and waits for that upload alone.  The
// replaced buffer is kept until the plan is destroyed.  Thread-safe.
int ensure_schedule(purin_cp_plan* p, int64_t iters, hipStream_t stream, bool at_create,
                    const void** sched = nullptr);
// *capturing = whether ``stream`` is under graph capture.
int stream_capturing(hipStream_t stream, bool* capturing);
// Record the timing of a call (purin_cp_last_timing).
void record_timing(purin_cp_plan* p, const purin_cp_timing& t);
// Make ``kernel`` accept ``bytes`` of dynamic LDS on the current device.  The
// cap only ever rises (under a lock), so a concurrent call on another plan or
// thread cannot lower it between another call's raise and its launch.
int raise_lds_cap(const void* kernel, size_t bytes);
// Samples of one resident tile (forward.hip): 16 bytes of samples, or 8 fp32
// samples in two LDS planes where one row and one column slot per thread hold
// the problem.
int res_tile_samples(const purin_cp_plan* p);

// Host-visible words for one call's reads of device flags: a slot of the
// plan's pinned pool, or, when concurrent calls hold every slot, host memory
// of the call's own (the reads are followed by a stream synchronisation, so
// an ordinary host buffer serves, staged by the runtime).
class HostWords {
 public:
  explicit HostWords(purin_cp_plan* p);
  ~HostWords();
  HostWords(const HostWords&) = delete;
  HostWords& operator=(const HostWords&) = delete;
  int32_t* get() { return ptr_; }

 private:
  purin_cp_plan* p_;
  int slot_ = -1;
  std::vector<int64_t> heap_;
  int32_t* ptr_ = nullptr;
};
// The no-allocation entry's scratch (forward.hip): look up this device's copy
// of the static array once, with the device current.
int scratch_init_device(int device);
}  // namespace purin

#define PURIN_HIP(call)                                        \
  do {                                                         \
    hipError_t e_ = (call);                                    \
    if (e_ != hipSuccess) return purin::hip_check(e_, #call);  \
  } while (0)
