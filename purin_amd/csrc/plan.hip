// Plan preparation: bound presolve classification, row scaling, step sizes,
// CSR/CSC construction and device upload.
//
// Mirrors the preparation in the reference (paths into SOULS-TAMU/Purin):
//   layout / kept rows          src/purin/solvers/chambolle_pock/solver.py:44-62
//   singleton bound rows        src/purin/solvers/chambolle_pock/bounds.py:320-326
//   row scaling + tolerance     src/purin/solvers/chambolle_pock/bounds.py:210-236
//   norm-bound steps            src/purin/solvers/chambolle_pock/kernels.py:209-227
//   adjoint power iteration     src/purin/solvers/chambolle_pock/bounds.py:83-101,
//                               src/purin/solvers/chambolle_pock/kernels.py:52-65
// With the constraint matrix shared by the batch every one of these is a
// property of the matrix alone, so it is computed once here, on the host, in
// the plan's precision.

#include <algorithm>
#include <functional>
#include <map>
#include <mutex>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "plan.hpp"

namespace purin {

static thread_local std::string g_error;

int set_error(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

int hip_check(hipError_t e, const char* what) {
  (void)hipGetLastError();  // reported here: do not leave it for a later call's launch check
  return set_error(PURIN_CP_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

int raise_lds_cap(const void* kernel, size_t bytes) {
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, size_t> caps;
  int dev = 0;
  PURIN_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  size_t& cap = caps[{dev, kernel}];
  if (bytes <= cap) return PURIN_CP_OK;
  PURIN_HIP(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
  cap = bytes;
  return PURIN_CP_OK;
}

size_t elem_size(const purin_cp_plan* p) { return p->dtype == PURIN_CP_F64 ? 8 : 4; }

int64_t padded_batch(const purin_cp_plan* p, int64_t batch) {
  const int64_t tile = p->dtype == PURIN_CP_F64 ? tile_samples<double>() : tile_samples<float>();
  return round_up(std::max<int64_t>(batch, 1), tile);
}

int stream_capturing(hipStream_t stream, bool* capturing) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  PURIN_HIP(hipStreamIsCapturing(stream, &cs));
  *capturing = cs != hipStreamCaptureStatusNone;
  return PURIN_CP_OK;
}

void record_timing(purin_cp_plan* p, const purin_cp_timing& t) {
  std::lock_guard<std::mutex> lock(p->mu);
  p->timing = t;
}

HostWords::HostWords(purin_cp_plan* p) : p_(p) {
  uint32_t busy = p->pinned ? p->pinned_busy.load() : ~0u;
  while (p->pinned) {
    int s = 0;
    while (s < kPinnedSlots && (busy >> s) & 1u) ++s;
    if (s == kPinnedSlots) break;
    if (p->pinned_busy.compare_exchange_weak(busy, busy | (1u << s))) {
      slot_ = s;
      ptr_ = p->pinned + (size_t)s * (kPinnedBytes / sizeof(int32_t));
      return;
    }
  }
  heap_.assign(kPinnedBytes / sizeof(int64_t), 0);
  ptr_ = reinterpret_cast<int32_t*>(heap_.data());
}

HostWords::~HostWords() {
  if (slot_ >= 0) p_->pinned_busy.fetch_and(~(1u << slot_));
}

void* workspace(purin_cp_plan* p, size_t bytes, hipStream_t stream, int* err, bool adjoint,
                void* caller, int64_t caller_bytes) {
  *err = PURIN_CP_OK;
  if (caller) {
    if (caller_bytes < 0 || (size_t)caller_bytes < bytes) {
      *err = set_error(PURIN_CP_ERR_ARG, "workspace too small: the call needs " +
                                             std::to_string(bytes) + " bytes, " +
                                             std::to_string(caller_bytes) + " given");
      return nullptr;
    }
    if (reinterpret_cast<uintptr_t>(caller) % 256 != 0) {
      *err = set_error(PURIN_CP_ERR_ARG, "workspace must be 256-byte aligned");
      return nullptr;
    }
    return caller;
  }
  void*& buf = adjoint ? p->aws : p->ws;
  size_t& have = adjoint ? p->aws_bytes : p->ws_bytes;
  if (bytes <= have && buf) return buf;
  bool cap = false;
  if ((*err = stream_capturing(stream, &cap))) return nullptr;
  if (cap) {
    *err = set_error(PURIN_CP_ERR_ARG,
                     "the plan's workspace must grow, which allocates: under stream capture "
                     "pass a workspace (purin_cp_workspace_bytes)");
    return nullptr;
  }
  // Stream-ordered growth: the new buffer is usable by work enqueued after it
  // on ``stream``, and the old one is released once the stream's earlier
  // kernels (which may still read it) are done.  No host or device-wide sync.
  bytes = (size_t)round_up((int64_t)bytes, 1 << 20);
  void* nb = nullptr;
  hipError_t e = hipMallocAsync(&nb, bytes, stream);
  if (e != hipSuccess) {
    *err = set_error(PURIN_CP_ERR_NOMEM, std::string("workspace hipMallocAsync: ") + hipGetErrorString(e));
    return nullptr;
  }
  if (buf) {
    e = hipFreeAsync(buf, stream);
    if (e != hipSuccess) {
      (void)hipFreeAsync(nb, stream);
      *err = hip_check(e, "workspace hipFreeAsync");
      return nullptr;
    }
  }
  buf = nb;
  have = bytes;
  return buf;
}

// Per-iteration step scalars (sigma, a, delta, theta) of the shared scalar
// schedule, in the plan's precision: the prox coefficients with q = 1
// (kernels.py:68-73) and, when accelerated, the update of kernels.py:279-283
// with gamma = min q = 1.  The streaming driver (forward.hip, run_iterations)
// performs the same operations in the same order on its host loop variables.
template <typename T>
static std::vector<T> step_schedule(const purin_cp_plan* p, int64_t iters) {
  std::vector<T> h((size_t)4 * iters);
  const T one = T(1);
  T tau = (T)p->tau0, sigma = (T)p->sigma0, theta = one;
  for (int64_t k = 0; k < iters; ++k) {
    const T a = one / (one + tau);
    h[4 * k] = sigma;
    h[4 * k + 1] = a;
    h[4 * k + 2] = tau * a;
    h[4 * k + 3] = theta;
    if (p->opts.accelerated) {
      const T nt = one / std::sqrt(one + tau);
      tau = nt * tau;
      sigma = sigma / nt;
      theta = nt;
    }
  }
  return h;
}

int ensure_schedule(purin_cp_plan* p, int64_t iters, hipStream_t stream, bool at_create,
                    const void** sched) {
  std::lock_guard<std::mutex> lock(p->mu);
  if (p->res_sched && p->res_sched_len >= iters) {
    if (sched) *sched = p->res_sched;
    return PURIN_CP_OK;
  }
  if (!at_create) {
    bool cap = false;
    if (int rc = stream_capturing(stream, &cap)) return rc;
    if (cap)
      return set_error(PURIN_CP_ERR_ARG,
                       "max_iterations exceeds the plan's step schedule (" +
                           std::to_string(p->res_sched_len) +
                           " iterations), whose extension allocates: not under stream capture");
  }
  const int64_t len = std::max(iters, p->res_sched_len * 2);
  const size_t es = elem_size(p);
  const size_t bytes = (size_t)4 * len * es;
  // the host schedule in pinned staging (kept until the plan is destroyed: no
  // host buffer is freed while a copy from it may be pending)
  void* staging = nullptr;
  hipError_t e = hipHostMalloc(&staging, bytes, hipHostMallocDefault);
  if (e != hipSuccess) return set_error(PURIN_CP_ERR_NOMEM, "schedule hipHostMalloc failed");
  p->sched_staging.push_back(staging);
  if (p->dtype == PURIN_CP_F64) {
    auto v = step_schedule<double>(p, len);
    std::memcpy(staging, v.data(), bytes);
  } else {
    auto v = step_schedule<float>(p, len);
    std::memcpy(staging, v.data(), bytes);
  }
  // upload on the plan's own stream and wait for it alone: the buffer is
  // complete before any call, on any stream, can read it
  void* d = nullptr;
  e = hipMallocAsync(&d, bytes, p->upload);
  if (e != hipSuccess) return set_error(PURIN_CP_ERR_NOMEM, "schedule hipMallocAsync failed");
  e = hipMemcpyAsync(d, staging, bytes, hipMemcpyHostToDevice, p->upload);
  if (e == hipSuccess) e = hipStreamSynchronize(p->upload);
  if (e != hipSuccess) {
    (void)hipFreeAsync(d, p->upload);
    return hip_check(e, "schedule upload");
  }
  // kernels enqueued earlier (on any stream) may still read the old schedule
  if (p->res_sched) p->sched_retired.push_back(p->res_sched);
  p->res_sched = d;
  p->res_sched_len = len;
  if (sched) *sched = d;
  return PURIN_CP_OK;
}

// Layout of one wavefront's pass in the resident kernels' matrix stream: slots
// of W[s] entries per lane packed back to back, a chunk being 4 entries.  A
// slot that would start and end inside a chunk it shares with the slot before
// starts on the next chunk instead (the previous slot is padded to the
// boundary), so a chunk holds two slots at most, and the pass's end is padded
// to a whole chunk.  Fills at[s] (the slot's first entry) and from[s] (its
// entries from its first whole chunk on, pads included) when given; returns
// the pass's chunk count.
static int64_t pass_layout(const int32_t* W, int64_t slots, int64_t* at, int32_t* from) {
  int64_t E = 0;
  int32_t prev = 0;  // entries of the previous slot from its first whole chunk
  for (int64_t s = 0; s < slots; ++s) {
    int64_t u = E % 4;
    if (u > 0 && W[s] < 4 - u) {
      prev += (int32_t)(4 - u);
      if (from) from[s - 1] = prev;
      E += 4 - u;
      u = 0;
    }
    const int64_t h = u > 0 ? 4 - u : 0;  // head in the chunk shared with slot s - 1
    prev = (int32_t)(W[s] - h);
    if (from) from[s] = prev;
    if (at) at[s] = E;
    E += W[s];
  }
  if (slots > 0) {
    const int64_t pad = (4 - E % 4) % 4;
    if (from) from[slots - 1] = prev + (int32_t)pad;
    E += pad;
  }
  return E / 4;
}

// splitmix64 start vector in [-1, 1) (the oracle's start_vector restates it).
static double start_value(uint64_t seed, uint64_t j) {
  uint64_t z = (seed << 32) + j + 0x9E3779B97F4A7C15ULL;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  z = z ^ (z >> 31);
  return (double)(z >> 11) * 0x1.0p-53 * 2.0 - 1.0;
}

template <typename T>
struct HostMatrix {
  // kept rows in CSR, values in T
  std::vector<int32_t> ptr, idx;
  std::vector<T> val_s, val_o;
  std::vector<int32_t> cptr, cidx;
  std::vector<T> cval_s, cval_o;
};

// LDS placement of the resident kernels' vectors.  A ds_read_b128 serves a
// wavefront's lanes in four cycle groups of 16 (kCycleLane) and is free of
// bank conflicts when a group's 16-byte entries differ mod 16 (lanes on one
// entry are a broadcast).  Over a slot, a group gathers the entries of its 16
// rows' columns (row pass) or columns' rows (column pass), and reads and
// writes its own 16 entries.  Those sets are the groups here (gptr/gmem:
// distinct entities per group; entities are columns [0, n), the zero entry n,
// rows n + 1 + [0, m)).  The entries of the columns and of the rows are
// permuted among themselves (so every entry class keeps its size and the LDS
// image its length) by a greedy swap search that lowers the number of
// same-class pairs summed over the groups, balancing the classes each group
// gathers; the gathers of a slot are then ordered step by step
// (schedule_group).  ent[e] is entity e's entry.  The search is deterministic
// (fixed seed) and bounded.
static void lds_placement(int64_t n, int64_t m, const std::vector<int32_t>& gptr,
                          const std::vector<int32_t>& gmem, std::vector<int32_t>& ent) {
  const int64_t E = n + 1 + m;
  const int64_t G = (int64_t)gptr.size() - 1;
  ent.resize(E);
  for (int64_t e = 0; e < E; ++e) ent[e] = (int32_t)e;
  if (G <= 0) return;
  std::vector<int32_t> eptr(E + 1, 0), egrp(gmem.size());
  for (int32_t e : gmem) eptr[e + 1]++;
  for (int64_t e = 0; e < E; ++e) eptr[e + 1] += eptr[e];
  {
    std::vector<int32_t> fill(eptr.begin(), eptr.end() - 1);
    for (int64_t g = 0; g < G; ++g)
      for (int32_t k = gptr[g]; k < gptr[g + 1]; ++k) egrp[fill[gmem[k]]++] = (int32_t)g;
  }
  std::vector<uint16_t> cnt((size_t)G * 16, 0);
  for (int64_t g = 0; g < G; ++g)
    for (int32_t k = gptr[g]; k < gptr[g + 1]; ++k) cnt[(size_t)g * 16 + (ent[gmem[k]] & 15)]++;
  auto in_group = [&](int32_t g, int32_t e) {
    for (int32_t k = gptr[g]; k < gptr[g + 1]; ++k)
      if (gmem[k] == e) return true;
    return false;
  };
  auto conflicted = [&](int32_t a) {
    const int ca = ent[a] & 15;
    for (int32_t k = eptr[a]; k < eptr[a + 1]; ++k)
      if (cnt[(size_t)egrp[k] * 16 + ca] > 1) return true;
    return false;
  };
  // change of the pair count when a and b exchange entries
  auto delta = [&](int32_t a, int32_t b) {
    const int ca = ent[a] & 15, cb = ent[b] & 15;
    int d = 0;
    for (int32_t k = eptr[a]; k < eptr[a + 1]; ++k) {
      const int32_t g = egrp[k];
      if (!in_group(g, b)) d += (int)cnt[(size_t)g * 16 + cb] - ((int)cnt[(size_t)g * 16 + ca] - 1);
    }
    for (int32_t k = eptr[b]; k < eptr[b + 1]; ++k) {
      const int32_t g = egrp[k];
      if (!in_group(g, a)) d += (int)cnt[(size_t)g * 16 + ca] - ((int)cnt[(size_t)g * 16 + cb] - 1);
    }
    return d;
  };
  auto swap_entries = [&](int32_t a, int32_t b) {
    const int ca = ent[a] & 15, cb = ent[b] & 15;
    for (int32_t k = eptr[a]; k < eptr[a + 1]; ++k) {
      const int32_t g = egrp[k];
      if (in_group(g, b)) continue;
      cnt[(size_t)g * 16 + ca]--;
      cnt[(size_t)g * 16 + cb]++;
    }
    for (int32_t k = eptr[b]; k < eptr[b + 1]; ++k) {
      const int32_t g = egrp[k];
      if (in_group(g, a)) continue;
      cnt[(size_t)g * 16 + cb]--;
      cnt[(size_t)g * 16 + ca]++;
    }
    std::swap(ent[a], ent[b]);
  };
  uint64_t rng = 0x9E3779B97F4A7C15ull;
  auto next = [&]() {
    rng ^= rng << 13;
    rng ^= rng >> 7;
    rng ^= rng << 17;
    return rng;
  };
  constexpr int kSweeps = 12, kCandidates = 32;
  const int64_t kinds[2][2] = {{0, n}, {n + 1, n + 1 + m}};
  std::vector<int32_t> order;
  for (int sweep = 0; sweep < kSweeps; ++sweep) {
    int64_t swaps = 0;
    for (const auto& kind : kinds) {
      const int64_t lo = kind[0], span = kind[1] - kind[0];
      if (span < 2) continue;
      order.resize(span);
      for (int64_t e = 0; e < span; ++e) order[e] = (int32_t)(lo + e);
      for (int64_t e = span - 1; e > 0; --e) std::swap(order[e], order[next() % (e + 1)]);
      for (int32_t a : order) {
        if (!conflicted(a)) continue;
        int best = 0;
        int32_t pick = -1;
        for (int c = 0; c < kCandidates; ++c) {
          const int32_t b = (int32_t)(lo + (int64_t)(next() % span));
          if ((ent[b] & 15) == (ent[a] & 15)) continue;
          const int d = delta(a, b);
          if (d < best) {
            best = d;
            pick = b;
          }
        }
        if (pick >= 0) {
          swap_entries(a, pick);
          ++swaps;
        }
      }
    }
    if (swaps == 0) break;
  }
}

// The lanes a ds_read_b128 serves together: the wavefront's 64 lanes take four
// cycles of 16, a cycle serving, within one half wavefront, lanes 0-3 and
// 12-15 of one quarter with lanes 4-11 of the other (measured on gfx950:
// 16-byte entries in distinct classes, entry index mod 16, within each of
// these groups read at the full rate whatever the other groups do; a class
// read at k distinct addresses in a group costs about k cycles).
static const int kCycleLane[4][16] = {
    {0, 1, 2, 3, 12, 13, 14, 15, 20, 21, 22, 23, 24, 25, 26, 27},
    {4, 5, 6, 7, 8, 9, 10, 11, 16, 17, 18, 19, 28, 29, 30, 31},
    {32, 33, 34, 35, 44, 45, 46, 47, 52, 53, 54, 55, 56, 57, 58, 59},
    {36, 37, 38, 39, 40, 41, 42, 43, 48, 49, 50, 51, 60, 61, 62, 63}};

// One gathered item of a lane's slot: its entry offset q in the row / column
// (-1: padding, the zero entry), the gathered entity (-1: the zero entry) and
// the entity's LDS entry class (its entry index mod 16).
struct GatherItem {
  int32_t q, e, cls;
};

// Order of one slot's gathers for the 16 lanes of a cycle group (kCycleLane),
// which gather together at each step (entries of one class at distinct
// addresses conflict; equal addresses broadcast).
// Step by step, a maximum matching of lanes to classes (lanes with fewer
// classes left first; classes with more items left tried first) gives each
// matched lane an item of its own class; an unmatched lane takes the item
// that adds the fewest addresses to a class this step.  Writes each lane's W
// items in step order to out[l * W + s] (the item's q).  The sums then run in
// this order instead of the row's / column's index order.
static void schedule_group(std::vector<GatherItem> (&lanes)[16], int W, int32_t* out) {
  for (int s = 0; s < W; ++s) {
    int left[16] = {0};
    for (int l = 0; l < 16; ++l)
      for (const GatherItem& it : lanes[l]) left[it.cls]++;
    int nopt[16], opt[16][16];
    for (int l = 0; l < 16; ++l) {
      bool has[16] = {false};
      for (const GatherItem& it : lanes[l]) has[it.cls] = true;
      nopt[l] = 0;
      for (int c = 0; c < 16; ++c)
        if (has[c]) opt[l][nopt[l]++] = c;
      std::stable_sort(opt[l], opt[l] + nopt[l], [&](int a, int b) { return left[a] > left[b]; });
    }
    int owner[16], lane_cls[16];
    for (int c = 0; c < 16; ++c) owner[c] = -1;
    for (int l = 0; l < 16; ++l) lane_cls[l] = -1;
    // Kuhn's augmenting paths over at most 16 x 16
    std::function<bool(int, bool*)> augment = [&](int l, bool* seen) -> bool {
      for (int k = 0; k < nopt[l]; ++k) {
        const int c = opt[l][k];
        if (seen[c]) continue;
        seen[c] = true;
        if (owner[c] < 0 || augment(owner[c], seen)) {
          owner[c] = l;
          lane_cls[l] = c;
          return true;
        }
      }
      return false;
    };
    int lorder[16];
    for (int l = 0; l < 16; ++l) lorder[l] = l;
    std::stable_sort(lorder, lorder + 16, [&](int a, int b) { return nopt[a] < nopt[b]; });
    for (int k = 0; k < 16; ++k) {
      if (lanes[lorder[k]].empty()) continue;
      bool seen[16] = {false};
      augment(lorder[k], seen);
    }
    for (int c = 0; c < 16; ++c)
      if (owner[c] >= 0) lane_cls[owner[c]] = c;
    // the step's addresses per class so far (entities; -1 the zero entry)
    std::vector<int32_t> picked[16];
    auto add_cost = [&](const GatherItem& it) {
      for (int32_t e : picked[it.cls])
        if (e == it.e) return 0;
      return (int)picked[it.cls].size() + 1;
    };
    auto take = [&](int l, size_t k) {
      const GatherItem it = lanes[l][k];
      lanes[l].erase(lanes[l].begin() + (std::ptrdiff_t)k);
      picked[it.cls].push_back(it.e);
      out[(size_t)l * W + s] = it.q;
    };
    for (int l = 0; l < 16; ++l) {
      if (lane_cls[l] < 0 || lanes[l].empty()) continue;
      for (size_t k = 0; k < lanes[l].size(); ++k)
        if (lanes[l][k].cls == lane_cls[l]) {
          take(l, k);
          break;
        }
    }
    for (int l = 0; l < 16; ++l) {
      if (lane_cls[l] >= 0 || lanes[l].empty()) continue;
      size_t best = 0;
      for (size_t k = 1; k < lanes[l].size(); ++k) {
        const int a = add_cost(lanes[l][k]), b = add_cost(lanes[l][best]);
        if (a < b || (a == b && left[lanes[l][k].cls] > left[lanes[l][best].cls])) best = k;
      }
      take(l, best);
    }
  }
}

template <typename T>
static int build(purin_cp_plan* p, const int64_t* indptr, const int32_t* indices,
                 const double* values) {
  const int64_t n = p->n, me = p->me, M = p->M;
  // --- classify rows --------------------------------------------------------
  std::vector<std::vector<std::pair<int64_t, double>>> bounds_of(n);
  for (int64_t r = 0; r < M; ++r) {
    const int64_t len = indptr[r + 1] - indptr[r];
    if (r >= me && len == 1 && p->opts.bound_presolve) {
      const int32_t j = indices[indptr[r]];
      bounds_of[j].push_back({r, values[indptr[r]]});
    } else {
      p->kept.push_back(r);
    }
  }
  p->m = (int64_t)p->kept.size();
  p->bound.clear();
  p->bvar.clear();
  p->bcoef.clear();
  std::vector<int32_t> bptr(n + 1, 0);
  for (int64_t j = 0; j < n; ++j) {
    bptr[j + 1] = bptr[j] + (int32_t)bounds_of[j].size();
    for (auto& rc : bounds_of[j]) {
      p->bound.push_back(rc.first);
      p->bvar.push_back((int32_t)j);
      p->bcoef.push_back(rc.second);
    }
  }
  // --- kept CSR, row scaling (bounds.py:210-214) ------------------------------
  HostMatrix<T> H;
  const int64_t m = p->m;
  H.ptr.assign(m + 1, 0);
  std::vector<T> scale(m, T(1));
  // entry maps into the caller's CSR order, for per-sample coefficients
  std::vector<int32_t> kcsr, kcsc, bpos;
  for (int64_t i = 0; i < m; ++i) {
    const int64_t r = p->kept[i];
    T sq = T(0);
    for (int64_t k = indptr[r]; k < indptr[r + 1]; ++k) {
      const T v = (T)values[k];
      sq = sq + v * v;
      H.idx.push_back(indices[k]);
      H.val_o.push_back(v);
      kcsr.push_back((int32_t)k);
    }
    H.ptr[i + 1] = (int32_t)H.idx.size();
    if (p->opts.row_scaling) {
      const T norm = std::sqrt(sq);
      scale[i] = norm > T(0) ? T(1) / std::max(norm, (T)1e-30) : T(1);
    }
  }
  p->nnz = (int64_t)H.idx.size();
  H.val_s.resize(p->nnz);
  T min_scale = T(1);
  for (int64_t i = 0; i < m; ++i) {
    for (int32_t k = H.ptr[i]; k < H.ptr[i + 1]; ++k) H.val_s[k] = H.val_o[k] * scale[i];
    min_scale = std::min(min_scale, scale[i]);
  }
  p->scale.assign(scale.begin(), scale.end());
  p->tol_factor = (double)std::min(T(1), min_scale);
  // --- CSC, increasing kept-row order per column ------------------------------
  H.cptr.assign(n + 1, 0);
  for (int64_t k = 0; k < p->nnz; ++k) H.cptr[H.idx[k] + 1]++;
  for (int64_t j = 0; j < n; ++j) H.cptr[j + 1] += H.cptr[j];
  H.cidx.resize(p->nnz);
  H.cval_s.resize(p->nnz);
  H.cval_o.resize(p->nnz);
  kcsc.resize(p->nnz);
  {
    std::vector<int32_t> fill(H.cptr.begin(), H.cptr.end() - 1);
    for (int64_t i = 0; i < m; ++i)
      for (int32_t k = H.ptr[i]; k < H.ptr[i + 1]; ++k) {
        const int32_t pos = fill[H.idx[k]]++;
        H.cidx[pos] = (int32_t)i;
        H.cval_s[pos] = H.val_s[k];
        H.cval_o[pos] = H.val_o[k];
        kcsc[pos] = kcsr[k];
      }
  }
  for (int64_t r : p->bound) bpos.push_back((int32_t)indptr[r]);
  p->nnz_full = indptr[M];
  // --- forward steps (kernels.py:209-227, norm_bound) -------------------------
  const T safety = (T)p->opts.safety;
  {
    T rmax = T(0), cmax = T(0);
    for (int64_t i = 0; i < m; ++i) {
      T s = T(0);
      for (int32_t k = H.ptr[i]; k < H.ptr[i + 1]; ++k) s = s + std::fabs(H.val_s[k]);
      rmax = std::max(rmax, s);
    }
    for (int64_t j = 0; j < n; ++j) {
      T s = T(0);
      for (int32_t k = H.cptr[j]; k < H.cptr[j + 1]; ++k) s = s + std::fabs(H.cval_s[k]);
      cmax = std::max(cmax, s);
    }
    T norm = std::sqrt(rmax * cmax);
    if (!p->opts.norm_bound) norm = T(0);  // replaced by the power iteration below
    p->L = (double)norm;
  }
  // --- diagonal steps (kernels.py:76-88), when diagonal_preconditioning and not
  // accelerated (kernels.py:209-210; the adjoint likewise, bounds.py:83-86):
  // tau_j = safety / colsum_j, sigma_i = safety / rowsum_i of |K~| (a zero sum
  // becomes 1, a positive one at least 1e-12); with q = 1 the prox coefficients
  // are a_j = 1/(1 + tau_j), delta_j = tau_j a_j (kernels.py:68-73)
  std::vector<T> dsig, da, dd;
  p->diag = p->opts.diagonal_preconditioning && !p->opts.accelerated;
  if (p->diag) {
    dsig.resize(m);
    da.resize(n);
    dd.resize(n);
    const T tiny = (T)1e-12, one = T(1);
    for (int64_t i = 0; i < m; ++i) {
      T s = T(0);
      for (int32_t k = H.ptr[i]; k < H.ptr[i + 1]; ++k) s = s + std::fabs(H.val_s[k]);
      s = s > T(0) ? std::max(s, tiny) : one;
      dsig[i] = safety / s;
    }
    for (int64_t j = 0; j < n; ++j) {
      T s = T(0);
      for (int32_t k = H.cptr[j]; k < H.cptr[j + 1]; ++k) s = s + std::fabs(H.cval_s[k]);
      s = s > T(0) ? std::max(s, tiny) : one;
      const T tau = safety / s;
      da[j] = one / (one + tau);
      dd[j] = tau * da[j];
    }
  }
  // --- power iteration on K^T K (kernels.py:52-65) ----------------------------
  T Lpi;
  std::vector<T> ps_start;
  {
    std::vector<T> x(n), z(m), w(n);
    const T eps = (T)1e-12;
    for (int64_t j = 0; j < n; ++j) x[j] = (T)start_value((uint64_t)p->opts.norm_seed, j);
    T nx = T(0);
    for (int64_t j = 0; j < n; ++j) nx = nx + x[j] * x[j];
    nx = std::sqrt(nx) + eps;
    for (int64_t j = 0; j < n; ++j) x[j] = x[j] / nx;
    ps_start = x;  // the normalised start vector, shared by every sample
    T eig = T(0);
    for (int it = 0; it < p->opts.norm_iterations; ++it) {
      for (int64_t i = 0; i < m; ++i) {
        T s = T(0);
        for (int32_t k = H.ptr[i]; k < H.ptr[i + 1]; ++k) s = s + H.val_s[k] * x[H.idx[k]];
        z[i] = s;
      }
      for (int64_t j = 0; j < n; ++j) {
        T s = T(0);
        for (int32_t k = H.cptr[j]; k < H.cptr[j + 1]; ++k) s = s + H.cval_s[k] * z[H.cidx[k]];
        w[j] = s;
      }
      eig = T(0);
      T nw = T(0);
      for (int64_t j = 0; j < n; ++j) {
        eig = eig + x[j] * w[j];
        nw = nw + w[j] * w[j];
      }
      nw = std::sqrt(nw) + eps;
      for (int64_t j = 0; j < n; ++j) x[j] = w[j] / nw;
    }
    Lpi = std::sqrt(std::max(eig, T(0))) + eps;
  }
  {
    const T Lf = std::max(p->opts.norm_bound ? (T)p->L : Lpi, (T)1e-12);
    p->L = (double)Lf;
    p->sigma0 = (double)(safety / Lf);
    p->tau0 = (double)(p->opts.accelerated ? safety / Lf : safety / (T(1) + Lf));
    const T La = std::max(Lpi, (T)1e-12);
    p->Ladj = (double)La;
    p->tau_adj = (double)(safety / (T(1) + La));
    p->sigma_adj = (double)(safety / La);
  }
  // --- resident schedule: slots sorted by degree, per-wavefront chunk streams --
  {
    const int64_t NT = kResThreads;
    const int64_t mr = std::max<int64_t>((m + NT - 1) / NT, 1);
    const int64_t mc = std::max<int64_t>((n + NT - 1) / NT, 1);
    // LDS: Gy (n) | zero | Gd (m) | trash, 16 bytes each
    const bool lds_fits = (n + 1 + m + 1) * 16 <= 160 * 1024;
    p->res_ok = mr <= kResMaxSlots && mc <= kResMaxSlots && n >= 1 && lds_fits;
    if (p->res_ok) {
      p->res_mr = (int32_t)mr;
      p->res_mc = (int32_t)mc;
      const uint32_t zero_off = (uint32_t)n * 16u;
      // Rows / columns go to slots k = slot * NT + thread.  Sorted by degree,
      // they form groups of 64 of nearly equal length (one group per slot of
      // one wavefront).  Within each slot the groups are dealt to the
      // wavefronts longest first to the wavefront with the least work so far,
      // which evens out the entries each wavefront walks between barriers.
      // (Dealing all groups widest-first to the least-loaded wavefront and
      // ordering each wavefront's slots for the fewest packed chunks took the
      // config 2 column pass's widest wavefront from 8 to 7 chunks and made no
      // measurable difference, so the simpler dealing stays.)
      auto assign = [&](int64_t K, int64_t count, const std::vector<int32_t>& ptr,
                        std::vector<int32_t>& map) {
        std::vector<int32_t> order(count);
        for (int64_t i = 0; i < count; ++i) order[i] = (int32_t)i;
        std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) {
          return ptr[a + 1] - ptr[a] > ptr[b + 1] - ptr[b];
        });
        const int64_t groups = K / 64;
        std::vector<int32_t> gch(groups, 0);  // entries per lane of each sorted group
        for (int64_t g = 0; g < groups; ++g)
          if (g * 64 < count) gch[g] = ptr[order[g * 64] + 1] - ptr[order[g * 64]];
        std::vector<int64_t> load(16, 0);
        std::vector<int64_t> slice_of(groups);
        for (int64_t slot = 0; slot < groups / 16; ++slot) {
          std::vector<int> gs(16), ws(16);
          for (int i = 0; i < 16; ++i) gs[i] = ws[i] = i;
          std::stable_sort(gs.begin(), gs.end(), [&](int a, int b) {
            return gch[slot * 16 + a] > gch[slot * 16 + b];
          });
          std::stable_sort(ws.begin(), ws.end(), [&](int a, int b) { return load[a] < load[b]; });
          for (int i = 0; i < 16; ++i) {
            slice_of[slot * 16 + gs[i]] = slot * 16 + ws[i];
            load[ws[i]] += gch[slot * 16 + gs[i]];
          }
        }
        map.assign(K, -1);
        for (int64_t k = 0; k < count; ++k) map[slice_of[k / 64] * 64 + k % 64] = order[k];
      };
      std::vector<int32_t> rmap, cmap;
      assign(mr * NT, m, H.ptr, rmap);
      assign(mc * NT, n, H.cptr, cmap);
      // LDS entries: columns in [0, n), the zero entry n, rows in n + 1 + [0, m),
      // placed to spread each cycle group's accesses over the 16 entry classes
      // (lds_placement)
      std::vector<int32_t> ent;
      {
        std::vector<int32_t> gptr(1, 0), gmem;
        auto add_group = [&](const int32_t* mem, size_t count) {
          const size_t at = gmem.size();
          for (size_t k = 0; k < count; ++k) {
            bool seen = false;
            for (size_t q = at; q < gmem.size(); ++q) seen |= gmem[q] == mem[k];
            if (!seen) gmem.push_back(mem[k]);
          }
          if (gmem.size() - at > 1) gptr.push_back((int32_t)gmem.size());
          else gmem.resize(at);  // a single entity cannot conflict
        };
        // slot z of a pass: lanes l own map[z * 64 + l].  A cycle group
        // (kCycleLane) reads its own entries together, and gathers its rows' /
        // columns' entities in an order scheduled after the placement
        // (schedule_group) that spreads each step over the classes as far as
        // the group's class counts allow, so the placement balances the classes
        // of all the entities a group gathers (the zero entry when a lane pads)
        auto slot_groups = [&](const std::vector<int32_t>& map, int64_t z,
                               const std::vector<int32_t>& ptr, const std::vector<int32_t>& idx,
                               int32_t own_base, int32_t gather_base) {
          int32_t width = 0;
          for (int l = 0; l < 64; ++l) {
            const int32_t r = map[z * 64 + l];
            if (r >= 0) width = std::max(width, ptr[r + 1] - ptr[r]);
          }
          std::vector<int32_t> mem;
          for (int g = 0; g < 4; ++g) {
            mem.clear();
            for (int i = 0; i < 16; ++i)
              if (map[z * 64 + kCycleLane[g][i]] >= 0)
                mem.push_back(own_base + map[z * 64 + kCycleLane[g][i]]);
            add_group(mem.data(), mem.size());
            mem.clear();
            for (int i = 0; i < 16; ++i) {
              const int32_t r = map[z * 64 + kCycleLane[g][i]];
              const int32_t d = r >= 0 ? ptr[r + 1] - ptr[r] : 0;
              for (int32_t k = 0; k < d; ++k) mem.push_back(gather_base + idx[ptr[r] + k]);
              if (d < width) mem.push_back((int32_t)n);
            }
            add_group(mem.data(), mem.size());
          }
        };
        for (int64_t z = 0; z < mr * 16; ++z)
          slot_groups(rmap, z, H.ptr, H.idx, (int32_t)(n + 1), 0);
        for (int64_t z = 0; z < mc * 16; ++z)
          slot_groups(cmap, z, H.cptr, H.cidx, 0, (int32_t)(n + 1));
        lds_placement(n, m, gptr, gmem, ent);
      }
      // chunk = 64 lanes x 4 entries: u32 LDS byte addresses, then the coefficients
      const size_t CB = 64 * 16 + 64 * 4 * sizeof(T);
      std::vector<unsigned char> stream;
      // per stream entry, [chunk][lane][4]: the kept CSR entry it takes its
      // coefficient from (row sections), the kept CSC entry | kResSrcCol
      // (column sections), or -1 (padding): the map that lays per-sample
      // coefficients out in stream order
      std::vector<int32_t> srcmap;
      std::vector<int32_t> wtab((size_t)kResWtab * 16, 0);
      int64_t nchunks = 0;
      auto put_chunk = [&](const uint32_t* off, const T* val,
                           const int32_t* src) {  // off, val, src: [64][4]
        srcmap.insert(srcmap.end(), src, src + 64 * 4);
        const size_t at = stream.size();
        stream.resize(at + CB);
        std::memcpy(&stream[at], off, 64 * 16);
        if (sizeof(T) == 8) {  // two blocks of (v0, v1) and (v2, v3) per lane
          T* dst = reinterpret_cast<T*>(&stream[at + 1024]);
          for (int l = 0; l < 64; ++l) {
            dst[2 * l] = val[4 * l];
            dst[2 * l + 1] = val[4 * l + 1];
            dst[128 + 2 * l] = val[4 * l + 2];
            dst[128 + 2 * l + 1] = val[4 * l + 3];
          }
        } else {
          std::memcpy(&stream[at + 1024], val, 64 * 4 * sizeof(T));
        }
        ++nchunks;
      };
      bool too_wide = false;
      // One pass of one wavefront (its row slots or its column slots): the
      // slots' entries packed back to back, slot s taking W_s entries per lane
      // (W_s = the longest row / column of its 64 lanes; shorter ones padded
      // with the zero entry), so a slot may start inside the chunk where the
      // one before it ends.  A chunk is shared by two slots at most: a slot
      // that would start and end inside a shared chunk starts on the next
      // chunk instead (the previous slot is padded to the boundary), and the
      // section's end is padded to a whole chunk.  Writes to width[] each
      // slot's entries from its first whole chunk on (W_s less the head it
      // has in the chunk it shares with the slot before) and returns the
      // section's chunk count.
      auto put_section = [&](const std::vector<int32_t>& map, int64_t slots, int w,
                             const std::vector<int32_t>& ptr, const std::vector<int32_t>& idx,
                             const std::vector<T>& val, int32_t gather_base,
                             int32_t* width) -> int64_t {
        std::vector<int32_t> W(slots, 0);
        for (int64_t s2 = 0; s2 < slots; ++s2)
          for (int l = 0; l < 64; ++l) {
            const int32_t r = map[(s2 * 16 + w) * 64 + l];
            if (r >= 0) W[s2] = std::max(W[s2], ptr[r + 1] - ptr[r]);
          }
        // entry positions: slot s2 starts at at[s2]; pads are zero entries
        std::vector<int64_t> at(slots, 0);
        const int64_t nch = pass_layout(W.data(), slots, at.data(), width);
        const int64_t E = nch * 4;
        if (nch >= (int64_t)1 << 20) {
          too_wide = true;
          return 0;
        }
        std::vector<uint32_t> off((size_t)64 * E, zero_off);
        std::vector<T> v((size_t)64 * E, T(0));
        std::vector<int32_t> src((size_t)64 * E, -1);
        const int32_t colflag = gather_base == 0 ? 0 : kResSrcCol;  // column sections gather rows
        const int32_t zcls = (int32_t)(n & 15);
        for (int64_t s2 = 0; s2 < slots; ++s2) {
          const int32_t Wd = W[s2];
          if (Wd == 0) continue;
          std::vector<int32_t> sched((size_t)16 * Wd);
          for (int g = 0; g < 4; ++g) {
            std::vector<GatherItem> lanes[16];
            for (int l = 0; l < 16; ++l) {
              const int32_t r = map[(s2 * 16 + w) * 64 + kCycleLane[g][l]];
              const int32_t d = r >= 0 ? ptr[r + 1] - ptr[r] : 0;
              for (int32_t k = 0; k < d; ++k) {
                const int32_t e = gather_base + idx[ptr[r] + k];
                lanes[l].push_back({k, e, ent[e] & 15});
              }
              for (int32_t k = d; k < Wd; ++k) lanes[l].push_back({-1, -1, zcls});
            }
            schedule_group(lanes, Wd, sched.data());
            for (int l = 0; l < 16; ++l) {
              const int lane = kCycleLane[g][l];
              const int32_t r = map[(s2 * 16 + w) * 64 + lane];
              for (int32_t st2 = 0; st2 < Wd; ++st2) {
                const int32_t k = sched[(size_t)l * Wd + st2];
                if (k < 0) continue;  // padding: the zero entry, coefficient 0
                off[(size_t)lane * E + at[s2] + st2] =
                    16u * (uint32_t)ent[gather_base + idx[ptr[r] + k]];
                v[(size_t)lane * E + at[s2] + st2] = val[ptr[r] + k];
                src[(size_t)lane * E + at[s2] + st2] = (ptr[r] + k) | colflag;
              }
            }
          }
        }
        uint32_t co[64 * 4];
        T cv[64 * 4];
        int32_t cs[64 * 4];
        for (int64_t ch = 0; ch < nch; ++ch) {
          for (int l = 0; l < 64; ++l)
            for (int u = 0; u < 4; ++u) {
              co[4 * l + u] = off[(size_t)l * E + 4 * ch + u];
              cv[4 * l + u] = v[(size_t)l * E + 4 * ch + u];
              cs[4 * l + u] = src[(size_t)l * E + 4 * ch + u];
            }
          put_chunk(co, cv, cs);
        }
        return nch;
      };
      // per slot: its whole chunks and the entries of the last one, 8 bits each
      auto pack_slots = [&](const int32_t* width, int64_t slots, int32_t& cnt, int32_t& last) {
        uint32_t c = 0, l = 0;
        for (int64_t s2 = 0; s2 < slots; ++s2) {
          const int32_t R = width[s2];
          const int32_t nch = (R + 3) / 4;
          const int32_t e = nch > 0 ? R - 4 * (nch - 1) : 4;
          if (nch > 255) too_wide = true;
          c |= (uint32_t)(nch & 255) << (8 * s2);
          l |= (uint32_t)e << (8 * s2);
        }
        cnt = (int32_t)c;
        last = (int32_t)l;
      };
      int64_t iter_chunks = 0;
      for (int w = 0; w < 16; ++w) {
        const int64_t first = nchunks;
        int32_t* wt = &wtab[(size_t)kResWtab * w];
        int32_t rw[kResMaxSlots] = {0, 0, 0, 0}, cw[kResMaxSlots] = {0, 0, 0, 0};
        const int64_t rch = put_section(rmap, mr, w, H.ptr, H.idx, H.val_s, 0, rw);
        const int64_t cch =
            put_section(cmap, mc, w, H.cptr, H.cidx, H.cval_s, (int32_t)(n + 1), cw);
        pack_slots(rw, mr, wt[1], wt[3]);
        pack_slots(cw, mc, wt[2], wt[4]);
        // the wrap chunk: a copy of the wave's first chunk (or zero padding),
        // prefetched at the end of each iteration for the next one
        if (nchunks > first) {
          const size_t at = stream.size();
          stream.resize(at + CB);
          std::memcpy(&stream[at], &stream[(size_t)first * CB], CB);
          const size_t sat = srcmap.size();
          srcmap.resize(sat + 64 * 4);
          std::copy(srcmap.begin() + (size_t)first * 256, srcmap.begin() + (size_t)first * 256 + 256,
                    srcmap.begin() + sat);
          ++nchunks;
        } else {
          uint32_t off[64 * 4];
          T v[64 * 4];
          int32_t src[64 * 4];
          for (int e = 0; e < 64 * 4; ++e) {
            off[e] = zero_off;
            v[e] = T(0);
            src[e] = -1;
          }
          put_chunk(off, v, src);
        }
        wt[0] = (int32_t)first;
        wt[5] = (int32_t)rch;
        wt[6] = (int32_t)cch;
        // a pass whose first slot spans two chunks has both of them loaded
        // before the barrier that opens it (k_resident)
        wt[7] = (mr > 0 && rw[0] > 4 ? 1 : 0) | (mc > 0 && cw[0] > 4 ? 2 : 0);
        iter_chunks += rch + cch;
      }
      if (too_wide || nchunks >= (int64_t)1 << 30) p->res_ok = false;
      if (p->res_ok) {
        // matrix-stream bytes one workgroup reads per iteration: every
        // wavefront's row and column chunks (the early-stop kernel reads the
        // same, plus one closing row sweep per launch)
        p->res_iter_bytes = iter_chunks * (int64_t)CB;
        p->res_iter_bytes_e = p->res_iter_bytes;
      }
      if (p->res_ok) {
        p->res_stream_bytes = (int64_t)stream.size();
        auto upr = [&](void** dst, const void* src, size_t bytes) -> int {
          if (bytes == 0) bytes = 16;
          hipError_t e = hipMalloc(dst, bytes);
          if (e != hipSuccess) return set_error(PURIN_CP_ERR_NOMEM, "plan hipMalloc failed");
          p->owned.push_back(*dst);
          if (src) {
            e = hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice);
            if (e != hipSuccess) return hip_check(e, "plan upload");
          }
          return PURIN_CP_OK;
        };
        int rc2;
#define UPR(dst, vec) \
  if ((rc2 = upr((void**)&(dst), (vec).empty() ? nullptr : (vec).data(), (vec).size() * sizeof((vec)[0]))) != PURIN_CP_OK) return rc2
        // each slot's own LDS entry: the (slot, thread) maps' entities placed
        std::vector<int32_t> rent(rmap.size()), cent(cmap.size());
        for (size_t k = 0; k < rmap.size(); ++k)
          rent[k] = rmap[k] >= 0 ? ent[n + 1 + rmap[k]] : -1;
        for (size_t k = 0; k < cmap.size(); ++k) cent[k] = cmap[k] >= 0 ? ent[cmap[k]] : -1;
        UPR(p->res_rowmap, rmap);
        UPR(p->res_colmap, cmap);
        UPR(p->res_rowent, rent);
        UPR(p->res_colent, cent);
        UPR(p->res_stream, stream);
        UPR(p->res_srcmap, srcmap);
        UPR(p->res_wtab, wtab);
#undef UPR
      }
    }
  }
  // --- upload -----------------------------------------------------------------
  auto up = [&](void** dst, const void* src, size_t bytes) -> int {
    *dst = nullptr;
    if (bytes == 0) bytes = 16;  // keep valid pointers for empty arrays
    hipError_t e = hipMalloc(dst, bytes);
    if (e != hipSuccess) return set_error(PURIN_CP_ERR_NOMEM, "plan hipMalloc failed");
    p->owned.push_back(*dst);
    if (src) {
      e = hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice);
      if (e != hipSuccess) return hip_check(e, "plan upload");
    }
    return PURIN_CP_OK;
  };
  std::vector<int32_t> kept32(p->kept.begin(), p->kept.end());
  std::vector<int32_t> brow32(p->bound.begin(), p->bound.end());
  std::vector<T> bcoefT(p->bcoef.begin(), p->bcoef.end());
  int rc = PURIN_CP_OK;
#define UP(dst, vec) \
  if ((rc = up((void**)&(dst), (vec).empty() ? nullptr : (vec).data(), (vec).size() * sizeof((vec)[0]))) != PURIN_CP_OK) return rc
  UP(p->rptr, H.ptr);
  UP(p->ridx, H.idx);
  UP(p->rval_s, H.val_s);
  UP(p->rval_o, H.val_o);
  UP(p->cptr, H.cptr);
  UP(p->cidx, H.cidx);
  UP(p->cval_s, H.cval_s);
  UP(p->cval_o, H.cval_o);
  UP(p->dscale, scale);
  if (p->diag) {
    UP(p->diag_sig, dsig);
    UP(p->diag_a, da);
    UP(p->diag_d, dd);
  }
  UP(p->dkept, kept32);
  UP(p->ps_kcsr, kcsr);
  UP(p->ps_kcsc, kcsc);
  UP(p->ps_bpos, bpos);
  UP(p->ps_start, ps_start);
  UP(p->bptr, bptr);
  UP(p->brow, brow32);
  UP(p->dbcoef, bcoefT);
#undef UP
  return PURIN_CP_OK;
}

}  // namespace purin

using namespace purin;

extern "C" {

void purin_cp_default_options(purin_cp_options* o) {
  if (!o) return;
  o->accelerated = 0;
  o->row_scaling = 1;
  o->norm_bound = 1;
  o->norm_iterations = 20;
  o->norm_seed = 42;
  o->diagonal_preconditioning = 0;
  o->safety = 0.95;
  o->bound_presolve = 1;
  o->reserved = 0;
}

void purin_cp_default_solve_options(purin_cp_solve_options* o) {
  if (!o) return;
  o->tolerance = 1e-9;
  o->max_iterations = 10000;
  o->early_stop = 1;
  o->check_every = 32;
  o->shared_bounds = 0;
  o->timing = 0;
  o->streaming = 0;
  o->reserved = 0;
  o->workspace = nullptr;
  o->workspace_bytes = 0;
}

void purin_cp_default_adjoint_options(purin_cp_adjoint_options* o) {
  if (!o) return;
  o->tolerance = 1e-9;
  o->atol = 0.0;
  o->restart = 30;
  o->max_iterations = 100;
  o->adjoint_tolerance = 1e-8;
  o->force_eligible = 0;
  o->reserved = 0;
  o->workspace = nullptr;
  o->workspace_bytes = 0;
  o->arnoldi_iterations = nullptr;
}

const char* purin_cp_last_error(void) { return g_error.c_str(); }

const char* purin_cp_build_info(void) {
  return "purin_cp abi=2 target=gfx950 (CDNA4) kernels=HIP";
}

int purin_cp_plan_create(purin_cp_plan** out, int32_t dtype, int64_t n, int64_t me, int64_t mi,
                         const int64_t* indptr, const int32_t* indices, const double* values,
                         const purin_cp_options* opts) {
  if (!out) return set_error(PURIN_CP_ERR_ARG, "plan pointer is NULL");
  *out = nullptr;
  if (dtype != PURIN_CP_F32 && dtype != PURIN_CP_F64)
    return set_error(PURIN_CP_ERR_ARG, "dtype must be PURIN_CP_F32 or PURIN_CP_F64");
  if (n < 1) return set_error(PURIN_CP_ERR_ARG, "batch_size and variable_size must be positive");
  if (me < 0 || mi < 0) return set_error(PURIN_CP_ERR_ARG, "row counts must be nonnegative");
  if (n > (1LL << 30) || me + mi > (1LL << 30))
    return set_error(PURIN_CP_ERR_ARG, "problem too large for 32-bit indices");
  if (!indptr) return set_error(PURIN_CP_ERR_ARG, "indptr is NULL");
  const int64_t M = me + mi;
  if (indptr[0] != 0) return set_error(PURIN_CP_ERR_ARG, "indptr[0] must be 0");
  for (int64_t r = 0; r < M; ++r) {
    if (indptr[r + 1] < indptr[r]) return set_error(PURIN_CP_ERR_ARG, "indptr must be nondecreasing");
    for (int64_t k = indptr[r]; k < indptr[r + 1]; ++k) {
      if (indices[k] < 0 || indices[k] >= n)
        return set_error(PURIN_CP_ERR_ARG, "column index out of range");
      if (k > indptr[r] && indices[k] <= indices[k - 1])
        return set_error(PURIN_CP_ERR_ARG, "columns must be strictly ascending within a row");
      if (!std::isfinite(values[k])) return set_error(PURIN_CP_ERR_ARG, "non-finite coefficient");
    }
  }
  if (indptr[M] > (1LL << 31) - 1) return set_error(PURIN_CP_ERR_ARG, "too many nonzeros");
  purin_cp_options o;
  purin_cp_default_options(&o);
  if (opts) o = *opts;
  if (!(o.safety > 0.0 && o.safety < 1.0))
    return set_error(PURIN_CP_ERR_ARG, "safety must be between zero and one");
  if (o.norm_iterations < 1) return set_error(PURIN_CP_ERR_ARG, "norm_iterations must be a positive integer");
  auto* p = new purin_cp_plan();
  p->dtype = dtype;
  p->n = n;
  p->me = me;
  p->mi = mi;
  p->M = M;
  p->opts = o;
  {
    hipError_t e = hipGetDevice(&p->device);
    if (e != hipSuccess) {
      delete p;
      return hip_check(e, "hipGetDevice");
    }
  }
  int rc = dtype == PURIN_CP_F64 ? build<double>(p, indptr, indices, values)
                                 : build<float>(p, indptr, indices, values);
  if (rc == PURIN_CP_OK) {
    hipError_t e = hipHostMalloc((void**)&p->pinned, (size_t)kPinnedSlots * kPinnedBytes,
                                 hipHostMallocDefault);
    if (e != hipSuccess) rc = hip_check(e, "hipHostMalloc");
  }
  if (rc == PURIN_CP_OK) {  // default priority, not synchronising with the null stream
    hipError_t e = hipStreamCreateWithFlags(&p->upload, hipStreamNonBlocking);
    if (e != hipSuccess) rc = hip_check(e, "hipStreamCreateWithFlags");
  }
  // the resident kernel's step schedule, for calls of up to kSchedCapacity iterations
  if (rc == PURIN_CP_OK && p->res_ok) rc = ensure_schedule(p, kSchedCapacity, nullptr, true);
  // this device's address of the no-allocation entry's scratch array
  if (rc == PURIN_CP_OK) rc = scratch_init_device(p->device);
  if (rc != PURIN_CP_OK) {
    purin_cp_plan_destroy(p);
    return rc;
  }
  *out = p;
  return PURIN_CP_OK;
}

void purin_cp_plan_destroy(purin_cp_plan* p) {
  if (!p) return;
  (void)hipDeviceSynchronize();
  for (void* ptr : p->owned) (void)hipFree(ptr);
  if (p->metric) (void)hipFree(p->metric);
  // the workspaces (and a grown schedule) are stream-ordered allocations
  if (p->ws) (void)hipFreeAsync(p->ws, nullptr);
  if (p->aws) (void)hipFreeAsync(p->aws, nullptr);
  if (p->res_sched) (void)hipFreeAsync(p->res_sched, nullptr);
  for (void* d : p->sched_retired) (void)hipFreeAsync(d, nullptr);
  (void)hipDeviceSynchronize();
  for (void* h : p->sched_staging) (void)hipHostFree(h);
  if (p->pinned) (void)hipHostFree(p->pinned);
  if (p->upload) (void)hipStreamDestroy(p->upload);
  delete p;
}

int purin_cp_plan_get_info(const purin_cp_plan* p, purin_cp_plan_info* info) {
  if (!p || !info) return set_error(PURIN_CP_ERR_ARG, "NULL argument");
  info->dtype = p->dtype;
  info->n = p->n;
  info->me = p->me;
  info->mi = p->mi;
  info->kept_rows = p->m;
  info->bound_rows = (int64_t)p->bound.size();
  info->nnz_kept = p->nnz;
  info->norm = p->L;
  info->tau0 = p->tau0;
  info->sigma0 = p->sigma0;
  info->adjoint_norm = p->Ladj;
  info->adjoint_tau = p->tau_adj;
  info->adjoint_sigma = p->sigma_adj;
  info->tolerance_factor = p->tol_factor;
  info->resident_stream_bytes = p->res_ok ? p->res_iter_bytes : 0;
  info->resident_stream_bytes_early = p->res_ok ? p->res_iter_bytes_e : 0;
  info->resident_row_slots = p->res_ok ? (int64_t)p->res_mr * kResThreads : 0;
  info->resident_col_slots = p->res_ok ? (int64_t)p->res_mc * kResThreads : 0;
  info->workspace_bytes = (int64_t)p->ws_bytes;
  info->adjoint_workspace_bytes = (int64_t)p->aws_bytes;
  info->resident_tile_samples = p->res_ok ? res_tile_samples(p) : 0;
  return PURIN_CP_OK;
}

int purin_cp_last_timing(const purin_cp_plan* p, purin_cp_timing* t) {
  if (!p || !t) return set_error(PURIN_CP_ERR_ARG, "NULL argument");
  std::lock_guard<std::mutex> lock(const_cast<purin_cp_plan*>(p)->mu);
  *t = p->timing;
  return PURIN_CP_OK;
}

int purin_cp_last_adjoint_stats(const purin_cp_plan* p, purin_cp_adjoint_stats* s) {
  if (!p || !s) return set_error(PURIN_CP_ERR_ARG, "NULL argument");
  std::lock_guard<std::mutex> lock(const_cast<purin_cp_plan*>(p)->mu);
  *s = p->adjoint_stats;
  return PURIN_CP_OK;
}

int purin_cp_last_adjoint_iterations(const purin_cp_plan* p, void* stream, int64_t batch,
                                     int32_t* iterations) {
  if (!p || !iterations) return set_error(PURIN_CP_ERR_ARG, "NULL argument");
  std::lock_guard<std::mutex> lock(const_cast<purin_cp_plan*>(p)->mu);
  if (!p->adj_steps)
    return set_error(PURIN_CP_ERR_ARG,
                     "no GMRES adjoint call on the plan's workspace has run on this plan");
  if (batch != p->adj_steps_batch)
    return set_error(PURIN_CP_ERR_ARG, "batch differs from the last adjoint call's");
  PURIN_HIP(hipMemcpyAsync(iterations, p->adj_steps, (size_t)batch * sizeof(int32_t),
                           hipMemcpyDeviceToDevice, (hipStream_t)stream));
  return PURIN_CP_OK;
}

int purin_cp_plan_kept_rows(const purin_cp_plan* p, int64_t* rows, double* scale) {
  if (!p) return set_error(PURIN_CP_ERR_ARG, "NULL plan");
  for (int64_t i = 0; i < p->m; ++i) {
    if (rows) rows[i] = p->kept[i];
    if (scale) scale[i] = p->scale[i];
  }
  return PURIN_CP_OK;
}

int purin_cp_plan_set_metric(purin_cp_plan* p, const double* sqrt_d) {
  if (!p) return set_error(PURIN_CP_ERR_ARG, "NULL plan");
  if (p->metric) {
    (void)hipDeviceSynchronize();
    (void)hipFree(p->metric);
    p->metric = nullptr;
    p->metric_host.clear();
  }
  if (!sqrt_d) return PURIN_CP_OK;
  for (int64_t j = 0; j < p->n; ++j)
    if (!(sqrt_d[j] > 0.0) || !std::isfinite(sqrt_d[j]))
      return set_error(PURIN_CP_ERR_ARG, "metric_diagonal must be positive and finite");
  p->metric_host.assign(sqrt_d, sqrt_d + p->n);
  const size_t es = elem_size(p);
  std::vector<char> buf(p->n * es);
  for (int64_t j = 0; j < p->n; ++j) {
    if (p->dtype == PURIN_CP_F64)
      reinterpret_cast<double*>(buf.data())[j] = sqrt_d[j];
    else
      reinterpret_cast<float*>(buf.data())[j] = (float)sqrt_d[j];
  }
  PURIN_HIP(hipMalloc(&p->metric, buf.size()));
  PURIN_HIP(hipMemcpy(p->metric, buf.data(), buf.size(), hipMemcpyHostToDevice));
  return PURIN_CP_OK;
}

}  // extern "C"
