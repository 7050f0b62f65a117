// tac_gpu.hip — C ABI and host driver of the gfx950 PQ build path.
//
// Reference interfaces replaced (paths in the reference repository):
//   pq.train     src/index/pq.zig:158-336
//   PQ.encode    src/index/pq.zig:59-76 (batched as src/index/storage.zig:384-401)
//   PQ.decode    src/index/pq.zig:79-88
//   kmeans.fit   src/tac/kmeans.zig:67-365
//   residuals    src/index/storage.zig:255-278,355-376 (storage.build stage 2)
//   doc layouts  src/index/storage.zig:674-686,705-749 and the image CRC-32
//   distance table / refine  src/index/pq.zig:92-123, src/retrieval/refine.zig:83-145
//
// One training call keeps the residuals resident in HBM as a subspace-major
// copy and runs every Lloyd iteration of all subspaces as a fixed sequence of
// kernels on one stream:
//   assign -> tile histogram -> scan -> stable scatter -> serial fold
//   -> (wcss fold) -> empty reseed -> convergence flags
// Subspaces that converged are skipped by every later kernel through a
// per-subspace flag, so the host never waits inside the loop.
#include "../../include/tac_gpu.h"
#include "pq_kernels.hpp"
#include "cand_kernels.hpp"
#include "cell_kernels.hpp"
#include "screen_kernels.hpp"
#include "kmeanspp.hpp"
#include "storage_kernels.hpp"
#include "query_kernels.hpp"
#include "tac_kernels.hpp"
#include "tac_phases.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdarg>
#include <map>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <deque>
#include <condition_variable>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

using namespace tacgpu;

namespace {

thread_local std::string g_last_error;

constexpr uint32_t kMaxDsub = 8;
constexpr uint32_t kMaxKsub = 1024;
constexpr int kMaxDevices = 64;

struct HipFailure {
  hipError_t err;
};

void set_error(const char *what, hipError_t e) {
  g_last_error = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
}

int hip_status(const char *what, hipError_t e) {
  set_error(what, e);
  return e == hipErrorOutOfMemory ? TAC_ERR_OUT_OF_MEMORY : TAC_ERR_HIP;
}

#define HIP_TRY(expr)                                            \
  do {                                                           \
    hipError_t _e = (expr);                                      \
    if (_e != hipSuccess) return hip_status(#expr, _e);          \
  } while (0)

#define LAUNCH_TRY(what)                                         \
  do {                                                           \
    hipError_t _e = hipGetLastError();                           \
    if (_e != hipSuccess) return hip_status(what, _e);           \
  } while (0)

struct Buffer {
  void *ptr = nullptr;
  size_t bytes = 0;
};

struct EventPair {
  hipEvent_t a = nullptr, b = nullptr;
};

struct DeviceState {
  std::mutex mu;
  hipStream_t own_stream = nullptr;
  hipStream_t last_stream = nullptr;
  hipEvent_t last_done = nullptr;
  // training / encode workspace
  Buffer xs, codes, e, hist, counts, start, sorted, flags, scal, trace, io_in, io_out, io_cb,
      io_init, counter, kpp_state, kpp_w, kpp_bsum, kpp_bad, status, io_aux, io_out2, scan_sums,
      io_x1, io_x2, io_x3, crc_tx, fold_pre, fold_chunks, cand_nbr, cand_defer, cand_count, cand_anchor, cand_grid, kpp_src,
      fold_order, cell_par, cell_cids, cell_ccnt, cell_rec, cell_list;
  // token-aware clustering
  Buffer tac_v, tac_idx, tac_offs, tac_G, tac_spreads, tac_w, tac_e, tac_code, tac_sorted,
      tac_tsum, tac_hist, tac_counts, tac_start, tac_C, tac_pre, tac_fch, tac_st, tac_bad,
      tac_done, tac_iters, tac_wcss, tac_prev, tac_empties, tac_assign, tac_probs, tac_tiles,
      tac_chl, tac_cprob, tac_inv, tac_rsum, tac_ranges, tac_h, tac_ktiles, tac_big, tac_ids,
      tac_pcnt, tac_pslots;
  hipEvent_t tac_pre_ev[16] = {};  // chunk arrivals for the early spreads (a ring)
  bool crc_tx_ready = false;
  // training's second stream (two halves of the subspaces) and its events
  hipStream_t aux_stream[1] = {};
  hipEvent_t aux_fork = nullptr, aux_join[1] = {};
  // pinned staging for large uploads from pageable host memory (upload_host)
  static constexpr int kStageThreads = 8, kStageBufs = 2 * kStageThreads;
  void *stage[kStageBufs] = {};
  hipEvent_t stage_ev[kStageBufs] = {};
  bool stage_pending[kStageBufs] = {};
  // measurement
  std::vector<hipEvent_t> events;
  std::vector<hipEvent_t> kevents;  // per-kernel timers
};

DeviceState *g_devices[kMaxDevices] = {};
std::mutex g_devices_mu;
bool g_profile = false;
std::mutex g_profile_mu;
tac_gpu_profile g_prof = {};

int device_count() {
  int c = 0;
  const hipError_t e = hipGetDeviceCount(&c);
  if (e != hipSuccess) {
    set_error("hipGetDeviceCount", e);
    return 0;
  }
  return c;
}

// Current device's state; NO_DEVICE when HIP reports none.
int acquire_device(DeviceState **out, int *dev_out) {
  if (device_count() <= 0) return TAC_ERR_NO_DEVICE;
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return TAC_ERR_NO_DEVICE;
  std::lock_guard<std::mutex> g(g_devices_mu);
  if (!g_devices[dev]) g_devices[dev] = new DeviceState();
  *out = g_devices[dev];
  if (dev_out) *dev_out = dev;
  return TAC_OK;
}

int ensure(DeviceState &ds, Buffer &b, size_t bytes) {
  if (bytes <= b.bytes) return TAC_OK;
  if (b.ptr) {
    if (ds.last_stream) HIP_TRY(hipStreamSynchronize(ds.last_stream));
    HIP_TRY(hipFree(b.ptr));
    b.ptr = nullptr;
    b.bytes = 0;
  }
  size_t want = bytes < 4096 ? 4096 : bytes;
  want = (want + 4095) & ~size_t(4095);
  const hipError_t e = hipMalloc(&b.ptr, want);
  if (e != hipSuccess) {
    b.ptr = nullptr;
    return hip_status("hipMalloc(workspace)", e);
  }
  b.bytes = want;
  return TAC_OK;
}

constexpr size_t kStageChunk = 8u << 20;  // bytes per staged copy
constexpr size_t kStageMin = 32u << 20;   // smaller uploads copy from pageable memory directly

// Host-to-device copy of `bytes` from pageable memory, enqueued on s.  Large
// copies pass through pinned staging buffers that kStageThreads host threads
// fill (two buffers each, used in turn), so the DMA of one chunk overlaps the
// memcpy of the next: about 56 GB/s with eight threads on an MI355X host (49
// with four), against 27 GB/s for a
// hipMemcpyAsync from the same pageable memory.  The source may be reused
// once this returns; a staging buffer is waited on before its next fill.
// With after_chunk, the chunks' copies are enqueued in order, and
// after_chunk(end) runs right after each (end: the bytes enqueued so far),
// from the thread that enqueued it; a non-zero status ends the upload.
int upload_host(DeviceState &ds, void *dst, const void *src, size_t bytes, hipStream_t s,
                const std::function<int(size_t)> *after_chunk = nullptr) {
  if (bytes < kStageMin) {
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
    return after_chunk ? (*after_chunk)(bytes) : TAC_OK;
  }
  constexpr int T = DeviceState::kStageThreads;
  for (int b = 0; b < DeviceState::kStageBufs; ++b) {
    if (!ds.stage[b]) HIP_TRY(hipHostMalloc(&ds.stage[b], kStageChunk, hipHostMallocDefault));
    if (!ds.stage_ev[b]) HIP_TRY(hipEventCreateWithFlags(&ds.stage_ev[b], hipEventDisableTiming));
  }
  const size_t nch = (bytes + kStageChunk - 1) / kStageChunk;
  hipError_t errs[T] = {};
  const char *what[T] = {};
  int cb_status[T] = {};
  std::atomic<size_t> next{0};  // the next chunk to enqueue (ordered mode)
  std::atomic<bool> failed{false};
  auto work = [&](int tid) {
    uint32_t k = 0;
    for (size_t c = (size_t)tid; c < nch; c += T, ++k) {
      const int b = tid + T * (int)(k & 1u);  // only this thread touches buffer b
      hipError_t e;
      if (ds.stage_pending[b] && (e = hipEventSynchronize(ds.stage_ev[b])) != hipSuccess) {
        errs[tid] = e;
        what[tid] = "hipEventSynchronize";
        failed = true;
        return;
      }
      const size_t off = c * kStageChunk, len = std::min(bytes - off, kStageChunk);
      memcpy(ds.stage[b], static_cast<const char *>(src) + off, len);
      if (after_chunk) {
        while (next.load(std::memory_order_acquire) != c) {
          if (failed.load(std::memory_order_acquire)) return;
          std::this_thread::yield();
        }
      }
      if ((e = hipMemcpyAsync(static_cast<char *>(dst) + off, ds.stage[b], len,
                              hipMemcpyHostToDevice, s)) != hipSuccess) {
        errs[tid] = e;
        what[tid] = "hipMemcpyAsync";
        failed = true;
        return;
      }
      if ((e = hipEventRecord(ds.stage_ev[b], s)) != hipSuccess) {
        errs[tid] = e;
        what[tid] = "hipEventRecord";
        failed = true;
        return;
      }
      ds.stage_pending[b] = true;
      if (after_chunk) {
        if ((cb_status[tid] = (*after_chunk)(off + len)) != TAC_OK) {
          failed = true;
          return;
        }
        next.store(c + 1, std::memory_order_release);
      }
    }
  };
  std::thread helpers[T - 1];
  for (int t = 1; t < T; ++t) helpers[t - 1] = std::thread(work, t);
  work(0);
  for (auto &h : helpers) h.join();
  for (int t = 0; t < T; ++t)
    if (errs[t] != hipSuccess) return hip_status(what[t], errs[t]);
  for (int t = 0; t < T; ++t)
    if (cb_status[t] != TAC_OK) return cb_status[t];
  return TAC_OK;
}

// Order this call after the previous one that used the workspace.
// The reference host's vector lane count (tac_gpu_set_lane_count), and the
// value each device's c_vec_lanes last received (0: never written).
std::atomic<uint32_t> g_vec_lanes{16};
std::atomic<uint32_t> g_dev_lanes[kMaxDevices] = {};
const uint32_t kLaneValues[3] = {4, 8, 16};  // copy sources that outlive the copies

// Brings the current device's c_vec_lanes up to the setting, ordered before
// the work the call enqueues on s.  No allocation.
int sync_lanes(hipStream_t s) {
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return TAC_ERR_NO_DEVICE;
  const uint32_t want = g_vec_lanes.load();
  if (g_dev_lanes[dev].load() == want) return TAC_OK;
  const uint32_t *src = want == 4 ? &kLaneValues[0] : want == 8 ? &kLaneValues[1] : &kLaneValues[2];
  HIP_TRY(hipMemcpyToSymbolAsync(HIP_SYMBOL(c_vec_lanes), src, sizeof(uint32_t), 0,
                                 hipMemcpyHostToDevice, s));
  g_dev_lanes[dev].store(want);
  return TAC_OK;
}

int begin_call(DeviceState &ds, hipStream_t s) {
  if (int st = sync_lanes(s)) return st;
  if (!ds.last_done) HIP_TRY(hipEventCreateWithFlags(&ds.last_done, hipEventDisableTiming));
  if (ds.last_stream && ds.last_stream != s) HIP_TRY(hipStreamWaitEvent(s, ds.last_done, 0));
  ds.last_stream = s;
  return TAC_OK;
}

int end_call(DeviceState &ds, hipStream_t s) {
  HIP_TRY(hipEventRecord(ds.last_done, s));
  return TAC_OK;
}

int resolve_stream(DeviceState &ds, void *stream, hipStream_t *out) {
  if (stream) {
    *out = reinterpret_cast<hipStream_t>(stream);
    return TAC_OK;
  }
  // A blocking stream: work on it is ordered with the null stream, so the
  // synchronous tac_gpu_memcpy_* helpers see finished results.
  if (!ds.own_stream) HIP_TRY(hipStreamCreateWithFlags(&ds.own_stream, hipStreamDefault));
  *out = ds.own_stream;
  return TAC_OK;
}

// ---- per-kernel timers (profiling only) ------------------------------------
// While profiling is on, a call installs a KernelClock for its thread; every
// instrumented launch is bracketed by two HIP events on its stream, and the
// call adds the elapsed times to g_kernel_times by kernel name (the name
// rocprofv3 reports, without the namespace) once its stream is synchronised.
struct KernelMark {
  char name[96];
  size_t ev;
};
struct KernelClock {
  DeviceState *ds = nullptr;
  hipStream_t s = nullptr;
  std::vector<KernelMark> marks;
};
thread_local KernelClock *tl_clock = nullptr;
// The stream of the launches being timed when it is not the call's own.
thread_local hipStream_t tl_kt_stream = nullptr;
std::map<std::string, std::pair<double, uint64_t>> g_kernel_times;  // under g_profile_mu

hipEvent_t kevent(DeviceState &ds, size_t idx) {
  while (ds.kevents.size() <= idx) {
    hipEvent_t ev = nullptr;
    if (hipEventCreate(&ev) != hipSuccess) return nullptr;
    ds.kevents.push_back(ev);
  }
  return ds.kevents[idx];
}

// Start of an instrumented launch; the name is printf-formatted.
void kt_begin(const char *fmt, ...) {
  KernelClock *c = tl_clock;
  if (!c) return;
  KernelMark mk;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(mk.name, sizeof mk.name, fmt, ap);
  va_end(ap);
  mk.ev = 2 * c->marks.size();
  hipEvent_t a = kevent(*c->ds, mk.ev);
  if (!a || hipEventRecord(a, tl_kt_stream ? tl_kt_stream : c->s) != hipSuccess) return;
  c->marks.push_back(mk);
}

void kt_end() {
  KernelClock *c = tl_clock;
  if (!c || c->marks.empty()) return;
  hipEvent_t b = kevent(*c->ds, c->marks.back().ev + 1);
  if (!b || hipEventRecord(b, tl_kt_stream ? tl_kt_stream : c->s) != hipSuccess)
    c->marks.pop_back();
}

// Brackets one launch statement (which may hold commas) with the timer.
#define KT(...) kt_begin(__VA_ARGS__)
#define KT_END() kt_end()

template <typename T> constexpr const char *code_name();
template <> constexpr const char *code_name<uint8_t>() { return "unsigned char"; }
template <> constexpr const char *code_name<uint16_t>() { return "unsigned short"; }

// Installs a clock on this thread for one call when profiling is on.
struct ClockScope {
  KernelClock clock;
  bool on;
  ClockScope(DeviceState &ds, hipStream_t s) : on(g_profile && !tl_clock) {
    if (on) {
      clock.ds = &ds;
      clock.s = s;
      tl_clock = &clock;
    }
  }
  ~ClockScope() {
    if (on) tl_clock = nullptr;
  }
  // Adds the call's kernel times; synchronises the stream.
  int collect() {
    if (!on || clock.marks.empty()) return TAC_OK;
    HIP_TRY(hipStreamSynchronize(clock.s));
    std::lock_guard<std::mutex> g(g_profile_mu);
    for (const KernelMark &mk : clock.marks) {
      float ms = 0.0f;
      HIP_TRY(hipEventElapsedTime(&ms, clock.ds->kevents[mk.ev], clock.ds->kevents[mk.ev + 1]));
      auto &t = g_kernel_times[mk.name];
      t.first += ms;
      t.second += 1;
    }
    clock.marks.clear();
    return TAC_OK;
  }
};

int event_at(DeviceState &ds, size_t idx, hipEvent_t *out) {
  while (ds.events.size() <= idx) {
    hipEvent_t ev;
    HIP_TRY(hipEventCreate(&ev));
    ds.events.push_back(ev);
  }
  *out = ds.events[idx];
  return TAC_OK;
}

// Device counter of vectors the pruned search resolved by a full reference
// scan; zeroed per call, added to the profile when measuring.
// Device counters: [0] exact rescans, [1] candidate-path deferrals,
// [2] candidate-path assignments, [3] cell-list encode subspaces,
// [4] screen deferrals, [5] screen searches.
constexpr int kCounters = 6;
int counter_begin(DeviceState &ds, hipStream_t s, unsigned long long **out) {
  int st = ensure(ds, ds.counter, kCounters * sizeof(unsigned long long));
  if (st) return st;
  HIP_TRY(hipMemsetAsync(ds.counter.ptr, 0, kCounters * sizeof(unsigned long long), s));
  *out = reinterpret_cast<unsigned long long *>(ds.counter.ptr);
  return TAC_OK;
}

int counter_collect(DeviceState &ds, hipStream_t s) {
  unsigned long long v[kCounters] = {0, 0, 0, 0, 0, 0};
  HIP_TRY(hipMemcpyAsync(v, ds.counter.ptr, sizeof(v), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  std::lock_guard<std::mutex> g(g_profile_mu);
  g_prof.exact_rescans += v[0];
  g_prof.cand_deferred += v[1];
  g_prof.cand_vectors += v[2];
  g_prof.cell_subspaces += v[3];
  g_prof.screen_deferred += v[4];
  g_prof.screen_vectors += v[5];
  return TAC_OK;
}

// Device word that kernels raise on invalid input (a centroid id or code out
// of range); cleared before the launch, read back after it.
int status_begin(DeviceState &ds, hipStream_t s, uint32_t **out) {
  int st = ensure(ds, ds.status, sizeof(uint32_t));
  if (st) return st;
  HIP_TRY(hipMemsetAsync(ds.status.ptr, 0, sizeof(uint32_t), s));
  *out = reinterpret_cast<uint32_t *>(ds.status.ptr);
  return TAC_OK;
}

int status_collect(DeviceState &ds, hipStream_t s) {
  uint32_t v = 0;
  HIP_TRY(hipMemcpyAsync(&v, ds.status.ptr, sizeof(v), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  if (v) {
    g_last_error = "input holds a centroid id or code out of range";
    return TAC_ERR_INVALID_ARGUMENT;
  }
  return TAC_OK;
}

uint32_t pad_of(uint32_t d) { return d <= 1 ? 1 : d <= 2 ? 2 : d <= 4 ? 4 : 8; }

uint32_t code_bits(uint32_t K) {
  uint32_t b = 0;
  while ((1u << b) < K) ++b;
  return b;
}

// ---- argument validation with the reference's precedence ----------------

// src/index/pq.zig:165-168, plus this build's shape limits.
int validate_pq(uint64_t n, uint32_t dim, uint32_t m, uint32_t ksub) {
  if (m == 0) return TAC_ERR_INVALID_ARGUMENT;
  if (dim == 0) return TAC_ERR_DIM_MISMATCH;
  if (dim % m != 0) return TAC_ERR_DIM_NOT_DIVISIBLE_BY_M;
  if (n == 0) return TAC_ERR_EMPTY_CORPUS;
  if (ksub == 0) return TAC_ERR_KMEANS_BUDGET_TOO_SMALL;
  const uint32_t dsub = dim / m;
  if (dsub > kMaxDsub || ksub > kMaxKsub) return TAC_ERR_UNSUPPORTED;
  if (n > 0xFFFFFFFFull) return TAC_ERR_UNSUPPORTED;
  return TAC_OK;
}

// ---- kernel launchers -------------------------------------------------------

// Raises a kernel's dynamic-LDS limit above the 64 KB default to the largest
// layout it has been launched with (at most kCandLdsMax).
int raise_lds(const void *fn, uint32_t bytes, uint32_t cells) {
  (void)cells;
  if (bytes <= 65536) return TAC_OK;
  if (bytes > kCandLdsMax) return TAC_ERR_UNSUPPORTED;
  static std::mutex mu;
  static std::vector<std::pair<const void *, uint32_t>> raised;
  std::lock_guard<std::mutex> g(mu);
  for (auto &f : raised)
    if (f.first == fn && f.second >= bytes) return TAC_OK;
  const hipError_t err =
      hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (err != hipSuccess) return hip_status("hipFuncSetAttribute(candidate kernel)", err);
  for (auto &f : raised)
    if (f.first == fn) {
      f.second = bytes;
      return TAC_OK;
    }
  raised.push_back({fn, bytes});
  return TAC_OK;
}

// Sort tiles a training candidate block counts (its chunk is whole tiles):
// kCandHistTiles, fewer when the tile histograms would not fit the LDS.
inline uint32_t cand_hist_tiles(uint32_t K, uint32_t DP, uint32_t cells, uint32_t anchor_bytes) {
  uint32_t tiles = kCandHistTiles;
  while (tiles > 1 && cand_lds(K, DP, cells, tiles, anchor_bytes).total > kCandLdsMax) tiles >>= 1;
  return tiles;
}
inline uint32_t nbr_threads(uint32_t K) { return K > 256 ? 256u : (uint32_t)kWave; }
// The full search at sub-dimensions 5-8 takes its first pass on the matrix
// cores (screen_kernels.hpp) up to K = 256: on 1.52M corpus rows at m8 K256
// the Lloyd loop took 15.7 ms against 19.8 with the vector-unit search.
// TAC_GPU_SCREEN=0 keeps the vector-unit search (for the tests that compare
// the two).
inline bool screen_wanted(uint32_t K) {
  const char *v = getenv("TAC_GPU_SCREEN");
  return K <= kScreenMaxK && !(v && v[0] == '0');
}
// The deferred-vector kernels can give each vector four lanes from K = 128
// on, where the blocks of kPruneBlock codewords split evenly over four lanes
// (TAC_GPU_LIST_LANES=1 keeps one lane per vector, for the tests that
// compare the two).  Four lanes serve a subspace with fewer than
// list_split(K) deferred vectors (one lane costs less once the many vectors
// fill the SIMDs: measured 118 against 133 us for 100,000 vectors per
// subspace at K = 256); 0 when they are not used.
inline bool list_lanes4(uint32_t K) {
  const char *v = getenv("TAC_GPU_LIST_LANES");
  const bool one = v != nullptr && v[0] == '1';
  const uint32_t Kp = (K + kPruneBlock - 1) / kPruneBlock * kPruneBlock;
  return !one && K >= 128 && (Kp / kPruneBlock) % 4 == 0;
}
inline uint32_t list_split(uint32_t K) {
  return !list_lanes4(K) ? 0u : K >= 512 ? 0xFFFFFFFFu : 32768u;
}

template <int D>
struct Launch {
  static int transpose(const float *x, float *xs, uint64_t n, uint32_t dim, hipStream_t s) {
    uint32_t rows = 16384 / (dim + 1);
    if (rows > 64) rows = 64;
    if (rows == 0) return TAC_ERR_UNSUPPORTED;
    const size_t lds = (size_t)rows * (dim + 1) * sizeof(float);
    KT("transpose_kernel<%d>", D);
    transpose_kernel<D><<<(unsigned)((n + rows - 1) / rows), kBlock, lds, s>>>(x, xs, n, dim,
                                                                            rows);
    KT_END();
    return TAC_OK;
  }
  static constexpr int VPT = D <= 4 ? 8 : 4;  // vectors per thread in assign / encode

  static void assign(const float *xs, const float *cb, uint16_t *codes, float *e,
                     const uint32_t *done, uint64_t n, uint32_t M, uint32_t K,
                     unsigned long long *rescans, hipStream_t s) {
    dim3 grid((unsigned)((n + kBlock * VPT - 1) / (kBlock * VPT)), M);
    const uint32_t Kp = (K + kPruneBlock - 1) / kPruneBlock * kPruneBlock;
    const size_t lds = (size_t)Kp * (Pad<D>::value + 1) * sizeof(float) + 2 * sizeof(uint32_t);
    KT("assign_kernel<%d, %d>", D, VPT);
    assign_kernel<D, VPT><<<grid, kBlock, lds, s>>>(xs, cb, codes, e, done, n, K, rescans);
    KT_END();
  }
  // The full search with its first pass on the matrix cores (sub-dimensions
  // 5-8, K <= 256; screen_kernels.hpp): one block per sort tile settles the
  // vectors the screen separates and counts them into hist[M][T][K], the
  // others take the pruned exact search of the deferred list.
  static int assign_screen(const float *xs, const float *cb, uint16_t *codes, float *e,
                           uint32_t *defer, uint32_t *defer_count, const uint32_t *done,
                           uint64_t n, uint32_t M, uint32_t K, uint32_t *hist, uint32_t T,
                           unsigned long long *rescans, hipStream_t s) {
    if constexpr (D >= 5 && D <= 8) {
      zero_words_kernel<<<1, kWave, 0, s>>>(defer_count, M);  // a dispatch, also in a graph
      KT("screen_kernel<%d, false, unsigned short>", D);
      screen_kernel<D, false, uint16_t><<<dim3(T, M), 256, 0, s>>>(
          xs, cb, codes, e, defer, defer_count, done, n, 0, M, K, hist, T);
      KT_END();
      assign_deferred(xs, cb, codes, e, defer, defer_count, done, n, M, K, hist, T, rescans,
                      g_profile ? rescans + 4 : nullptr, s);
      return TAC_OK;
    } else {
      return TAC_ERR_INVALID_ARGUMENT;  // no matrix-core screen outside 5-8 sub-dimensions
    }
  }
  // Candidate-set assignment (cand_kernels.hpp): neighbour tables of the
  // current codebooks, the assignment from grid anchors (GRID, the first
  // Lloyd iteration) or from the previous codes, then the pruned full search
  // of the deferred vectors.  Both passes also count the new codes per sort
  // tile into hist[M][T][K] for the update.
  template <bool GRID, typename AnchorT>
  static int assign_cand(const float *xs, const float *cb, uint32_t *nbr, AnchorT *anchors,
                         float *grid, uint16_t *codes, float *e, uint32_t *slice,
                         uint32_t *defer, uint32_t *defer_count, const uint32_t *done,
                         uint64_t n, uint32_t M, uint32_t K, uint32_t L, uint32_t *hist,
                         uint32_t T, unsigned long long *rescans, hipStream_t s) {
    KT("nbr_build_kernel<%d>", D);
    nbr_build_kernel<D><<<dim3(K, M), nbr_threads(K), nbr_lds_bytes(K), s>>>(
        cb, nbr, defer_count, done, K, L);
    KT_END();
    uint32_t G = 0, cells = 0;
    constexpr uint32_t NA = cand_anchors<false>();
    if (GRID) {
      G = cand_grid_side(D);
      cells = 1;
      for (int k = 0; k < D; ++k) cells *= G;
      KT("grid_build_kernel<%d, %uu, %s>", D, NA, code_name<AnchorT>());
      grid_build_kernel<D, NA, AnchorT><<<dim3((cells + kBlock - 1) / kBlock, M), kBlock, 0, s>>>(
          cb, anchors, grid, K, G, cells, nullptr);
      KT_END();
    }
    // About 1,024 blocks over all subspaces; a chunk is whole sort tiles
    // (whole groups of kCandThreads vectors), at most as many as the block's
    // tile histograms can hold in LDS.
    const uint32_t abytes = GRID ? NA * (uint32_t)sizeof(AnchorT) : 0u;
    const uint32_t max_tiles = cand_hist_tiles(K, Pad<D>::value, cells, abytes);
    const uint64_t per_sub = std::max<uint64_t>(1, (1024 + M - 1) / M);
    uint64_t chunk = (n + per_sub - 1) / per_sub;
    chunk = (chunk + kSortTile - 1) / kSortTile * kSortTile;
    chunk = std::min<uint64_t>(chunk, (uint64_t)max_tiles * kSortTile);
    const uint64_t nblk = (n + chunk - 1) / chunk;
    const CandLds lay = cand_lds(K, Pad<D>::value, cells, (uint32_t)(chunk / kSortTile), abytes);
    if (int st = raise_lds((const void *)cand_kernel<D, GRID, false, uint16_t, AnchorT>,
                           lay.total, cells))
      return st;
    KT("cand_kernel<%d, %s, false, unsigned short, %s>", D, GRID ? "true" : "false",
       code_name<AnchorT>());
    cand_kernel<D, GRID, false, uint16_t, AnchorT><<<dim3((unsigned)nblk, M), kCandThreads,
                                                     lay.total, s>>>(
        xs, cb, nbr, anchors, grid, codes, e, nullptr, slice, defer, defer_count, done, n, 0, M, K,
        L, (uint32_t)chunk, (uint32_t)nblk, G, cells, hist, T);
    KT_END();
    assign_deferred(xs, cb, codes, e, defer, defer_count, done, n, M, K, hist, T, rescans,
                    g_profile ? rescans + 1 : nullptr, s);
    return TAC_OK;
  }
  // The pruned exact search of the deferred vectors defer[m][..], which also
  // counts their codes into hist[M][T][K]; stats (profiling): [0] += the
  // deferred vectors, [1] += n per subspace.
  static void assign_deferred(const float *xs, const float *cb, uint16_t *codes, float *e,
                              const uint32_t *defer, const uint32_t *defer_count,
                              const uint32_t *done, uint64_t n, uint32_t M, uint32_t K,
                              uint32_t *hist, uint32_t T, unsigned long long *rescans,
                              unsigned long long *stats, hipStream_t s) {
    const uint32_t Kp = (K + kPruneBlock - 1) / kPruneBlock * kPruneBlock;
    const size_t lds = (size_t)Kp * (Pad<D>::value + 1) * sizeof(float) + 2 * sizeof(uint32_t);
    // About 2% of the vectors are deferred, each a serial chain over all K
    // codewords: four lanes share a vector's search when the blocks of
    // kPruneBlock codewords split evenly over them (list_lanes4), so that
    // four times as many waves hide the chains, else one vector per thread;
    // about 4,096 blocks over all subspaces, looping when there are more.
    const uint32_t split = list_split(K);
    const uint64_t per = split ? kBlock / 4 : kBlock;  // the smaller tiles of the two widths
    const uint64_t g =
        std::max<uint64_t>(1, std::min<uint64_t>((n + per - 1) / per, (4096 + M - 1) / M));
    if (split) {
      KT("assign_list_kernel<%d, 1, 4>", D);
      assign_list_kernel<D, 1, 4><<<dim3((unsigned)g, M), kBlock, lds, s>>>(
          xs, cb, codes, e, defer, defer_count, done, n, K, rescans,
          stats, hist, T, split);
    } else {
      KT("assign_list_kernel<%d, 1, 1>", D);
      assign_list_kernel<D, 1, 1><<<dim3((unsigned)g, M), kBlock, lds, s>>>(
          xs, cb, codes, e, defer, defer_count, done, n, K, rescans,
          stats, hist, T, 0u);
    }
    KT_END();
  }
  // Encode through the matrix-core screen (sub-dimensions 5-8, K <= 256;
  // screen_kernels.hpp), then the deferred rows' pruned exact search with
  // PQ.encode's scan; defer holds M * n words.
  template <typename CodeT>
  static int encode_screen(const float *x, const float *cb, CodeT *codes, uint32_t *defer,
                           uint32_t *defer_count, uint64_t n, uint32_t dim, uint32_t M,
                           uint32_t K, unsigned long long *rescans, unsigned long long *stats,
                           hipStream_t s) {
    if constexpr (D >= 5 && D <= 8) {
      const uint64_t tiles = (n + kSortTile - 1) / kSortTile;
      const uint64_t total = tiles * M;
      if (total > 0xFFFFFFF0ull) return TAC_ERR_UNSUPPORTED;
      zero_words_kernel<<<1, kWave, 0, s>>>(defer_count, M);  // a dispatch, also in a graph
      const uint32_t blocks = (uint32_t)(8 * ((total + 7) / 8));
      KT("screen_kernel<%d, true, %s>", D, code_name<CodeT>());
      screen_kernel<D, true, CodeT><<<blocks, 256, 0, s>>>(x, cb, codes, nullptr, defer,
                                                           defer_count, nullptr, n, dim, M, K,
                                                           nullptr, (uint32_t)tiles);
      KT_END();
      return encode_deferred<CodeT>(x, cb, codes, defer, defer_count, n, dim, M, K, rescans,
                                    stats, s);
    } else {
      return TAC_ERR_INVALID_ARGUMENT;  // no matrix-core screen outside 5-8 sub-dimensions
    }
  }
  // Candidate-set encode: neighbour rows and grid anchors of the codebooks,
  // the candidate pass over token-major input, then the reference scan of
  // the deferred vectors.
  template <typename CodeT>
  static int encode_cand(const float *x, const float *cb, CodeT *codes, uint32_t *nbr,
                         CodeT *anchors, float *grid, uint32_t *slice, uint32_t *defer,
                         uint32_t *defer_count, uint64_t n, uint32_t dim, uint32_t M, uint32_t K,
                         uint32_t L, unsigned long long *rescans, hipStream_t s) {
    encode_tables<CodeT>(cb, nbr, anchors, grid, defer_count, M, K, L, s);
    return encode_rows<CodeT>(x, cb, codes, nbr, anchors, grid, slice, defer, defer_count, n, dim,
                              M, K, L, rescans, g_profile ? rescans + 1 : nullptr, s);
  }
  // The codebooks' neighbour rows and grid anchors (also clears defer_count).
  template <typename AnchorT>
  static void encode_tables(const float *cb, uint32_t *nbr, AnchorT *anchors, float *grid,
                            uint32_t *defer_count, uint32_t M, uint32_t K, uint32_t L,
                            hipStream_t s, const uint32_t *skip = nullptr) {
    const uint32_t G = cand_grid_side(D);
    uint32_t cells = 1;
    for (int k = 0; k < D; ++k) cells *= G;
    KT("nbr_build_kernel<%d>", D);
    nbr_build_kernel<D><<<dim3(K, M), nbr_threads(K), nbr_lds_bytes(K), s>>>(
        cb, nbr, defer_count, skip, K, L);
    KT_END();
    KT("grid_build_kernel<%d, %uu, %s>", D, cand_anchors<true>(), code_name<AnchorT>());
    grid_build_kernel<D, cand_anchors<true>(), AnchorT><<<dim3((cells + kBlock - 1) / kBlock, M),
                                                          kBlock, 0, s>>>(
        cb, anchors, grid, K, G, cells, skip);
    KT_END();
  }
  // The candidate pass over n token-major rows from the tables, then the
  // reference scan of the deferred vectors; defer_count must be zero, and
  // slice / defer hold M * n words each.
  template <typename CodeT>
  static int encode_rows(const float *x, const float *cb, CodeT *codes, const uint32_t *nbr,
                         const CodeT *anchors, const float *grid, uint32_t *slice,
                         uint32_t *defer, uint32_t *defer_count, uint64_t n, uint32_t dim,
                         uint32_t M, uint32_t K, uint32_t L, unsigned long long *rescans,
                         unsigned long long *stats, hipStream_t s,
                         const uint32_t *skip = nullptr, bool deferred_pass = true) {
    const uint32_t G = cand_grid_side(D);
    uint32_t cells = 1;
    for (int k = 0; k < D; ++k) cells *= G;
    const CandLds lay =
        cand_lds(K, Pad<D>::value, cells, 0, cand_anchors<true>() * (uint32_t)sizeof(CodeT));
    if (int st = raise_lds((const void *)cand_kernel<D, true, true, CodeT, CodeT>, lay.total, cells))
      return st;
    // Chunks of 8,192 rows; the M blocks of a chunk run on one XCD, so a row
    // crosses HBM once and its other subspaces come from L2.
    const uint64_t chunk = 8192;
    const uint64_t nchunks = (n + chunk - 1) / chunk;
    const uint64_t total = nchunks * M;
    if (total > 0xFFFFFFF0ull) return TAC_ERR_UNSUPPORTED;
    const uint32_t blocks = (uint32_t)(8 * ((total + 7) / 8));
    KT("cand_kernel<%d, true, true, %s, %s>", D, code_name<CodeT>(), code_name<CodeT>());
    cand_kernel<D, true, true, CodeT, CodeT><<<blocks, kCandThreads, lay.total, s>>>(
        x, cb, nbr, anchors, grid, nullptr, nullptr, codes, slice, defer, defer_count, skip, n,
        dim, M, K, L, (uint32_t)chunk, (uint32_t)nchunks, G, cells, nullptr, 0);
    KT_END();
    if (!deferred_pass) return TAC_OK;
    return encode_deferred<CodeT>(x, cb, codes, defer, defer_count, n, dim, M, K, rescans, stats, s);
  }
  // The deferred vectors of an encode pass: one per thread on about 4,096
  // blocks over all subspaces when they are few, eight per thread when more
  // than a quarter of a subspace's rows were deferred (each launch serves the
  // subspaces of its width, blocks loop when there are more).
  template <typename CodeT>
  static int encode_deferred(const float *x, const float *cb, CodeT *codes,
                             const uint32_t *defer, const uint32_t *defer_count, uint64_t n,
                             uint32_t dim, uint32_t M, uint32_t K, unsigned long long *rescans,
                             unsigned long long *stats, hipStream_t s) {
    const uint32_t Kp = (K + kPruneBlock - 1) / kPruneBlock * kPruneBlock;
    const size_t lds = (size_t)Kp * (Pad<D>::value + 1) * sizeof(float) + 2 * sizeof(uint32_t);
    const uint32_t split = list_split(K);
    const uint64_t per1 = split ? kBlock / 4 : kBlock;  // the smaller tiles of the two widths
    const uint64_t g1 = std::max<uint64_t>(
        1, std::min<uint64_t>((n + per1 - 1) / per1, (4096 + M - 1) / M));
    const uint64_t g8 = std::max<uint64_t>(
        1, std::min<uint64_t>((n + kBlock * 8 - 1) / (kBlock * 8), (4096 + M - 1) / M));
    if (split) {
      KT("encode_list_kernel<%d, 1, %s, 4>", D, code_name<CodeT>());
      encode_list_kernel<D, 1, CodeT, 4><<<dim3((unsigned)g1, M), kBlock, lds, s>>>(
          x, cb, codes, defer, defer_count, n, dim, M, K, rescans, stats, split);
    } else {
      KT("encode_list_kernel<%d, 1, %s, 1>", D, code_name<CodeT>());
      encode_list_kernel<D, 1, CodeT, 1><<<dim3((unsigned)g1, M), kBlock, lds, s>>>(
          x, cb, codes, defer, defer_count, n, dim, M, K, rescans, stats, 0u);
    }
    KT_END();
    KT("encode_list_kernel<%d, 8, %s, 1>", D, code_name<CodeT>());
    encode_list_kernel<D, 8, CodeT><<<dim3((unsigned)g8, M), kBlock, lds, s>>>(
        x, cb, codes, defer, defer_count, n, dim, M, K, rescans, stats, split);
    KT_END();
    return TAC_OK;
  }
  // Encode at sub-dimensions 1-4 with K <= 256: per subspace, the box
  // kernel picks the cell-list encode (cell_kernels.hpp) when more than
  // kCellOutside of a sample of the rows lies outside the codebook's box (the
  // anchored encode would leave them to the full search), else the anchored
  // candidate encode; every kernel of the other pass returns at once for that
  // subspace.  mode 1 / 0 forces the cell lists / the anchored pass.  Then
  // the reference scan of the deferred vectors of both.  slice / defer hold
  // M * n words each.
  template <typename CodeT>
  static int encode_auto(const float *x, const float *cb, CodeT *codes, uint32_t *nbr,
                         CodeT *anchors, float *grid, uint32_t *par, uint32_t *sel,
                         uint8_t *cids, uint32_t *ccnt, uint32_t *rec, uint8_t *lists,
                         uint32_t cap_items, uint32_t *slice, uint32_t *defer,
                         uint32_t *defer_count, uint64_t n, uint32_t dim, uint32_t M, uint32_t K,
                         uint32_t L, int mode, unsigned long long *rescans,
                         unsigned long long *stats, unsigned long long *cells_stat,
                         hipStream_t s) {
    if constexpr (D > 4) {
      return TAC_ERR_UNSUPPORTED;
    } else {
      constexpr uint32_t Cc = cell_coarse_count(D), F = cell_fine_per_coarse(D), CPB = 256 / F;
      KT("cell_box_kernel<%d>", D);
      cell_box_kernel<D><<<M, 256, 0, s>>>(x, cb, par, sel, defer_count, n, dim, K, mode,
                                           cells_stat);
      KT_END();
      encode_tables<CodeT>(cb, nbr, anchors, grid, defer_count, M, K, L, s, sel);
      if (int st = encode_rows<CodeT>(x, cb, codes, nbr, anchors, grid, slice, defer,
                                      defer_count, n, dim, M, K, L, rescans, stats, s, sel,
                                      false))
        return st;
      KT("cell_coarse_kernel<%d>", D);
      cell_coarse_kernel<D><<<dim3((Cc + 3) / 4, M), 256, 0, s>>>(cb, par, cids, ccnt, K);
      KT_END();
      KT("cell_fine_kernel<%d>", D);
      cell_fine_kernel<D><<<dim3((Cc + CPB - 1) / CPB, M), CPB * F, 0, s>>>(
          cb, par, cids, ccnt, rec, lists, K, cap_items);
      KT_END();
      const CellLds lay = cell_lds(K, Pad<D>::value);
      if (int st = raise_lds((const void *)cell_encode_kernel<D, CodeT>, lay.total, 0)) return st;
      // Chunks of 8,192 rows; the M blocks of a chunk run on one XCD, so a
      // row crosses HBM once and its other subspaces come from L2.
      const uint64_t chunk = 8192;
      const uint64_t nchunks = (n + chunk - 1) / chunk;
      const uint64_t total = nchunks * M;
      if (total > 0xFFFFFFF0ull) return TAC_ERR_UNSUPPORTED;
      const uint32_t blocks = (uint32_t)(8 * ((total + 7) / 8));
      KT("cell_encode_kernel<%d, %s>", D, code_name<CodeT>());
      cell_encode_kernel<D, CodeT><<<blocks, kCandThreads, lay.total, s>>>(
          x, cb, par, rec, lists, codes, slice, defer, defer_count, n, dim, M, K,
          (uint32_t)chunk, (uint32_t)nchunks, cap_items);
      KT_END();
      return encode_deferred<CodeT>(x, cb, codes, defer, defer_count, n, dim, M, K, rescans,
                                    stats, s);
    }
  }
  static int scatter(const float *xs, const uint16_t *codes, const uint32_t *hist,
                     const uint32_t *start, float *sorted, const uint32_t *done, uint64_t n,
                     uint32_t M, uint32_t K, uint32_t T, hipStream_t s) {
    const size_t lds = (size_t)kSortTile * Pad<D>::value * sizeof(float) +
                       (size_t)kSortTile * sizeof(uint32_t) + (size_t)5 * K * sizeof(uint32_t);
    if (lds > 65536) {
      static bool raised = false;
      if (!raised) {
        const hipError_t e = hipFuncSetAttribute((const void *)scatter_kernel<D>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)lds);
        if (e != hipSuccess) return hip_status("hipFuncSetAttribute(scatter_kernel)", e);
        raised = true;
      }
    }
    const uint32_t total = M * T;
    const uint32_t blocks = 8 * ((total + 7) / 8);
    KT("scatter_kernel<%d>", D);
    scatter_kernel<D><<<blocks, kBlock, lds, s>>>(xs, codes, hist, start, sorted, done, n, K, T,
                                                  M, code_bits(K));
    KT_END();
    return TAC_OK;
  }
  static void kpp_update(const float *xs, float *w, uint16_t *src, double *bsum, uint32_t *bad,
                         const KppState *st, float *cb, uint64_t n, uint32_t M, uint32_t K,
                         uint32_t c, uint32_t NB, hipStream_t s) {
    kpp_update_kernel<D><<<dim3(NB, M), kKppThreads, 0, s>>>(xs, w, src, bsum, bad, st, cb, n,
                                                              K, c, NB);
  }
  static void fold(const float *sorted, const uint32_t *counts, const uint32_t *start,
                   float *cb, const uint32_t *done, const uint32_t *order, uint64_t n, uint32_t M,
                   uint32_t K, hipStream_t s) {
    KT("fold_kernel<%d>", D);
    constexpr uint32_t FP = fold_per_wave<D>();
    fold_kernel<D><<<M * ((K + FP - 1) / FP), kWave, 0, s>>>(sorted, counts, start, cb, done,
                                                             order, n, M, K);
    KT_END();
  }
  static void reseed(const float *xs, float *e, const uint32_t *counts, float *cb,
                     uint32_t *empties, uint32_t *done, const float *wcss, float *prev,
                     uint32_t *iters_run, uint64_t n, uint32_t M, uint32_t K, uint32_t iter,
                     float tol, int check, hipStream_t s) {
    KT("reseed_kernel<%d>", D);
    reseed_kernel<D><<<M, 1024, 0, s>>>(xs, e, counts, cb, empties, done, wcss, prev, iters_run,
                                        n, K, iter, tol, check);
    KT_END();
  }
  template <typename CodeT>
  static int encode(const float *x, const float *cb, CodeT *codes, uint64_t n, uint32_t dim,
                    uint32_t M, uint32_t K, unsigned long long *rescans, hipStream_t s) {
    const uint32_t Kp = (K + kPruneBlock - 1) / kPruneBlock * kPruneBlock;
    const size_t lds = (size_t)Kp * (Pad<D>::value + 1) * sizeof(float) + 2 * sizeof(uint32_t);
    const uint64_t tiles = (n + kBlock * VPT - 1) / (kBlock * VPT);
    const uint64_t total = tiles * M;
    if (total > 0xFFFFFFF0ull) return TAC_ERR_UNSUPPORTED;
    const uint32_t blocks = (uint32_t)(8 * ((total + 7) / 8));
    KT("encode_kernel<%d, %d, %s>", D, VPT, code_name<CodeT>());
    encode_kernel<D, VPT, CodeT><<<blocks, kBlock, lds, s>>>(x, cb, codes, n, dim, M, K,
                                                              (uint32_t)tiles, rescans);
    KT_END();
    return TAC_OK;
  }
};

#define DISPATCH_D_ST(D_, CALL)                          \
  switch (D_) {                                          \
    case 1: st = Launch<1>::CALL; break;                 \
    case 2: st = Launch<2>::CALL; break;                 \
    case 3: st = Launch<3>::CALL; break;                 \
    case 4: st = Launch<4>::CALL; break;                 \
    case 5: st = Launch<5>::CALL; break;                 \
    case 6: st = Launch<6>::CALL; break;                 \
    case 7: st = Launch<7>::CALL; break;                 \
    case 8: st = Launch<8>::CALL; break;                 \
    default: st = TAC_ERR_UNSUPPORTED;                   \
  }

#define DISPATCH_D(D_, CALL)                 \
  switch (D_) {                              \
    case 1: { Launch<1>::CALL; } break;      \
    case 2: { Launch<2>::CALL; } break;      \
    case 3: { Launch<3>::CALL; } break;      \
    case 4: { Launch<4>::CALL; } break;      \
    case 5: { Launch<5>::CALL; } break;      \
    case 6: { Launch<6>::CALL; } break;      \
    case 7: { Launch<7>::CALL; } break;      \
    case 8: { Launch<8>::CALL; } break;      \
    default: return TAC_ERR_UNSUPPORTED;     \
  }

template <typename T>
T *as(Buffer &b) {
  return reinterpret_cast<T *>(b.ptr);
}

struct TrainOut {
  float *cb;                 // device [M][K][D]: init in (unless kpp), result out
  bool kpp;                  // seed with k-means++ (seed +% subspace) instead of cb
  uint64_t seed;
  uint32_t *d_assign;        // device [n] u32 (M == 1) or null
  tac_pq_train_extras *ex;   // host extras or null
  float *h_wcss_single;      // host scalar (kmeans.fit) or null
  uint32_t *h_iters_single;  // host scalar (kmeans.fit) or null
  void *codes_out = nullptr;  // device token-major [n][M] codes (u8, u16 past K = 256) or null
  bool *encoded = nullptr;    // set when train_core wrote codes_out itself
};

// A run of consecutive subspaces [m0, m0 + Mh) and the stream it runs on.
struct SubspaceGroup {
  uint32_t m0, Mh;
  hipStream_t s;
};

// k-means++ seeding of all subspaces (src/tac/kmeans.zig:106-136) into cb,
// each group of subspaces on its own stream (groups[0] on s, the call's
// stream, which waits for the others before the states are read back).
// Returns the lowest subspace's error, as a serial run of the reference
// (src/index/pq.zig:180-191) would.
int kmeanspp(DeviceState &ds, hipStream_t s, const SubspaceGroup *groups, uint32_t H,
             const float *xs, uint64_t n, uint32_t M, uint32_t K, uint32_t D, uint64_t seed,
             float *cb) {
  const uint32_t NB = (uint32_t)((n + kKppBlock - 1) / kKppBlock);
  const uint32_t DP = pad_of(D);
  int st;
  if ((st = ensure(ds, ds.kpp_state, (size_t)M * sizeof(KppState))) ||
      (st = ensure(ds, ds.kpp_w, (size_t)M * n * sizeof(float))) ||
      (st = ensure(ds, ds.kpp_src, (size_t)M * n * sizeof(uint16_t))) ||
      (st = ensure(ds, ds.kpp_bsum, (size_t)M * NB * sizeof(double))) ||
      (st = ensure(ds, ds.kpp_bad, (size_t)M * sizeof(uint32_t))))
    return st;
  // exact weight folds of the fallback: chunk prefixes / start values and
  // descriptors (the same buffers, and sizes, as the wcss fold of training)
  const uint32_t nfc = (uint32_t)((n + kFoldChunk - 1) / kFoldChunk);
  if ((st = ensure(ds, ds.fold_pre, (size_t)M * nfc * sizeof(double))) ||
      (st = ensure(ds, ds.fold_chunks, (size_t)M * nfc * sizeof(FoldChunk))))
    return st;
  double *fold_pre = as<double>(ds.fold_pre);
  FoldChunk *fold_chunks = as<FoldChunk>(ds.fold_chunks);
  // TAC_GPU_KPP_EXACT=1: every draw takes the exact sequential evaluation
  // (the same picks, slower; the parallel band test is skipped).
  const char *exact_env = getenv("TAC_GPU_KPP_EXACT");
  const uint32_t exact_only = exact_env != nullptr && exact_env[0] == '1';
  KppState *state = as<KppState>(ds.kpp_state);
  float *w = as<float>(ds.kpp_w);
  uint16_t *src = as<uint16_t>(ds.kpp_src);
  double *bsum = as<double>(ds.kpp_bsum);
  uint32_t *bad = as<uint32_t>(ds.kpp_bad);
  auto launch_all = [&]() -> int {
    for (uint32_t h = 0; h < H; ++h) {
      const SubspaceGroup &g = groups[h];
      kpp_init_kernel<<<(g.Mh + 63) / 64, 64, 0, g.s>>>(state + g.m0, bad + g.m0, seed + g.m0,
                                                       n, g.Mh);
      LAUNCH_TRY("kpp_init_kernel");
    }
    for (uint32_t c = 0; c < K; ++c) {
      for (uint32_t h = 0; h < H; ++h) {
        const SubspaceGroup &g = groups[h];
        const uint64_t m0 = g.m0;
        DISPATCH_D(D, kpp_update(xs + m0 * n * DP, w + m0 * n, src + m0 * n, bsum + m0 * NB,
                                 bad + m0, state + m0, cb + m0 * K * D, n, g.Mh, K, c, NB, g.s));
        LAUNCH_TRY("kpp_update_kernel");
        if (c + 1 == K) continue;
        kpp_select_kernel<<<g.Mh, 1024, 0, g.s>>>(w + m0 * n, bsum + m0 * NB, bad + m0,
                                                  state + m0, n, NB, exact_only);
        LAUNCH_TRY("kpp_select_kernel");
        kpp_fallback_kernel<<<g.Mh, kKppFallbackThreads, 0, g.s>>>(
            w + m0 * n, state + m0, n, fold_pre + m0 * nfc, fold_chunks + m0 * nfc, nfc);
        LAUNCH_TRY("kpp_fallback_kernel");
      }
    }
    return TAC_OK;
  };
  st = launch_all();
  // The call's stream waits for the other groups, also after an error.
  for (uint32_t h = 1; h < H; ++h) {
    HIP_TRY(hipEventRecord(ds.aux_join[h - 1], groups[h].s));
    HIP_TRY(hipStreamWaitEvent(s, ds.aux_join[h - 1], 0));
  }
  if (st) return st;
  std::vector<KppState> hs(M);
  HIP_TRY(hipMemcpyAsync(hs.data(), state, M * sizeof(KppState), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  for (uint32_t m = 0; m < M; ++m)
    if (hs[m].err) return hs[m].err;
  return TAC_OK;
}

// Whether the candidate-set passes serve a shape.  Past a few dimensions the
// candidate ball around an anchor holds most of a 256-codeword book (its
// volume grows as 2^D): the rows run out and most vectors fall through to the
// full search anyway.  With the vector-unit pruned search the Lloyd loop on
// 1.52M corpus rows at m8 K256 was faster through the full search from dsub
// 7 on (19.7 against 24.4 ms at dsub 8; a tie at 6) and encode from dsub 5
// on (0.83 against 1.14 ms at 8).  With the full search's first pass on the
// matrix cores (screen_kernels.hpp, K <= 256) the Lloyd loop is faster
// through it from dsub 5 on (corpus columns, 20 iterations: 19.5 against
// 20.9 ms at m12 dsub 5, 13.3 against 16.7 ms at m8 dsub 6); without the
// screen (TAC_GPU_SCREEN=0) the candidate passes keep dsub 5-6.  Larger
// books keep the candidate passes: the full search costs K per vector.
// TAC_GPU_FULL_SEARCH=1 turns the candidate passes off everywhere,
// TAC_GPU_CANDIDATES=1 keeps them at every dsub (both for auditing).
bool cand_wanted(uint32_t D, uint32_t K, bool encode) {
  const char *full_env = getenv("TAC_GPU_FULL_SEARCH");
  if (full_env && full_env[0] == '1') return false;
  const char *cand_env = getenv("TAC_GPU_CANDIDATES");
  if (cand_env && cand_env[0] == '1') return true;
  if (K > 256 || D <= 4u) return true;
  return !encode && D <= 6u && !screen_wanted(K);
}

// Lloyd training of all subspaces.  `out.cb` holds the initial codebooks on
// entry and the trained ones on return.
int train_core(DeviceState &ds, hipStream_t s, const float *d_x, uint64_t n, uint32_t dim,
               uint32_t M, uint32_t K, uint32_t max_iters, float tol, const TrainOut &out) {
  const uint32_t D = dim / M;
  const uint32_t DP = pad_of(D);
  tac_pq_train_extras *ex = out.ex;
  const bool want_trace = ex && ex->trace && max_iters > 0;
  const size_t cb_elems = (size_t)M * K * D;

  // Degenerate branch: k >= n (src/tac/kmeans.zig:88-104).
  if ((uint64_t)K >= n) {
    const uint64_t total = cb_elems;
    degenerate_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(d_x, out.cb, n, dim, M, K,
                                                                       D);
    LAUNCH_TRY("degenerate_kernel");
    if (out.d_assign) {
      std::vector<uint32_t> iota(n);
      for (uint64_t i = 0; i < n; ++i) iota[i] = (uint32_t)i;
      HIP_TRY(hipMemcpyAsync(out.d_assign, iota.data(), n * sizeof(uint32_t),
                             hipMemcpyHostToDevice, s));
      HIP_TRY(hipStreamSynchronize(s));
    }
    if (ex) {
      if (ex->iters_run) std::fill(ex->iters_run, ex->iters_run + M, 0u);
      if (ex->wcss) std::fill(ex->wcss, ex->wcss + M, 0.0f);
      if (ex->empties) std::fill(ex->empties, ex->empties + M, 0u);
      if (want_trace) {
        HIP_TRY(hipStreamSynchronize(s));
        for (uint32_t t = 0; t < max_iters; ++t)
          HIP_TRY(hipMemcpy(ex->trace + (size_t)t * cb_elems, out.cb, cb_elems * sizeof(float),
                            hipMemcpyDeviceToHost));
      }
    }
    if (out.h_wcss_single) *out.h_wcss_single = 0.0f;
    if (out.h_iters_single) *out.h_iters_single = 0;
    return TAC_OK;
  }

  const uint32_t T = (uint32_t)((n + kSortTile - 1) / kSortTile);
  int st;
  if ((st = ensure(ds, ds.xs, (size_t)M * n * DP * sizeof(float)))) return st;
  if ((st = ensure(ds, ds.codes, (size_t)M * n * sizeof(uint16_t)))) return st;
  if ((st = ensure(ds, ds.e, (size_t)M * n * sizeof(float)))) return st;
  if ((st = ensure(ds, ds.hist, (size_t)M * T * K * sizeof(uint32_t)))) return st;
  if ((st = ensure(ds, ds.counts, (size_t)M * K * sizeof(uint32_t)))) return st;
  if ((st = ensure(ds, ds.start, (size_t)M * K * sizeof(uint32_t)))) return st;
  if ((st = ensure(ds, ds.fold_order, (size_t)M * K * sizeof(uint32_t)))) return st;
  const uint32_t G = T < kScanRanges ? T : kScanRanges;
  const uint32_t nfc = (uint32_t)((n + kFoldChunk - 1) / kFoldChunk);  // wcss chunks
  if ((st = ensure(ds, ds.fold_pre, (size_t)M * nfc * sizeof(double)))) return st;
  if ((st = ensure(ds, ds.fold_chunks, (size_t)M * nfc * sizeof(FoldChunk)))) return st;
  if ((st = ensure(ds, ds.scan_sums, (size_t)M * G * K * sizeof(uint32_t)))) return st;
  if ((st = ensure(ds, ds.sorted, (size_t)M * n * DP * sizeof(float)))) return st;
  if ((st = ensure(ds, ds.flags, (size_t)3 * M * sizeof(uint32_t)))) return st;
  if ((st = ensure(ds, ds.scal, (size_t)2 * M * sizeof(float)))) return st;
  if (want_trace && (st = ensure(ds, ds.trace, (size_t)max_iters * cb_elems * sizeof(float))))
    return st;
  // Candidate-set assignment (cand_kernels.hpp) when the codeword ids fit the
  // neighbour keys and the tables fit in LDS: iterations after the first
  // start from the previous codes, and the first, on 16,384 vectors or more,
  // from grid anchors; cand_wanted decides the sub-dimensions and switches.
  const uint32_t Lc = K >= 2 ? std::min<uint32_t>(dim / M <= 4 ? kCandList : kCandListWide, K - 1) : 0;
  // Anchors (first iteration) are u8 ids up to K = 256, u16 beyond; the
  // block's tables must fit the LDS with at least one sort tile.
  const uint32_t anchor_size = K <= 256 ? 1u : 2u;
  const bool cand_ok = cand_wanted(D, K, false) && K >= 2 && K <= kCandMaxK &&
                       cand_lds(K, DP, kCandCells, 1, cand_anchors<false>() * anchor_size).total <=
                           kCandLdsMax &&
                       n <= 0xFFFFFFFFull;
  const bool cand = cand_ok && max_iters > 1;
  const bool cand_first = cand_ok && n >= 16384;
  // The full search's iterations take the matrix-core screen where it applies.
  const bool screen = D >= 5 && D <= 8 && screen_wanted(K) && n <= 0xFFFFFFFFull;
  if ((cand || cand_first) &&
      (st = ensure(ds, ds.cand_nbr, (size_t)M * K * cand_row_len(Lc) * sizeof(uint32_t))))
    return st;
  if ((cand || cand_first || screen) &&
      ((st = ensure(ds, ds.cand_defer, (size_t)2 * M * n * sizeof(uint32_t))) ||
       (st = ensure(ds, ds.cand_count, (size_t)M * sizeof(uint32_t)))))
    return st;
  if (cand_first && ((st = ensure(ds, ds.cand_anchor,
                                  (size_t)M * kCandCells * kCandAnchorsMax * anchor_size)) ||
                     (st = ensure(ds, ds.cand_grid, (size_t)M * 16 * sizeof(float)))))
    return st;

  float *xs = as<float>(ds.xs);
  uint16_t *codes = as<uint16_t>(ds.codes);
  float *e = as<float>(ds.e);
  uint32_t *hist = as<uint32_t>(ds.hist);
  uint32_t *counts = as<uint32_t>(ds.counts);
  uint32_t *start = as<uint32_t>(ds.start);
  uint32_t *scan_part = as<uint32_t>(ds.scan_sums);
  double *fold_pre = as<double>(ds.fold_pre);
  FoldChunk *fold_chunks = as<FoldChunk>(ds.fold_chunks);
  float *sorted = as<float>(ds.sorted);
  uint32_t *done = as<uint32_t>(ds.flags);
  uint32_t *iters_run = done + M;
  uint32_t *empties = done + 2 * M;
  float *wcss = as<float>(ds.scal);
  float *prev = wcss + M;
  HIP_TRY(hipMemsetAsync(done, 0, 3 * M * sizeof(uint32_t), s));
  HIP_TRY(hipMemsetAsync(wcss, 0, 2 * M * sizeof(float), s));
  unsigned long long *rescans = nullptr;
  if ((st = counter_begin(ds, s, &rescans))) return st;

  const bool profile = g_profile;
  ClockScope clock(ds, s);
  size_t ev = 0;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (profile) {
    if ((st = event_at(ds, ev++, &e0))) return st;
    HIP_TRY(hipEventRecord(e0, s));
  }
  DISPATCH_D_ST(D, transpose(d_x, xs, n, dim, s));
  if (st) return st;
  LAUNCH_TRY("transpose_kernel");
  // Two halves of the subspaces on two streams (M even), for the k-means++
  // seeding and the Lloyd loop: every subspace's kernels see only its own
  // buffers, so each half runs the same arithmetic as one stream would, and
  // one half's latency-bound steps (the fold's longest chains, the
  // deferred-vector scans, the draws, the small scans) overlap the other
  // half's VALU- or HBM-bound work.  TAC_GPU_TRAIN_STREAMS=1 keeps one
  // stream.
  const char *streams_env = getenv("TAC_GPU_TRAIN_STREAMS");
  const bool one_stream = streams_env && streams_env[0] == '1';
  const uint32_t H = (!one_stream && M >= 2 && M % 2 == 0) ? 2u : 1u;
  SubspaceGroup halves[2];
  for (uint32_t h = 0; h < H; ++h) halves[h] = {h * (M / H), M / H, s};
  if (H > 1) {
    if (!ds.aux_fork) HIP_TRY(hipEventCreateWithFlags(&ds.aux_fork, hipEventDisableTiming));
    HIP_TRY(hipEventRecord(ds.aux_fork, s));
    for (uint32_t h = 1; h < H; ++h) {
      if (!ds.aux_stream[h - 1])
        HIP_TRY(hipStreamCreateWithFlags(&ds.aux_stream[h - 1], hipStreamNonBlocking));
      if (!ds.aux_join[h - 1])
        HIP_TRY(hipEventCreateWithFlags(&ds.aux_join[h - 1], hipEventDisableTiming));
      halves[h].s = ds.aux_stream[h - 1];
      HIP_TRY(hipStreamWaitEvent(halves[h].s, ds.aux_fork, 0));
    }
  }
  if (out.kpp && (st = kmeanspp(ds, s, halves, H, xs, n, M, K, D, out.seed, out.cb))) {
    // the other half joins the call's stream inside kmeanspp
    return st;
  }
  if (profile) {
    if ((st = event_at(ds, ev++, &e1))) return st;
    HIP_TRY(hipEventRecord(e1, s));
  }

  // The reference breaks on rel < tol; only a tol above -inf can ever fire.
  const bool check = tol > -INFINITY;
  const bool want_wcss = (ex && ex->wcss) || out.h_wcss_single;
  const size_t hist_lds = (size_t)K * sizeof(uint32_t);
  std::vector<size_t> it_events;  // event index triples per iteration
  uint32_t gcells = 1;
  for (uint32_t k = 0; k < D; ++k) gcells *= cand_grid_side(D);

  struct StreamScope {
    explicit StreamScope(hipStream_t hs) { tl_kt_stream = hs; }
    ~StreamScope() { tl_kt_stream = nullptr; }
  };
  uint32_t *slices_all =
      (cand || cand_first || screen) ? as<uint32_t>(ds.cand_defer) : nullptr;

  // One Lloyd iteration t of the subspaces m0 .. m0+Mh-1 on stream hs.
  auto iterate = [&](const SubspaceGroup &h, uint32_t t) -> int {
    int st = TAC_OK;
    const uint32_t m0 = h.m0, Mh = h.Mh;
    hipStream_t hs = h.s;
    StreamScope scope(hs);
    float *xs_h = xs + (size_t)m0 * n * DP;
    uint16_t *codes_h = codes + (size_t)m0 * n;
    float *e_h = e + (size_t)m0 * n;
    uint32_t *hist_h = hist + (size_t)m0 * T * K;
    uint32_t *counts_h = counts + (size_t)m0 * K;
    uint32_t *start_h = start + (size_t)m0 * K;
    uint32_t *scan_h = scan_part + (size_t)m0 * G * K;
    double *pre_h = fold_pre + (size_t)m0 * nfc;
    FoldChunk *chunks_h = fold_chunks + (size_t)m0 * nfc;
    float *sorted_h = sorted + (size_t)m0 * n * DP;
    uint32_t *done_h = done + m0;
    float *cb_h = out.cb + (size_t)m0 * K * D;
    uint32_t *order_h = as<uint32_t>(ds.fold_order) + (size_t)m0 * K;
    hipEvent_t a = nullptr, b = nullptr, c = nullptr;
    const bool timed = profile && m0 == 0;
    if (timed) {
      it_events.push_back(ev);
      if ((st = event_at(ds, ev++, &a)) || (st = event_at(ds, ev++, &b)) ||
          (st = event_at(ds, ev++, &c)))
        return st;
      HIP_TRY(hipEventRecord(a, hs));
    }
    // The candidate passes and the screened full search count the sort
    // tiles themselves; the vector-unit full search leaves that to hist_kernel.
    const bool cand_now = (cand && t > 0) || (cand_first && t == 0);
    const bool screen_now = !cand_now && screen;
    if (cand_now) {
      uint32_t *nbr_h = as<uint32_t>(ds.cand_nbr) + (size_t)m0 * K * cand_row_len(Lc);
      uint32_t *slices_h = slices_all + (size_t)m0 * n;
      uint32_t *defer_h = slices_all + (size_t)M * n + (size_t)m0 * n;
      uint32_t *count_h = as<uint32_t>(ds.cand_count) + m0;
      if (t == 0) {
        const size_t aoff = (size_t)m0 * gcells * cand_anchors<false>();
        float *grid_h = as<float>(ds.cand_grid) + (size_t)m0 * 16;
        if (anchor_size == 1) {
          DISPATCH_D_ST(D, assign_cand<true>(xs_h, cb_h, nbr_h, as<uint8_t>(ds.cand_anchor) + aoff,
                                             grid_h, codes_h, e_h, slices_h, defer_h, count_h,
                                             done_h, n, Mh, K, Lc, hist_h, T, rescans, hs));
        } else {
          DISPATCH_D_ST(D, assign_cand<true>(xs_h, cb_h, nbr_h, as<uint16_t>(ds.cand_anchor) + aoff,
                                             grid_h, codes_h, e_h, slices_h, defer_h, count_h,
                                             done_h, n, Mh, K, Lc, hist_h, T, rescans, hs));
        }
      } else {
        DISPATCH_D_ST(D, assign_cand<false>(xs_h, cb_h, nbr_h, (uint8_t *)nullptr, nullptr,
                                            codes_h, e_h, slices_h, defer_h, count_h, done_h, n,
                                            Mh, K, Lc, hist_h, T, rescans, hs));
      }
      if (st) return st;
      LAUNCH_TRY("assign_cand kernels");
    } else if (screen_now) {
      uint32_t *defer_h = slices_all + (size_t)M * n + (size_t)m0 * n;
      uint32_t *count_h = as<uint32_t>(ds.cand_count) + m0;
      DISPATCH_D_ST(D, assign_screen(xs_h, cb_h, codes_h, e_h, defer_h, count_h, done_h, n, Mh, K,
                                     hist_h, T, rescans, hs));
      if (st) return st;
      LAUNCH_TRY("assign_screen kernels");
    } else {
      DISPATCH_D(D, assign(xs_h, cb_h, codes_h, e_h, done_h, n, Mh, K, rescans, hs));
      LAUNCH_TRY("assign_kernel");
    }
    if (timed) HIP_TRY(hipEventRecord(b, hs));
    if (!cand_now && !screen_now) {
      KT("hist_kernel");
      hist_kernel<<<dim3(T, Mh), kBlock, hist_lds, hs>>>(codes_h, hist_h, done_h, n, K, T);
      KT_END();
      LAUNCH_TRY("hist_kernel");
    }
    // codes per scan thread: ceil(K / kBlock), rounded up to 1, 2 or 4
    const uint32_t scan_per = K <= kBlock ? 1u : K <= 2u * kBlock ? 2u : 4u;
    // the fold's order: bins of 1/32 of the mean cluster size
    const uint32_t order_unit = (uint32_t)std::max<uint64_t>(1, n / K / 32);
#define SCAN_PASSES(P)                                                                    \
  do {                                                                                    \
    KT("scan_partial_kernel<%uu>", P);                                                    \
    scan_partial_kernel<P><<<dim3(G, Mh), kBlock, 0, hs>>>(hist_h, scan_h, done_h, K, T, G); \
    KT_END();                                                                             \
    KT("scan_apply_kernel<%uu>", P);                                                      \
    scan_apply_kernel<P><<<dim3(G, Mh), kBlock, 0, hs>>>(hist_h, scan_h, counts_h, start_h,  \
                                                         order_h, done_h, K, T, G,        \
                                                         order_unit);                     \
    KT_END();                                                                             \
  } while (0)
    if (scan_per == 1)
      SCAN_PASSES(1u);
    else if (scan_per == 2)
      SCAN_PASSES(2u);
    else
      SCAN_PASSES(4u);
#undef SCAN_PASSES
    LAUNCH_TRY("scan kernels");
    DISPATCH_D_ST(D, scatter(xs_h, codes_h, hist_h, start_h, sorted_h, done_h, n, Mh, K, T, hs));
    if (st) return st;
    LAUNCH_TRY("scatter_kernel");
    DISPATCH_D(D, fold(sorted_h, counts_h, start_h, cb_h, done_h, order_h, n, Mh, K, hs));
    LAUNCH_TRY("fold_kernel");
    if (check || (want_wcss && t + 1 == max_iters)) {
      const uint32_t fgrid = (nfc + kBlock / kWave - 1) / (kBlock / kWave);
      KT("wcss_chunk_sums_kernel");
      wcss_chunk_sums_kernel<<<dim3(fgrid, Mh), kBlock, 0, hs>>>(e_h, pre_h, done_h, n, nfc);
      KT_END();
      KT("wcss_prefix_kernel");
      wcss_prefix_kernel<<<Mh, kBlock, 0, hs>>>(pre_h, done_h, nfc);
      KT_END();
      KT("wcss_quantize_kernel");
      wcss_quantize_kernel<<<dim3(fgrid, Mh), kBlock, 0, hs>>>(e_h, pre_h, chunks_h, done_h, n,
                                                                nfc);
      KT_END();
      KT("wcss_apply_kernel");
      wcss_apply_kernel<<<Mh, kWave, 0, hs>>>(e_h, chunks_h, wcss + m0, done_h, n, nfc);
      KT_END();
      LAUNCH_TRY("wcss kernels");
    }
    DISPATCH_D(D, reseed(xs_h, e_h, counts_h, cb_h, empties + m0, done_h, wcss + m0, prev + m0,
                         iters_run + m0, n, Mh, K, t, tol, check ? 1 : 0, hs));
    LAUNCH_TRY("reseed_kernel");
    if (want_trace)
      HIP_TRY(hipMemcpyAsync(as<float>(ds.trace) + (size_t)t * cb_elems + (size_t)m0 * K * D,
                             cb_h, (size_t)Mh * K * D * sizeof(float), hipMemcpyDeviceToDevice,
                             hs));
    if (timed) HIP_TRY(hipEventRecord(c, hs));
    return TAC_OK;
  };

  st = TAC_OK;
  for (uint32_t t = 0; t < max_iters && !st; ++t)
    for (uint32_t h = 0; h < H && !st; ++h) st = iterate(halves[h], t);
  // The caller's stream waits for the other half, also after an error.
  for (uint32_t h = 1; h < H; ++h) {
    HIP_TRY(hipEventRecord(ds.aux_join[h - 1], halves[h].s));
    HIP_TRY(hipStreamWaitEvent(s, ds.aux_join[h - 1], 0));
  }
  if (st) return st;
  // Encode of the residuals just trained on, as storage.build chains train
  // and encode (src/index/storage.zig:380-401): one more candidate pass with
  // the final codebooks, anchored at the last Lloyd codes (any anchor gives
  // the exact argmin; these are the nearest at hand), over every subspace,
  // then the codes turned token-major.  Without the candidate tables the
  // caller runs the ordinary encode.
  if (out.codes_out && (cand || cand_first) && max_iters >= 1 && cand_wanted(D, K, true)) {
    hipEvent_t ea = nullptr, eb = nullptr;
    if (profile) {
      if ((st = event_at(ds, ev++, &ea)) || (st = event_at(ds, ev++, &eb))) return st;
      HIP_TRY(hipEventRecord(ea, s));
    }
    if (H > 1) {
      HIP_TRY(hipEventRecord(ds.aux_fork, s));
      for (uint32_t h = 1; h < H; ++h) HIP_TRY(hipStreamWaitEvent(halves[h].s, ds.aux_fork, 0));
    }
    for (uint32_t h = 0; h < H && !st; ++h) {
      const uint32_t m0 = halves[h].m0, Mh = halves[h].Mh;
      hipStream_t hs = halves[h].s;
      StreamScope scope(hs);
      uint32_t *done_h = done + m0;
      HIP_TRY(hipMemsetAsync(done_h, 0, Mh * sizeof(uint32_t), hs));  // every subspace
      uint32_t *nbr_h = as<uint32_t>(ds.cand_nbr) + (size_t)m0 * K * cand_row_len(Lc);
      uint32_t *slices_h = slices_all + (size_t)m0 * n;
      uint32_t *defer_h = slices_all + (size_t)M * n + (size_t)m0 * n;
      DISPATCH_D_ST(D, assign_cand<false>(xs + (size_t)m0 * n * DP, out.cb + (size_t)m0 * K * D,
                                          nbr_h, (uint8_t *)nullptr, nullptr,
                                          codes + (size_t)m0 * n, e + (size_t)m0 * n, slices_h,
                                          defer_h, as<uint32_t>(ds.cand_count) + m0, done_h, n,
                                          Mh, K, Lc, hist + (size_t)m0 * T * K, T, rescans, hs));
    }
    for (uint32_t h = 1; h < H; ++h) {
      HIP_TRY(hipEventRecord(ds.aux_join[h - 1], halves[h].s));
      HIP_TRY(hipStreamWaitEvent(s, ds.aux_join[h - 1], 0));
    }
    if (st) return st;
    LAUNCH_TRY("final candidate pass");
    const unsigned tb = (unsigned)((n + 255) / 256);
    if (K <= 256)
      codes_to_tokens_kernel<uint8_t><<<tb, 256, 0, s>>>(codes, (uint8_t *)out.codes_out, n, M);
    else
      codes_to_tokens_kernel<uint16_t><<<tb, 256, 0, s>>>(codes, (uint16_t *)out.codes_out, n, M);
    LAUNCH_TRY("codes_to_tokens_kernel");
    if (profile) {
      HIP_TRY(hipEventRecord(eb, s));
      HIP_TRY(hipEventSynchronize(eb));
      float ms = 0.0f;
      HIP_TRY(hipEventElapsedTime(&ms, ea, eb));
      std::lock_guard<std::mutex> g(g_profile_mu);
      g_prof.encode_ms += ms;
      g_prof.encode_launches += 1;
    }
    if (out.encoded) *out.encoded = true;
  }
  if (out.d_assign && max_iters == 0) HIP_TRY(hipMemsetAsync(codes, 0, n * sizeof(uint16_t), s));
  if (out.d_assign) {
    widen_codes_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(codes, out.d_assign, n);
    LAUNCH_TRY("widen_codes_kernel");
  }

  const bool need_host = profile || ex || out.h_wcss_single || out.h_iters_single;
  if (need_host) {
    std::vector<uint32_t> h_flags(3 * M);
    std::vector<float> h_scal(2 * M);
    HIP_TRY(hipMemcpyAsync(h_flags.data(), done, 3 * M * sizeof(uint32_t),
                           hipMemcpyDeviceToHost, s));
    HIP_TRY(hipMemcpyAsync(h_scal.data(), wcss, 2 * M * sizeof(float), hipMemcpyDeviceToHost,
                           s));
    HIP_TRY(hipStreamSynchronize(s));
    if (ex) {
      if (ex->iters_run) std::memcpy(ex->iters_run, &h_flags[M], M * sizeof(uint32_t));
      if (ex->empties) std::memcpy(ex->empties, &h_flags[2 * M], M * sizeof(uint32_t));
      if (ex->wcss) std::memcpy(ex->wcss, &h_scal[0], M * sizeof(float));
      if (want_trace) {
        HIP_TRY(hipMemcpy(ex->trace, ds.trace.ptr, (size_t)max_iters * cb_elems * sizeof(float),
                          hipMemcpyDeviceToHost));
        // Iterations a converged subspace skipped repeat its final codebook.
        for (uint32_t m = 0; m < M; ++m) {
          const uint32_t ran = h_flags[M + m];
          for (uint32_t t = ran; t < max_iters; ++t)
            if (ran > 0)
              std::memcpy(ex->trace + ((size_t)t * M + m) * K * D,
                          ex->trace + ((size_t)(ran - 1) * M + m) * K * D,
                          (size_t)K * D * sizeof(float));
        }
      }
    }
    if (out.h_wcss_single) *out.h_wcss_single = h_scal[0];
    if (out.h_iters_single) *out.h_iters_single = h_flags[M];
    if (profile) {
      if ((st = counter_collect(ds, s))) return st;
      if ((st = clock.collect())) return st;
      std::lock_guard<std::mutex> g(g_profile_mu);
      float ms = 0.0f;
      HIP_TRY(hipEventElapsedTime(&ms, e0, e1));
      g_prof.transpose_ms += ms;
      g_prof.transpose_launches += 1;
      g_prof.train_streams = H;
      for (size_t t = 0; t < it_events.size(); ++t) {
        const size_t q = it_events[t];
        HIP_TRY(hipEventElapsedTime(&ms, ds.events[q], ds.events[q + 1]));
        g_prof.assign_ms += ms;
        g_prof.assign_launches += 1;
        if (cand && t > 0) {
          g_prof.cand_assign_ms += ms;
          g_prof.cand_assign_iters += 1;
        }
        HIP_TRY(hipEventElapsedTime(&ms, ds.events[q + 1], ds.events[q + 2]));
        g_prof.update_ms += ms;
        g_prof.update_iters += 1;
      }
    }
  }
  return TAC_OK;
}

// Fine and coarse cells per subspace of the cell-list encode at a runtime
// sub-dimension (1-4).
inline uint32_t cell_count_of(uint32_t D) {
  return D == 1 ? cell_count(1) : D == 2 ? cell_count(2) : D == 3 ? cell_count(3) : cell_count(4);
}
inline uint32_t cell_coarse_count_of(uint32_t D) {
  return D == 1   ? cell_coarse_count(1)
         : D == 2 ? cell_coarse_count(2)
         : D == 3 ? cell_coarse_count(3)
                  : cell_coarse_count(4);
}

int encode_core(DeviceState &ds, hipStream_t s, const float *d_x, uint64_t n, uint32_t dim,
                uint32_t M, uint32_t K, const float *d_cb, void *d_codes) {
  const uint32_t D = dim / M;
  const bool profile = g_profile;
  ClockScope clock(ds, s);
  hipEvent_t a = nullptr, b = nullptr;
  int st;
  unsigned long long *rescans = nullptr;
  if ((st = counter_begin(ds, s, &rescans))) return st;
  if (profile) {
    if ((st = event_at(ds, 0, &a)) || (st = event_at(ds, 1, &b))) return st;
    HIP_TRY(hipEventRecord(a, s));
  }
  st = TAC_OK;
  // Batches of 16,384 vectors or more take the candidate-set encode
  // (cand_kernels.hpp) where cand_wanted says so.
  const uint32_t L = K >= 2 ? std::min<uint32_t>(kCandListEncode, K - 1) : 0;
  // Codes and grid anchors share one width: u8 up to K = 256, u16 beyond.
  const uint32_t code_size = K <= 256 ? 1u : 2u;
  const uint32_t G = cand_grid_side(D), D_pad = pad_of(D);
  uint32_t cells = 1;
  for (uint32_t k = 0; k < D; ++k) cells *= G;
  const bool cand = cand_wanted(D, K, true) && K >= 2 && K <= kCandMaxK &&
                    n >= 16384 && n <= 0xFFFFFFFFull &&
                    cand_lds(K, D_pad, cells, 0, cand_anchors<true>() * code_size).total <=
                        kCandLdsMax;
  // Sub-dimensions 1-4 with K <= 256 on kCellMinRows rows or more choose per
  // subspace between the cell-list and the anchored encode (encode_auto).
  // TAC_GPU_ENCODE_CELLS=1 or 0 forces one of them, =auto makes the choice
  // at any size.
  const char *cells_env = getenv("TAC_GPU_ENCODE_CELLS");
  const int cell_mode = !cells_env ? -1 : cells_env[0] == '1' ? 1 : cells_env[0] == '0' ? 0 : -1;
  const bool by_cells = cand && D >= 1 && D <= 4 && K <= 256 && (cells_env || n >= kCellMinRows);
  if (by_cells) {
    const uint32_t ncell = cell_count_of(D), ncoarse = cell_coarse_count_of(D);
    const uint32_t cap_items = ncell * kCellItemsPerCell;
    if ((st = ensure(ds, ds.cand_nbr, (size_t)M * K * cand_row_len(L) * sizeof(uint32_t))) ||
        (st = ensure(ds, ds.cand_defer, (size_t)2 * M * n * sizeof(uint32_t))) ||
        (st = ensure(ds, ds.cand_count, (size_t)M * sizeof(uint32_t))) ||
        (st = ensure(ds, ds.cand_anchor, (size_t)M * kCandCells * kCandAnchorsMax * code_size)) ||
        (st = ensure(ds, ds.cand_grid, (size_t)M * 16 * sizeof(float))) ||
        (st = ensure(ds, ds.cell_par, (size_t)M * (kCellParWords + 1) * sizeof(uint32_t))) ||
        (st = ensure(ds, ds.cell_cids, (size_t)M * ncoarse * K)) ||
        (st = ensure(ds, ds.cell_ccnt, (size_t)M * ncoarse * sizeof(uint32_t))) ||
        (st = ensure(ds, ds.cell_rec, (size_t)M * ncell * sizeof(uint32_t))) ||
        (st = ensure(ds, ds.cell_list, (size_t)M * cap_items * kCellItem)))
      return st;
    uint32_t *slices = as<uint32_t>(ds.cand_defer);
    uint32_t *par = as<uint32_t>(ds.cell_par);
    DISPATCH_D_ST(D, encode_auto<uint8_t>(
                         d_x, d_cb, (uint8_t *)d_codes, as<uint32_t>(ds.cand_nbr),
                         as<uint8_t>(ds.cand_anchor), as<float>(ds.cand_grid), par,
                         par + (size_t)M * kCellParWords, as<uint8_t>(ds.cell_cids),
                         as<uint32_t>(ds.cell_ccnt), as<uint32_t>(ds.cell_rec),
                         as<uint8_t>(ds.cell_list), cap_items, slices, slices + (size_t)M * n,
                         as<uint32_t>(ds.cand_count), n, dim, M, K, L, cell_mode, rescans,
                         g_profile ? rescans + 1 : nullptr, g_profile ? rescans + 3 : nullptr, s));
  } else if (cand) {
    if ((st = ensure(ds, ds.cand_nbr, (size_t)M * K * cand_row_len(L) * sizeof(uint32_t))) ||
        (st = ensure(ds, ds.cand_defer, (size_t)2 * M * n * sizeof(uint32_t))) ||
        (st = ensure(ds, ds.cand_count, (size_t)M * sizeof(uint32_t))) ||
        (st = ensure(ds, ds.cand_anchor, (size_t)M * kCandCells * kCandAnchorsMax * code_size)) ||
        (st = ensure(ds, ds.cand_grid, (size_t)M * 16 * sizeof(float))))
      return st;
    uint32_t *slices = as<uint32_t>(ds.cand_defer);
    if (code_size == 1) {
      DISPATCH_D_ST(D, encode_cand<uint8_t>(d_x, d_cb, (uint8_t *)d_codes,
                                            as<uint32_t>(ds.cand_nbr), as<uint8_t>(ds.cand_anchor),
                                            as<float>(ds.cand_grid), slices,
                                            slices + (size_t)M * n, as<uint32_t>(ds.cand_count),
                                            n, dim, M, K, L, rescans, s));
    } else {
      DISPATCH_D_ST(D, encode_cand<uint16_t>(d_x, d_cb, (uint16_t *)d_codes,
                                             as<uint32_t>(ds.cand_nbr),
                                             as<uint16_t>(ds.cand_anchor),
                                             as<float>(ds.cand_grid), slices,
                                             slices + (size_t)M * n, as<uint32_t>(ds.cand_count),
                                             n, dim, M, K, L, rescans, s));
    }
  } else if (D >= 5 && D <= 8 && screen_wanted(K) && n <= 0xFFFFFFFFull) {
    if ((st = ensure(ds, ds.cand_defer, (size_t)2 * M * n * sizeof(uint32_t))) ||
        (st = ensure(ds, ds.cand_count, (size_t)M * sizeof(uint32_t))))
      return st;
    DISPATCH_D_ST(D, encode_screen<uint8_t>(d_x, d_cb, (uint8_t *)d_codes,
                                            as<uint32_t>(ds.cand_defer) + (size_t)M * n,
                                            as<uint32_t>(ds.cand_count), n, dim, M, K, rescans,
                                            g_profile ? rescans + 4 : nullptr, s));
  } else if (K <= 256) {
    DISPATCH_D_ST(D, encode<uint8_t>(d_x, d_cb, (uint8_t *)d_codes, n, dim, M, K, rescans, s));
  } else {
    DISPATCH_D_ST(D, encode<uint16_t>(d_x, d_cb, (uint16_t *)d_codes, n, dim, M, K, rescans, s));
  }
  if (st) return st;
  LAUNCH_TRY("encode_kernel");
  if (profile) {
    HIP_TRY(hipEventRecord(b, s));
    HIP_TRY(hipEventSynchronize(b));
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, a, b));
    if ((st = counter_collect(ds, s))) return st;
    if ((st = clock.collect())) return st;
    std::lock_guard<std::mutex> g(g_profile_mu);
    g_prof.encode_ms += ms;
    g_prof.encode_launches += 1;
  }
  return TAC_OK;
}

const char *kNames[] = {"Ok",
                        "DimNotDivisibleByM",
                        "DimMismatch",
                        "EmptyCorpus",
                        "OutBufferWrongSize",
                        "NQMismatch",
                        "KmeansBudgetTooSmall",
                        "EmptyVectorSet",
                        "EmptyDistribution",
                        "NonFinite",
                        "AllZero",
                        "OutOfMemory",
                        "NoDevice",
                        "HipError",
                        "InvalidArgument",
                        "Unsupported",
                        "QueryShapeMismatch",
                        "TableSizeMismatch",
                        "DocOutOfRange",
                        "DocLayoutCorrupt",
                        "BufferTooSmall",
                        "BudgetTooSmall",
                        "BudgetTooLarge",
                        "InvalidThresholds",
                        "EmptyTokenDump"};

}  // namespace

// ===========================================================================
// Scratch of the entry point that allocates nothing
// ===========================================================================
// tac_pq_encode_device_noalloc takes its counters, neighbour rows, grid
// anchors and deferred-vector lists from this array instead of the cached
// workspace.  Each GPU the library runs on holds its own copy, at its own
// address, until the process ends.  The name is a host-side stand-in: host
// code uses only the device address scratch_address returns.
// 32 MiB: batches of 245,760 rows at m16 (49,152 at m64).
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

std::mutex g_scratch_mu;
uint8_t *g_scratch[kMaxDevices] = {};

// The scratch array's address on device `dev`, which must be current;
// resolved on the first call on that device and kept.
int scratch_address(int dev, uint8_t **out) {
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status("hipGetSymbolAddress(scratch)", e);
    if (!p) return TAC_ERR_HIP;
    g_scratch[dev] = static_cast<uint8_t *>(p);
  }
  *out = g_scratch[dev];
  return TAC_OK;
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
namespace {
// One kmeans.fit problem run through the token engine (tac_kmeans_fit at
// dims past the PQ kernels'): every row belongs to token 0, which gets k
// centroids without the spreads and budget phases; init (k x dim, host),
// when given, replaces k-means++; the problem's iteration count goes to
// *iters_out.
struct TacFixedFit {
  uint32_t k;
  const float *init;
  uint32_t *iters_out;
};

int tac_cluster_core(DeviceState &ds, hipStream_t s, const uint32_t *ids, uint64_t N,
                     const float *vectors, bool vectors_on_device, uint32_t dim,
                     const tac_cluster_params &prm, uint64_t nd, float *cent_out,
                     uint32_t *assign_out, uint32_t *kpt_out, float *wcss_out,
                     const TacFixedFit *fixed = nullptr);
}  // namespace

extern "C" {

const char *tac_gpu_strerror(int status) {
  if (status < 0 || status >= (int)(sizeof(kNames) / sizeof(kNames[0]))) return "Unknown";
  return kNames[status];
}

const char *tac_gpu_last_error(void) { return g_last_error.c_str(); }

int tac_gpu_device_count(int *count) {
  if (!count) return TAC_ERR_INVALID_ARGUMENT;
  *count = device_count();
  return *count > 0 ? TAC_OK : TAC_ERR_NO_DEVICE;
}

int tac_gpu_get_device_info(int device, tac_gpu_device_info *info) {
  if (!info) return TAC_ERR_INVALID_ARGUMENT;
  const int c = device_count();
  if (c <= 0) return TAC_ERR_NO_DEVICE;
  if (device < 0 || device >= c) return TAC_ERR_INVALID_ARGUMENT;
  hipDeviceProp_t p;
  HIP_TRY(hipGetDeviceProperties(&p, device));
  std::memset(info, 0, sizeof(*info));
  std::snprintf(info->name, sizeof(info->name), "%s", p.name);
  std::snprintf(info->arch, sizeof(info->arch), "%s", p.gcnArchName);
  info->compute_units = p.multiProcessorCount;
  info->clock_khz = p.clockRate;
  info->global_mem_bytes = p.totalGlobalMem;
  info->lds_bytes_per_block = p.sharedMemPerBlock;
  return TAC_OK;
}

int tac_gpu_set_lane_count(uint32_t lanes) {
  if (lanes != 4 && lanes != 8 && lanes != 16) return TAC_ERR_INVALID_ARGUMENT;
  g_vec_lanes.store(lanes);
  return TAC_OK;
}

int tac_gpu_get_lane_count(uint32_t *lanes) {
  if (!lanes) return TAC_ERR_INVALID_ARGUMENT;
  *lanes = g_vec_lanes.load();
  return TAC_OK;
}

int tac_gpu_set_device(int device) {
  const int c = device_count();
  if (c <= 0) return TAC_ERR_NO_DEVICE;
  if (device < 0 || device >= c) return TAC_ERR_INVALID_ARGUMENT;
  HIP_TRY(hipSetDevice(device));
  return TAC_OK;
}

int tac_gpu_malloc(void **ptr, uint64_t bytes) {
  if (!ptr) return TAC_ERR_INVALID_ARGUMENT;
  *ptr = nullptr;
  if (device_count() <= 0) return TAC_ERR_NO_DEVICE;
  HIP_TRY(hipMalloc(ptr, bytes ? bytes : 1));
  return TAC_OK;
}

int tac_gpu_free(void *ptr) {
  if (!ptr) return TAC_OK;
  if (device_count() <= 0) return TAC_ERR_NO_DEVICE;
  HIP_TRY(hipFree(ptr));
  return TAC_OK;
}

int tac_gpu_memcpy_htod(void *dst, const void *src, uint64_t bytes) {
  if ((!dst || !src) && bytes) return TAC_ERR_INVALID_ARGUMENT;
  if (device_count() <= 0) return TAC_ERR_NO_DEVICE;
  if (bytes) HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return TAC_OK;
}

int tac_gpu_memcpy_dtoh(void *dst, const void *src, uint64_t bytes) {
  if ((!dst || !src) && bytes) return TAC_ERR_INVALID_ARGUMENT;
  if (device_count() <= 0) return TAC_ERR_NO_DEVICE;
  if (bytes) HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return TAC_OK;
}

int tac_gpu_memcpy_dtod(void *dst, const void *src, uint64_t bytes) {
  if ((!dst || !src) && bytes) return TAC_ERR_INVALID_ARGUMENT;
  if (device_count() <= 0) return TAC_ERR_NO_DEVICE;
  if (bytes) HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
  return TAC_OK;
}

int tac_gpu_synchronize(void) {
  if (device_count() <= 0) return TAC_ERR_NO_DEVICE;
  HIP_TRY(hipDeviceSynchronize());
  return TAC_OK;
}

int tac_gpu_release_workspace(void) {
  DeviceState *ds = nullptr;
  int st = acquire_device(&ds, nullptr);
  if (st) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  HIP_TRY(hipDeviceSynchronize());
  Buffer *bufs[] = {&ds->xs,        &ds->codes,   &ds->e,         &ds->hist,     &ds->counts,
                    &ds->start,     &ds->sorted,  &ds->flags,     &ds->scal,     &ds->trace,
                    &ds->io_in,     &ds->io_out,  &ds->io_cb,     &ds->io_init,  &ds->counter,
                    &ds->kpp_state, &ds->kpp_w,   &ds->kpp_bsum,  &ds->kpp_bad,  &ds->status,
                    &ds->io_aux,    &ds->io_out2, &ds->scan_sums, &ds->io_x1,    &ds->io_x2,
                    &ds->io_x3,     &ds->crc_tx,  &ds->fold_pre,  &ds->fold_chunks,
                    &ds->tac_v,     &ds->tac_idx, &ds->tac_offs,  &ds->tac_G,
                    &ds->tac_spreads, &ds->tac_w, &ds->tac_e,     &ds->tac_code,
                    &ds->tac_sorted, &ds->tac_tsum, &ds->tac_hist, &ds->tac_counts,
                    &ds->tac_start, &ds->tac_C,   &ds->tac_pre,   &ds->tac_fch,
                    &ds->tac_st,    &ds->tac_bad, &ds->tac_done,  &ds->tac_iters,
                    &ds->tac_wcss,  &ds->tac_prev, &ds->tac_empties, &ds->tac_assign,
                    &ds->tac_probs, &ds->tac_tiles, &ds->tac_chl, &ds->tac_cprob,
                    &ds->tac_inv,   &ds->tac_rsum, &ds->tac_ranges, &ds->cand_nbr,
                    &ds->cand_defer, &ds->cand_count, &ds->cand_anchor, &ds->cand_grid,
                    &ds->kpp_src,   &ds->fold_order, &ds->tac_h, &ds->tac_ktiles,
                    &ds->tac_big};
  ds->crc_tx_ready = false;
  for (Buffer *b : bufs) {
    if (b->ptr) HIP_TRY(hipFree(b->ptr));
    b->ptr = nullptr;
    b->bytes = 0;
  }
  for (int b = 0; b < DeviceState::kStageBufs; ++b) {
    if (ds->stage[b]) HIP_TRY(hipHostFree(ds->stage[b]));
    if (ds->stage_ev[b]) HIP_TRY(hipEventDestroy(ds->stage_ev[b]));
    ds->stage[b] = nullptr;
    ds->stage_ev[b] = nullptr;
    ds->stage_pending[b] = false;
  }
  return TAC_OK;
}

int tac_gpu_profile_enable(int enable) {
  g_profile = enable != 0;
  return TAC_OK;
}

int tac_gpu_profile_read(tac_gpu_profile *out, int reset) {
  if (!out) return TAC_ERR_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> g(g_profile_mu);
  *out = g_prof;
  if (reset) g_prof = tac_gpu_profile{};
  return TAC_OK;
}

int tac_gpu_profile_kernels(tac_gpu_kernel_time *out, uint32_t cap, uint32_t *count, int reset) {
  if (!count || (cap && !out)) return TAC_ERR_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> g(g_profile_mu);
  uint32_t i = 0;
  for (const auto &kv : g_kernel_times) {
    if (i < cap) {
      std::snprintf(out[i].name, sizeof out[i].name, "%s", kv.first.c_str());
      out[i].ms = kv.second.first;
      out[i].launches = kv.second.second;
    }
    ++i;
  }
  *count = i;
  if (reset) g_kernel_times.clear();
  return TAC_OK;
}

int tac_pq_train_device(const float *d_residuals, uint64_t n, uint32_t dim, uint32_t m,
                        uint32_t ksub, const float *d_init_codebooks, uint64_t seed,
                        uint32_t max_iters, float tol, float *d_codebooks_out,
                        tac_pq_train_extras *extras, void *stream) {
  int st = validate_pq(n, dim, m, ksub);
  if (st) return st;
  if (!d_residuals || !d_codebooks_out) return TAC_ERR_INVALID_ARGUMENT;
  DeviceState *ds = nullptr;
  if ((st = acquire_device(&ds, nullptr))) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, stream, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  const size_t cb_bytes = (size_t)m * ksub * (dim / m) * sizeof(float);
  if (d_init_codebooks && d_init_codebooks != d_codebooks_out)
    HIP_TRY(hipMemcpyAsync(d_codebooks_out, d_init_codebooks, cb_bytes, hipMemcpyDeviceToDevice,
                           s));
  TrainOut out{d_codebooks_out, d_init_codebooks == nullptr, seed, nullptr, extras, nullptr,
               nullptr};
  st = train_core(*ds, s, d_residuals, n, dim, m, ksub, max_iters, tol, out);
  if (st) return st;
  return end_call(*ds, s);
}

int tac_pq_train_encode_device(const float *d_residuals, uint64_t n, uint32_t dim, uint32_t m,
                               uint32_t ksub, const float *d_init_codebooks, uint64_t seed,
                               uint32_t max_iters, float tol, float *d_codebooks_out,
                               void *d_codes_out, tac_pq_train_extras *extras, void *stream) {
  int st = validate_pq(n, dim, m, ksub);
  if (st) return st;
  if (!d_residuals || !d_codebooks_out || !d_codes_out) return TAC_ERR_INVALID_ARGUMENT;
  DeviceState *ds = nullptr;
  if ((st = acquire_device(&ds, nullptr))) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, stream, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  const size_t cb_bytes = (size_t)m * ksub * (dim / m) * sizeof(float);
  if (d_init_codebooks && d_init_codebooks != d_codebooks_out)
    HIP_TRY(hipMemcpyAsync(d_codebooks_out, d_init_codebooks, cb_bytes, hipMemcpyDeviceToDevice,
                           s));
  bool encoded = false;
  TrainOut out{d_codebooks_out, d_init_codebooks == nullptr, seed, nullptr, extras, nullptr,
               nullptr, d_codes_out, &encoded};
  st = train_core(*ds, s, d_residuals, n, dim, m, ksub, max_iters, tol, out);
  if (st) return st;
  if (!encoded &&
      (st = encode_core(*ds, s, d_residuals, n, dim, m, ksub, d_codebooks_out, d_codes_out)))
    return st;
  return end_call(*ds, s);
}

int tac_pq_train(const float *residuals, uint64_t n, uint32_t dim, uint32_t m, uint32_t ksub,
                 const float *init_codebooks, uint64_t seed, uint32_t max_iters, float tol,
                 float *codebooks_out, tac_pq_train_extras *extras) {
  int st = validate_pq(n, dim, m, ksub);
  if (st) return st;
  if (!residuals || !codebooks_out) return TAC_ERR_INVALID_ARGUMENT;
  DeviceState *ds = nullptr;
  if ((st = acquire_device(&ds, nullptr))) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, nullptr, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  const size_t x_bytes = (size_t)n * dim * sizeof(float);
  const size_t cb_bytes = (size_t)m * ksub * (dim / m) * sizeof(float);
  if ((st = ensure(*ds, ds->io_in, x_bytes)) || (st = ensure(*ds, ds->io_cb, cb_bytes))) return st;
  if ((st = upload_host(*ds, ds->io_in.ptr, residuals, x_bytes, s))) return st;
  if (init_codebooks)
    HIP_TRY(hipMemcpyAsync(ds->io_cb.ptr, init_codebooks, cb_bytes, hipMemcpyHostToDevice, s));
  TrainOut out{as<float>(ds->io_cb), init_codebooks == nullptr, seed, nullptr, extras, nullptr,
               nullptr};
  st = train_core(*ds, s, as<float>(ds->io_in), n, dim, m, ksub, max_iters, tol, out);
  if (st) return st;
  HIP_TRY(hipMemcpyAsync(codebooks_out, ds->io_cb.ptr, cb_bytes, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return end_call(*ds, s);
}

int tac_pq_encode_device(const float *d_residuals, uint64_t n, uint32_t dim, uint32_t m,
                         uint32_t ksub, const float *d_codebooks, void *d_codes_out,
                         void *stream) {
  if (m == 0 || ksub == 0) return TAC_ERR_INVALID_ARGUMENT;
  if (dim == 0 || dim % m != 0) return TAC_ERR_DIM_MISMATCH;
  if (dim / m > kMaxDsub || ksub > kMaxKsub) return TAC_ERR_UNSUPPORTED;
  if (n == 0) return TAC_OK;
  if (!d_residuals || !d_codebooks || !d_codes_out) return TAC_ERR_INVALID_ARGUMENT;
  DeviceState *ds = nullptr;
  int st = acquire_device(&ds, nullptr);
  if (st) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, stream, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  if ((st = encode_core(*ds, s, d_residuals, n, dim, m, ksub, d_codebooks, d_codes_out)))
    return st;
  return end_call(*ds, s);
}

// PQ.encode with no device allocation: the candidate encode's scratch comes
// from one static device array per GPU (see scratch_address), and rows run
// in batches that fit it.
int tac_pq_encode_device_noalloc(const float *d_residuals, uint64_t n, uint32_t dim, uint32_t m,
                                 uint32_t ksub, const float *d_codebooks, void *d_codes_out,
                                 void *stream) {
  if (m == 0 || ksub == 0) return TAC_ERR_INVALID_ARGUMENT;
  if (dim == 0 || dim % m != 0) return TAC_ERR_DIM_MISMATCH;
  if (dim / m > kMaxDsub || ksub > kMaxKsub) return TAC_ERR_UNSUPPORTED;
  if (n == 0) return TAC_OK;
  if (!d_residuals || !d_codebooks || !d_codes_out) return TAC_ERR_INVALID_ARGUMENT;
  if (device_count() <= 0) return TAC_ERR_NO_DEVICE;
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return TAC_ERR_NO_DEVICE;
  uint8_t *base = nullptr;
  int st = scratch_address(dev, &base);
  if (st) return st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);  // NULL: the null stream
  if ((st = sync_lanes(s))) return st;
  const uint32_t D = dim / m;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    uint8_t *p = base + off;
    off += (bytes + 255) & ~(size_t)255;
    return p;
  };
  // [0] exact rescans, [1] and [2] stay unused (no profiling here)
  auto *counters = reinterpret_cast<unsigned long long *>(take(3 * sizeof(unsigned long long)));
  zero_words_kernel<<<1, kWave, 0, s>>>(reinterpret_cast<uint32_t *>(counters), 6);
  LAUNCH_TRY("zero_words_kernel");
  // Sub-dimensions 5-8 with ksub <= 256: the matrix-core screen, its
  // deferred list (one word per row and subspace) and count in the scratch,
  // in batches of whole sort tiles that fit.
  if (D >= 5 && D <= 8 && screen_wanted(ksub)) {
    uint32_t *dcount = reinterpret_cast<uint32_t *>(take((size_t)m * sizeof(uint32_t)));
    const size_t left = off < kNoAllocScratchBytes ? kNoAllocScratchBytes - off : 0;
    uint64_t sb = left / (sizeof(uint32_t) * (size_t)m) / kSortTile * kSortTile;
    sb = std::min<uint64_t>(sb, 0xFFFF0000ull / kSortTile * kSortTile);
    uint32_t *dlist = reinterpret_cast<uint32_t *>(base + off);
    if (sb > 0) {
      for (uint64_t r0 = 0; r0 < n; r0 += sb) {
        const uint64_t nb = std::min<uint64_t>(sb, n - r0);
        DISPATCH_D_ST(D, encode_screen<uint8_t>(d_residuals + r0 * dim, d_codebooks,
                                                static_cast<uint8_t *>(d_codes_out) + r0 * m,
                                                dlist, dcount, nb, dim, m, ksub, counters,
                                                nullptr, s));
        if (st) return st;
        LAUNCH_TRY("screen encode");
      }
      return TAC_OK;
    }
  }
  const uint32_t L = ksub >= 2 ? std::min<uint32_t>(kCandListEncode, ksub - 1) : 0;
  bool cand = cand_wanted(D, ksub, true) && ksub >= 2 && ksub <= 256 && n >= 16384;
  uint64_t batch = 0;
  uint32_t *count = nullptr, *nbr = nullptr, *lists = nullptr;
  uint8_t *anchors = nullptr;
  float *grid = nullptr;
  if (cand) {
    count = reinterpret_cast<uint32_t *>(take((size_t)m * sizeof(uint32_t)));
    nbr = reinterpret_cast<uint32_t *>(
        take((size_t)m * ksub * cand_row_len(L) * sizeof(uint32_t)));
    anchors = take((size_t)m * kCandCells * kCandAnchorsMax);
    grid = reinterpret_cast<float *>(take((size_t)m * 16 * sizeof(float)));
    // the rest holds a batch's slices and deferred lists: 2 words per row and subspace
    const size_t left = off < kNoAllocScratchBytes ? kNoAllocScratchBytes - off : 0;
    batch = left / (2 * sizeof(uint32_t) * (size_t)m) / 8192 * 8192;
    batch = std::min<uint64_t>(batch, 0xFFFF0000ull);
    lists = reinterpret_cast<uint32_t *>(base + off);
    cand = batch >= 16384;
  }
  if (!cand) {
    if (ksub <= 256) {
      DISPATCH_D_ST(D, encode<uint8_t>(d_residuals, d_codebooks, (uint8_t *)d_codes_out, n, dim,
                                       m, ksub, counters, s));
    } else {
      DISPATCH_D_ST(D, encode<uint16_t>(d_residuals, d_codebooks, (uint16_t *)d_codes_out, n,
                                        dim, m, ksub, counters, s));
    }
    if (st) return st;
    LAUNCH_TRY("encode_kernel");
    return TAC_OK;
  }
  DISPATCH_D(D, encode_tables<uint8_t>(d_codebooks, nbr, anchors, grid, count, m, ksub, L, s));
  LAUNCH_TRY("encode tables");
  for (uint64_t r0 = 0; r0 < n; r0 += batch) {
    const uint64_t nb = std::min<uint64_t>(batch, n - r0);
    const float *x = d_residuals + r0 * dim;
    uint8_t *codes = static_cast<uint8_t *>(d_codes_out) + r0 * m;
    if (nb >= 16384) {
      if (r0) {  // the tables' launch cleared the first batch's count
        zero_words_kernel<<<1, kWave, 0, s>>>(count, m);
        LAUNCH_TRY("zero_words_kernel");
      }
      DISPATCH_D_ST(D, encode_rows<uint8_t>(x, d_codebooks, codes, nbr, anchors, grid, lists,
                                            lists + (size_t)m * nb, count, nb, dim, m, ksub, L,
                                            counters, nullptr, s));
    } else {
      DISPATCH_D_ST(D, encode<uint8_t>(x, d_codebooks, codes, nb, dim, m, ksub, counters, s));
    }
    if (st) return st;
    LAUNCH_TRY("encode_kernel");
  }
  return TAC_OK;
}

int tac_pq_encode(const float *residuals, uint64_t n, uint32_t dim, uint32_t m, uint32_t ksub,
                  const float *codebooks, void *codes_out) {
  if (m == 0 || ksub == 0) return TAC_ERR_INVALID_ARGUMENT;
  if (dim == 0 || dim % m != 0) return TAC_ERR_DIM_MISMATCH;
  if (dim / m > kMaxDsub || ksub > kMaxKsub) return TAC_ERR_UNSUPPORTED;
  if (n == 0) return TAC_OK;
  if (!residuals || !codebooks || !codes_out) return TAC_ERR_INVALID_ARGUMENT;
  DeviceState *ds = nullptr;
  int st = acquire_device(&ds, nullptr);
  if (st) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, nullptr, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  const size_t x_bytes = (size_t)n * dim * sizeof(float);
  const size_t cb_bytes = (size_t)ksub * dim * sizeof(float);
  const size_t code_bytes = (size_t)n * m * (ksub <= 256 ? 1 : 2);
  if ((st = ensure(*ds, ds->io_in, x_bytes)) || (st = ensure(*ds, ds->io_cb, cb_bytes)) ||
      (st = ensure(*ds, ds->io_out, code_bytes)))
    return st;
  if ((st = upload_host(*ds, ds->io_in.ptr, residuals, x_bytes, s))) return st;
  HIP_TRY(hipMemcpyAsync(ds->io_cb.ptr, codebooks, cb_bytes, hipMemcpyHostToDevice, s));
  if ((st = encode_core(*ds, s, as<float>(ds->io_in), n, dim, m, ksub, as<float>(ds->io_cb),
                        ds->io_out.ptr)))
    return st;
  HIP_TRY(hipMemcpyAsync(codes_out, ds->io_out.ptr, code_bytes, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return end_call(*ds, s);
}

int tac_pq_decode(const void *codes, uint64_t n, uint32_t dim, uint32_t m, uint32_t ksub,
                  const float *codebooks, float *out) {
  if (m == 0 || ksub == 0) return TAC_ERR_INVALID_ARGUMENT;
  if (dim == 0 || dim % m != 0) return TAC_ERR_DIM_MISMATCH;
  if (dim / m > kMaxDsub || ksub > kMaxKsub) return TAC_ERR_UNSUPPORTED;
  if (n == 0) return TAC_OK;
  if (!codes || !codebooks || !out) return TAC_ERR_INVALID_ARGUMENT;
  DeviceState *ds = nullptr;
  int st = acquire_device(&ds, nullptr);
  if (st) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, nullptr, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  const uint32_t D = dim / m;
  const size_t code_bytes = (size_t)n * m * (ksub <= 256 ? 1 : 2);
  const size_t cb_bytes = (size_t)ksub * dim * sizeof(float);
  const size_t out_bytes = (size_t)n * dim * sizeof(float);
  if ((st = ensure(*ds, ds->io_in, code_bytes)) || (st = ensure(*ds, ds->io_cb, cb_bytes)) ||
      (st = ensure(*ds, ds->io_out, out_bytes)))
    return st;
  HIP_TRY(hipMemcpyAsync(ds->io_in.ptr, codes, code_bytes, hipMemcpyHostToDevice, s));
  HIP_TRY(hipMemcpyAsync(ds->io_cb.ptr, codebooks, cb_bytes, hipMemcpyHostToDevice, s));
  uint32_t *status = nullptr;
  if ((st = status_begin(*ds, s, &status))) return st;
  const uint64_t total = n * dim;
  const unsigned blocks = (unsigned)((total + 255) / 256);
  if (ksub <= 256)
    decode_kernel<uint8_t><<<blocks, 256, 0, s>>>(as<uint8_t>(ds->io_in), as<float>(ds->io_cb),
                                                  as<float>(ds->io_out), status, n, m, ksub, D);
  else
    decode_kernel<uint16_t><<<blocks, 256, 0, s>>>(as<uint16_t>(ds->io_in), as<float>(ds->io_cb),
                                                   as<float>(ds->io_out), status, n, m, ksub, D);
  LAUNCH_TRY("decode_kernel");
  if ((st = status_collect(*ds, s))) return st;
  HIP_TRY(hipMemcpyAsync(out, ds->io_out.ptr, out_bytes, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return end_call(*ds, s);
}

int tac_kmeans_fit(const float *vectors, uint64_t n, uint32_t dim, uint32_t k,
                   uint32_t max_iters, float tol, uint64_t seed, const float *init_centroids,
                   float *centroids_out, uint32_t *assignments_out, float *wcss_out,
                   uint32_t *iters_run_out) {
  // src/tac/kmeans.zig:73-76
  if (k == 0) return TAC_ERR_KMEANS_BUDGET_TOO_SMALL;
  if (dim == 0) return TAC_ERR_DIM_MISMATCH;
  if (n == 0) return TAC_ERR_EMPTY_VECTOR_SET;
  // dims up to 8 run on the PQ kernels (one subspace of the whole vector);
  // wider rows, up to 512 floats, on the token-clustering engine as a single
  // problem.  Both compute vec.l2sq in the reference's form for the dim.
  const bool wide = dim > kMaxDsub;
  if ((wide ? dim > kTacMaxDim : k > kMaxKsub) || n > 0xFFFFFFFFull) return TAC_ERR_UNSUPPORTED;
  if (!vectors || !centroids_out || !assignments_out) return TAC_ERR_INVALID_ARGUMENT;
  DeviceState *ds = nullptr;
  int st = acquire_device(&ds, nullptr);
  if (st) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, nullptr, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  if (wide) {
    tac_cluster_params prm{};
    prm.kappa_total = k;
    prm.max_iters = max_iters;
    prm.tol = tol;
    prm.seed = seed;  // token 0: the problem's seed is seed ^ 0
    prm.n_threads = 1;
    uint32_t kpt = 0, iters = 0;
    float wcss = 0.0f;
    const TacFixedFit fx{k, init_centroids, &iters};
    st = tac_cluster_core(*ds, s, nullptr, n, vectors, false, dim, prm, 1, centroids_out,
                          assignments_out, &kpt, &wcss, &fx);
    if (st) return st;
    if (wcss_out) *wcss_out = wcss;
    if (iters_run_out) *iters_run_out = iters;
    return end_call(*ds, s);
  }
  const size_t x_bytes = (size_t)n * dim * sizeof(float);
  const size_t cb_bytes = (size_t)k * dim * sizeof(float);
  if ((st = ensure(*ds, ds->io_in, x_bytes)) || (st = ensure(*ds, ds->io_cb, cb_bytes)) ||
      (st = ensure(*ds, ds->io_out, (size_t)n * sizeof(uint32_t))))
    return st;
  if ((st = upload_host(*ds, ds->io_in.ptr, vectors, x_bytes, s))) return st;
  if (init_centroids)
    HIP_TRY(hipMemcpyAsync(ds->io_cb.ptr, init_centroids, cb_bytes, hipMemcpyHostToDevice, s));
  float wcss = 0.0f;
  uint32_t iters = 0;
  TrainOut out{as<float>(ds->io_cb), init_centroids == nullptr, seed, as<uint32_t>(ds->io_out),
               nullptr, &wcss, &iters};
  st = train_core(*ds, s, as<float>(ds->io_in), n, dim, 1, k, max_iters, tol, out);
  if (st) return st;
  HIP_TRY(hipMemcpyAsync(centroids_out, ds->io_cb.ptr, cb_bytes, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipMemcpyAsync(assignments_out, ds->io_out.ptr, (size_t)n * sizeof(uint32_t),
                         hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  if (wcss_out) *wcss_out = wcss;
  if (iters_run_out) *iters_run_out = iters;
  return end_call(*ds, s);
}

}  // extern "C"

// ---- storage.build stage 2: residuals and norms ----------------------------

namespace {

int validate_residuals(uint64_t n, uint32_t dim) {
  if (dim == 0) return TAC_ERR_DIM_MISMATCH;
  if (dim > 4096) return TAC_ERR_UNSUPPORTED;
  (void)n;
  return TAC_OK;
}

int residuals_core(DeviceState &ds, hipStream_t s, const float *v, uint64_t n, uint32_t dim,
                   const float *cent, uint32_t n_cent, const uint32_t *assign, float *out,
                   float *norms) {
  uint32_t *status = nullptr;
  int st = status_begin(ds, s, &status);
  if (st) return st;
  const uint32_t R = residual_rows(dim);
  const uint64_t blocks = (n + R - 1) / R;
  if (blocks > 0x7FFFFFFFull) return TAC_ERR_UNSUPPORTED;
  const size_t lds = ((size_t)R * (dim + 1) + 2 * R) * sizeof(float);
  const bool vec4 = dim % 4 == 0 && ((uintptr_t)v % 16 == 0) && ((uintptr_t)cent % 16 == 0) &&
                    ((uintptr_t)out % 16 == 0);
  const bool profile = g_profile;
  hipEvent_t a = nullptr, b = nullptr;
  if (profile) {
    if ((st = event_at(ds, 0, &a)) || (st = event_at(ds, 1, &b))) return st;
    HIP_TRY(hipEventRecord(a, s));
  }
  if (vec4)
    residual_kernel<4><<<(unsigned)blocks, kResBlock, lds, s>>>(v, cent, assign, out, norms,
                                                                status, n, dim, n_cent, R);
  else
    residual_kernel<1><<<(unsigned)blocks, kResBlock, lds, s>>>(v, cent, assign, out, norms,
                                                                status, n, dim, n_cent, R);
  LAUNCH_TRY("residual_kernel");
  if (profile) HIP_TRY(hipEventRecord(b, s));
  if ((st = status_collect(ds, s))) return st;
  if (profile) {
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, a, b));
    std::lock_guard<std::mutex> g(g_profile_mu);
    g_prof.residual_ms += ms;
    g_prof.residual_launches += 1;
  }
  return TAC_OK;
}

}  // namespace

extern "C" {

int tac_residuals_device(const float *d_vectors, uint64_t n, uint32_t dim,
                         const float *d_centroids, uint32_t n_centroids,
                         const uint32_t *d_assignments, float *d_residuals_out,
                         float *d_norms_out, void *stream) {
  int st = validate_residuals(n, dim);
  if (st) return st;
  if (n == 0) return TAC_OK;
  if (!d_vectors || !d_centroids || !d_assignments || !d_residuals_out || !d_norms_out)
    return TAC_ERR_INVALID_ARGUMENT;
  DeviceState *ds = nullptr;
  if ((st = acquire_device(&ds, nullptr))) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, stream, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  if ((st = residuals_core(*ds, s, d_vectors, n, dim, d_centroids, n_centroids, d_assignments,
                           d_residuals_out, d_norms_out)))
    return st;
  return end_call(*ds, s);
}

int tac_residuals(const float *vectors, uint64_t n, uint32_t dim, const float *centroids,
                  uint32_t n_centroids, const uint32_t *assignments, float *residuals_out,
                  float *norms_out) {
  int st = validate_residuals(n, dim);
  if (st) return st;
  if (n == 0) return TAC_OK;
  if (!vectors || !centroids || !assignments || !residuals_out || !norms_out)
    return TAC_ERR_INVALID_ARGUMENT;
  DeviceState *ds = nullptr;
  if ((st = acquire_device(&ds, nullptr))) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, nullptr, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  const size_t x_bytes = (size_t)n * dim * sizeof(float);
  const size_t c_bytes = (size_t)n_centroids * dim * sizeof(float);
  const size_t a_bytes = (size_t)n * sizeof(uint32_t);
  if ((st = ensure(*ds, ds->io_in, x_bytes)) || (st = ensure(*ds, ds->io_cb, c_bytes)) ||
      (st = ensure(*ds, ds->io_aux, a_bytes)) || (st = ensure(*ds, ds->io_out, x_bytes)) ||
      (st = ensure(*ds, ds->io_out2, (size_t)n * sizeof(float))))
    return st;
  if ((st = upload_host(*ds, ds->io_in.ptr, vectors, x_bytes, s))) return st;
  if (c_bytes)
    HIP_TRY(hipMemcpyAsync(ds->io_cb.ptr, centroids, c_bytes, hipMemcpyHostToDevice, s));
  HIP_TRY(hipMemcpyAsync(ds->io_aux.ptr, assignments, a_bytes, hipMemcpyHostToDevice, s));
  if ((st = residuals_core(*ds, s, as<float>(ds->io_in), n, dim, as<float>(ds->io_cb),
                           n_centroids, as<uint32_t>(ds->io_aux), as<float>(ds->io_out),
                           as<float>(ds->io_out2))))
    return st;
  HIP_TRY(hipMemcpyAsync(residuals_out, ds->io_out.ptr, x_bytes, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipMemcpyAsync(norms_out, ds->io_out2.ptr, (size_t)n * sizeof(float),
                         hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return end_call(*ds, s);
}

}  // extern "C"

// ---- .tac doc layouts, CRC-32, distance table, refine ----------------------

namespace {

uint64_t align8_host(uint64_t x) { return (x + 7u) & ~(uint64_t)7u; }

int doc_layouts_core(DeviceState &ds, hipStream_t s, const uint64_t *d_off, uint64_t n_docs,
                     uint64_t n_tokens, const uint32_t *d_assign, const uint8_t *d_codes,
                     uint32_t m, uint32_t cb, uint64_t *d_index, uint8_t *d_payload,
                     uint64_t payload_len, uint64_t *total_out) {
  uint32_t *status = nullptr;
  int st = status_begin(ds, s, &status);
  if (st) return st;
  if (n_docs == 0) {
    HIP_TRY(hipMemsetAsync(d_index, 0, sizeof(uint64_t), s));
    HIP_TRY(hipStreamSynchronize(s));
    *total_out = 0;
    return TAC_OK;
  }
  const uint64_t per = (uint64_t)kScanBlock * kScanPer;
  const uint64_t nb = (n_docs + per - 1) / per;
  if (nb > 0x7FFFFFFFull) return TAC_ERR_UNSUPPORTED;
  if ((st = ensure(ds, ds.scan_sums, (size_t)nb * sizeof(uint64_t)))) return st;
  uint64_t *sums = as<uint64_t>(ds.scan_sums);
  doc_sizes_scan_kernel<<<(unsigned)nb, kScanBlock, 0, s>>>(d_off, n_docs, n_tokens, m, cb,
                                                           d_index, sums, status);
  doc_sums_scan_kernel<<<1, kScanBlock, 0, s>>>(sums, (uint32_t)nb, d_index, n_docs);
  doc_scan_add_kernel<<<(unsigned)nb, kScanBlock, 0, s>>>(d_index, sums, n_docs);
  LAUNCH_TRY("doc layout scan");
  uint64_t total = 0;
  HIP_TRY(hipMemcpyAsync(&total, d_index + n_docs, sizeof(total), hipMemcpyDeviceToHost, s));
  if ((st = status_collect(ds, s))) return st;  // synchronises the stream
  *total_out = total;
  if (total > payload_len) {
    g_last_error = "payload buffer smaller than the document layouts";
    return TAC_ERR_BUFFER_TOO_SMALL;
  }
  const uint64_t waves_wanted = n_docs < (1ull << 20) ? n_docs : (1ull << 20);
  const unsigned blocks = (unsigned)((waves_wanted + 3) / 4);
  doc_write_kernel<<<blocks, 256, 0, s>>>(d_off, n_docs, d_assign, d_codes, m, cb, d_index,
                                          d_payload);
  LAUNCH_TRY("doc_write_kernel");
  HIP_TRY(hipStreamSynchronize(s));
  return TAC_OK;
}

int crc_core(DeviceState &ds, hipStream_t s, const uint8_t *d_buf, uint64_t len, uint32_t *out) {
  const uint64_t mis = (uintptr_t)d_buf % 16;
  const uint64_t head = mis ? ((16 - mis) < len ? (16 - mis) : len) : 0;
  const uint64_t leaves = (len - head) / kCrcLeaf;
  const uint64_t tail = len - head - leaves * kCrcLeaf;
  const uint64_t nb = (leaves + kCrcBlock - 1) / kCrcBlock;
  if (nb > 0x7FFFFFFFull) return TAC_ERR_UNSUPPORTED;
  int st;
  if ((st = ensure(ds, ds.scan_sums, (size_t)(nb ? nb : 1) * sizeof(CrcNode) + 16))) return st;
  CrcNode *nodes = as<CrcNode>(ds.scan_sums);
  uint32_t *d_crc = reinterpret_cast<uint32_t *>(nodes + (nb ? nb : 1));
  if (!ds.crc_tx_ready) {  // the [64][32] shift table, uploaded once per device
    static const std::vector<uint32_t> host_tx = [] {
      std::vector<uint32_t> t(kCrcTxRows * 32);
      crc_tx_host(t.data());
      return t;
    }();
    if ((st = ensure(ds, ds.crc_tx, host_tx.size() * sizeof(uint32_t)))) return st;
    HIP_TRY(hipMemcpy(ds.crc_tx.ptr, host_tx.data(), host_tx.size() * sizeof(uint32_t),
                      hipMemcpyHostToDevice));
    ds.crc_tx_ready = true;
  }
  const uint32_t *tx = as<uint32_t>(ds.crc_tx);
  const bool profile = g_profile;
  hipEvent_t a = nullptr, b = nullptr;
  if (profile) {
    if ((st = event_at(ds, 0, &a)) || (st = event_at(ds, 1, &b))) return st;
    HIP_TRY(hipEventRecord(a, s));
  }
  if (nb) crc_leaf_kernel<<<(unsigned)nb, kCrcBlock, 0, s>>>(d_buf + head, leaves, tx, nodes);
  crc_final_kernel<<<1, kCrcBlock, 0, s>>>(d_buf, head, leaves, tail, nodes, (uint32_t)nb, tx,
                                           d_crc);
  LAUNCH_TRY("crc kernels");
  if (profile) HIP_TRY(hipEventRecord(b, s));
  HIP_TRY(hipMemcpyAsync(out, d_crc, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  if (profile) {
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, a, b));
    std::lock_guard<std::mutex> g(g_profile_mu);
    g_prof.crc_ms += ms;
    g_prof.crc_launches += 1;
  }
  return TAC_OK;
}

int refine_smem(uint32_t n_q, uint32_t dim, size_t *bytes) {
  if (dim > 4096 || n_q > 65536) return TAC_ERR_UNSUPPORTED;
  const uint64_t floats = refine_lds_floats(n_q, dim);
  if (floats * sizeof(float) > 65536) return TAC_ERR_UNSUPPORTED;
  *bytes = (size_t)floats * sizeof(float);
  return TAC_OK;
}

// refine.zig:99-105 argument checks, shared by both entry points.
int validate_refine(const tac_doc_index *ix, uint64_t table_len, uint32_t n_q) {
  if (!ix) return TAC_ERR_INVALID_ARGUMENT;
  if (n_q == 0) return TAC_ERR_QUERY_SHAPE_MISMATCH;
  if (table_len != (uint64_t)ix->m * ix->ksub * n_q) return TAC_ERR_TABLE_SIZE_MISMATCH;
  if (ix->dim == 0 || ix->m == 0 || ix->ksub == 0 || ix->ksub > 65536)
    return TAC_ERR_INVALID_ARGUMENT;
  size_t smem;
  return refine_smem(n_q, ix->dim, &smem);
}

int refine_core(DeviceState &ds, hipStream_t s, const tac_doc_index &ix, const float *d_table,
                const float *d_q, uint32_t n_q, const uint32_t *d_ids, uint32_t n_cand,
                float *d_scores) {
  size_t smem = 0;
  int st = refine_smem(n_q, ix.dim, &smem);
  if (st) return st;
  if ((st = ensure(ds, ds.io_x3, (size_t)n_cand * sizeof(uint32_t) + 16))) return st;
  uint32_t *status = as<uint32_t>(ds.io_x3);
  uint32_t *first_bad = status + n_cand;
  HIP_TRY(hipMemsetAsync(first_bad, 0xFF, sizeof(uint32_t), s));
  RefineIndex r{ix.centroids, ix.doc_index, ix.doc_payload, ix.doc_token_offsets,
                ix.residual_norms, ix.n_docs, ix.n_tokens, ix.payload_len, ix.dim, ix.kappa,
                ix.m, ix.ksub};
  const uint32_t want = (n_cand + kRefineWaves - 1) / kRefineWaves;
  const unsigned blocks = want < 8192 ? want : 8192;
  const bool profile = g_profile;
  hipEvent_t ea = nullptr, eb = nullptr;
  if (profile) {
    if ((st = event_at(ds, 0, &ea)) || (st = event_at(ds, 1, &eb))) return st;
    HIP_TRY(hipEventRecord(ea, s));
  }
  refine_kernel<<<blocks, 64 * kRefineWaves, smem, s>>>(r, d_q, n_q, d_table, d_ids, n_cand,
                                                       d_scores, status, first_bad);
  LAUNCH_TRY("refine_kernel");
  if (profile) HIP_TRY(hipEventRecord(eb, s));
  uint32_t bad = 0xFFFFFFFFu;
  HIP_TRY(hipMemcpyAsync(&bad, first_bad, sizeof(bad), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  if (profile) {
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, ea, eb));
    std::lock_guard<std::mutex> g(g_profile_mu);
    g_prof.refine_ms += ms;
    g_prof.refine_launches += 1;
  }
  if (bad != 0xFFFFFFFFu) {
    uint32_t code = 0;
    HIP_TRY(hipMemcpy(&code, status + bad, sizeof(code), hipMemcpyDeviceToHost));
    g_last_error = "refine failed at candidate " + std::to_string(bad);
    return (int)code;
  }
  return TAC_OK;
}

}  // namespace

extern "C" {

int tac_doc_payload_bytes(const uint64_t *doc_offsets, uint64_t n_docs, uint32_t m,
                          uint32_t code_bytes, uint64_t *bytes_out) {
  if (!bytes_out || (n_docs && !doc_offsets) || m == 0 || (code_bytes != 1 && code_bytes != 2))
    return TAC_ERR_INVALID_ARGUMENT;
  uint64_t total = 0;
  for (uint64_t d = 0; d < n_docs; ++d) {
    if (doc_offsets[d + 1] < doc_offsets[d]) return TAC_ERR_INVALID_ARGUMENT;
    const uint64_t n_d = doc_offsets[d + 1] - doc_offsets[d];
    total += align8_host(4 + 4 * n_d + n_d * (uint64_t)m * code_bytes);
  }
  *bytes_out = total;
  return TAC_OK;
}

int tac_write_doc_layouts_device(const uint64_t *d_doc_offsets, uint64_t n_docs,
                                 uint64_t n_tokens, const uint32_t *d_assignments,
                                 const void *d_codes, uint32_t m, uint32_t code_bytes,
                                 uint64_t *d_doc_index_out, uint8_t *d_payload_out,
                                 uint64_t payload_len, void *stream) {
  if (m == 0 || (code_bytes != 1 && code_bytes != 2)) return TAC_ERR_INVALID_ARGUMENT;
  if (!d_doc_offsets || !d_doc_index_out || (n_tokens && (!d_assignments || !d_codes)) ||
      (payload_len && !d_payload_out) || ((uintptr_t)d_payload_out % 8))
    return TAC_ERR_INVALID_ARGUMENT;
  DeviceState *ds = nullptr;
  int st = acquire_device(&ds, nullptr);
  if (st) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, stream, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  uint64_t total = 0;
  if ((st = doc_layouts_core(*ds, s, d_doc_offsets, n_docs, n_tokens, d_assignments,
                             static_cast<const uint8_t *>(d_codes), m, code_bytes,
                             d_doc_index_out, d_payload_out, payload_len, &total)))
    return st;
  return end_call(*ds, s);
}

int tac_write_doc_layouts(const uint64_t *doc_offsets, uint64_t n_docs, uint64_t n_tokens,
                          const uint32_t *assignments, const void *codes, uint32_t m,
                          uint32_t code_bytes, uint64_t *doc_index_out, uint8_t *payload_out,
                          uint64_t payload_len) {
  if (m == 0 || (code_bytes != 1 && code_bytes != 2)) return TAC_ERR_INVALID_ARGUMENT;
  if (!doc_offsets || !doc_index_out || (n_tokens && (!assignments || !codes)) ||
      (payload_len && !payload_out))
    return TAC_ERR_INVALID_ARGUMENT;
  // Host-side checks first: the reference's BufferTooSmall precedes any write.
  uint64_t need = 0;
  int st = tac_doc_payload_bytes(doc_offsets, n_docs, m, code_bytes, &need);
  if (st) return st;
  if (n_docs && doc_offsets[n_docs] > n_tokens) return TAC_ERR_INVALID_ARGUMENT;
  if (need > payload_len) return TAC_ERR_BUFFER_TOO_SMALL;
  DeviceState *ds = nullptr;
  if ((st = acquire_device(&ds, nullptr))) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, nullptr, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  const size_t off_b = (size_t)(n_docs + 1) * sizeof(uint64_t);
  const size_t a_b = (size_t)n_tokens * sizeof(uint32_t);
  const size_t c_b = (size_t)n_tokens * m * code_bytes;
  if ((st = ensure(*ds, ds->io_x1, off_b)) || (st = ensure(*ds, ds->io_aux, a_b + 4)) ||
      (st = ensure(*ds, ds->io_in, c_b + 4)) || (st = ensure(*ds, ds->io_x2, off_b)) ||
      (st = ensure(*ds, ds->io_out, need + 8)))
    return st;
  HIP_TRY(hipMemcpyAsync(ds->io_x1.ptr, doc_offsets, off_b, hipMemcpyHostToDevice, s));
  if (a_b) HIP_TRY(hipMemcpyAsync(ds->io_aux.ptr, assignments, a_b, hipMemcpyHostToDevice, s));
  if (c_b) HIP_TRY(hipMemcpyAsync(ds->io_in.ptr, codes, c_b, hipMemcpyHostToDevice, s));
  uint64_t total = 0;
  if ((st = doc_layouts_core(*ds, s, as<uint64_t>(ds->io_x1), n_docs, n_tokens,
                             as<uint32_t>(ds->io_aux), as<uint8_t>(ds->io_in), m, code_bytes,
                             as<uint64_t>(ds->io_x2), as<uint8_t>(ds->io_out), need + 8, &total)))
    return st;
  HIP_TRY(hipMemcpyAsync(doc_index_out, ds->io_x2.ptr, off_b, hipMemcpyDeviceToHost, s));
  if (total) HIP_TRY(hipMemcpyAsync(payload_out, ds->io_out.ptr, total, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return end_call(*ds, s);
}

int tac_crc32_device(const void *d_bytes, uint64_t len, uint32_t *crc_out, void *stream) {
  if (!crc_out || (len && !d_bytes)) return TAC_ERR_INVALID_ARGUMENT;
  if (len == 0) {
    *crc_out = 0;
    return TAC_OK;
  }
  DeviceState *ds = nullptr;
  int st = acquire_device(&ds, nullptr);
  if (st) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, stream, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  if ((st = crc_core(*ds, s, static_cast<const uint8_t *>(d_bytes), len, crc_out))) return st;
  return end_call(*ds, s);
}

int tac_crc32(const void *bytes, uint64_t len, uint32_t *crc_out) {
  if (!crc_out || (len && !bytes)) return TAC_ERR_INVALID_ARGUMENT;
  if (len == 0) {
    *crc_out = 0;
    return TAC_OK;
  }
  DeviceState *ds = nullptr;
  int st = acquire_device(&ds, nullptr);
  if (st) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, nullptr, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  if ((st = ensure(*ds, ds->io_in, len))) return st;
  HIP_TRY(hipMemcpyAsync(ds->io_in.ptr, bytes, len, hipMemcpyHostToDevice, s));
  if ((st = crc_core(*ds, s, as<uint8_t>(ds->io_in), len, crc_out))) return st;
  return end_call(*ds, s);
}

int tac_pq_distance_table_device(const float *d_query_tokens, uint32_t n_q, uint32_t dim,
                                 uint32_t m, uint32_t ksub, const float *d_codebooks,
                                 float *d_table_out, uint64_t table_len, void *stream) {
  if (m == 0 || ksub == 0) return TAC_ERR_INVALID_ARGUMENT;
  if (n_q == 0) return TAC_ERR_NQ_MISMATCH;  // pq.zig:99
  if (dim == 0 || dim % m != 0) return TAC_ERR_DIM_MISMATCH;
  if (table_len != (uint64_t)m * ksub * n_q) return TAC_ERR_OUT_BUFFER_WRONG_SIZE;  // :106
  if (!d_query_tokens || !d_codebooks || !d_table_out) return TAC_ERR_INVALID_ARGUMENT;
  DeviceState *ds = nullptr;
  int st = acquire_device(&ds, nullptr);
  if (st) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, stream, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  const uint64_t blocks = (table_len + 255) / 256;
  if (blocks > 0x7FFFFFFFull) return TAC_ERR_UNSUPPORTED;
  distance_table_kernel<<<(unsigned)blocks, 256, 0, s>>>(d_query_tokens, d_codebooks,
                                                          d_table_out, n_q, dim, m, ksub,
                                                          dim / m);
  LAUNCH_TRY("distance_table_kernel");
  return end_call(*ds, s);
}

int tac_pq_distance_table(const float *query_tokens, uint32_t n_q, uint32_t dim, uint32_t m,
                          uint32_t ksub, const float *codebooks, float *table_out,
                          uint64_t table_len) {
  if (m == 0 || ksub == 0) return TAC_ERR_INVALID_ARGUMENT;
  if (n_q == 0) return TAC_ERR_NQ_MISMATCH;
  if (dim == 0 || dim % m != 0) return TAC_ERR_DIM_MISMATCH;
  if (table_len != (uint64_t)m * ksub * n_q) return TAC_ERR_OUT_BUFFER_WRONG_SIZE;
  if (!query_tokens || !codebooks || !table_out) return TAC_ERR_INVALID_ARGUMENT;
  DeviceState *ds = nullptr;
  int st = acquire_device(&ds, nullptr);
  if (st) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, nullptr, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  const size_t q_b = (size_t)n_q * dim * sizeof(float);
  const size_t c_b = (size_t)ksub * dim * sizeof(float);
  const size_t t_b = (size_t)table_len * sizeof(float);
  if ((st = ensure(*ds, ds->io_in, q_b)) || (st = ensure(*ds, ds->io_cb, c_b)) ||
      (st = ensure(*ds, ds->io_out, t_b)))
    return st;
  HIP_TRY(hipMemcpyAsync(ds->io_in.ptr, query_tokens, q_b, hipMemcpyHostToDevice, s));
  HIP_TRY(hipMemcpyAsync(ds->io_cb.ptr, codebooks, c_b, hipMemcpyHostToDevice, s));
  distance_table_kernel<<<(unsigned)((table_len + 255) / 256), 256, 0, s>>>(
      as<float>(ds->io_in), as<float>(ds->io_cb), as<float>(ds->io_out), n_q, dim, m, ksub,
      dim / m);
  LAUNCH_TRY("distance_table_kernel");
  HIP_TRY(hipMemcpyAsync(table_out, ds->io_out.ptr, t_b, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return end_call(*ds, s);
}

int tac_refine_device(const tac_doc_index *d_index, const float *d_table, uint64_t table_len,
                      const float *d_query_tokens, uint32_t n_q, const uint32_t *d_doc_ids,
                      uint32_t n_candidates, float *d_scores_out, void *stream) {
  int st = validate_refine(d_index, table_len, n_q);
  if (st) return st;
  if (n_candidates == 0) return TAC_OK;
  const tac_doc_index &ix = *d_index;
  if (!d_table || !d_query_tokens || !d_doc_ids || !d_scores_out || !ix.centroids ||
      !ix.doc_index || !ix.doc_token_offsets || (ix.payload_len && !ix.doc_payload) ||
      (ix.n_tokens && !ix.residual_norms))
    return TAC_ERR_INVALID_ARGUMENT;
  DeviceState *ds = nullptr;
  if ((st = acquire_device(&ds, nullptr))) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, stream, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  if ((st = refine_core(*ds, s, ix, d_table, d_query_tokens, n_q, d_doc_ids, n_candidates,
                        d_scores_out)))
    return st;
  return end_call(*ds, s);
}

int tac_refine(const tac_doc_index *index, const float *table, uint64_t table_len,
               const float *query_tokens, uint32_t n_q, const uint32_t *doc_ids,
               uint32_t n_candidates, float *scores_out) {
  int st = validate_refine(index, table_len, n_q);
  if (st) return st;
  if (n_candidates == 0) return TAC_OK;
  const tac_doc_index &h = *index;
  if (!table || !query_tokens || !doc_ids || !scores_out || !h.centroids || !h.doc_index ||
      !h.doc_token_offsets || (h.payload_len && !h.doc_payload) ||
      (h.n_tokens && !h.residual_norms))
    return TAC_ERR_INVALID_ARGUMENT;
  DeviceState *ds = nullptr;
  if ((st = acquire_device(&ds, nullptr))) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, nullptr, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  // One staging allocation, 256-byte aligned pieces.
  const size_t pieces[] = {(size_t)h.kappa * h.dim * sizeof(float),
                           (size_t)(h.n_docs + 1) * sizeof(uint64_t),
                           (size_t)h.payload_len,
                           (size_t)(h.n_docs + 1) * sizeof(uint64_t),
                           (size_t)h.n_tokens * sizeof(float),
                           (size_t)table_len * sizeof(float),
                           (size_t)n_q * h.dim * sizeof(float),
                           (size_t)n_candidates * sizeof(uint32_t),
                           (size_t)n_candidates * sizeof(float)};
  const void *srcs[] = {h.centroids, h.doc_index, h.doc_payload, h.doc_token_offsets,
                        h.residual_norms, table, query_tokens, doc_ids, nullptr};
  size_t offs[9], total = 0;
  for (int i = 0; i < 9; ++i) {
    offs[i] = total;
    total += (pieces[i] + 255) & ~size_t(255);
  }
  if ((st = ensure(*ds, ds->io_x1, total + 256))) return st;
  uint8_t *base = as<uint8_t>(ds->io_x1);
  for (int i = 0; i < 8; ++i)
    if (pieces[i]) HIP_TRY(hipMemcpyAsync(base + offs[i], srcs[i], pieces[i], hipMemcpyHostToDevice, s));
  tac_doc_index d = h;
  d.centroids = reinterpret_cast<const float *>(base + offs[0]);
  d.doc_index = reinterpret_cast<const uint64_t *>(base + offs[1]);
  d.doc_payload = base + offs[2];
  d.doc_token_offsets = reinterpret_cast<const uint64_t *>(base + offs[3]);
  d.residual_norms = reinterpret_cast<const float *>(base + offs[4]);
  float *d_scores = reinterpret_cast<float *>(base + offs[8]);
  if ((st = refine_core(*ds, s, d, reinterpret_cast<const float *>(base + offs[5]),
                        reinterpret_cast<const float *>(base + offs[6]), n_q,
                        reinterpret_cast<const uint32_t *>(base + offs[7]), n_candidates,
                        d_scores)))
    return st;
  HIP_TRY(hipMemcpyAsync(scores_out, d_scores, pieces[8], hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return end_call(*ds, s);
}

}  // extern "C"

// ---- token-aware clustering (src/tac/tac.zig:563-830) -------------------------

namespace {

template <typename T>
int upload_vec(DeviceState &ds, Buffer &b, const std::vector<T> &v, hipStream_t s) {
  const size_t bytes = (v.empty() ? 1 : v.size()) * sizeof(T);
  if (int st = ensure(ds, b, bytes)) return st;
  if (!v.empty())
    HIP_TRY(hipMemcpyAsync(b.ptr, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice, s));
  return TAC_OK;
}

// The batch of per-token fits: problems ordered by k descending (degenerate
// problems, which skip seeding, last), their tiles and wcss chunks.
struct TacPlan {
  std::vector<TacProblem> probs;
  std::vector<TacTile> tiles;
  std::vector<TacChunk> chunks;
  std::vector<TacRange> ranges;      // scan ranges of the tile histograms
  std::vector<uint32_t> cprob;       // problem of every centroid
  std::vector<uint32_t> token;       // token id of every problem
  std::vector<uint32_t> tiles_upto;  // [c]: tiles of problems still seeding in round c
  std::vector<uint32_t> probs_upto;  // [c]: problems with more than c seeds
  uint64_t hist_total = 0;
  uint64_t rsum_total = 0;
  uint32_t kmax = 0;      // largest k of a non-degenerate problem
  void reset() {  // empty, keeping the lists' capacity
    probs.clear();
    tiles.clear();
    chunks.clear();
    ranges.clear();
    cprob.clear();
    token.clear();
    tiles_upto.clear();
    probs_upto.clear();
    hist_total = rsum_total = 0;
    kmax = 0;
  }
};

int tac_plan(const std::vector<uint32_t> &freqs, const std::vector<uint32_t> &offs,
             const std::vector<uint32_t> &kappa, const std::vector<uint64_t> &goff,
             uint64_t seed, uint32_t rt, uint64_t kappa_total, TacPlan *pl) {
  // Problems in order of effective k (0 for degenerate ones), descending,
  // ties in token order: a stable counting sort over the tokens in id order.
  pl->reset();
  const uint32_t nd = (uint32_t)freqs.size();
  auto keff = [&](uint32_t j) { return kappa[j] >= freqs[j] ? 0u : kappa[j]; };
  size_t P = 0;
  uint32_t kx = 0;
  for (uint32_t j = 0; j < nd; ++j) {
    if (kappa[j] == 0 || freqs[j] == 0) continue;
    ++P;
    kx = std::max(kx, keff(j));
  }
  std::vector<uint32_t> slot((size_t)kx + 2, 0);  // bucket kx - keff, descending k
  for (uint32_t j = 0; j < nd; ++j)
    if (kappa[j] != 0 && freqs[j] != 0) ++slot[kx - keff(j) + 1];
  for (size_t b = 1; b < slot.size(); ++b) slot[b] += slot[b - 1];
  pl->probs.assign(P, TacProblem{});
  pl->token.assign(P, 0u);
  size_t n_tiles = 0, n_chunks = 0, n_ranges = 0;
  for (uint32_t j = 0; j < nd; ++j) {
    if (kappa[j] == 0 || freqs[j] == 0) continue;
    const uint32_t q = slot[kx - keff(j)]++;
    TacProblem &p = pl->probs[q];
    p.off = offs[j];
    p.n = freqs[j];
    p.k = kappa[j];
    p.goff = (uint32_t)goff[j];
    p.seed = seed ^ (uint64_t)j;
    p.degenerate = p.k >= p.n ? 1u : 0u;
    pl->token[q] = j;
    const size_t nt = (p.n + rt - 1) / rt;
    n_tiles += nt;
    n_chunks += (p.n + kFoldChunk - 1) / kFoldChunk;
    n_ranges += (nt + kTacScanTiles - 1) / kTacScanTiles;
  }
  pl->tiles.reserve(n_tiles);
  pl->chunks.reserve(n_chunks);
  pl->ranges.reserve(n_ranges);
  pl->cprob.assign(kappa_total, 0);
  uint32_t t0 = 0, c0 = 0;
  for (uint32_t q = 0; q < (uint32_t)P; ++q) {
    TacProblem &p = pl->probs[q];
    p.tile0 = t0;
    p.ntiles = (p.n + rt - 1) / rt;
    p.chunk0 = c0;
    p.nchunks = (p.n + kFoldChunk - 1) / kFoldChunk;
    p.code_bits = p.k <= 1 ? 0u : 32u - (uint32_t)__builtin_clz(p.k - 1);
    p.hist0 = pl->hist_total;
    p.range0 = (uint32_t)pl->ranges.size();
    p.nranges = (p.ntiles + kTacScanTiles - 1) / kTacScanTiles;
    p.rsum0 = pl->rsum_total;
    if (!p.degenerate) {
      pl->hist_total += (uint64_t)p.ntiles * p.k;
      pl->rsum_total += (uint64_t)p.nranges * p.k;
      if (p.k > pl->kmax) pl->kmax = p.k;
    }
    for (uint32_t r = 0; r < p.nranges; ++r) pl->ranges.push_back(TacRange{q, r});
    for (uint32_t t = 0; t < p.ntiles; ++t) pl->tiles.push_back(TacTile{q, t * rt});
    for (uint32_t j = 0; j < p.nchunks; ++j) pl->chunks.push_back(TacChunk{q, j});
    for (uint32_t c = 0; c < p.k; ++c) pl->cprob[(uint64_t)p.goff + c] = q;
    t0 += p.ntiles;
    c0 += p.nchunks;
  }
  // prefixes for the k-means++ rounds (k descending)
  pl->tiles_upto.assign((size_t)pl->kmax + 1, 0);
  pl->probs_upto.assign((size_t)pl->kmax + 1, 0);
  for (uint32_t q = 0; q < (uint32_t)P; ++q) {
    const TacProblem &p = pl->probs[q];
    if (p.degenerate) break;
    for (uint32_t c = 0; c < p.k && c <= pl->kmax; ++c) {
      pl->tiles_upto[c] = p.tile0 + p.ntiles;
      pl->probs_upto[c] = q + 1;
    }
  }
  return TAC_OK;
}

int tac_cluster_core(DeviceState &ds, hipStream_t s, const uint32_t *ids, uint64_t N,
                     const float *vectors, bool vectors_on_device, uint32_t dim,
                     const tac_cluster_params &prm, uint64_t nd, float *cent_out,
                     uint32_t *assign_out, uint32_t *kpt_out, float *wcss_out,
                     const TacFixedFit *fixed) {
  const auto wall0 = std::chrono::steady_clock::now();
  const uint32_t rt = tac_rows_per_tile(dim);
  if (rt < 64 || dim > kTacMaxDim) return TAC_ERR_UNSUPPORTED;
  const uint32_t per = (dim + 63) / 64;  // dimensions per lane in the wave kernels
  // 32-bit row ids; the gather grid stays below 2^31 blocks
  if (N > 0xFFFFFFFFull || (uint64_t)N * dim > (1ull << 38) || nd > 0x7FFFFFFFull)
    return TAC_ERR_UNSUPPORTED;
  int st;
  // CSR grouping by token id, ascending input order inside a token (tac.zig:575-602).
  // The call's large host lists live in per-thread caches that keep their
  // capacity, so repeated calls do not fault in fresh pages for them.
  static thread_local std::vector<uint32_t> idx_cache, cnt_cache;
  static thread_local std::vector<uint64_t> goff_cache;
  static thread_local std::vector<KppState> hst_cache;
  static thread_local std::vector<KppTile> ktiles_cache;
  static thread_local TacPlan plan_cache;
  std::vector<uint32_t> freqs(nd, 0), offs(nd + 1, 0);
  std::vector<uint32_t> &idx = idx_cache;
  idx.resize(N);
  auto group = [&] {
    if (fixed) {  // one token: the rows in input order
      freqs[0] = (uint32_t)N;
      offs[1] = (uint32_t)N;
      for (uint64_t i = 0; i < N; ++i) idx[i] = (uint32_t)i;
      return;
    }
    for (uint64_t i = 0; i < N; ++i) freqs[ids[i]] += 1;
    for (uint64_t j = 0; j < nd; ++j) offs[j + 1] = offs[j] + freqs[j];
    std::vector<uint32_t> cur(offs.begin(), offs.end() - 1);
    for (uint64_t i = 0; i < N; ++i) idx[cur[ids[i]]++] = (uint32_t)i;
  };
  // The same grouping on T host threads, each over a contiguous slice of the
  // rows: per-slice counts, then each slice's run of token j placed after the
  // runs of the slices before it, so the order inside a token stays the
  // input order and idx, offs and freqs equal the one-thread result.
  auto group_threads = [&](uint32_t T) {
    std::vector<uint32_t> &cnt = cnt_cache;
    cnt.assign((size_t)T * nd, 0u);
    auto each = [&](auto fn) {
      std::vector<std::thread> th;
      for (uint32_t t = 1; t < T; ++t) th.emplace_back(fn, t);
      fn(0u);
      for (auto &x : th) x.join();
    };
    each([&](uint32_t t) {
      uint32_t *c = cnt.data() + (size_t)t * nd;
      for (uint64_t i = N * t / T, e = N * (t + 1) / T; i < e; ++i) c[ids[i]] += 1;
    });
    uint32_t at = 0;
    for (uint64_t j = 0; j < nd; ++j) {
      offs[j] = at;
      for (uint32_t t = 0; t < T; ++t) {
        const uint32_t v = cnt[(size_t)t * nd + j];
        cnt[(size_t)t * nd + j] = at;
        at += v;
      }
      freqs[j] = at - offs[j];
    }
    offs[nd] = at;
    each([&](uint32_t t) {
      uint32_t *c = cnt.data() + (size_t)t * nd;
      for (uint64_t i = N * t / T, e = N * (t + 1) / T; i < e; ++i) idx[c[ids[i]]++] = (uint32_t)i;
    });
  };
  const size_t vbytes = (size_t)N * dim * sizeof(float);
  // G carries tac_spread_pad_floats of slack: the spread kernel's full-batch
  // loads run up to one batch past a token's last row, and the fold kernel's
  // lanes past dim up to 64 * per floats past a row
  const size_t gbytes = vbytes + tac_spread_pad_floats(dim) * sizeof(float);
  if ((!vectors_on_device && (st = ensure(ds, ds.tac_v, vbytes))) ||
      (st = ensure(ds, ds.tac_G, gbytes)))
    return st;
  // Early spreads of the largest tokens (64-float rows): on the second
  // stream the ids go up, the kTacPreSlots tokens with the most rows (at
  // least pre_min) take slots, and as the rows arrive (each staged chunk of a
  // host upload, or all at once when they are resident) those tokens' rows
  // are copied into G and their Welford chains advance, beside the upload
  // and the host grouping.  The main gather waits for the second stream.
  // TAC_GPU_TAC_PRESPREAD=0 turns it off; TAC_GPU_TAC_PRESPREAD_MIN sets
  // pre_min (16,384 rows).
  const char *pre_env = getenv("TAC_GPU_TAC_PRESPREAD");
  const char *pre_min_env = getenv("TAC_GPU_TAC_PRESPREAD_MIN");
  const uint32_t pre_min = pre_min_env ? (uint32_t)std::max(1, atoi(pre_min_env)) : 16384u;
  // (resident rows need 16-byte alignment: the copies move 16-byte pieces)
  const bool early = dim == 64 && !fixed && nd <= (1ull << 17) && N >= pre_min &&
                     (vectors_on_device ? ((uintptr_t)vectors & 15u) == 0 : vbytes >= kStageMin) &&
                     !(pre_env && pre_env[0] == '0');
  hipStream_t s2 = nullptr;
  TacPreSlot *slots = nullptr;
  uint64_t pre_rows = 0;  // input rows the slots have been advanced over
  if (early) {
    const uint64_t ninv_pre = N + kTacSpreadSlackRows;  // covers any token's rows
    if ((st = ensure(ds, ds.tac_ids, N * sizeof(uint32_t))) ||
        (st = ensure(ds, ds.tac_pcnt, (nd + kTacPreMaxSegs * kTacPreSlots) * sizeof(uint32_t))) ||
        (st = ensure(ds, ds.tac_pslots, kTacPreSlots * sizeof(TacPreSlot))) ||
        (st = ensure(ds, ds.tac_inv, ninv_pre * sizeof(float))))
      return st;
    if (!ds.aux_stream[0])
      HIP_TRY(hipStreamCreateWithFlags(&ds.aux_stream[0], hipStreamNonBlocking));
    if (!ds.aux_fork) HIP_TRY(hipEventCreateWithFlags(&ds.aux_fork, hipEventDisableTiming));
    if (!ds.aux_join[0]) HIP_TRY(hipEventCreateWithFlags(&ds.aux_join[0], hipEventDisableTiming));
    for (hipEvent_t &ev : ds.tac_pre_ev)
      if (!ev) HIP_TRY(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    s2 = ds.aux_stream[0];
    slots = as<TacPreSlot>(ds.tac_pslots);
    HIP_TRY(hipEventRecord(ds.aux_fork, s));
    HIP_TRY(hipStreamWaitEvent(s2, ds.aux_fork, 0));
    HIP_TRY(hipMemcpyAsync(ds.tac_ids.ptr, ids, N * sizeof(uint32_t), hipMemcpyHostToDevice, s2));
    HIP_TRY(hipMemsetAsync(ds.tac_pcnt.ptr, 0, nd * sizeof(uint32_t), s2));
    const dim3 hgrid((unsigned)std::min<uint64_t>((N + 16383) / 16384, 128),
                     (unsigned)((nd + kTacHistTile - 1) / kTacHistTile));
    tac_id_hist_kernel<<<hgrid, 1024, 0, s2>>>(as<uint32_t>(ds.tac_ids), N, (uint32_t)nd,
                                              as<uint32_t>(ds.tac_pcnt));
    LAUNCH_TRY("tac_id_hist_kernel");
    tac_pre_select_kernel<<<1, 1024, 0, s2>>>(as<uint32_t>(ds.tac_pcnt), (uint32_t)nd, pre_min,
                                              slots);
    LAUNCH_TRY("tac_pre_select_kernel");
    tac_inv_table_kernel<<<(unsigned)std::min<uint64_t>((ninv_pre + 255) / 256, 1u << 20), 256, 0,
                           s2>>>(as<float>(ds.tac_inv), ninv_pre);
    LAUNCH_TRY("tac_inv_table_kernel");
  }
  // advance the slots over input rows [pre_rows, r1) of rows (on the device),
  // in pieces of kTacPreMaxSegs segments: count, copy, fold
  auto pre_advance = [&](const float *rows, uint64_t r1) -> int {
    constexpr uint64_t piece = (uint64_t)kTacPreSeg * kTacPreMaxSegs;
    uint32_t *segcnt = as<uint32_t>(ds.tac_pcnt) + nd;  // past the id counts
    const uint32_t *dids = as<uint32_t>(ds.tac_ids);
    for (; pre_rows < r1;) {
      const uint64_t e = std::min<uint64_t>(r1, pre_rows + piece);
      const uint32_t a = (uint32_t)pre_rows, b = (uint32_t)e;
      const uint32_t nseg = (uint32_t)((e - pre_rows + kTacPreSeg - 1) / kTacPreSeg);
      tac_pre_count_kernel<<<nseg, 256, 0, s2>>>(dids, a, b, slots, segcnt);
      LAUNCH_TRY("tac_pre_count_kernel");
      tac_pre_copy_kernel<<<nseg, 256, 0, s2>>>(rows, dids, a, b, slots, segcnt,
                                                as<float>(ds.tac_G));
      LAUNCH_TRY("tac_pre_copy_kernel");
      tac_spread64_kernel<<<kTacPreSlots, kTacSpread64Threads, 0, s2>>>(
          as<float>(ds.tac_G), nullptr, as<float>(ds.tac_inv), nullptr, 0, slots, 1u, segcnt,
          nseg);
      LAUNCH_TRY("tac_spread64_kernel (resume)");
      pre_rows = e;
    }
    return TAC_OK;
  };
  // Host upload: after the last staged chunk of each piece of rows (the
  // callback runs in chunk order) an event goes on the upload stream, and a
  // launcher thread makes the second stream wait for it and advances the
  // slots, so the upload threads make one extra call per piece.  Re-recording
  // one of the 16 ring events before its wait is issued only makes that wait
  // later.
  constexpr uint64_t kPrePieceRows = (uint64_t)kTacPreSeg * kTacPreMaxSegs;
  uint32_t pre_chunk = 0;
  uint64_t pre_mark = 0;  // rows covered by the pieces handed over so far
  std::mutex pre_mu;
  std::condition_variable pre_cv;
  std::deque<std::pair<hipEvent_t, uint64_t>> pre_q;
  bool pre_end = false;
  int pre_st = TAC_OK;
  const std::function<int(size_t)> after_chunk = [&](size_t end) -> int {
    const uint64_t r1 = end / ((size_t)dim * sizeof(float));
    if (r1 < pre_mark + kPrePieceRows && end < vbytes) return TAC_OK;
    pre_mark = r1;
    hipEvent_t ev = ds.tac_pre_ev[pre_chunk++ % 16u];
    HIP_TRY(hipEventRecord(ev, s));
    {
      std::lock_guard<std::mutex> g(pre_mu);
      pre_q.emplace_back(ev, r1);
    }
    pre_cv.notify_one();
    return TAC_OK;
  };
  auto launcher = [&] {
    for (;;) {
      std::pair<hipEvent_t, uint64_t> item;
      {
        std::unique_lock<std::mutex> g(pre_mu);
        pre_cv.wait(g, [&] { return pre_end || !pre_q.empty(); });
        if (pre_q.empty()) return;  // pre_end
        item = pre_q.front();
        pre_q.pop_front();
      }
      if (pre_st != TAC_OK) continue;  // drain after a failure
      const hipError_t e = hipStreamWaitEvent(s2, item.first, 0);
      pre_st = e != hipSuccess ? hip_status("hipStreamWaitEvent", e)
                               : pre_advance(as<float>(ds.tac_v), item.second);
    }
  };
  // Host vectors go up once (the grouping runs on a second thread meanwhile,
  // the copy from pageable memory holding this one); device-resident ones
  // are gathered in place.
  const float *dv = vectors;
  if (!vectors_on_device) {
    std::thread grouper(group);
    std::thread pre_launcher;
    if (early) pre_launcher = std::thread(launcher);
    const int up =
        upload_host(ds, ds.tac_v.ptr, vectors, vbytes, s, early ? &after_chunk : nullptr);
    if (early) {
      {
        std::lock_guard<std::mutex> g(pre_mu);
        pre_end = true;
      }
      pre_cv.notify_one();
      pre_launcher.join();
    }
    grouper.join();
    if (up) return up;
    if (pre_st) return pre_st;
    dv = as<float>(ds.tac_v);
  } else {
    if (early && (st = pre_advance(vectors, N))) return st;
    // Nothing to overlap with here: the grouping runs on up to 8 threads when
    // the rows are many and the per-thread counts stay small.
    const uint32_t hc = std::thread::hardware_concurrency();
    const uint32_t T = std::max<uint32_t>(1u, std::min<uint32_t>(8u, hc));
    if (!fixed && T > 1 && N >= (1u << 16) && (uint64_t)nd * T <= (1ull << 24))
      group_threads(T);
    else
      group();
  }
  if ((st = upload_vec(ds, ds.tac_idx, idx, s)) || (st = upload_vec(ds, ds.tac_offs, offs, s)) ||
      (st = ensure(ds, ds.tac_spreads, nd * sizeof(float))))
    return st;
  float *G = as<float>(ds.tac_G);
  const uint64_t nf = (uint64_t)N * dim;
  if (early) {  // the early spreads are done with G before the gather fills it
    HIP_TRY(hipEventRecord(ds.aux_join[0], s2));
    HIP_TRY(hipStreamWaitEvent(s, ds.aux_join[0], 0));
  }
  // Grids stay far below a dispatch's 2^32 work-items: the gather and the
  // reciprocal table are grid-stride loops, the spreads run in token slices.
  constexpr uint64_t kMaxBlocks = 1ull << 20;
  tac_gather_kernel<<<(unsigned)std::min<uint64_t>((nf + 255) / 256, kMaxBlocks), 256, 0, s>>>(
      dv, as<uint32_t>(ds.tac_idx), G, N, dim);
  LAUNCH_TRY("tac_gather_kernel");
  uint32_t max_n = 0;
  for (uint64_t j = 0; j < nd; ++j) max_n = freqs[j] > max_n ? freqs[j] : max_n;
  const uint64_t ninv = (uint64_t)max_n + kTacSpreadSlackRows;  // slack, as for G
  if ((st = ensure(ds, ds.tac_inv, (size_t)ninv * sizeof(float)))) return st;
  tac_inv_table_kernel<<<(unsigned)std::min<uint64_t>((ninv + 255) / 256, kMaxBlocks), 256, 0,
                         s>>>(as<float>(ds.tac_inv), ninv);
  LAUNCH_TRY("tac_inv_table_kernel");
  if (!fixed) {  // a fixed problem needs no spreads: its k is given
    const uint32_t *doffs = as<uint32_t>(ds.tac_offs);
    const float *dinv = as<float>(ds.tac_inv);
    float *dsp = as<float>(ds.tac_spreads);
    const size_t lds = dim * sizeof(float);
    constexpr uint64_t kSlice = 1ull << 24;  // tokens per launch (2^30 work-items)
    for (uint64_t j0 = 0; j0 < nd; j0 += kSlice) {
      const unsigned nb = (unsigned)std::min<uint64_t>(nd - j0, kSlice);
#define TAC_SPREAD(P) tac_spread_kernel<P><<<nb, kWave, lds, s>>>(G, doffs, dinv, dim, dsp, j0)
      if (dim == 64) {
        tac_spread64_kernel<<<nb, kTacSpread64Threads, 0, s>>>(G, doffs, dinv, dsp, j0, slots,
                                                               0u);
      } else {
        switch (per) {  // dim <= kTacMaxDim: at most 8 dimensions per lane
          case 1: TAC_SPREAD(1); break;
          case 2: TAC_SPREAD(2); break;
          case 3: TAC_SPREAD(3); break;
          case 4: TAC_SPREAD(4); break;
          case 5: TAC_SPREAD(5); break;
          case 6: TAC_SPREAD(6); break;
          case 7: TAC_SPREAD(7); break;
          default: TAC_SPREAD(8); break;
        }
      }
#undef TAC_SPREAD
      LAUNCH_TRY("tac_spread_kernel");
    }
  }
  std::vector<uint32_t> kappa(nd, 0);
  if (fixed) {
    kappa[0] = fixed->k;
  } else {
    std::vector<float> spreads(nd);
    HIP_TRY(hipMemcpyAsync(spreads.data(), ds.tac_spreads.ptr, nd * sizeof(float),
                           hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));

    // budgets (tac.zig:641-668)
    const tacphase::Params pp{prm.kappa_total, prm.mu, prm.tau, prm.epsilon, prm.theta};
    if ((st = tacphase::allocate(freqs, spreads, kappa, pp))) return st;
  }
  for (uint64_t j = 0; j < nd; ++j)
    if (freqs[j] > 0 && kappa[j] == 0) return TAC_ERR_BUDGET_TOO_SMALL;
  std::vector<uint64_t> &goff = goff_cache;
  goff.assign(nd + 1, 0);
  for (uint64_t j = 0; j < nd; ++j) goff[j + 1] = goff[j] + kappa[j];
  if (goff[nd] != prm.kappa_total) return TAC_ERR_BUDGET_TOO_SMALL;
  const uint64_t K = prm.kappa_total;

  TacPlan &pl = plan_cache;
  if ((st = tac_plan(freqs, offs, kappa, goff, prm.seed, rt, K, &pl))) return st;

  // The Lloyd kernels launch one block of at most 256 work-items per tile,
  // problem, chunk or scan range; a dispatch's grid holds under 2^32.
  constexpr uint64_t kMaxUnits = (1ull << 32) / 256;
  if (pl.tiles.size() >= kMaxUnits || pl.probs.size() >= kMaxUnits ||
      pl.ranges.size() >= kMaxUnits || pl.chunks.size() >= kMaxUnits)
    return TAC_ERR_UNSUPPORTED;
  const uint32_t P = (uint32_t)pl.probs.size();
  const uint32_t NT = (uint32_t)pl.tiles.size(), NCH = (uint32_t)pl.chunks.size();
  std::vector<uint32_t> done0(P);
  for (uint32_t q = 0; q < P; ++q) done0[q] = pl.probs[q].degenerate;
  // the tiles of the k-means++ rounds (problems in k-descending order, so
  // round c covers the first tiles_upto[c])
  std::vector<KppTile> &ktiles = ktiles_cache;
  ktiles.assign(std::max<uint32_t>(pl.tiles_upto.empty() ? 0u : pl.tiles_upto[0], 1u), KppTile{});
  for (uint32_t b = 0; b < (pl.tiles_upto.empty() ? 0u : pl.tiles_upto[0]); ++b) {
    const TacTile &tl = pl.tiles[b];
    const TacProblem &pq = pl.probs[tl.prob];
    ktiles[b] = KppTile{tl.prob, tl.row0, pq.off, pq.n, pq.goff, pq.tile0, pq.ntiles, 0u};
  }
  if ((st = upload_vec(ds, ds.tac_probs, pl.probs, s)) ||
      (st = upload_vec(ds, ds.tac_tiles, pl.tiles, s)) ||
      (st = upload_vec(ds, ds.tac_ktiles, ktiles, s)) ||
      (st = upload_vec(ds, ds.tac_chl, pl.chunks, s)) ||
      (st = upload_vec(ds, ds.tac_ranges, pl.ranges, s)) ||
      (st = ensure(ds, ds.tac_rsum, (pl.rsum_total + 1) * sizeof(uint32_t))) ||
      (st = upload_vec(ds, ds.tac_cprob, pl.cprob, s)) ||
      (st = upload_vec(ds, ds.tac_done, done0, s)) ||
      (st = ensure(ds, ds.tac_w, 2 * N * sizeof(float))) ||
      (st = ensure(ds, ds.tac_e, N * sizeof(float))) ||
      (st = ensure(ds, ds.tac_code, N * sizeof(uint32_t))) ||
      (st = ensure(ds, ds.tac_sorted, N * sizeof(uint32_t))) ||
      (st = ensure(ds, ds.tac_assign, N * sizeof(uint32_t))) ||
      (st = ensure(ds, ds.tac_tsum, 2 * (size_t)NT * sizeof(double))) ||
      (st = ensure(ds, ds.tac_hist, (pl.hist_total + 1) * sizeof(uint32_t))) ||
      (st = ensure(ds, ds.tac_counts, K * sizeof(uint32_t))) ||
      (st = ensure(ds, ds.tac_start, K * sizeof(uint32_t))) ||
      (st = ensure(ds, ds.tac_C, K * dim * sizeof(float))) ||
      (st = ensure(ds, ds.tac_pre, (size_t)NCH * sizeof(double))) ||
      (st = ensure(ds, ds.tac_fch, (size_t)NCH * sizeof(FoldChunk))) ||
      (st = ensure(ds, ds.tac_st, 2 * (size_t)P * sizeof(KppState))) ||
      (st = ensure(ds, ds.tac_big, (K + 1) * sizeof(uint32_t))) ||
      (st = ensure(ds, ds.tac_bad, (size_t)P * sizeof(uint32_t))) ||
      (st = ensure(ds, ds.tac_iters, (size_t)P * sizeof(uint32_t))) ||
      (st = ensure(ds, ds.tac_wcss, (size_t)P * sizeof(float))) ||
      (st = ensure(ds, ds.tac_prev, (size_t)P * sizeof(float))) ||
      (st = ensure(ds, ds.tac_empties, (size_t)P * sizeof(uint32_t))))
    return st;
  // 64-float rows take the matrix-core assignment (tac_assign_mfma_kernel);
  // TAC_GPU_TAC_VALU_ASSIGN=1 keeps the exact search for every row.
  const char *valu_env = getenv("TAC_GPU_TAC_VALU_ASSIGN");
  const bool mfma = dim == 64 && rt == kTacMfmaRows && !(valu_env && valu_env[0] == '1');
  // Problems are sorted by k, descending: the tiles of those with at least
  // kmin centroids (a prefix) take the matrix cores, the rest the exact
  // search, which costs less for a few centroids.
  const char *kmin_env = getenv("TAC_GPU_TAC_MFMA_KMIN");
  const uint32_t kmin = kmin_env ? (uint32_t)std::max(1, atoi(kmin_env)) : 8u;
  const uint32_t mfma_tiles = !mfma ? 0u : pl.kmax >= kmin ? pl.tiles_upto[kmin - 1] : 0u;
  if (mfma_tiles > 0 && (st = ensure(ds, ds.tac_h, K * sizeof(float)))) return st;
  float *w = as<float>(ds.tac_w), *e = as<float>(ds.tac_e), *C = as<float>(ds.tac_C);
  uint32_t *code = as<uint32_t>(ds.tac_code), *sorted = as<uint32_t>(ds.tac_sorted);
  uint32_t *done = as<uint32_t>(ds.tac_done), *bad = as<uint32_t>(ds.tac_bad);
  uint32_t *hist = as<uint32_t>(ds.tac_hist), *counts = as<uint32_t>(ds.tac_counts);
  uint32_t *start = as<uint32_t>(ds.tac_start), *iters = as<uint32_t>(ds.tac_iters);
  float *wcss = as<float>(ds.tac_wcss), *prev = as<float>(ds.tac_prev);
  double *tsum = as<double>(ds.tac_tsum), *pre = as<double>(ds.tac_pre);
  FoldChunk *fch = as<FoldChunk>(ds.tac_fch);
  KppState *kst = as<KppState>(ds.tac_st);
  const TacProblem *probs = as<TacProblem>(ds.tac_probs);
  const TacTile *tiles = as<TacTile>(ds.tac_tiles);
  const TacChunk *chl = as<TacChunk>(ds.tac_chl);
  const TacRange *ranges = as<TacRange>(ds.tac_ranges);
  uint32_t *rsum = as<uint32_t>(ds.tac_rsum);
  const uint32_t NR = (uint32_t)pl.ranges.size();
  HIP_TRY(hipMemsetAsync(code, 0, N * sizeof(uint32_t), s));
  HIP_TRY(hipMemsetAsync(iters, 0, (size_t)P * sizeof(uint32_t), s));
  HIP_TRY(hipMemsetAsync(ds.tac_empties.ptr, 0, (size_t)P * sizeof(uint32_t), s));
  HIP_TRY(hipMemsetAsync(wcss, 0, (size_t)P * sizeof(float), s));
  if (P == 0) return TAC_ERR_BUDGET_TOO_SMALL;  // unreachable: some token has rows

  const size_t rows_lds = (size_t)rt * (dim + 1);
  // the rows of a tile, then (assignment) a chunk of centroids or (k-means++
  // round) the drawn row; rt and the budget leave room for one centroid at least
  uint32_t chunk_c = (uint32_t)((tac_tile_lds_floats(dim) - rows_lds) / dim);
  if (chunk_c > 64) chunk_c = 64;
  const size_t upd_lds = (rows_lds + dim) * sizeof(float);
  const size_t asg_lds = (rows_lds + (size_t)chunk_c * dim) * sizeof(float);
  // Wide rows take more than the 64 KB of dynamic LDS a launch gets by default.
  if (upd_lds > 65536 || asg_lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void *)tac_kpp_round_kernel<0>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)upd_lds);
    if (e == hipSuccess)
      e = hipFuncSetAttribute((const void *)tac_assign_kernel<0>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)asg_lds);
    if (e != hipSuccess) return hip_status("hipFuncSetAttribute(tac tile kernels)", e);
  }
  // hist / scatter: per-code counters up to kTacMaxCodes codes, the tile's
  // codes beyond
  const size_t code_lds =
      (size_t)std::max<uint32_t>(std::min<uint32_t>(std::max<uint32_t>(pl.kmax, 1u), kTacMaxCodes),
                                 rt) *
      sizeof(uint32_t);
  const bool profile = g_profile;
  const double prep_ms =
      std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - wall0).count();

  hipEvent_t ev0 = nullptr, ev1 = nullptr, ev2 = nullptr;
  if (profile) {
    if ((st = event_at(ds, 0, &ev0)) || (st = event_at(ds, 1, &ev1)) ||
        (st = event_at(ds, 2, &ev2)))
      return st;
    HIP_TRY(hipEventRecord(ev0, s));
  }

  tac_degenerate_kernel<<<P, 256, 0, s>>>(G, probs, P, C, code, wcss, dim);
  LAUNCH_TRY("tac_degenerate_kernel");
  // k-means++ seeding (kmeans.zig:106-136), round c for every problem with k > c
  // states, weights and tile sums alternate between two halves by round
  // parity; the states "after round -1" (the first draws) go to half 1
  tac_kpp_init_kernel<<<(P + 63) / 64, 64, 0, s>>>(probs, P, kst + P, bad);
  LAUNCH_TRY("tac_kpp_init_kernel");
  // TAC_GPU_KPP_EXACT=v: the draws of round c for problem q with (c + q) % v
  // == 0 take the exact sequential evaluation (v = 1: every draw; the same
  // picks, through the stall-and-replay path)
  const char *exact_env = getenv("TAC_GPU_KPP_EXACT");
  const uint32_t exact_every = exact_env != nullptr ? (uint32_t)std::max(0, atoi(exact_env)) : 0u;
  // dim 64: one 128-row tile per block of 128 threads, staged 64 rows at a time
  if (dim == 64 && rt != 128) return TAC_ERR_UNSUPPORTED;
  const size_t round_lds = dim == 64 ? (64 * 64 + 64) * sizeof(float) : upd_lds;
  const KppTile *ktl = as<KppTile>(ds.tac_ktiles);
  auto round = [&](uint32_t c, uint32_t replay) -> int {
    const uint32_t T = pl.tiles_upto[c];
    const uint32_t in = (c + 1) & 1u, out = c & 1u;
    const KppRound rb{w + in * N,      w + out * N,  tsum + in * NT,
                      tsum + out * NT, kst + in * P, kst + out * P};
    if (dim == 64)
      tac_kpp_round_kernel<64><<<T, rt, round_lds, s>>>(G, rb, bad, ktl, C, c, dim, exact_every,
                                                        replay);
    else if (dim == 128)
      tac_kpp_round_kernel<128><<<T, rt, round_lds, s>>>(G, rb, bad, ktl, C, c, dim,
                                                         exact_every, replay);
    else
      tac_kpp_round_kernel<0><<<T, rt, round_lds, s>>>(G, rb, bad, ktl, C, c, dim, exact_every,
                                                       replay);
    LAUNCH_TRY("tac_kpp_round_kernel");
    return TAC_OK;
  };
  auto exact_round = [&](uint32_t c) -> int {
    const uint32_t Pc = pl.probs_upto[c];
    const uint32_t in = (c + 1) & 1u, out = c & 1u;
    const KppRound rb{w + in * N,      w + out * N,  tsum + in * NT,
                      tsum + out * NT, kst + in * P, kst + out * P};
    const size_t ex_lds = (size_t)dim * sizeof(float);
    if (dim == 64)
      tac_kpp_exact_round_kernel<64><<<Pc, kKppFallbackThreads, ex_lds, s>>>(
          G, rb, bad, probs, C, pre, fch, c, dim, rt);
    else if (dim == 128)
      tac_kpp_exact_round_kernel<128><<<Pc, kKppFallbackThreads, ex_lds, s>>>(
          G, rb, bad, probs, C, pre, fch, c, dim, rt);
    else
      tac_kpp_exact_round_kernel<0><<<Pc, kKppFallbackThreads, ex_lds, s>>>(
          G, rb, bad, probs, C, pre, fch, c, dim, rt);
    LAUNCH_TRY("tac_kpp_exact_round_kernel");
    return TAC_OK;
  };
  // a problem's state after its last round k - 1 sits in half (k - 1) & 1;
  // returns the earliest pending round (kmax if none)
  std::vector<KppState> &hst = hst_cache;
  hst.resize(2 * (size_t)P);
  auto final_states = [&](uint32_t *pending) -> int {
    HIP_TRY(hipMemcpyAsync(hst.data(), kst, 2 * (size_t)P * sizeof(KppState),
                           hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    *pending = pl.kmax;
    for (uint32_t q = 0; q < P; ++q) {
      const TacProblem &pq = pl.probs[q];
      if (pq.degenerate || pq.k == 0) continue;
      const KppState &hq = hst[(size_t)((pq.k - 1) & 1u) * P + q];
      if (!hq.err && hq.fallback) *pending = std::min(*pending, hq.pad);
    }
    return TAC_OK;
  };
  // Caller-supplied centroids (a fixed problem with init) replace the
  // seeding; a degenerate problem keeps the rows the degenerate kernel wrote.
  const bool given_init = fixed && fixed->init && !pl.probs[0].degenerate;
  if (given_init)
    HIP_TRY(hipMemcpyAsync(C, fixed->init, (size_t)fixed->k * dim * sizeof(float),
                           hipMemcpyHostToDevice, s));
  for (uint32_t c = 0; !given_init && c < pl.kmax && pl.tiles_upto[c] > 0; ++c)
    if ((st = round(c, 0))) return st;
  uint32_t pending = pl.kmax;
  if (!given_init && (st = final_states(&pending))) return st;
  if (pending < pl.kmax) {
    // replay the stalled problems from their earliest pending draw
    for (uint32_t c = pending; c < pl.kmax; ++c) {
      if ((st = exact_round(c))) return st;
      if (c + 1 < pl.kmax && pl.tiles_upto[c + 1] > 0 && (st = round(c + 1, 1))) return st;
    }
    if ((st = final_states(&pending))) return st;
    if (pending < pl.kmax) {
      g_last_error = "k-means++ replay left a draw pending";
      return TAC_ERR_HIP;
    }
  }
  if (!given_init) {
    // the reference fits tokens in id order and stops at the first error
    uint32_t first_tok = 0xFFFFFFFFu;
    int first_err = 0;
    for (uint32_t q = 0; q < P; ++q) {
      const TacProblem &pq = pl.probs[q];
      if (pq.degenerate || pq.k == 0) continue;
      const KppState &hq = hst[(size_t)((pq.k - 1) & 1u) * P + q];
      if (hq.err && pl.token[q] < first_tok) {
        first_tok = pl.token[q];
        first_err = hq.err;
      }
    }
    if (first_err) return first_err;
  }
  if (profile) HIP_TRY(hipEventRecord(ev1, s));

  // Lloyd iterations (kmeans.zig:149-224) for every problem not yet converged.
  // Problems are sorted by k, descending, and their tiles, scan ranges and
  // wcss chunks are listed in problem order, so the problems still running
  // lie in a prefix of each list.  At a few iterations the done flags are
  // read back once and the per-tile, per-range, per-chunk and per-problem
  // launches shrink to the prefix up to the last problem still running
  // (the one-centroid tail converges within the first iterations); when
  // none is left the loop ends.  The kernels skip finished problems
  // themselves, so the results are those of the full launches.
  std::vector<uint32_t> range_upto(P + 1, 0), chunk_upto(P + 1, 0);
  for (uint32_t q = 0; q < P; ++q) {
    range_upto[q + 1] = range_upto[q] + pl.probs[q].nranges;
    chunk_upto[q + 1] = chunk_upto[q] + pl.probs[q].nchunks;
  }
  uint32_t Pa = P, NTa = NT, NRa = NR, NCHa = NCH;
  std::vector<uint32_t> hdone;
  for (uint32_t t = 0; t < prm.max_iters; ++t) {
    if (t == 3 || t == 6 || t == 10 || t == 15 || t == 21) {
      hdone.resize(P);
      HIP_TRY(hipMemcpyAsync(hdone.data(), done, (size_t)P * sizeof(uint32_t),
                             hipMemcpyDeviceToHost, s));
      HIP_TRY(hipStreamSynchronize(s));
      uint32_t qa = 0;
      for (uint32_t q = Pa; q > 0; --q)
        if (!hdone[q - 1]) {
          qa = q;
          break;
        }
      if (qa == 0) break;  // every problem has converged
      Pa = qa;
      NTa = pl.probs[qa - 1].tile0 + pl.probs[qa - 1].ntiles;
      NRa = range_upto[qa];
      NCHa = chunk_upto[qa];
    }
    const uint32_t mt = std::min(mfma_tiles, NTa);
    if (mt > 0) {
      tac_cnorm_kernel<<<(unsigned)((K + 255) / 256), 256, 0, s>>>(
          C, as<uint32_t>(ds.tac_cprob), done, (uint32_t)K, as<float>(ds.tac_h));
      LAUNCH_TRY("tac_cnorm_kernel");
      tac_assign_mfma_kernel<<<mt, kTacMfmaThreads, 0, s>>>(
          G, C, as<float>(ds.tac_h), probs, tiles, done, code, e);
      LAUNCH_TRY("tac_assign_mfma_kernel");
    }
    if (mfma_tiles < NTa) {
      const uint32_t nt = NTa - mfma_tiles;
      const TacTile *rest = tiles + mfma_tiles;
      if (dim == 64)
        tac_assign_kernel<64><<<nt, rt, asg_lds, s>>>(G, C, probs, rest, done, code, e, dim,
                                                      chunk_c);
      else if (dim == 128)
        tac_assign_kernel<128><<<nt, rt, asg_lds, s>>>(G, C, probs, rest, done, code, e, dim,
                                                       chunk_c);
      else
        tac_assign_kernel<0><<<nt, rt, asg_lds, s>>>(G, C, probs, rest, done, code, e, dim,
                                                     chunk_c);
      LAUNCH_TRY("tac_assign_kernel");
    }
    tac_hist_kernel<<<NTa, rt, code_lds, s>>>(code, probs, tiles, done, hist);
    LAUNCH_TRY("tac_hist_kernel");
    tac_scan_partial_kernel<<<NRa, 256, 0, s>>>(hist, probs, ranges, done, rsum);
    tac_scan_apply_kernel<<<NRa, 256, 0, s>>>(hist, probs, ranges, done, rsum, counts, start);
    LAUNCH_TRY("tac scan kernels");
    tac_scatter_kernel<<<NTa, rt, code_lds, s>>>(code, hist, start, probs, tiles, done, sorted);
    LAUNCH_TRY("tac_scatter_kernel");
    {
      const uint32_t *cp = as<uint32_t>(ds.tac_cprob);
      const unsigned fb = (unsigned)((K + 3) / 4);
      // dim 64: clusters of kTacFoldBig members or more go to the block kernel
      uint32_t *big = dim == 64 ? as<uint32_t>(ds.tac_big) : nullptr;
      if (big) HIP_TRY(hipMemsetAsync(big, 0, sizeof(uint32_t), s));
#define TAC_FOLD(P, BIG) \
  tac_fold_kernel<P><<<fb, 256, 0, s>>>(G, sorted, counts, start, cp, probs, done, C, (uint32_t)K, dim, BIG)
      switch (per) {  // dim <= kTacMaxDim: at most 8 dimensions per lane
        case 1: TAC_FOLD(1, big); break;
        case 2: TAC_FOLD(2, nullptr); break;
        case 3: TAC_FOLD(3, nullptr); break;
        case 4: TAC_FOLD(4, nullptr); break;
        case 5: TAC_FOLD(5, nullptr); break;
        case 6: TAC_FOLD(6, nullptr); break;
        case 7: TAC_FOLD(7, nullptr); break;
        default: TAC_FOLD(8, nullptr); break;
      }
#undef TAC_FOLD
      LAUNCH_TRY("tac_fold_kernel");
      if (big) {
        tac_fold_big_kernel<<<kTacFoldBigBlocks, kTacFoldBigThreads, 0, s>>>(
            G, sorted, counts, start, cp, probs, C, big);
        LAUNCH_TRY("tac_fold_big_kernel");
      }
    }
    tac_chunk_sums_kernel<<<(NCHa + 3) / 4, 256, 0, s>>>(e, probs, chl, NCHa, done, pre);
    tac_chunk_prefix_kernel<<<Pa, 256, 0, s>>>(pre, probs, done);
    tac_quantize_kernel<<<(NCHa + 3) / 4, 256, 0, s>>>(e, pre, probs, chl, NCHa, done, fch);
    tac_wcss_apply_kernel<<<Pa, kWave, 0, s>>>(e, fch, probs, done, wcss);
    LAUNCH_TRY("tac wcss kernels");
    tac_reseed_kernel<<<Pa, 256, 0, s>>>(G, e, counts, probs, done, C,
                                         as<uint32_t>(ds.tac_empties), dim);
    LAUNCH_TRY("tac_reseed_kernel");
    tac_converge_kernel<<<(Pa + 255) / 256, 256, 0, s>>>(wcss, prev, done, iters, Pa, t, prm.tol);
    LAUNCH_TRY("tac_converge_kernel");
  }
  if (profile) HIP_TRY(hipEventRecord(ev2, s));
  tac_output_kernel<<<NT, rt, 0, s>>>(code, as<uint32_t>(ds.tac_idx), probs, tiles,
                                     as<uint32_t>(ds.tac_assign));
  LAUNCH_TRY("tac_output_kernel");
  std::vector<float> pw(P);
  HIP_TRY(hipMemcpyAsync(assign_out, ds.tac_assign.ptr, N * sizeof(uint32_t),
                         hipMemcpyDeviceToHost, s));
  HIP_TRY(hipMemcpyAsync(cent_out, C, K * dim * sizeof(float), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipMemcpyAsync(pw.data(), wcss, (size_t)P * sizeof(float), hipMemcpyDeviceToHost, s));
  if (fixed && fixed->iters_out)
    HIP_TRY(hipMemcpyAsync(fixed->iters_out, iters, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  if (profile) {
    float a = 0.0f, b = 0.0f;
    HIP_TRY(hipEventElapsedTime(&a, ev0, ev1));
    HIP_TRY(hipEventElapsedTime(&b, ev1, ev2));
    std::lock_guard<std::mutex> g(g_profile_mu);
    g_prof.cluster_kpp_ms += a;
    g_prof.cluster_lloyd_ms += b;
    g_prof.cluster_calls += 1;
    g_prof.cluster_prep_ms += prep_ms;
    g_prof.cluster_call_ms +=
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - wall0)
            .count();
  }
  for (uint64_t j = 0; j < nd; ++j) kpt_out[j] = kappa[j];
  // wcss_total: the per-token wcss in token order, grouped by thread slices
  std::vector<float> tok_w(nd, 0.0f);
  std::vector<uint8_t> has(nd, 0);
  for (uint32_t q = 0; q < P; ++q) {
    tok_w[pl.token[q]] = pw[q];
    has[pl.token[q]] = 1;
  }
  const uint32_t nt = prm.n_threads > 1 ? prm.n_threads : 1;
  const uint64_t chunk = nt > 1 ? (nd + nt - 1) / nt : nd;
  std::vector<float> parts(nt, 0.0f);
  for (uint64_t j = 0; j < nd; ++j)
    if (has[j]) parts[nt > 1 ? j / chunk : 0] += tok_w[j];
  float total = 0.0f;
  for (uint32_t q = 0; q < nt; ++q) total += parts[q];
  *wcss_out = total;
  return TAC_OK;
}

}  // namespace

extern "C" {

namespace {
int cluster_flat_entry(const uint32_t *token_ids, uint64_t n_tokens, const float *vectors,
                       bool on_device, uint64_t vectors_len, uint32_t dim,
                       const tac_cluster_params *params, float *centroids_out,
                       uint32_t *assignments_out, uint32_t *kappa_per_token_out,
                       uint64_t kappa_per_token_len, float *wcss_total_out,
                       uint64_t *n_distinct_out) {
  if (!params) return TAC_ERR_INVALID_ARGUMENT;
  // validation in the reference's order (tac.zig:570-573)
  if (n_tokens == 0) return TAC_ERR_EMPTY_TOKEN_DUMP;
  if (dim == 0) return TAC_ERR_INVALID_THRESHOLDS;
  if (vectors_len != n_tokens * (uint64_t)dim) return TAC_ERR_INVALID_THRESHOLDS;
  if (params->kappa_total == 0) return TAC_ERR_BUDGET_TOO_SMALL;
  if (!token_ids || !vectors || !centroids_out || !assignments_out || !kappa_per_token_out ||
      !wcss_total_out)
    return TAC_ERR_INVALID_ARGUMENT;
  uint32_t max_id = 0;
  for (uint64_t i = 0; i < n_tokens; ++i)
    if (token_ids[i] > max_id) max_id = token_ids[i];
  const uint64_t nd = (uint64_t)max_id + 1;
  if (n_distinct_out) *n_distinct_out = nd;
  if (kappa_per_token_len < nd) return TAC_ERR_BUFFER_TOO_SMALL;
  DeviceState *ds = nullptr;
  int st;
  if ((st = acquire_device(&ds, nullptr))) return st;
  std::lock_guard<std::mutex> g(ds->mu);
  hipStream_t s;
  if ((st = resolve_stream(*ds, nullptr, &s))) return st;
  if ((st = begin_call(*ds, s))) return st;
  st = tac_cluster_core(*ds, s, token_ids, n_tokens, vectors, on_device, dim, *params, nd,
                        centroids_out, assignments_out, kappa_per_token_out, wcss_total_out);
  if (st) {
    HIP_TRY(hipStreamSynchronize(s));
    return st;
  }
  return end_call(*ds, s);
}
}  // namespace

int tac_cluster_flat(const uint32_t *token_ids, uint64_t n_tokens, const float *vectors,
                     uint64_t vectors_len, uint32_t dim, const tac_cluster_params *params,
                     float *centroids_out, uint32_t *assignments_out,
                     uint32_t *kappa_per_token_out, uint64_t kappa_per_token_len,
                     float *wcss_total_out, uint64_t *n_distinct_out) {
  return cluster_flat_entry(token_ids, n_tokens, vectors, false, vectors_len, dim, params,
                            centroids_out, assignments_out, kappa_per_token_out,
                            kappa_per_token_len, wcss_total_out, n_distinct_out);
}

int tac_cluster_flat_device(const uint32_t *token_ids, uint64_t n_tokens,
                            const float *d_vectors, uint64_t vectors_len, uint32_t dim,
                            const tac_cluster_params *params, float *centroids_out,
                            uint32_t *assignments_out, uint32_t *kappa_per_token_out,
                            uint64_t kappa_per_token_len, float *wcss_total_out,
                            uint64_t *n_distinct_out) {
  return cluster_flat_entry(token_ids, n_tokens, d_vectors, true, vectors_len, dim, params,
                            centroids_out, assignments_out, kappa_per_token_out,
                            kappa_per_token_len, wcss_total_out, n_distinct_out);
}

}  // extern "C"
