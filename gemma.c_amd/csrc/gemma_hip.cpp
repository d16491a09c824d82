// gemma_hip.cpp -- the C ABI declared in include/gemma_hip.h.
//
// Host-side responsibilities: the error channel (the reference's
// log_error/get_error, gemma.c:577-587: return 1 and keep a message), the
// device and stream, the weight registry (host range -> device copy, so the
// reference's host weight pointers, interior ones included, stay the
// handles), argument validation (every shape/stride/pointer a kernel's grid
// relies on is checked here before a launch), and kernel selection: M == 1
// goes to the bandwidth-bound GEMV, M > 1 to the MFMA GEMM.
#include "../../include/gemma_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "gh_kernels.h"

namespace {

thread_local char g_err[256] = "";

int fail(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return 1;
}

int hip_fail(const char *what, hipError_t e) {
  return fail("%s: %s", what, hipGetErrorString(e));
}

#define GH_CHECK(what, expr)                  \
  do {                                        \
    hipError_t gh_e_ = (expr);                \
    if (gh_e_ != hipSuccess) return hip_fail(what, gh_e_); \
  } while (0)

struct Region {
  size_t bytes;
  char *device;
};

struct State {
  bool ready = false;
  int device = -1;
  hipStream_t stream = nullptr;
  gh::DeviceInfo info{};
  std::map<uintptr_t, Region> regions;  // keyed by host start address
  std::mutex lock;
  // serialises the _host entry points, which share the staging buffer and
  // may be called from several threads at once (the reference's prefill QKV
  // site calls gemm_int8 from inside an OpenMP loop, gemma.c:5050-5089)
  std::recursive_mutex host;
  // device staging for the _host entry points, grown on demand
  char *staging = nullptr;
  size_t staging_bytes = 0;
  // im2col workspace of the patch embedding, grown on demand
  float *work = nullptr;
  size_t work_bytes = 0;
  // pinned host staging of the _host entry points: small activations are
  // read by the kernels and small outputs written by them in place, so a
  // decode call costs one launch and one synchronisation
  char *pinned = nullptr;
  char *pinned_dev = nullptr;  // the same memory as kernels address it
  size_t pinned_bytes = 0;
  // the last activations a _host quantize produced: the device copy, and a
  // pinned mirror of what the caller received.  A following matmul whose
  // int8 input and scales are byte-equal to (part of) the mirror reads the
  // device copy instead of uploading them again.
  struct {
    bool valid = false;
    const int8_t *host_q = nullptr;  // the caller's dst
    int m = 0, n = 0;
    int8_t *dev_q = nullptr;
    float *dev_s = nullptr;
    int8_t *mir_q = nullptr;  // pinned mirror, host view
    float *mir_s = nullptr;
    int8_t *mir_q_dev = nullptr;  // pinned mirror, device view
    float *mir_s_dev = nullptr;
    size_t cap_q = 0, cap_s = 0;
  } act;
};

State g;

// ---- per-op GPU timing (the reference's PerfBench, gemma.c:2402-2431) ----
// When enabled, every device entry point records a HIP event before and
// after its launches on its stream; the pairs are resolved into totals per
// (phase, op) lazily (when many are pending, and on read).  Launches on a
// stream that is being captured into a graph are not timed, so the decoder
// runs its steps eagerly while timing is on.  The ops are the reference's,
// in its report order (gemma.c:2409-2431).
enum PerfOp {
  kOpRmsnorm, kOpLayernorm, kOpQuantizeAct, kOpGemvFpx, kOpGemvInt8, kOpGemvFpxNn,
  kOpGemmFpx, kOpGemmFpxNn, kOpGemmInt8, kOpSoftmax, kOpGelu, kOpRope, kOpSample, kOpCount
};
const char *const kOpName[kOpCount] = {
    "rmsnorm",     "layernorm", "quantize_act", "gemv_fpx",  "gemv_int8",
    "gemv_fpx_nn", "gemm_fpx",  "gemm_fpx_nn",  "gemm_int8", "softmax",
    "gelu",        "rope",      "sample_from_logits"};
// PerfPhase (gemma.c:2402-2407)
enum PerfPhase { kPhasePrefill, kPhaseDecode, kPhaseVision, kPhases };

struct Perf {
  std::mutex mu;
  std::atomic<bool> on{false};  // read unlocked by every PerfScope
  int phase = 0;
  struct Pending {
    int op, phase;
    hipEvent_t a, b;
  };
  std::vector<Pending> pending;
  std::vector<hipEvent_t> pool;
  double sec[kPhases][kOpCount] = {};
  long calls[kPhases][kOpCount] = {};

  hipEvent_t take() {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    return hipEventCreate(&e) == hipSuccess ? e : nullptr;
  }
  // resolves every pending pair (waits for its end event)
  hipError_t drain() {
    hipError_t err = hipSuccess;
    for (const Pending &p : pending) {
      float ms = 0.0f;
      hipError_t e = hipEventSynchronize(p.b);
      if (e == hipSuccess) e = hipEventElapsedTime(&ms, p.a, p.b);
      if (e == hipSuccess) {
        sec[p.phase][p.op] += ms * 1e-3;
        calls[p.phase][p.op] += 1;
      } else if (err == hipSuccess) {
        err = e;
      }
      pool.push_back(p.a);
      pool.push_back(p.b);
    }
    pending.clear();
    return err;
  }
  void release() {
    (void)drain();
    for (hipEvent_t e : pool) (void)hipEventDestroy(e);
    pool.clear();
  }
};
Perf g_perf;

// Times the launches made during its lifetime on `stream` as one call of op,
// in `phase` (default: the current one).
class PerfScope {
 public:
  PerfScope(int op, hipStream_t stream, int phase = -1)
      : op_(op), phase_(phase), stream_(stream) {
    if (!g_perf.on.load(std::memory_order_relaxed)) return;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
      return;
    std::lock_guard<std::mutex> lock(g_perf.mu);
    a_ = g_perf.take();
    b_ = g_perf.take();
    if (a_ == nullptr || b_ == nullptr || hipEventRecord(a_, stream) != hipSuccess) {
      if (a_ != nullptr) g_perf.pool.push_back(a_);
      if (b_ != nullptr) g_perf.pool.push_back(b_);
      a_ = b_ = nullptr;
    }
  }
  ~PerfScope() {
    if (a_ == nullptr) return;
    std::lock_guard<std::mutex> lock(g_perf.mu);
    if (hipEventRecord(b_, stream_) != hipSuccess) {
      g_perf.pool.push_back(a_);
      g_perf.pool.push_back(b_);
      return;
    }
    g_perf.pending.push_back(Perf::Pending{op_, phase_ >= 0 ? phase_ : g_perf.phase, a_, b_});
    if (g_perf.pending.size() >= 512) (void)g_perf.drain();
  }
  PerfScope(const PerfScope &) = delete;
  PerfScope &operator=(const PerfScope &) = delete;

 private:
  int op_, phase_;
  hipStream_t stream_;
  hipEvent_t a_ = nullptr, b_ = nullptr;
};

// One launch (or a few that make one op) timed as one call of op.
template <class F>
hipError_t timed(int op, hipStream_t stream, F &&launch, int phase = -1) {
  PerfScope perf(op, stream, phase);
  return launch();
}

// A whole-forward entry point attributes the ops that follow to its phase,
// as the reference's forward_gemma_* do with PERF_PHASE (gemma.c:5463,
// 5509, 5568).
void perf_enter(int phase) {
  std::lock_guard<std::mutex> lock(g_perf.mu);
  g_perf.phase = phase;
}

// NULL is HIP's default (null) stream, so work on it is ordered with the
// caller's own default-stream copies.
hipStream_t pick_stream(void *stream) { return static_cast<hipStream_t>(stream); }

int need_init() {
  if (!g.ready) return fail("gemma_hip: library not initialised (call gemma_hip_init)");
  return 0;
}

// Device address of [host, host+bytes) inside a registered range, or null.
char *resolve(const void *host, size_t bytes) {
  const uintptr_t h = reinterpret_cast<uintptr_t>(host);
  std::lock_guard<std::mutex> guard(g.lock);
  auto it = g.regions.upper_bound(h);
  if (it == g.regions.begin()) return nullptr;
  --it;
  const uintptr_t begin = it->first;
  if (h + bytes > begin + it->second.bytes) return nullptr;
  return it->second.device + (h - begin);
}

int staging_reserve(size_t bytes) {
  if (bytes <= g.staging_bytes) return 0;
  if (g.staging != nullptr) {
    GH_CHECK("gemma_hip staging sync", hipStreamSynchronize(g.stream));
    GH_CHECK("gemma_hip staging free", hipFree(g.staging));
    g.staging = nullptr;
    g.staging_bytes = 0;
  }
  size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
  GH_CHECK("gemma_hip staging alloc", hipMalloc(&g.staging, want));
  g.staging_bytes = want;
  return 0;
}

int pinned_reserve(size_t bytes) {
  if (bytes <= g.pinned_bytes) return 0;
  if (g.pinned != nullptr) {
    GH_CHECK("gemma_hip pinned sync", hipStreamSynchronize(g.stream));
    GH_CHECK("gemma_hip pinned free", hipHostFree(g.pinned));
    g.pinned = nullptr;
    g.pinned_bytes = 0;
  }
  size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
  GH_CHECK("gemma_hip pinned alloc",
           hipHostMalloc((void **)&g.pinned, want, hipHostMallocMapped));
  g.pinned_bytes = want;
  GH_CHECK("gemma_hip pinned map",
           hipHostGetDevicePointer((void **)&g.pinned_dev, g.pinned, 0));
  return 0;
}

// Room for m x n quantized activations in the activation cache.
int act_reserve(int m, int n) {
  g.act.valid = false;
  const size_t q = (size_t)m * n, sc = (size_t)m * 4;
  if (q > g.act.cap_q || sc > g.act.cap_s) {
    GH_CHECK("gemma_hip act sync", hipStreamSynchronize(g.stream));
    if (g.act.dev_q != nullptr) GH_CHECK("gemma_hip act free", hipFree(g.act.dev_q));
    if (g.act.mir_q != nullptr) GH_CHECK("gemma_hip act free", hipHostFree(g.act.mir_q));
    g.act.dev_q = nullptr;
    g.act.mir_q = nullptr;
    g.act.cap_q = g.act.cap_s = 0;
    const size_t want_q = (q < (1u << 16) ? (1u << 16) : q + 255) / 256 * 256;
    const size_t want_s = (sc < 4096 ? 4096 : sc + 255) / 256 * 256;
    char *dev = nullptr, *mir = nullptr;
    GH_CHECK("gemma_hip act alloc", hipMalloc((void **)&dev, want_q + want_s));
    char *mir_dev = nullptr;
    hipError_t e = hipHostMalloc((void **)&mir, want_q + want_s, hipHostMallocMapped);
    if (e == hipSuccess) e = hipHostGetDevicePointer((void **)&mir_dev, mir, 0);
    if (e != hipSuccess) {
      (void)hipFree(dev);
      if (mir != nullptr) (void)hipHostFree(mir);
      return hip_fail("gemma_hip act alloc", e);
    }
    g.act.dev_q = (int8_t *)dev;
    g.act.dev_s = (float *)(dev + want_q);
    g.act.mir_q = (int8_t *)mir;
    g.act.mir_s = (float *)(mir + want_q);
    g.act.mir_q_dev = (int8_t *)mir_dev;
    g.act.mir_s_dev = (float *)(mir_dev + want_q);
    g.act.cap_q = want_q;
    g.act.cap_s = want_s;
  }
  return 0;
}

// Row r0 of the cached activations when the caller's int8 rows [src, m rows
// of stride sstr, k used bytes each] and their scales are byte-equal to what
// the last _host quantize handed out from rows r0.. of the cache; else -1.
// `scales` is the caller's scale array, or null with `one_scale` holding the
// by-value scale of a single row (gemv_int8's vsc).
int act_lookup(const int8_t *src, int sstr, const float *scales, float one_scale,
               int m, int k) {
  const auto &a = g.act;
  if (!a.valid || src == nullptr || k > a.n || (m > 1 && sstr != a.n)) return -1;
  const uintptr_t off = (uintptr_t)src - (uintptr_t)a.host_q;
  if ((uintptr_t)src < (uintptr_t)a.host_q || off % (size_t)a.n != 0) return -1;
  const size_t r0 = off / (size_t)a.n;
  if (r0 + (size_t)m > (size_t)a.m) return -1;
  const size_t span = (size_t)(m - 1) * a.n + k;
  if (memcmp(src, a.mir_q + r0 * a.n, span) != 0) return -1;
  if (scales != nullptr) {
    if (memcmp(scales, a.mir_s + r0, (size_t)m * 4) != 0) return -1;
  } else if (m != 1 || memcmp(&one_scale, a.mir_s + r0, 4) != 0) {
    return -1;
  }
  return (int)r0;
}

// Carves aligned pieces out of the staging buffer.
struct Carver {
  size_t used = 0;
  size_t take(size_t bytes) {
    size_t at = used;
    used += (bytes + 255) / 256 * 256;
    return at;
  }
};

int check_matmul_shape(const char *fn, int m, int n, int k, int dstr, int mstr,
                       int sstr) {
  if (m < 0 || n <= 0 || k <= 0)
    return fail("%s: bad shape m=%d n=%d k=%d", fn, m, n, k);
  if (dstr < n || mstr < k || sstr < k)
    return fail("%s: stride smaller than row (dstr=%d n=%d mstr=%d sstr=%d k=%d)",
                fn, dstr, n, mstr, sstr, k);
  return 0;
}

int build_jobs(const char *fn, const gemma_hip_job *jobs, int njobs,
               gh::GemvJobs *out) {
  if (jobs == nullptr || njobs < 1 || njobs > GEMMA_HIP_MAX_JOBS)
    return fail("%s: njobs must be 1..%d (got %d)", fn, GEMMA_HIP_MAX_JOBS,
                njobs);
  memset(out, 0, sizeof(*out));
  long total = 0;
  for (int j = 0; j < njobs; ++j) {
    if (jobs[j].m < 0) return fail("%s: job %d has m=%d", fn, j, jobs[j].m);
    if (jobs[j].m > 0 && (jobs[j].w == nullptr || jobs[j].dst == nullptr))
      return fail("%s: job %d has a null pointer", fn, j);
    total += jobs[j].m;
    if (total > (1l << 30)) return fail("%s: too many rows", fn);
    out->w[j] = jobs[j].w;
    out->sc[j] = jobs[j].sc;
    out->dst[j] = jobs[j].dst;
    out->end[j] = (int)total;
  }
  for (int j = njobs; j < gh::kMaxJobs; ++j) out->end[j] = (int)total;
  out->njobs = njobs;
  return 0;
}

constexpr int kMaxGemvK8 = 65536;   // int8 vector staged in 64 KB of LDS
constexpr int kMaxGemvK32 = 16384;  // fp32 vector staged in 64 KB of LDS

}  // namespace

extern "C" {

int gemma_hip_init(int device) {
  if (g.ready) {
    if (device == g.device) return 0;
    return fail("gemma_hip_init: already initialised on device %d", g.device);
  }
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0)
    return fail("gemma_hip_init: no HIP device available (%s)",
                e == hipSuccess ? "0 devices" : hipGetErrorString(e));
  if (device < 0 || device >= count)
    return fail("gemma_hip_init: device %d out of range (0..%d)", device,
                count - 1);
  hipDeviceProp_t prop;
  GH_CHECK("gemma_hip_init: hipGetDeviceProperties",
           hipGetDeviceProperties(&prop, device));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail("gemma_hip_init: device %d is %s; this library is built for gfx950",
                device, prop.gcnArchName);
  GH_CHECK("gemma_hip_init: hipSetDevice", hipSetDevice(device));
  GH_CHECK("gemma_hip_init: scratch address", gh::gemm_scratch_init(device));
  GH_CHECK("gemma_hip_init: hipStreamCreate",
           hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking));
  g.info.cus = prop.multiProcessorCount;
  g.device = device;
  g.ready = true;
  g_err[0] = '\0';
  return 0;
}

void gemma_hip_shutdown(void) {
  if (!g.ready) return;
  (void)hipStreamSynchronize(g.stream);
  {
    std::lock_guard<std::mutex> lock(g_perf.mu);
    g_perf.release();
    g_perf.on = false;
  }
  gh::release_gemm_workspaces();
  {
    std::lock_guard<std::mutex> guard(g.lock);
    for (auto &kv : g.regions) (void)hipFree(kv.second.device);
    g.regions.clear();
  }
  if (g.staging != nullptr) (void)hipFree(g.staging);
  g.staging = nullptr;
  g.staging_bytes = 0;
  if (g.work != nullptr) (void)hipFree(g.work);
  g.work = nullptr;
  g.work_bytes = 0;
  if (g.pinned != nullptr) (void)hipHostFree(g.pinned);
  g.pinned = nullptr;
  g.pinned_dev = nullptr;
  g.pinned_bytes = 0;
  if (g.act.dev_q != nullptr) (void)hipFree(g.act.dev_q);
  if (g.act.mir_q != nullptr) (void)hipHostFree(g.act.mir_q);
  g.act = {};
  (void)hipStreamDestroy(g.stream);
  g.stream = nullptr;
  g.ready = false;
  g.device = -1;
}

const char *gemma_hip_last_error(void) { return g_err; }

int gemma_hip_sync(void *stream) {
  if (need_init()) return 1;
  GH_CHECK("gemma_hip_sync", hipStreamSynchronize(pick_stream(stream)));
  return 0;
}

int gemma_hip_perf_enable(int on) {
  if (need_init()) return 1;
  std::lock_guard<std::mutex> lock(g_perf.mu);
  if (on && !g_perf.on) {
    (void)g_perf.drain();
    memset(g_perf.sec, 0, sizeof(g_perf.sec));
    memset(g_perf.calls, 0, sizeof(g_perf.calls));
  }
  g_perf.on = on != 0;
  return 0;
}

int gemma_hip_perf_phase(int phase) {
  if (phase < 0 || phase >= kPhases)
    return fail("gemma_hip_perf_phase: phase %d outside 0..%d", phase, kPhases - 1);
  std::lock_guard<std::mutex> lock(g_perf.mu);
  g_perf.phase = phase;
  return 0;
}

int gemma_hip_perf_read(gemma_hip_perf_entry *out, int max, int *count) {
  if (need_init()) return 1;
  if (count == nullptr || max < 0 || (max > 0 && out == nullptr))
    return fail("gemma_hip_perf_read: bad arguments");
  std::lock_guard<std::mutex> lock(g_perf.mu);
  const hipError_t e = g_perf.drain();
  if (e != hipSuccess) return hip_fail("gemma_hip_perf_read", e);
  int n = 0;
  for (int ph = 0; ph < kPhases; ++ph)
    for (int op = 0; op < kOpCount; ++op) {
      if (g_perf.calls[ph][op] == 0) continue;
      if (n < max) out[n] = gemma_hip_perf_entry{kOpName[op], ph, g_perf.sec[ph][op],
                                                 g_perf.calls[ph][op]};
      ++n;
    }
  *count = n;
  return 0;
}

int gemma_hip_register_weights(const void *host, size_t bytes) {
  if (need_init()) return 1;
  if (host == nullptr || bytes == 0)
    return fail("gemma_hip_register_weights: empty range");
  const uintptr_t h = reinterpret_cast<uintptr_t>(host);
  {
    std::lock_guard<std::mutex> guard(g.lock);
    auto it = g.regions.upper_bound(h + bytes - 1);
    if (it != g.regions.begin()) {
      --it;
      if (it->first + it->second.bytes > h)
        return fail("gemma_hip_register_weights: range overlaps a registered one");
    }
  }
  char *device = nullptr;
  GH_CHECK("gemma_hip_register_weights: hipMalloc", hipMalloc(&device, bytes));
  hipError_t e = hipMemcpy(device, host, bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(device);
    return hip_fail("gemma_hip_register_weights: upload", e);
  }
  std::lock_guard<std::mutex> guard(g.lock);
  g.regions[h] = Region{bytes, device};
  return 0;
}

int gemma_hip_release_weights(const void *host) {
  if (need_init()) return 1;
  const uintptr_t h = reinterpret_cast<uintptr_t>(host);
  char *device = nullptr;
  {
    std::lock_guard<std::mutex> guard(g.lock);
    auto it = g.regions.find(h);
    if (it == g.regions.end())
      return fail("gemma_hip_release_weights: %p is not a registered range start",
                  host);
    device = it->second.device;
    g.regions.erase(it);
  }
  GH_CHECK("gemma_hip_release_weights: sync", hipStreamSynchronize(g.stream));
  GH_CHECK("gemma_hip_release_weights: hipFree", hipFree(device));
  return 0;
}

void *gemma_hip_device_ptr(const void *host) {
  if (!g.ready) return nullptr;
  return resolve(host, 1);
}

/* ---- device entry points ---------------------------------------------- */

int gemma_hip_quantize(int8_t *dst, float *dsc, const float *src, int sstr,
                       int m, int n, void *stream) {
  if (need_init()) return 1;
  if (sstr == 0) sstr = n;
  if (m < 0 || n <= 0 || sstr < n)
    return fail("gemma_hip_quantize: bad shape m=%d n=%d sstr=%d", m, n, sstr);
  if (m == 0) return 0;
  if (dst == nullptr || dsc == nullptr || src == nullptr)
    return fail("gemma_hip_quantize: null pointer");
  PerfScope perf(kOpQuantizeAct, pick_stream(stream));
  GH_CHECK("gemma_hip_quantize: launch",
           gh::launch_quantize(dst, dsc, src, sstr, m, n, pick_stream(stream)));
  return 0;
}

}  // extern "C"

namespace {

// gemma_hip_matmul and gemma_hip_matmul_noalloc: `noalloc` takes the GEMM's
// workspace from the library's static scratch instead of memory it allocates.
int matmul_impl(const char *name, float *dst, int dstr, const int8_t *mat, int mstr,
                const float *matsc, const int8_t *src, int sstr, const float *ssc, int m,
                int n, int k, void *stream, bool noalloc, int op = -1) {
  if (need_init()) return 1;
  if (dstr == 0) dstr = n;
  if (mstr == 0) mstr = k;
  if (sstr == 0) sstr = k;
  if (check_matmul_shape(name, m, n, k, dstr, mstr, sstr)) return 1;
  if (m == 0) return 0;
  if (!dst || !mat || !matsc || !src || !ssc) return fail("%s: null pointer", name);
  hipStream_t s = pick_stream(stream);
  const int perf_op = op >= 0 ? op : m == 1 ? kOpGemvInt8 : kOpGemmInt8;
  if (m == 1 && mstr == k && k <= kMaxGemvK8) {
    gh::GemvJobs jobs{};
    jobs.w[0] = mat;
    jobs.sc[0] = matsc;
    jobs.dst[0] = dst;
    for (int j = 0; j < gh::kMaxJobs; ++j) jobs.end[j] = n;
    jobs.njobs = 1;
    PerfScope perf(perf_op, s);
    const hipError_t e =
        gh::launch_gemv_i8(jobs, k, src, ssc, nullptr, nullptr, nullptr, g.info, s);
    if (e != hipSuccess) return fail("%s: gemv launch: %s", name, hipGetErrorString(e));
    return 0;
  }
  gh::GemmWs ws{};
  if (noalloc) {
    ws = gh::gemm_scratch(g.device);
    if (ws.base == nullptr) return fail("%s: scratch not resolved on device %d", name, g.device);
    const size_t need =
        gh::gemm_i8_scratch_bytes(m, n, k, false, mat, mstr, src, sstr, dstr, g.info);
    if (need > ws.bytes)
      return fail("%s: m=%d n=%d k=%d needs %zu bytes of scratch, more than the %zu it has",
                  name, m, n, k, need, ws.bytes);
  }
  PerfScope perf(perf_op, s);  // after the checks: a refused call is not timed
  const hipError_t e = gh::launch_gemm_i8(dst, dstr, 0, mat, mstr, matsc, src, sstr, ssc, m,
                                          n, k, g.info, s, noalloc ? &ws : nullptr);
  if (e != hipSuccess) return fail("%s: gemm launch: %s", name, hipGetErrorString(e));
  return 0;
}

}  // namespace

extern "C" {

int gemma_hip_matmul(float *dst, int dstr, const int8_t *mat, int mstr,
                     const float *matsc, const int8_t *src, int sstr,
                     const float *ssc, int m, int n, int k, void *stream) {
  return matmul_impl("gemma_hip_matmul", dst, dstr, mat, mstr, matsc, src, sstr, ssc, m, n, k,
                     stream, false);
}

int gemma_hip_matmul_noalloc(float *dst, int dstr, const int8_t *mat, int mstr,
                             const float *matsc, const int8_t *src, int sstr,
                             const float *ssc, int m, int n, int k, void *stream) {
  return matmul_impl("gemma_hip_matmul_noalloc", dst, dstr, mat, mstr, matsc, src, sstr, ssc, m,
                     n, k, stream, true);
}

int gemma_hip_matmul_cols(float *dst, int dstr, const gemma_hip_job *jobs, int njobs,
                          const int8_t *src, int sstr, const float *ssc, int m, int k,
                          void *stream) {
  const char *name = "gemma_hip_matmul_cols";
  if (need_init()) return 1;
  if (jobs == nullptr || njobs < 1 || njobs > gh::kMaxGemmSegs)
    return fail("%s: njobs=%d outside 1..%d", name, njobs, gh::kMaxGemmSegs);
  gh::GemmSegs bs{};
  long n = 0;
  for (int j = 0; j < njobs; ++j) {
    if (jobs[j].m <= 0) return fail("%s: job %d has m=%d rows", name, j, jobs[j].m);
    if (jobs[j].w == nullptr || jobs[j].sc == nullptr)
      return fail("%s: job %d has a null weight or scale pointer", name, j);
    n += jobs[j].m;
    if (n > (1l << 30)) return fail("%s: %ld output columns", name, n);
    bs.w[j] = static_cast<const int8_t *>(jobs[j].w);
    bs.s[j] = jobs[j].sc;
    bs.end[j] = (int)n;
  }
  bs.nseg = njobs;
  if (dstr == 0) dstr = (int)n;
  if (sstr == 0) sstr = k;
  if (check_matmul_shape(name, m, (int)n, k, dstr, k, sstr)) return 1;
  if (m == 0) return 0;
  if (!dst || !src || !ssc) return fail("%s: null pointer", name);
  hipStream_t s = pick_stream(stream);
  PerfScope perf(kOpGemmInt8, s);
  GH_CHECK("gemma_hip_matmul_cols: launch",
           gh::launch_gemm_i8_segs(dst, dstr, bs, src, sstr, ssc, m, k, g.info, s));
  return 0;
}

int gemma_hip_matmul_f32_cols(float *dst, int dstr, const gemma_hip_job *jobs, int njobs,
                              const float *src, int sstr, int m, int k, void *stream) {
  const char *name = "gemma_hip_matmul_f32_cols";
  if (need_init()) return 1;
  if (jobs == nullptr || njobs < 1 || njobs > gh::kMaxGemmSegs)
    return fail("%s: njobs=%d outside 1..%d", name, njobs, gh::kMaxGemmSegs);
  gh::F32Segs bs{};
  long n = 0;
  for (int j = 0; j < njobs; ++j) {
    if (jobs[j].m <= 0) return fail("%s: job %d has m=%d rows", name, j, jobs[j].m);
    if (jobs[j].w == nullptr) return fail("%s: job %d has a null weight pointer", name, j);
    n += jobs[j].m;
    if (n > (1l << 30)) return fail("%s: %ld output columns", name, n);
    bs.w[j] = static_cast<const float *>(jobs[j].w);
    bs.end[j] = (int)n;
  }
  bs.nseg = njobs;
  if (dstr == 0) dstr = (int)n;
  if (sstr == 0) sstr = k;
  if (check_matmul_shape(name, m, (int)n, k, dstr, k, sstr)) return 1;
  if (m == 0) return 0;
  if (!dst || !src) return fail("%s: null pointer", name);
  hipStream_t s = pick_stream(stream);
  PerfScope perf(kOpGemmFpx, s);
  GH_CHECK("gemma_hip_matmul_f32_cols: launch",
           gh::launch_gemm_f32_segs(dst, dstr, bs, k, src, sstr, m, k, gh::F32Epilogue{},
                                    g.info, s, false));
  return 0;
}

int gemma_hip_matmul_heads(float *dst, const int8_t *mat, const float *matsc,
                           const int8_t *src, const float *ssc, int m,
                           int heads, int hdim, int k, void *stream) {
  if (need_init()) return 1;
  if (m < 0 || heads <= 0 || hdim <= 0 || k <= 0 || (long)heads * hdim > (1l << 30))
    return fail("gemma_hip_matmul_heads: bad shape m=%d heads=%d hdim=%d k=%d", m,
                heads, hdim, k);
  if (m == 0) return 0;
  if (!dst || !mat || !matsc || !src || !ssc)
    return fail("gemma_hip_matmul_heads: null pointer");
  PerfScope perf(kOpGemmInt8, pick_stream(stream));
  GH_CHECK("gemma_hip_matmul_heads: launch",
           gh::launch_gemm_i8(dst, hdim, hdim, mat, k, matsc, src, k, ssc, m,
                              heads * hdim, k, g.info, pick_stream(stream)));
  return 0;
}

int gemma_hip_matmul_multi(const gemma_hip_job *jobs, int njobs,
                           const int8_t *x, const float *xs, int k,
                           void *stream) {
  if (need_init()) return 1;
  gh::GemvJobs gj;
  if (build_jobs("gemma_hip_matmul_multi", jobs, njobs, &gj)) return 1;
  if (k <= 0 || k > kMaxGemvK8)
    return fail("gemma_hip_matmul_multi: k=%d outside 1..%d", k, kMaxGemvK8);
  if (x == nullptr || xs == nullptr)
    return fail("gemma_hip_matmul_multi: null activation pointer");
  for (int j = 0; j < njobs; ++j)
    if (jobs[j].m > 0 && jobs[j].sc == nullptr)
      return fail("gemma_hip_matmul_multi: job %d has no scales", j);
  if (gj.end[njobs - 1] == 0) return 0;
  PerfScope perf(kOpGemvInt8, pick_stream(stream));
  GH_CHECK("gemma_hip_matmul_multi: launch",
           gh::launch_gemv_i8(gj, k, x, xs, nullptr, nullptr, nullptr, g.info,
                              pick_stream(stream)));
  return 0;
}

int gemma_hip_quantize_matmul(const gemma_hip_job *jobs, int njobs,
                              const float *x, int k, int8_t *xq, float *xs,
                              void *stream) {
  if (need_init()) return 1;
  gh::GemvJobs gj;
  if (build_jobs("gemma_hip_quantize_matmul", jobs, njobs, &gj)) return 1;
  if (k <= 0 || k > kMaxGemvK8)
    return fail("gemma_hip_quantize_matmul: k=%d outside 1..%d", k, kMaxGemvK8);
  if (x == nullptr) return fail("gemma_hip_quantize_matmul: null activation pointer");
  for (int j = 0; j < njobs; ++j)
    if (jobs[j].m > 0 && jobs[j].sc == nullptr)
      return fail("gemma_hip_quantize_matmul: job %d has no scales", j);
  hipStream_t s = pick_stream(stream);
  // the quantize is fused into the GEMV kernel: one launch, timed as gemv_int8
  PerfScope perf(gj.end[njobs - 1] == 0 ? kOpQuantizeAct : kOpGemvInt8, s);
  if (gj.end[njobs - 1] == 0) {
    // no rows: still produce the quantized vector when asked for
    if (xq != nullptr && xs != nullptr)
      GH_CHECK("gemma_hip_quantize_matmul: quantize",
               gh::launch_quantize(xq, xs, x, k, 1, k, s));
    return 0;
  }
  GH_CHECK("gemma_hip_quantize_matmul: launch",
           gh::launch_gemv_i8(gj, k, nullptr, nullptr, x, xq, xs, g.info, s));
  return 0;
}

}  // extern "C"

namespace {
int matmul_f32_impl(float *dst, int dstr, const float *mat, int mstr, const float *src,
                    int sstr, int m, int n, int k, void *stream, int op);
}  // namespace

extern "C" {

int gemma_hip_matmul_f32(float *dst, int dstr, const float *mat, int mstr,
                         const float *src, int sstr, int m, int n, int k,
                         void *stream) {
  return matmul_f32_impl(dst, dstr, mat, mstr, src, sstr, m, n, k, stream, -1);
}

}  // extern "C"

namespace {
// gemma_hip_matmul_f32; op >= 0 names the timed op (the _host gemm_fpx
// drop-in counts m == 1 calls as gemm_fpx, as the reference does)
int matmul_f32_impl(float *dst, int dstr, const float *mat, int mstr, const float *src,
                    int sstr, int m, int n, int k, void *stream, int op) {
  if (need_init()) return 1;
  if (dstr == 0) dstr = n;
  if (mstr == 0) mstr = k;
  if (sstr == 0) sstr = k;
  if (check_matmul_shape("gemma_hip_matmul_f32", m, n, k, dstr, mstr, sstr)) return 1;
  if (m == 0) return 0;
  if (!dst || !mat || !src) return fail("gemma_hip_matmul_f32: null pointer");
  hipStream_t s = pick_stream(stream);
  PerfScope perf(op >= 0 ? op : m == 1 ? kOpGemvFpx : kOpGemmFpx, s);
  if (m == 1 && mstr == k && k <= kMaxGemvK32) {
    gh::GemvJobs jobs{};
    jobs.w[0] = mat;
    jobs.dst[0] = dst;
    for (int j = 0; j < gh::kMaxJobs; ++j) jobs.end[j] = n;
    jobs.njobs = 1;
    GH_CHECK("gemma_hip_matmul_f32: gemv launch",
             gh::launch_gemv_f32(jobs, k, src, g.info, s));
    return 0;
  }
  GH_CHECK("gemma_hip_matmul_f32: gemm launch",
           gh::launch_gemm_f32(dst, dstr, mat, mstr, src, sstr, m, n, k, nullptr, false,
                               g.info, s));
  return 0;
}
}  // namespace

extern "C" {

int gemma_hip_matmul_f32_multi(const gemma_hip_job *jobs, int njobs,
                               const float *x, int k, void *stream) {
  if (need_init()) return 1;
  gh::GemvJobs gj;
  if (build_jobs("gemma_hip_matmul_f32_multi", jobs, njobs, &gj)) return 1;
  if (k <= 0 || k > kMaxGemvK32)
    return fail("gemma_hip_matmul_f32_multi: k=%d outside 1..%d", k, kMaxGemvK32);
  if (x == nullptr) return fail("gemma_hip_matmul_f32_multi: null activation pointer");
  if (gj.end[njobs - 1] == 0) return 0;
  PerfScope perf(kOpGemvFpx, pick_stream(stream));
  GH_CHECK("gemma_hip_matmul_f32_multi: launch",
           gh::launch_gemv_f32(gj, k, x, g.info, pick_stream(stream)));
  return 0;
}

int gemma_hip_patch_embed(float *dst, const float *img, const float *pe,
                          const float *pe_b, int img_px, int psize, int dim,
                          float *work, void *stream) {
  if (need_init()) return 1;
  if (psize <= 0 || img_px <= 0 || dim <= 0 || img_px % psize != 0)
    return fail("gemma_hip_patch_embed: bad shape img_px=%d psize=%d dim=%d", img_px,
                psize, dim);
  if (!dst || !img || !pe || !pe_b) return fail("gemma_hip_patch_embed: null pointer");
  const long ppi = img_px / psize;
  const long npatch = ppi * ppi;
  const long kdim = 3l * psize * psize;
  if (npatch * kdim > (1l << 30) || npatch * dim > (1l << 30) ||
      (long)img_px * img_px * 3 > (1l << 30))
    return fail("gemma_hip_patch_embed: image too large");
  hipStream_t st = pick_stream(stream);
  if (work == nullptr) {
    const size_t need = (size_t)npatch * kdim * sizeof(float);
    if (need > g.work_bytes) {
      if (g.work != nullptr) {
        GH_CHECK("gemma_hip_patch_embed: sync", hipDeviceSynchronize());
        GH_CHECK("gemma_hip_patch_embed: free", hipFree(g.work));
        g.work = nullptr;
        g.work_bytes = 0;
      }
      GH_CHECK("gemma_hip_patch_embed: workspace", hipMalloc(&g.work, need));
      g.work_bytes = need;
    }
    work = g.work;
  }
  GH_CHECK("gemma_hip_patch_embed: im2col",
           gh::launch_im2col(work, img, img_px, psize, st));
  GH_CHECK("gemma_hip_patch_embed: gemm",
           gh::launch_gemm_f32(dst, dim, pe, (int)kdim, work, (int)kdim, (int)npatch, dim,
                               (int)kdim, pe_b, true, g.info, st));
  return 0;
}

int gemma_hip_vision_attention(float *out, const float *qkv, const float *bias, int n,
                               int n_heads, int dim, int mode, void *stream) {
  if (need_init()) return 1;
  if (!out || !qkv || !bias) return fail("gemma_hip_vision_attention: null pointer");
  const int hdim = n_heads > 0 && dim % n_heads == 0 ? dim / n_heads : 0;
  if (n < 1 || (hdim != 16 && hdim != 32 && hdim != 64 && hdim != 72 && hdim != 128) ||
      (long)n * 3 * dim > (1l << 30))
    return fail("gemma_hip_vision_attention: unsupported shape n=%d heads=%d dim=%d "
                "(head dim 16, 32, 64, 72 or 128)", n, n_heads, dim);
  if (mode != GEMMA_HIP_ATTN_F64 && mode != GEMMA_HIP_ATTN_F32)
    return fail("gemma_hip_vision_attention: unknown mode %d", mode);
  const gh::VisAttn at{qkv, 3 * dim, bias, out, n, n_heads, dim, 1.0f / sqrtf((float)hdim)};
  GH_CHECK("gemma_hip_vision_attention: launch",
           gh::launch_vis_attention(at, hdim, mode == GEMMA_HIP_ATTN_F32, pick_stream(stream)));
  return 0;
}

int gemma_hip_prefill_attention(float *out, const float *q, int q_stride, const float *kc,
                                const float *vc, int n, int pos0, int n_heads, int nkv,
                                int hdim, int clen, int slide, float asc, float sc_att,
                                int dense, int mode, void *stream) {
  const char *name = "gemma_hip_prefill_attention";
  if (need_init()) return 1;
  if (!out || !q || !kc || !vc) return fail("%s: null pointer", name);
  const int hn = nkv > 0 && n_heads % nkv == 0 ? n_heads / nkv : 0;
  if (n < 1 || pos0 < 0 || hn < 1 || 32 % hn != 0 || (hdim != 128 && hdim != 256) ||
      n_heads > gh::kPfMaxMergeHeads || (long)n_heads * hdim > q_stride ||
      n_heads * hdim > 4 * 256 * gh::kPfMaxNpt ||
      (long)pos0 + n > clen || slide < 0 || (long)n * q_stride > (1l << 30) ||
      (long)nkv * clen * hdim > (1l << 30))
    return fail("%s: unsupported shape n=%d pos0=%d heads=%d/%d hdim=%d clen=%d stride=%d",
                name, n, pos0, n_heads, nkv, hdim, clen, q_stride);
  if (mode != GEMMA_HIP_ATTN_F64 && mode != GEMMA_HIP_ATTN_F32)
    return fail("%s: unknown mode %d", name, mode);
  hipStream_t s = pick_stream(stream);
  double *part = nullptr;
  GH_CHECK("gemma_hip_prefill_attention: workspace",
           hipMalloc(&part, gh::pf_attn_part_doubles(n, n_heads, hdim) * sizeof(double)));
  const gh::PfAttn at{q, q_stride, kc, vc, out, n_heads * hdim, n, pos0, n_heads, nkv, clen,
                      slide, asc, sc_att, part, 0, 0, 0, dense ? 1 : 0};
  hipError_t e = gh::launch_pf_attention(at, hdim, mode == GEMMA_HIP_ATTN_F32, g.info, s);
  const hipError_t e2 = hipStreamSynchronize(s);
  (void)hipFree(part);
  if (e != hipSuccess || (e = e2) != hipSuccess)
    return fail("%s: %s", name, hipGetErrorString(e));
  return 0;
}

/* ---- host drop-ins ------------------------------------------------------ */

// Inputs up to this size are read by the kernels straight from pinned host
// memory; larger ones are first copied to the device (DMA at full PCIe rate).
constexpr size_t kZeroCopyIn = 256u << 10;

int gemma_hip_quantize_act_host(int8_t *dst, float *scale, const float *vec,
                                int dim) {
  std::lock_guard<std::recursive_mutex> serial(g.host);
  if (need_init()) return 1;
  if (dim <= 0 || !dst || !scale || !vec)
    return fail("gemma_hip_quantize_act_host: bad arguments (dim=%d)", dim);
  return gemma_hip_quantize_acts_host(dst, scale, vec, dim, 1, dim);
}

int gemma_hip_quantize_acts_host(int8_t *dst, float *dsc, const float *src,
                                 int sstr, int m, int n) {
  std::lock_guard<std::recursive_mutex> serial(g.host);
  if (need_init()) return 1;
  if (sstr == 0) sstr = n;
  if (m < 0 || n <= 0 || sstr < n || !dst || !dsc || !src)
    return fail("gemma_hip_quantize_acts_host: bad arguments");
  if (m == 0) return 0;
  const size_t in_bytes = ((size_t)(m - 1) * sstr + n) * 4;
  if (act_reserve(m, n) || pinned_reserve(in_bytes)) return 1;
  memcpy(g.pinned, src, in_bytes);
  const float *in = (const float *)g.pinned_dev;
  if (in_bytes > kZeroCopyIn) {
    if (staging_reserve(in_bytes)) return 1;
    GH_CHECK("quantize_acts_host: H2D",
             hipMemcpyAsync(g.staging, g.pinned, in_bytes, hipMemcpyHostToDevice, g.stream));
    in = (const float *)g.staging;
  }
  PerfScope perf(kOpQuantizeAct, g.stream);
  GH_CHECK("quantize_acts_host: launch",
           gh::launch_quantize(g.act.dev_q, g.act.dev_s, in, sstr, m, n, g.stream,
                               g.act.mir_q_dev, g.act.mir_s_dev));
  GH_CHECK("quantize_acts_host: sync", hipStreamSynchronize(g.stream));
  memcpy(dst, g.act.mir_q, (size_t)m * n);
  memcpy(dsc, g.act.mir_s, (size_t)m * 4);
  g.act.host_q = dst;
  g.act.m = m;
  g.act.n = n;
  g.act.valid = true;
  return 0;
}

int gemma_hip_gemv_int8_host(float *dst, const int8_t *mat, const float *matsc,
                             const int8_t *vec, float vsc, int m, int n) {
  gemma_hip_job job{mat, matsc, dst, m};
  return gemma_hip_gemv_int8_multi_host(&job, 1, vec, vsc, n);
}

int gemma_hip_gemv_int8_multi_host(const gemma_hip_job *jobs, int njobs,
                                   const int8_t *vec, float vsc, int n) {
  std::lock_guard<std::recursive_mutex> serial(g.host);
  if (need_init()) return 1;
  if (jobs == nullptr || njobs < 1 || njobs > GEMMA_HIP_MAX_JOBS || n <= 0 || !vec)
    return fail("gemma_hip_gemv_int8_multi_host: bad arguments");
  gemma_hip_job djobs[GEMMA_HIP_MAX_JOBS];
  // outputs go straight to pinned memory; the int8 input comes from the
  // activation cache when it is what the last quantize returned
  Carver c;
  size_t o_y[GEMMA_HIP_MAX_JOBS];
  for (int j = 0; j < njobs; ++j) {
    if (jobs[j].m < 0) return fail("gemma_hip_gemv_int8_multi_host: job %d m<0", j);
    o_y[j] = c.take((size_t)jobs[j].m * 4);
  }
  const size_t o_x = c.take(n), o_s = c.take(4);
  if (pinned_reserve(c.used)) return 1;
  char *pin = g.pinned;
  for (int j = 0; j < njobs; ++j) {
    const size_t rows = (size_t)jobs[j].m;
    const void *w = rows ? resolve(jobs[j].w, rows * n) : nullptr;
    const void *sc = rows ? resolve(jobs[j].sc, rows * 4) : nullptr;
    if (rows && (w == nullptr || sc == nullptr))
      return fail("gemma_hip_gemv_int8_multi_host: job %d weights are not registered", j);
    djobs[j] = gemma_hip_job{w, (const float *)sc, (float *)(g.pinned_dev + o_y[j]),
                             jobs[j].m};
  }
  const int8_t *xq;
  const float *xs;
  const int r0 = act_lookup(vec, n, nullptr, vsc, 1, n);
  if (r0 >= 0) {
    xq = g.act.dev_q + (size_t)r0 * g.act.n;
    xs = g.act.dev_s + r0;
  } else {
    if (staging_reserve(256 + (size_t)n)) return 1;
    memcpy(pin + o_x, vec, n);
    memcpy(pin + o_s, &vsc, 4);
    GH_CHECK("gemv_int8_host: H2D",
             hipMemcpyAsync(g.staging + 256, pin + o_x, n, hipMemcpyHostToDevice, g.stream));
    GH_CHECK("gemv_int8_host: H2D",
             hipMemcpyAsync(g.staging, pin + o_s, 4, hipMemcpyHostToDevice, g.stream));
    xq = (const int8_t *)(g.staging + 256);
    xs = (const float *)g.staging;
  }
  if (gemma_hip_matmul_multi(djobs, njobs, xq, xs, n, g.stream)) return 1;
  GH_CHECK("gemv_int8_host: sync", hipStreamSynchronize(g.stream));
  for (int j = 0; j < njobs; ++j)
    if (jobs[j].m > 0) memcpy(jobs[j].dst, pin + o_y[j], (size_t)jobs[j].m * 4);
  return 0;
}

int gemma_hip_gemm_int8_host(float *dst, int dstr, const int8_t *mat, int mstr,
                             const float *matsc, const int8_t *src, int sstr,
                             const float *ssc, int m, int n, int k) {
  std::lock_guard<std::recursive_mutex> serial(g.host);
  if (need_init()) return 1;
  if (dstr == 0) dstr = n;
  if (mstr == 0) mstr = k;
  if (sstr == 0) sstr = k;
  if (check_matmul_shape("gemma_hip_gemm_int8_host", m, n, k, dstr, mstr, sstr))
    return 1;
  if (m == 0) return 0;
  if (!dst || !mat || !matsc || !src || !ssc)
    return fail("gemma_hip_gemm_int8_host: null pointer");
  const void *dmat = resolve(mat, (size_t)(n - 1) * mstr + k);
  const void *dsc = resolve(matsc, (size_t)n * 4);
  if (dmat == nullptr || dsc == nullptr)
    return fail("gemma_hip_gemm_int8_host: weights are not registered");
  const size_t src_bytes = (size_t)(m - 1) * sstr + k;
  Carver c;
  size_t o_a = c.take(src_bytes), o_as = c.take((size_t)m * 4),
         o_y = c.take((size_t)m * dstr * 4);
  if (staging_reserve(c.used)) return 1;
  char *base = g.staging;
  const int8_t *a = (const int8_t *)(base + o_a);
  const float *as = (const float *)(base + o_as);
  const int r0 = act_lookup(src, sstr, ssc, 0.0f, m, k);
  if (r0 >= 0) {
    a = g.act.dev_q + (size_t)r0 * g.act.n;
    as = g.act.dev_s + r0;
  } else {
    GH_CHECK("gemm_int8_host: H2D",
             hipMemcpyAsync(base + o_a, src, src_bytes, hipMemcpyHostToDevice, g.stream));
    GH_CHECK("gemm_int8_host: H2D",
             hipMemcpyAsync(base + o_as, ssc, (size_t)m * 4, hipMemcpyHostToDevice, g.stream));
  }
  if (matmul_impl("gemma_hip_gemm_int8_host", (float *)(base + o_y), dstr,
                  (const int8_t *)dmat, mstr, (const float *)dsc, a, sstr, as, m, n, k,
                  g.stream, false, kOpGemmInt8))
    return 1;
  GH_CHECK("gemm_int8_host: D2H",
           hipMemcpy2DAsync(dst, (size_t)dstr * 4, base + o_y, (size_t)dstr * 4,
                            (size_t)n * 4, m, hipMemcpyDeviceToHost, g.stream));
  GH_CHECK("gemm_int8_host: sync", hipStreamSynchronize(g.stream));
  return 0;
}

int gemma_hip_gemv_fpx_host(float *dst, const float *mat, const float *vec,
                            int m, int n) {
  gemma_hip_job job{mat, nullptr, dst, m};
  return gemma_hip_gemv_fpx_multi_host(&job, 1, vec, n);
}

int gemma_hip_gemv_fpx_multi_host(const gemma_hip_job *jobs, int njobs,
                                  const float *vec, int n) {
  std::lock_guard<std::recursive_mutex> serial(g.host);
  if (need_init()) return 1;
  if (jobs == nullptr || njobs < 1 || njobs > GEMMA_HIP_MAX_JOBS || n <= 0 || !vec)
    return fail("gemma_hip_gemv_fpx_multi_host: bad arguments");
  gemma_hip_job djobs[GEMMA_HIP_MAX_JOBS];
  Carver c;
  size_t o_x = c.take((size_t)n * 4), o_y[GEMMA_HIP_MAX_JOBS];
  for (int j = 0; j < njobs; ++j) {
    if (jobs[j].m < 0) return fail("gemma_hip_gemv_fpx_multi_host: job %d m<0", j);
    o_y[j] = c.take((size_t)jobs[j].m * 4);
  }
  if (staging_reserve(c.used)) return 1;
  char *base = g.staging;
  for (int j = 0; j < njobs; ++j) {
    const size_t rows = (size_t)jobs[j].m;
    const void *w = rows ? resolve(jobs[j].w, rows * n * 4) : nullptr;
    if (rows && w == nullptr)
      return fail("gemma_hip_gemv_fpx_multi_host: job %d weights are not registered", j);
    djobs[j] = gemma_hip_job{w, nullptr, (float *)(base + o_y[j]), jobs[j].m};
  }
  GH_CHECK("gemv_fpx_host: H2D",
           hipMemcpyAsync(base + o_x, vec, (size_t)n * 4, hipMemcpyHostToDevice, g.stream));
  if (gemma_hip_matmul_f32_multi(djobs, njobs, (const float *)(base + o_x), n, g.stream))
    return 1;
  for (int j = 0; j < njobs; ++j)
    if (jobs[j].m > 0)
      GH_CHECK("gemv_fpx_host: D2H",
               hipMemcpyAsync(jobs[j].dst, base + o_y[j], (size_t)jobs[j].m * 4,
                              hipMemcpyDeviceToHost, g.stream));
  GH_CHECK("gemv_fpx_host: sync", hipStreamSynchronize(g.stream));
  return 0;
}

int gemma_hip_gemm_fpx_host(float *dst, int dstr, const float *mat, int mstr,
                            const float *src, int sstr, int m, int n, int k) {
  std::lock_guard<std::recursive_mutex> serial(g.host);
  if (need_init()) return 1;
  if (dstr == 0) dstr = n;
  if (mstr == 0) mstr = k;
  if (sstr == 0) sstr = k;
  if (check_matmul_shape("gemma_hip_gemm_fpx_host", m, n, k, dstr, mstr, sstr))
    return 1;
  if (m == 0) return 0;
  if (!dst || !mat || !src) return fail("gemma_hip_gemm_fpx_host: null pointer");
  const void *dmat = resolve(mat, ((size_t)(n - 1) * mstr + k) * 4);
  if (dmat == nullptr) return fail("gemma_hip_gemm_fpx_host: weights are not registered");
  const size_t src_floats = (size_t)(m - 1) * sstr + k;
  Carver c;
  size_t o_a = c.take(src_floats * 4), o_y = c.take((size_t)m * dstr * 4);
  if (staging_reserve(c.used)) return 1;
  char *base = g.staging;
  GH_CHECK("gemm_fpx_host: H2D",
           hipMemcpyAsync(base + o_a, src, src_floats * 4, hipMemcpyHostToDevice, g.stream));
  if (matmul_f32_impl((float *)(base + o_y), dstr, (const float *)dmat, mstr,
                      (const float *)(base + o_a), sstr, m, n, k, g.stream, kOpGemmFpx))
    return 1;
  GH_CHECK("gemm_fpx_host: D2H",
           hipMemcpy2DAsync(dst, (size_t)dstr * 4, base + o_y, (size_t)dstr * 4,
                            (size_t)n * 4, m, hipMemcpyDeviceToHost, g.stream));
  GH_CHECK("gemm_fpx_host: sync", hipStreamSynchronize(g.stream));
  return 0;
}


int gemma_hip_patch_embed_host(float *dst, const float *img, const float *pe,
                               const float *pe_b, int img_px, int psize, int dim) {
  std::lock_guard<std::recursive_mutex> serial(g.host);
  if (need_init()) return 1;
  if (psize <= 0 || img_px <= 0 || dim <= 0 || img_px % psize != 0 || !dst || !img ||
      !pe || !pe_b)
    return fail("gemma_hip_patch_embed_host: bad arguments");
  const size_t kdim = 3ul * psize * psize;
  const size_t npatch = (size_t)(img_px / psize) * (img_px / psize);
  const void *dpe = resolve(pe, (size_t)dim * kdim * 4);
  const void *db = resolve(pe_b, (size_t)dim * 4);
  if (dpe == nullptr || db == nullptr)
    return fail("gemma_hip_patch_embed_host: weights are not registered");
  const size_t img_bytes = (size_t)img_px * img_px * 3 * 4;
  Carver c;
  size_t o_img = c.take(img_bytes), o_y = c.take(npatch * dim * 4);
  if (staging_reserve(c.used)) return 1;
  char *base = g.staging;
  GH_CHECK("patch_embed_host: H2D",
           hipMemcpyAsync(base + o_img, img, img_bytes, hipMemcpyHostToDevice, g.stream));
  if (gemma_hip_patch_embed((float *)(base + o_y), (const float *)(base + o_img),
                            (const float *)dpe, (const float *)db, img_px, psize, dim,
                            nullptr, g.stream))
    return 1;
  GH_CHECK("patch_embed_host: D2H",
           hipMemcpyAsync(dst, base + o_y, npatch * dim * 4, hipMemcpyDeviceToHost, g.stream));
  GH_CHECK("patch_embed_host: sync", hipStreamSynchronize(g.stream));
  return 0;
}

}  // extern "C"

/* ---- device-resident decoder -------------------------------------------- */

struct gemma_hip_decoder {
  gemma_hip_text_config cfg{};
  std::vector<unsigned char> swa;
  int clen = 0, max_blocks = 0, nparts = 256;
  bool attn_f32 = true;  // prefill attention on the fp32 matrix cores (false: fp64)
  bool quant = true;     // W8A8 weights; false: an fp32 ('U') model
  struct Layer {
    const int8_t *w[7];  // wq wk wv wo w1(up) w2(gate) w3(down), device
    const float *s[7];
    const float *wf[7];  // the same, fp32 ('U'), device
    float *nq, *nk, *n1, *n2, *n3, *n4;  // device copies
  };
  std::vector<Layer> layers;
  const int8_t *emb = nullptr;
  const float *emb_s = nullptr;
  const float *emb_f = nullptr;  // fp32 embedding / LM head ('U')
  float *fnorm = nullptr;
  char *mem = nullptr;  // every device buffer below lives in this allocation
  float *x[2]{}, *xq = nullptr, *xk = nullptr, *xv = nullptr, *xo = nullptr;
  float *yattn = nullptr, *gbuf = nullptr, *ymlp = nullptr, *h = nullptr;
  float *logits = nullptr, *rope_l = nullptr, *rope_g = nullptr;
  double *part = nullptr;
  float *kv = nullptr, *pval = nullptr;
  int *pidx = nullptr, *step = nullptr, *tokens = nullptr;
  int *pin = nullptr;  // pinned: step upload [4] and token readback [1]
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  // row buffers of the batched prefill, allocated on first use for pf_rows rows
  char *pf_mem = nullptr;
  int pf_rows = 0;
  float *pf_x = nullptr, *pf_y = nullptr, *pf_qkv = nullptr, *pf_xo = nullptr, *pf_g = nullptr;
  float *pf_as = nullptr;
  int8_t *pf_a8 = nullptr;
  float *pf_h = nullptr;  // normalized rows ('U': the fp32 GEMMs' input)
  int *pf_tok = nullptr;
  double *pf_part = nullptr;  // attention key-split partials
};

namespace {

void decoder_free(gemma_hip_decoder *d) {
  if (d == nullptr) return;
  if (d->exec != nullptr) (void)hipGraphExecDestroy(d->exec);
  if (d->graph != nullptr) (void)hipGraphDestroy(d->graph);
  if (d->mem != nullptr) (void)hipFree(d->mem);
  if (d->pf_mem != nullptr) (void)hipFree(d->pf_mem);
  if (d->pin != nullptr) (void)hipHostFree(d->pin);
  delete d;
}

// Row buffers of the batched prefill for n rows (kept, and regrown only for
// a larger n): x, y [n][dim]; q/k/v [n][q_sz + 2 kv_sz]; attention output
// [n][q_sz]; gate|up [n][2 mlp]; quantized rows [n][max K] + their scales.
int prefill_reserve(gemma_hip_decoder *d, int n) {
  if (n <= d->pf_rows) return 0;
  const gemma_hip_text_config &c = d->cfg;
  const size_t rows = (size_t)n, q_sz = (size_t)c.n_heads * c.hdim,
               kv_sz = (size_t)c.nkv * c.hdim, dim = c.dim, mlp = c.mlp_dim;
  const size_t kmax = std::max(dim, std::max(q_sz, mlp));
  Carver cv;
  const size_t o_x = cv.take(rows * dim * 4), o_y = cv.take(rows * dim * 4),
               o_qkv = cv.take(rows * (q_sz + 2 * kv_sz) * 4), o_xo = cv.take(rows * q_sz * 4),
               o_g = cv.take(rows * 2 * mlp * 4), o_a8 = cv.take(rows * kmax),
               o_as = cv.take(rows * 4), o_tok = cv.take(rows * 4),
               o_part = cv.take(gh::pf_attn_part_doubles(rows, c.n_heads, c.hdim) * 8),
               o_h = cv.take(d->quant ? 0 : rows * dim * 4);
  if (d->pf_mem != nullptr) {
    (void)hipStreamSynchronize(g.stream);
    (void)hipFree(d->pf_mem);
    d->pf_mem = nullptr;
    d->pf_rows = 0;
  }
  hipError_t e = hipMalloc((void **)&d->pf_mem, cv.used);
  if (e != hipSuccess) return hip_fail("gemma_hip_decoder_prefill: alloc", e);
  char *m = d->pf_mem;
  d->pf_x = (float *)(m + o_x);
  d->pf_y = (float *)(m + o_y);
  d->pf_qkv = (float *)(m + o_qkv);
  d->pf_xo = (float *)(m + o_xo);
  d->pf_g = (float *)(m + o_g);
  d->pf_a8 = (int8_t *)(m + o_a8);
  d->pf_as = (float *)(m + o_as);
  d->pf_tok = (int *)(m + o_tok);
  d->pf_part = (double *)(m + o_part);
  d->pf_h = d->quant ? nullptr : (float *)(m + o_h);
  d->pf_rows = n;
  return 0;
}

// Enqueues the prompt pass of rows pos .. pos+n-1 (forward_text_chunk,
// gemma.c:4985-5453) and the decode step's tail on the last row.  The step
// record must hold {last token, pos + n - 1, 0} (the argmax advances it).
// embed: the rows are the tokens in pf_tok, embedded here; else pf_x holds
// them already.  dense: mask=false, every row attends to every key up to the
// last row, with no sliding window (gemma.c:5258-5290).
constexpr int kWarmRows = 256;  // rows from which a GEMM's weights are read ahead of it

// Each launch is timed as the reference op it stands for when timing is on
// (fused kernels as the op they open with; the attention kernels, which hold
// the reference's score and value products too, as softmax).
#define GH_OP(op, expr) timed((op), st, [&] { return (expr); })

hipError_t prefill_enqueue_f32(gemma_hip_decoder *d, int n, int pos, bool embed, bool dense,
                               hipStream_t st);
hipError_t decoder_enqueue_f32(gemma_hip_decoder *d, hipStream_t st);

hipError_t prefill_enqueue(gemma_hip_decoder *d, int n, int pos, bool embed, bool dense,
                           hipStream_t st) {
  const gemma_hip_text_config &c = d->cfg;
  const int q_sz = c.n_heads * c.hdim, kv_sz = c.nkv * c.hdim, dim = c.dim, mlp = c.mlp_dim;
  const int stride = q_sz + 2 * kv_sz;
  const size_t cache = (size_t)d->clen * kv_sz;
  hipError_t e;
  auto gemm = [&](float *dst, int dstr, const int8_t *w, const float *ws, int nout, int k) {
    return GH_OP(kOpGemmInt8, gh::launch_gemm_i8(dst, dstr, 0, w, k, ws, d->pf_a8, k, d->pf_as,
                                                 n, nout, k, g.info, st));
  };
  if (!d->quant) return prefill_enqueue_f32(d, n, pos, embed, dense, st);
  if (embed && (e = gh::launch_pf_embed(d->pf_tok, n, d->emb, d->emb_s, nullptr, d->pf_x, dim,
                                        c.mlp_pre ? 1.0f : sqrtf((float)dim), st)) != hipSuccess)
    return e;
  for (int l = 0; l < c.nl; ++l) {
    const auto &L = d->layers[l];
    // residual of the previous MLP (post-FFN norm), pre-attention norm, quantize
    const gh::PfNorm n1{d->pf_x, l > 0 ? d->pf_y : nullptr,
                        (l > 0 && c.mlp_pst) ? d->layers[l - 1].n4 : nullptr, L.n1, d->pf_a8,
                        d->pf_as, dim, c.eps};
    if ((e = GH_OP(kOpRmsnorm, gh::launch_pf_norm_rows(n1, n, st))) != hipSuccess) return e;
    // q, k, v rows (gemma.c:5045-5089)
    const gh::GemmSegs qkv{{L.w[0], L.w[1], L.w[2]}, {L.s[0], L.s[1], L.s[2]},
                           {q_sz, q_sz + kv_sz, q_sz + 2 * kv_sz}, 3};
    if ((e = GH_OP(kOpGemmInt8, gh::launch_gemm_i8_segs(d->pf_qkv, stride, qkv, d->pf_a8, dim,
                                                        d->pf_as, n, dim, g.info, st))) !=
        hipSuccess)
      return e;
    // q/k norm, RoPE, KV append, attention
    const bool sliding = d->swa[l] != 0;
    float *kc = d->kv + (size_t)l * 2 * cache;
    const gh::PfRope rp{d->pf_qkv, stride, q_sz, c.qk_norm ? L.nq : nullptr,
                        c.qk_norm ? L.nk : nullptr, sliding ? d->rope_l : d->rope_g, kc,
                        kc + cache, d->clen, pos, c.n_heads, c.nkv, c.eps};
    if ((e = GH_OP(kOpRope, gh::launch_pf_qk_rope(rp, n, c.hdim, st))) != hipSuccess) return e;
    // the attention's merge pass also quantizes its rows for the o projection
    const gh::PfAttn at{d->pf_qkv, stride, kc, kc + cache, d->pf_xo, q_sz, n, pos, c.n_heads,
                        c.nkv, d->clen, sliding ? c.slide : 0,
                        (float)(1.0f / sqrtf((float)c.q_scale)), c.sc_att, d->pf_part, 0, 0,
                        0, dense ? 1 : 0, d->pf_a8, d->pf_as};
    if ((e = GH_OP(kOpSoftmax, gh::launch_pf_attention(at, c.hdim, d->attn_f32, g.info, st))) !=
        hipSuccess)
      return e;
    // o projection
    if ((e = gemm(d->pf_y, dim, L.w[3], L.s[3], dim, q_sz)) != hipSuccess) return e;
    // residual of the attention (post-attention norm), pre-FFN norm, quantize
    const gh::PfNorm n3{d->pf_x, d->pf_y, c.mlp_pre ? L.n2 : nullptr, c.mlp_pre ? L.n3 : L.n2,
                        d->pf_a8, d->pf_as, dim, c.eps};
    if ((e = GH_OP(kOpRmsnorm, gh::launch_pf_norm_rows(n3, n, st))) != hipSuccess) return e;
    // The GELU kernel reads the down weights after its rows, so that the down
    // GEMM finds them in the Infinity Cache: a GEMM whose weights stream from
    // HBM runs latency-bound on them (gemma-3-4b down alone: 70 us with its
    // weights cached, 93 us from HBM).  Measured on the prefill: 4b 2048
    // tokens 20.30 -> 19.49 ms, 1b 512 tokens 3.20 -> 3.15 ms; at 270m's 32
    // rows 1.16 -> 1.19 ms, hence the row threshold.
    gh::WarmRegions wdown{};
    if (n >= kWarmRows) wdown = {{L.w[6]}, {(size_t)dim * mlp}, 1};
    // gate (w2), up (w1) (gemma.c:5365-5373), GELU(gate) * up, quantize, down
    const gh::GemmSegs gu{{L.w[5], L.w[4], nullptr}, {L.s[5], L.s[4], nullptr},
                          {mlp, 2 * mlp, 2 * mlp}, 2};
    if ((e = GH_OP(kOpGemmInt8, gh::launch_gemm_i8_segs(d->pf_g, 2 * mlp, gu, d->pf_a8, dim,
                                                        d->pf_as, n, dim, g.info, st))) !=
            hipSuccess ||
        (e = GH_OP(kOpGelu, gh::launch_pf_gelu_quant(d->pf_g, n, mlp, d->pf_a8, d->pf_as, wdown,
                                                     st))) != hipSuccess ||
        (e = gemm(d->pf_y, dim, L.w[6], L.s[6], dim, mlp)) != hipSuccess)
      return e;
  }
  // the last row: last residual, final norm, LM head, softcap, argmax
  const size_t last = (size_t)(n - 1) * dim;
  gh::DecNorm fn{d->pf_x + last, d->pf_y + last,
                 c.mlp_pst ? d->layers[c.nl - 1].n4 : nullptr, d->fnorm, nullptr, d->h, dim,
                 c.eps};
  if ((e = GH_OP(kOpRmsnorm, gh::launch_dec_final_norm(fn, st))) != hipSuccess) return e;
  gh::GemvJobs lm{};
  lm.w[0] = d->emb; lm.sc[0] = d->emb_s; lm.dst[0] = d->logits;
  for (int j = 0; j < gh::kMaxJobs; ++j) lm.end[j] = c.nvocab;
  lm.njobs = 1;
  if ((e = GH_OP(kOpGemvInt8, gh::launch_gemv_i8(lm, dim, nullptr, nullptr, d->h, nullptr,
                                                  nullptr, g.info, st))) != hipSuccess)
    return e;
  // the softcap and argmax are sample_from_logits, which the reference
  // counts in the decode phase (gemma.c:5776)
  return timed(kOpSample, st, [&] {
    hipError_t es = hipSuccess;
    if (c.sc_log != 0.0f) es = gh::launch_dec_softcap(d->logits, c.nvocab, c.sc_log, st);
    if (es != hipSuccess) return es;
    return gh::launch_dec_argmax(d->logits, c.nvocab, d->pval, d->pidx, d->nparts, d->step,
                                 d->tokens, d->clen, st);
  }, kPhaseDecode);
}

// The checks every prefill entry point makes of n rows at pos.
int prefill_check(const gemma_hip_decoder *dec, const char *name, int n, int pos) {
  const gemma_hip_text_config &c = dec->cfg;
  if (n < 1 || pos < 0 || pos > dec->clen - n)
    return fail("%s: %d rows at pos %d out of range (clen %d)", name, n, pos, dec->clen);
  const int hn = c.n_heads / c.nkv;
  if ((c.hdim != 128 && c.hdim != 256) || 32 % hn != 0 || c.mlp_dim > 4 * 1024 * gh::kPfMaxNpt ||
      c.n_heads * c.hdim > 4 * 256 * gh::kPfMaxNpt)
    return fail("%s: unsupported shape (head dim %d must be 128 or 256, "
                "%d q heads per kv head must divide 32, mlp %d at most %d, q width %d at "
                "most %d)", name, c.hdim, hn, c.mlp_dim, 4 * 1024 * gh::kPfMaxNpt,
                c.n_heads * c.hdim, 4 * 256 * gh::kPfMaxNpt);
  return 0;
}

#define PF_CHECK(what, expr)                                                           \
  do {                                                                                 \
    hipError_t gh_e_ = (expr);                                                         \
    if (gh_e_ != hipSuccess) return fail("%s: %s: %s", kName, what, hipGetErrorString(gh_e_)); \
  } while (0)

// Waits for earlier work on the stream and makes room for n rows.
int prefill_stage(gemma_hip_decoder *dec, const char *kName, int n) {
  PF_CHECK("sync", hipStreamSynchronize(g.stream));
  return prefill_reserve(dec, n);
}

// With the rows staged (tokens in pf_tok when embed, else the rows in pf_x):
// sets the step record to {last token, pos + n - 1}, runs the pass and
// returns the last row's logits and argmax (both nullable).
int prefill_run(gemma_hip_decoder *dec, const char *kName, int n, int pos, int last_token,
                bool embed, bool dense, float *logits, int *next) {
  dec->pin[0] = last_token;
  dec->pin[1] = pos + n - 1;
  dec->pin[2] = 0;
  dec->pin[3] = 0;
  PF_CHECK("step H2D", hipMemcpyAsync(dec->step, dec->pin, 16, hipMemcpyHostToDevice, g.stream));
  PF_CHECK("launch", prefill_enqueue(dec, n, pos, embed, dense, g.stream));
  if (logits != nullptr)
    PF_CHECK("logits D2H", hipMemcpyAsync(logits, dec->logits, (size_t)dec->cfg.nvocab * 4,
                                          hipMemcpyDeviceToHost, g.stream));
  if (next != nullptr)
    PF_CHECK("D2H", hipMemcpyAsync(dec->pin + 4, dec->tokens, 4, hipMemcpyDeviceToHost, g.stream));
  PF_CHECK("sync", hipStreamSynchronize(g.stream));
  if (next != nullptr) *next = dec->pin[4];
  return 0;
}

// Enqueues one decode step on `st` (captured into the decoder's graph).
hipError_t decoder_enqueue(gemma_hip_decoder *d, hipStream_t st) {
  if (!d->quant) return decoder_enqueue_f32(d, st);
  const gemma_hip_text_config &c = d->cfg;
  const int q_sz = c.n_heads * c.hdim, kv_sz = c.nkv * c.hdim;
  hipError_t e;
  gh::DecEmbed em{d->emb, d->emb_s, d->x[0], d->step, c.dim, c.nvocab, d->clen,
                  c.mlp_pre ? 1.0f : sqrtf((float)c.dim)};
  if ((e = gh::launch_dec_embed(em, st)) != hipSuccess) return e;
  int cur = 0;
  for (int l = 0; l < c.nl; ++l) {
    const auto &L = d->layers[l];
    // residual of the previous MLP (post-FFN norm), pre-attention norm, q/k/v
    gh::DecNorm n1{d->x[cur], l > 0 ? d->ymlp : nullptr,
                   (l > 0 && c.mlp_pst) ? d->layers[l - 1].n4 : nullptr, L.n1,
                   d->x[cur ^ 1], nullptr, c.dim, c.eps};
    gh::GemvJobs qkv{};
    qkv.w[0] = L.w[0]; qkv.w[1] = L.w[1]; qkv.w[2] = L.w[2];
    qkv.sc[0] = L.s[0]; qkv.sc[1] = L.s[1]; qkv.sc[2] = L.s[2];
    qkv.dst[0] = d->xq; qkv.dst[1] = d->xk; qkv.dst[2] = d->xv;
    qkv.end[0] = q_sz; qkv.end[1] = q_sz + kv_sz; qkv.end[2] = qkv.end[3] = q_sz + 2 * kv_sz;
    qkv.njobs = 3;
    if ((e = GH_OP(kOpGemvInt8, gh::launch_dec_norm_gemv(n1, qkv, q_sz + 2 * kv_sz, c.dim,
                                                         false, g.info, st))) != hipSuccess)
      return e;
    cur ^= 1;
    // attention
    const size_t cache = (size_t)d->clen * kv_sz;
    float *kc = d->kv + (size_t)l * 2 * cache;
    const bool sliding = d->swa[l] != 0;
    gh::DecAttn at{d->xq, d->xk, d->xv, c.qk_norm ? L.nq : nullptr, c.qk_norm ? L.nk : nullptr,
                   sliding ? d->rope_l : d->rope_g, kc, kc + cache, d->part, d->xo, d->step,
                   c.n_heads, c.nkv, c.hdim, d->clen, sliding ? c.slide : 0,
                   d->max_blocks, c.nvocab, (float)(1.0f / sqrtf((float)c.q_scale)), c.sc_att,
                   c.eps};
    if ((e = GH_OP(kOpSoftmax, gh::launch_dec_attention(at, st))) != hipSuccess) return e;
    // o projection (quantize fused)
    gh::GemvJobs o{};
    o.w[0] = L.w[3]; o.sc[0] = L.s[3]; o.dst[0] = d->yattn;
    for (int j = 0; j < gh::kMaxJobs; ++j) o.end[j] = c.dim;
    o.njobs = 1;
    if ((e = GH_OP(kOpGemvInt8, gh::launch_gemv_i8(o, q_sz, nullptr, nullptr, d->xo, nullptr,
                                                   nullptr, g.info, st))) != hipSuccess)
      return e;
    // residual of the attention (post-attention norm), pre-FFN norm, gate/up + GELU
    gh::DecNorm n3{d->x[cur], d->yattn, c.mlp_pre ? L.n2 : nullptr, c.mlp_pre ? L.n3 : L.n2,
                   d->x[cur ^ 1], nullptr, c.dim, c.eps};
    gh::GemvJobs gu{};
    gu.w[0] = L.w[5]; gu.w[1] = L.w[4];  // gate (w2), up (w1): gemma.c:4911-4915
    gu.sc[0] = L.s[5]; gu.sc[1] = L.s[4];
    gu.dst[0] = d->gbuf; gu.dst[1] = d->gbuf;
    gu.end[0] = gu.end[1] = gu.end[2] = gu.end[3] = 2 * c.mlp_dim;
    gu.njobs = 2;
    if ((e = GH_OP(kOpGemvInt8, gh::launch_dec_norm_gemv(n3, gu, 2 * c.mlp_dim, c.dim, true,
                                                         g.info, st))) != hipSuccess)
      return e;
    cur ^= 1;
    // down projection (quantize fused)
    gh::GemvJobs dn{};
    dn.w[0] = L.w[6]; dn.sc[0] = L.s[6]; dn.dst[0] = d->ymlp;
    for (int j = 0; j < gh::kMaxJobs; ++j) dn.end[j] = c.dim;
    dn.njobs = 1;
    if ((e = GH_OP(kOpGemvInt8, gh::launch_gemv_i8(dn, c.mlp_dim, nullptr, nullptr, d->gbuf,
                                                   nullptr, nullptr, g.info, st))) != hipSuccess)
      return e;
  }
  // last residual, final norm, LM head (tied embedding), softcap, argmax
  gh::DecNorm fn{d->x[cur], d->ymlp, c.mlp_pst ? d->layers[c.nl - 1].n4 : nullptr, d->fnorm,
                 nullptr, d->h, c.dim, c.eps};
  if ((e = GH_OP(kOpRmsnorm, gh::launch_dec_final_norm(fn, st))) != hipSuccess) return e;
  gh::GemvJobs lm{};
  lm.w[0] = d->emb; lm.sc[0] = d->emb_s; lm.dst[0] = d->logits;
  for (int j = 0; j < gh::kMaxJobs; ++j) lm.end[j] = c.nvocab;
  lm.njobs = 1;
  if ((e = GH_OP(kOpGemvInt8, gh::launch_gemv_i8(lm, c.dim, nullptr, nullptr, d->h, nullptr,
                                                  nullptr, g.info, st))) != hipSuccess)
    return e;
  return GH_OP(kOpSample, [&] {
    hipError_t es = hipSuccess;
    if (c.sc_log != 0.0f) es = gh::launch_dec_softcap(d->logits, c.nvocab, c.sc_log, st);
    if (es != hipSuccess) return es;
    return gh::launch_dec_argmax(d->logits, c.nvocab, d->pval, d->pidx, d->nparts, d->step,
                                 d->tokens, d->clen, st);
  }());
}

// The fp32 ('U') model's prompt pass: forward_text_chunk's !quant branches
// (gemma.c:5079, 5297, 5358, 5384, 5431): the norms store fp32 rows, the
// projections are fp32 GEMMs on the matrix cores (gemm_fpx), GELU(gate) * up
// is computed in place, and the LM head is an fp32 GEMV; everything else is
// the W8A8 pass's kernels.
hipError_t prefill_enqueue_f32(gemma_hip_decoder *d, int n, int pos, bool embed, bool dense,
                               hipStream_t st) {
  const gemma_hip_text_config &c = d->cfg;
  const int q_sz = c.n_heads * c.hdim, kv_sz = c.nkv * c.hdim, dim = c.dim, mlp = c.mlp_dim;
  const int stride = q_sz + 2 * kv_sz;
  const size_t cache = (size_t)d->clen * kv_sz;
  hipError_t e;
  // dst[r][0..nout) = src[r] . w rows (gemm_fpx, gemma.c:3308)
  auto gemm = [&](float *dst, int dstr, const float *w, int nout, const float *src, int sstr,
                  int k) {
    return GH_OP(kOpGemmFpx, gh::launch_gemm_f32(dst, dstr, w, k, src, sstr, n, nout, k, nullptr,
                                                 false, g.info, st));
  };
  // adjacent output columns from several weight matrices of one K: one launch
  auto gemm_cols = [&](float *dst, int dstr, const gh::F32Segs &b, const float *src, int sstr,
                       int k) {
    return GH_OP(kOpGemmFpx, gh::launch_gemm_f32_segs(dst, dstr, b, k, src, sstr, n, k,
                                                      gh::F32Epilogue{}, g.info, st, false));
  };
  if (embed && (e = gh::launch_pf_embed(d->pf_tok, n, nullptr, nullptr, d->emb_f, d->pf_x, dim,
                                        c.mlp_pre ? 1.0f : sqrtf((float)dim), st)) != hipSuccess)
    return e;
  for (int l = 0; l < c.nl; ++l) {
    const auto &L = d->layers[l];
    gh::PfNorm n1{d->pf_x, l > 0 ? d->pf_y : nullptr,
                  (l > 0 && c.mlp_pst) ? d->layers[l - 1].n4 : nullptr, L.n1, nullptr, nullptr,
                  dim, c.eps, d->pf_h};
    if ((e = GH_OP(kOpRmsnorm, gh::launch_pf_norm_rows(n1, n, st))) != hipSuccess) return e;
    // q, k, v into the fused rows (gemma.c:5079)
    const gh::F32Segs qkv{{L.wf[0], L.wf[1], L.wf[2]}, {q_sz, q_sz + kv_sz, stride}, 3};
    if ((e = gemm_cols(d->pf_qkv, stride, qkv, d->pf_h, dim, dim)) != hipSuccess) return e;
    const bool sliding = d->swa[l] != 0;
    float *kc = d->kv + (size_t)l * 2 * cache;
    const gh::PfRope rp{d->pf_qkv, stride, q_sz, c.qk_norm ? L.nq : nullptr,
                        c.qk_norm ? L.nk : nullptr, sliding ? d->rope_l : d->rope_g, kc,
                        kc + cache, d->clen, pos, c.n_heads, c.nkv, c.eps};
    if ((e = GH_OP(kOpRope, gh::launch_pf_qk_rope(rp, n, c.hdim, st))) != hipSuccess) return e;
    const gh::PfAttn at{d->pf_qkv, stride, kc, kc + cache, d->pf_xo, q_sz, n, pos, c.n_heads,
                        c.nkv, d->clen, sliding ? c.slide : 0,
                        (float)(1.0f / sqrtf((float)c.q_scale)), c.sc_att, d->pf_part, 0, 0,
                        0, dense ? 1 : 0};
    if ((e = GH_OP(kOpSoftmax, gh::launch_pf_attention(at, c.hdim, d->attn_f32, g.info, st))) !=
        hipSuccess)
      return e;
    // o (gemma.c:5297), residual, norms
    if ((e = gemm(d->pf_y, dim, L.wf[3], dim, d->pf_xo, q_sz, q_sz)) != hipSuccess) return e;
    const gh::PfNorm n3{d->pf_x, d->pf_y, c.mlp_pre ? L.n2 : nullptr, c.mlp_pre ? L.n3 : L.n2,
                        nullptr, nullptr, dim, c.eps, d->pf_h};
    if ((e = GH_OP(kOpRmsnorm, gh::launch_pf_norm_rows(n3, n, st))) != hipSuccess) return e;
    // gate (w2) and up (w1) side by side in pf_g (gemma.c:5358), GELU, down (5384)
    const gh::F32Segs gu{{L.wf[5], L.wf[4], nullptr}, {mlp, 2 * mlp, 2 * mlp}, 2};
    if ((e = gemm_cols(d->pf_g, 2 * mlp, gu, d->pf_h, dim, dim)) != hipSuccess ||
        (e = GH_OP(kOpGelu, gh::launch_gelu_mul_rows(d->pf_g, n, mlp, st))) != hipSuccess ||
        (e = gemm(d->pf_y, dim, L.wf[6], dim, d->pf_g, 2 * mlp, mlp)) != hipSuccess)
      return e;
  }
  // the last row: last residual, final norm, LM head (gemma.c:5431), softcap, argmax
  const size_t last = (size_t)(n - 1) * dim;
  gh::DecNorm fn{d->pf_x + last, d->pf_y + last,
                 c.mlp_pst ? d->layers[c.nl - 1].n4 : nullptr, d->fnorm, nullptr, d->h, dim,
                 c.eps};
  if ((e = GH_OP(kOpRmsnorm, gh::launch_dec_final_norm(fn, st))) != hipSuccess) return e;
  gh::GemvJobs lm{};
  lm.w[0] = d->emb_f; lm.dst[0] = d->logits;
  for (int j = 0; j < gh::kMaxJobs; ++j) lm.end[j] = c.nvocab;
  lm.njobs = 1;
  if ((e = GH_OP(kOpGemvFpx, gh::launch_gemv_f32(lm, dim, d->h, g.info, st))) != hipSuccess)
    return e;
  return timed(kOpSample, st, [&] {
    hipError_t es = hipSuccess;
    if (c.sc_log != 0.0f) es = gh::launch_dec_softcap(d->logits, c.nvocab, c.sc_log, st);
    if (es != hipSuccess) return es;
    return gh::launch_dec_argmax(d->logits, c.nvocab, d->pval, d->pidx, d->nparts, d->step,
                                 d->tokens, d->clen, st);
  }, kPhaseDecode);
}

// The fp32 ('U') model's decode step: forward_text_decode's !quant branches
// (gemma.c:4762, 4855, 4906, 4925, 4960), launched as the W8A8 step is: the
// pre-attention and pre-FFN norms are the prologues of the q/k/v and gate/up
// fp32 GEMVs (every workgroup normalizes into LDS; workgroup 0 stores the new
// residual), the gate/up launch stores GELU(gate) * up, and o, down and the
// LM head are plain fp32 GEMVs (gemv_fpx / gemv_fpx_multi).
hipError_t decoder_enqueue_f32(gemma_hip_decoder *d, hipStream_t st) {
  const gemma_hip_text_config &c = d->cfg;
  const int q_sz = c.n_heads * c.hdim, kv_sz = c.nkv * c.hdim, mlp = c.mlp_dim;
  hipError_t e;
  gh::DecEmbed em{nullptr, nullptr, d->x[0], d->step, c.dim, c.nvocab, d->clen,
                  c.mlp_pre ? 1.0f : sqrtf((float)c.dim), d->emb_f};
  if ((e = gh::launch_dec_embed(em, st)) != hipSuccess) return e;
  auto gemv = [&](const gh::GemvJobs &jobs, int k, const float *x) {
    return GH_OP(kOpGemvFpx, gh::launch_gemv_f32(jobs, k, x, g.info, st));
  };
  auto one_job = [](const float *w, float *dst, int rows) {
    gh::GemvJobs j{};
    j.w[0] = w; j.dst[0] = dst;
    for (int t = 0; t < gh::kMaxJobs; ++t) j.end[t] = rows;
    j.njobs = 1;
    return j;
  };
  int cur = 0;
  for (int l = 0; l < c.nl; ++l) {
    const auto &L = d->layers[l];
    // residual of the previous MLP (post-FFN norm), pre-attention norm, q/k/v
    gh::DecNorm n1{d->x[cur], l > 0 ? d->ymlp : nullptr,
                   (l > 0 && c.mlp_pst) ? d->layers[l - 1].n4 : nullptr, L.n1,
                   d->x[cur ^ 1], nullptr, c.dim, c.eps};
    gh::GemvJobs qkv{};
    qkv.w[0] = L.wf[0]; qkv.w[1] = L.wf[1]; qkv.w[2] = L.wf[2];
    qkv.dst[0] = d->xq; qkv.dst[1] = d->xk; qkv.dst[2] = d->xv;
    qkv.end[0] = q_sz; qkv.end[1] = q_sz + kv_sz; qkv.end[2] = qkv.end[3] = q_sz + 2 * kv_sz;
    qkv.njobs = 3;
    if ((e = GH_OP(kOpGemvFpx, gh::launch_dec_norm_gemv_f32(n1, qkv, q_sz + 2 * kv_sz, c.dim,
                                                            false, g.info, st))) != hipSuccess)
      return e;
    cur ^= 1;
    const size_t cache = (size_t)d->clen * kv_sz;
    float *kc = d->kv + (size_t)l * 2 * cache;
    const bool sliding = d->swa[l] != 0;
    gh::DecAttn at{d->xq, d->xk, d->xv, c.qk_norm ? L.nq : nullptr, c.qk_norm ? L.nk : nullptr,
                   sliding ? d->rope_l : d->rope_g, kc, kc + cache, d->part, d->xo, d->step,
                   c.n_heads, c.nkv, c.hdim, d->clen, sliding ? c.slide : 0,
                   d->max_blocks, c.nvocab, (float)(1.0f / sqrtf((float)c.q_scale)), c.sc_att,
                   c.eps};
    if ((e = GH_OP(kOpSoftmax, gh::launch_dec_attention(at, st))) != hipSuccess) return e;
    if ((e = gemv(one_job(L.wf[3], d->yattn, c.dim), q_sz, d->xo)) != hipSuccess) return e;
    // residual of the attention (post-attention norm), pre-FFN norm, gate/up
    // and GELU(gate) * up into gbuf (gemma.c:4906-4915)
    gh::DecNorm n3{d->x[cur], d->yattn, c.mlp_pre ? L.n2 : nullptr, c.mlp_pre ? L.n3 : L.n2,
                   d->x[cur ^ 1], nullptr, c.dim, c.eps};
    gh::GemvJobs gu{};
    gu.w[0] = L.wf[5]; gu.w[1] = L.wf[4];  // gate (w2), up (w1): gemma.c:4906-4910
    gu.dst[0] = d->gbuf; gu.dst[1] = d->gbuf;
    gu.end[0] = gu.end[1] = gu.end[2] = gu.end[3] = 2 * mlp;
    gu.njobs = 2;
    if ((e = GH_OP(kOpGemvFpx, gh::launch_dec_norm_gemv_f32(n3, gu, 2 * mlp, c.dim, true, g.info,
                                                            st))) != hipSuccess)
      return e;
    cur ^= 1;
    if ((e = gemv(one_job(L.wf[6], d->ymlp, c.dim), mlp, d->gbuf)) != hipSuccess) return e;
  }
  gh::DecNorm fn{d->x[cur], d->ymlp, c.mlp_pst ? d->layers[c.nl - 1].n4 : nullptr, d->fnorm,
                 nullptr, d->h, c.dim, c.eps};
  if ((e = GH_OP(kOpRmsnorm, gh::launch_dec_final_norm(fn, st))) != hipSuccess) return e;
  if ((e = gemv(one_job(d->emb_f, d->logits, c.nvocab), c.dim, d->h)) != hipSuccess) return e;
  return GH_OP(kOpSample, [&] {
    hipError_t es = hipSuccess;
    if (c.sc_log != 0.0f) es = gh::launch_dec_softcap(d->logits, c.nvocab, c.sc_log, st);
    if (es != hipSuccess) return es;
    return gh::launch_dec_argmax(d->logits, c.nvocab, d->pval, d->pidx, d->nparts, d->step,
                                 d->tokens, d->clen, st);
  }());
}

}  // namespace

extern "C" {

}  // extern "C"

namespace {

// One layer's tensors as a create entry point passes them: the seven
// projections (int8 with row scales, or fp32), the norm weights.
struct LayerSrc {
  const void *w[7];  // wq wk wv wo w1 w2 w3
  const float *s[7];
  const float *norm[6];  // nq nk n1 n2 n3 n4
};

// gemma_hip_decoder_create(_f32): quant selects W8A8 weights (emb int8 with
// emb_s) or fp32 ones (emb fp32, emb_s unused).
gemma_hip_decoder *decoder_build(const char *name, const gemma_hip_text_config *cfg,
                                 const LayerSrc *layers, bool quant, const void *emb,
                                 const float *emb_s, const float *fnorm, int clen) {
  if (cfg == nullptr || layers == nullptr || emb == nullptr || (quant && emb_s == nullptr) ||
      fnorm == nullptr || cfg->swa == nullptr) {
    fail("%s: null argument", name);
    return nullptr;
  }
  const gemma_hip_text_config c = *cfg;
  if (c.nl <= 0 || c.n_heads <= 0 || c.nkv <= 0 || c.n_heads % c.nkv != 0 || c.hdim <= 0 ||
      c.hdim % 2 != 0 || c.dim <= 0 || c.dim % 16 != 0 || c.dim > 6144 || c.mlp_dim <= 0 ||
      c.mlp_dim % 16 != 0 || c.nvocab <= 0 || c.q_scale <= 0 || clen <= 0 || c.slide < 0 ||
      (c.n_heads * c.hdim) % 16 != 0) {
    fail("%s: unsupported config (nl=%d heads=%d/%d hdim=%d dim=%d "
         "mlp=%d vocab=%d clen=%d)", name, c.nl, c.n_heads, c.nkv, c.hdim, c.dim, c.mlp_dim, c.nvocab,
         clen);
    return nullptr;
  }
  for (int l = 0; l < c.nl; ++l)
    if (c.swa[l] && c.slide <= 0) {
      fail("%s: layer %d slides but slide = %d", name, l, c.slide);
      return nullptr;
    }
  gemma_hip_decoder *d = new gemma_hip_decoder();
  d->cfg = c;
  d->quant = quant;
  d->swa.assign(c.swa, c.swa + c.nl);
  d->cfg.swa = nullptr;
  d->clen = clen;
  d->max_blocks = (clen + gh::kDecAttnBlock - 1) / gh::kDecAttnBlock;
  const int hn = c.n_heads / c.nkv;
  if (gh::dec_attn_lds(hn, c.hdim) > 65536 || (size_t)d->max_blocks * 8 > 65536 ||
      c.hdim % 128 != 0 || c.hdim > 512) {
    fail("%s: unsupported attention shape (head dim %d must be a "
         "multiple of 128 up to 512; %d q heads per kv head; context %d)", name, c.hdim, hn,
         clen);
    decoder_free(d);
    return nullptr;
  }
  const size_t q_sz = (size_t)c.n_heads * c.hdim, kv_sz = (size_t)c.nkv * c.hdim;
  const size_t dim = c.dim, mlp = c.mlp_dim;
  // resolve every weight; rows must be 16-byte aligned on the device
  auto weight = [&](const void *host, size_t bytes, const char *what, const void **out) {
    const char *p = resolve(host, bytes);
    if (p == nullptr) return fail("%s: %s is not registered", name, what);
    if ((uintptr_t)p % 16 != 0)
      return fail("%s: %s is not 16-byte aligned on the device "
                  "(register each tensor as its own range)", name, what);
    *out = p;
    return 0;
  };
  const void *ptr = nullptr;
  const size_t wbytes = quant ? 1 : 4;  // bytes per weight
  if (weight(emb, (size_t)c.nvocab * dim * wbytes, "emb", &ptr)) {
    decoder_free(d);
    return nullptr;
  }
  if (quant) {
    d->emb = (const int8_t *)ptr;
    if (weight(emb_s, (size_t)c.nvocab * 4, "emb scales", &ptr)) {
      decoder_free(d);
      return nullptr;
    }
    d->emb_s = (const float *)ptr;
  } else {
    d->emb_f = (const float *)ptr;
  }
  d->layers.resize(c.nl);
  for (int l = 0; l < c.nl; ++l) {
    const LayerSrc &src = layers[l];
    const size_t rows[7] = {q_sz, kv_sz, kv_sz, dim, mlp, mlp, dim};
    const size_t cols[7] = {dim, dim, dim, q_sz, dim, dim, mlp};
    static const char *names[7] = {"wq", "wk", "wv", "wo", "w1", "w2", "w3"};
    for (int t = 0; t < 7; ++t) {
      if (weight(src.w[t], rows[t] * cols[t] * wbytes, names[t], &ptr)) {
        decoder_free(d);
        return nullptr;
      }
      if (!quant) {
        d->layers[l].wf[t] = (const float *)ptr;
        continue;
      }
      d->layers[l].w[t] = (const int8_t *)ptr;
      if (weight(src.s[t], rows[t] * 4, names[t], &ptr)) { decoder_free(d); return nullptr; }
      d->layers[l].s[t] = (const float *)ptr;
    }
    const float *const *nm = src.norm;  // nq nk n1 n2 n3 n4
    if (nm[2] == nullptr || nm[3] == nullptr || (c.qk_norm && (!nm[0] || !nm[1])) ||
        (c.mlp_pre && !nm[4]) || (c.mlp_pst && !nm[5])) {
      fail("%s: layer %d lacks a norm weight", name, l);
      decoder_free(d);
      return nullptr;
    }
  }
  // one device allocation for norms, activations, tables and the KV cache
  Carver cv;
  std::vector<size_t> o_norm(c.nl);
  const size_t norm_floats = 2 * (size_t)c.hdim + 4 * dim;
  for (int l = 0; l < c.nl; ++l) o_norm[l] = cv.take(norm_floats * 4);
  const size_t o_fnorm = cv.take(dim * 4), o_x0 = cv.take(dim * 4), o_x1 = cv.take(dim * 4),
               o_xq = cv.take(q_sz * 4), o_xk = cv.take(kv_sz * 4), o_xv = cv.take(kv_sz * 4),
               o_xo = cv.take(q_sz * 4), o_ya = cv.take(dim * 4), o_g = cv.take((quant ? 1 : 2) * mlp * 4),
               o_ym = cv.take(dim * 4), o_h = cv.take(dim * 4),
               o_lg = cv.take((size_t)c.nvocab * 4),
               o_part = cv.take((size_t)c.n_heads * d->max_blocks * (c.hdim + 2) * 8),
               o_rl = cv.take((size_t)clen * c.hdim * 4), o_rg = cv.take((size_t)clen * c.hdim * 4),
               o_kv = cv.take((size_t)c.nl * 2 * clen * kv_sz * 4),
               o_pv = cv.take((size_t)d->nparts * 4), o_pi = cv.take((size_t)d->nparts * 4),
               o_st = cv.take(16), o_tok = cv.take((size_t)clen * 4);
  hipError_t e = hipMalloc((void **)&d->mem, cv.used);
  if (e == hipSuccess) e = hipHostMalloc((void **)&d->pin, 64, hipHostMallocDefault);
  if (e != hipSuccess) {
    hip_fail(name, e);
    decoder_free(d);
    return nullptr;
  }
  char *m = d->mem;
  d->fnorm = (float *)(m + o_fnorm);
  d->x[0] = (float *)(m + o_x0);
  d->x[1] = (float *)(m + o_x1);
  d->xq = (float *)(m + o_xq);
  d->xk = (float *)(m + o_xk);
  d->xv = (float *)(m + o_xv);
  d->xo = (float *)(m + o_xo);
  d->yattn = (float *)(m + o_ya);
  d->gbuf = (float *)(m + o_g);
  d->ymlp = (float *)(m + o_ym);
  d->h = (float *)(m + o_h);
  d->logits = (float *)(m + o_lg);
  d->part = (double *)(m + o_part);
  d->rope_l = (float *)(m + o_rl);
  d->rope_g = (float *)(m + o_rg);
  d->kv = (float *)(m + o_kv);
  d->pval = (float *)(m + o_pv);
  d->pidx = (int *)(m + o_pi);
  d->step = (int *)(m + o_st);
  d->tokens = (int *)(m + o_tok);
  // norms and RoPE tables, staged on the host
  std::vector<float> host(norm_floats * c.nl + dim, 0.0f);
  for (int l = 0; l < c.nl; ++l) {
    float *dst = host.data() + norm_floats * l;
    const float *const *parts = layers[l].norm;
    const size_t lens[6] = {(size_t)c.hdim, (size_t)c.hdim, dim, dim, dim, dim};
    float *devp[6];
    size_t off = 0;
    for (int t = 0; t < 6; ++t) {
      if (parts[t] != nullptr) memcpy(dst + off, parts[t], lens[t] * 4);
      devp[t] = (float *)(m + o_norm[l]) + off;
      off += lens[t];
    }
    d->layers[l].nq = devp[0];
    d->layers[l].nk = devp[1];
    d->layers[l].n1 = devp[2];
    d->layers[l].n2 = devp[3];
    d->layers[l].n3 = devp[4];
    d->layers[l].n4 = devp[5];
    e = hipMemcpy(m + o_norm[l], dst, norm_floats * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) break;
  }
  if (e == hipSuccess) e = hipMemcpy(d->fnorm, fnorm, dim * 4, hipMemcpyHostToDevice);
  // rope_freqs_pos (gemma.c:4178-4196): freq = theta^(-2d/hdim) and the
  // angle freq*pos as the reference's floats, each rounded once; cos and sin
  // of that angle rounded once to float
  if (e == hipSuccess) {
    std::vector<float> tab((size_t)clen * c.hdim);
    for (int which = 0; which < 2 && e == hipSuccess; ++which) {
      const float theta = which == 0 ? c.theta_l : c.theta_g;
      for (int dd = 0; dd < c.hdim / 2; ++dd) {
        const float ex = (float)(-2 * dd) / (float)c.hdim;
        const float freq = (float)pow((double)theta, (double)ex);
        for (int p = 0; p < clen; ++p) {
          const float ang = freq * (float)p;
          tab[(size_t)p * c.hdim + 2 * dd] = (float)cos((double)ang);
          tab[(size_t)p * c.hdim + 2 * dd + 1] = (float)sin((double)ang);
        }
      }
      e = hipMemcpy(which == 0 ? d->rope_l : d->rope_g, tab.data(), tab.size() * 4,
                    hipMemcpyHostToDevice);
    }
  }
  if (e != hipSuccess) {
    hip_fail(name, e);
    decoder_free(d);
    return nullptr;
  }
  // capture the step graph
  e = hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal);
  if (e == hipSuccess) {
    hipError_t le = decoder_enqueue(d, g.stream);
    e = hipStreamEndCapture(g.stream, &d->graph);
    if (le != hipSuccess) e = le;
  }
  if (e == hipSuccess) e = hipGraphInstantiate(&d->exec, d->graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    hip_fail(name, e);
    decoder_free(d);
    return nullptr;
  }
  return d;
}

}  // namespace

extern "C" {

gemma_hip_decoder *gemma_hip_decoder_create(const gemma_hip_text_config *cfg,
                                            const gemma_hip_layer *layers,
                                            const int8_t *emb, const float *emb_s,
                                            const float *fnorm, int clen) {
  static const char *kName = "gemma_hip_decoder_create";
  if (need_init()) return nullptr;
  if (cfg == nullptr || layers == nullptr || cfg->nl <= 0) {
    fail("%s: null argument", kName);
    return nullptr;
  }
  std::vector<LayerSrc> src(cfg->nl);
  for (int l = 0; l < cfg->nl; ++l) {
    const gemma_hip_layer &a = layers[l];
    src[l] = LayerSrc{{a.wq, a.wk, a.wv, a.wo, a.w1, a.w2, a.w3},
                      {a.wq_s, a.wk_s, a.wv_s, a.wo_s, a.w1_s, a.w2_s, a.w3_s},
                      {a.nq, a.nk, a.n1, a.n2, a.n3, a.n4}};
  }
  return decoder_build(kName, cfg, src.data(), true, emb, emb_s, fnorm, clen);
}

gemma_hip_decoder *gemma_hip_decoder_create_f32(const gemma_hip_text_config *cfg,
                                                const gemma_hip_layer_f32 *layers,
                                                const float *emb, const float *fnorm,
                                                int clen) {
  static const char *kName = "gemma_hip_decoder_create_f32";
  if (need_init()) return nullptr;
  if (cfg == nullptr || layers == nullptr || cfg->nl <= 0) {
    fail("%s: null argument", kName);
    return nullptr;
  }
  std::vector<LayerSrc> src(cfg->nl);
  for (int l = 0; l < cfg->nl; ++l) {
    const gemma_hip_layer_f32 &a = layers[l];
    src[l] = LayerSrc{{a.wq, a.wk, a.wv, a.wo, a.w1, a.w2, a.w3},
                      {},
                      {a.nq, a.nk, a.n1, a.n2, a.n3, a.n4}};
  }
  return decoder_build(kName, cfg, src.data(), false, emb, nullptr, fnorm, clen);
}

void gemma_hip_decoder_destroy(gemma_hip_decoder *dec) {
  if (dec == nullptr) return;
  if (g.ready) (void)hipStreamSynchronize(g.stream);
  decoder_free(dec);
}

}  // extern "C"

namespace {
// One decode step on the library's stream: the captured graph, or the same
// launches made eagerly while per-op timing is on (a graph's kernels cannot
// be timed one by one).
hipError_t run_step(gemma_hip_decoder *dec) {
  if (g_perf.on.load(std::memory_order_relaxed)) return decoder_enqueue(dec, g.stream);
  return hipGraphLaunch(dec->exec, g.stream);
}
}  // namespace

extern "C" {

int gemma_hip_decoder_step(gemma_hip_decoder *dec, int token, int pos, float *logits,
                           int *next) {
  if (need_init()) return 1;
  if (dec == nullptr) return fail("gemma_hip_decoder_step: null decoder");
  if (token < 0 || token >= dec->cfg.nvocab || pos < 0 || pos >= dec->clen)
    return fail("gemma_hip_decoder_step: token %d / pos %d out of range (vocab %d, clen %d)",
                token, pos, dec->cfg.nvocab, dec->clen);
  GH_CHECK("gemma_hip_decoder_step: sync", hipStreamSynchronize(g.stream));
  dec->pin[0] = token;
  dec->pin[1] = pos;
  dec->pin[2] = 0;
  dec->pin[3] = 0;
  GH_CHECK("gemma_hip_decoder_step: H2D",
           hipMemcpyAsync(dec->step, dec->pin, 16, hipMemcpyHostToDevice, g.stream));
  perf_enter(kPhaseDecode);
  GH_CHECK("gemma_hip_decoder_step: step", run_step(dec));
  if (logits != nullptr)
    GH_CHECK("gemma_hip_decoder_step: logits D2H",
             hipMemcpyAsync(logits, dec->logits, (size_t)dec->cfg.nvocab * 4,
                            hipMemcpyDeviceToHost, g.stream));
  if (next != nullptr)
    GH_CHECK("gemma_hip_decoder_step: D2H",
             hipMemcpyAsync(dec->pin + 4, dec->tokens, 4, hipMemcpyDeviceToHost, g.stream));
  GH_CHECK("gemma_hip_decoder_step: sync", hipStreamSynchronize(g.stream));
  if (next != nullptr) *next = dec->pin[4];
  return 0;
}

int gemma_hip_decoder_generate(gemma_hip_decoder *dec, int token, int pos, int n,
                               int *tokens) {
  if (need_init()) return 1;
  if (dec == nullptr || tokens == nullptr) return fail("gemma_hip_decoder_generate: null argument");
  if (token < 0 || token >= dec->cfg.nvocab || pos < 0 || n < 0 || n > dec->clen - pos)
    return fail("gemma_hip_decoder_generate: token %d / pos %d / n %d out of range", token,
                pos, n);
  if (n == 0) return 0;
  GH_CHECK("gemma_hip_decoder_generate: sync", hipStreamSynchronize(g.stream));
  dec->pin[0] = token;
  dec->pin[1] = pos;
  dec->pin[2] = 0;
  dec->pin[3] = 0;
  GH_CHECK("gemma_hip_decoder_generate: H2D",
           hipMemcpyAsync(dec->step, dec->pin, 16, hipMemcpyHostToDevice, g.stream));
  perf_enter(kPhaseDecode);
  for (int i = 0; i < n; ++i) GH_CHECK("gemma_hip_decoder_generate: step", run_step(dec));
  GH_CHECK("gemma_hip_decoder_generate: D2H",
           hipMemcpyAsync(tokens, dec->tokens, (size_t)n * 4, hipMemcpyDeviceToHost, g.stream));
  GH_CHECK("gemma_hip_decoder_generate: sync", hipStreamSynchronize(g.stream));
  for (int i = 0; i < n; ++i)
    if (tokens[i] < 0 || tokens[i] >= dec->cfg.nvocab)
      return fail("gemma_hip_decoder_generate: step %d produced no token (NaN logits?)", i);
  return 0;
}

int gemma_hip_decoder_prefill(gemma_hip_decoder *dec, const int *tokens, int n, int pos,
                              float *logits, int *next) {
  static const char *kName = "gemma_hip_decoder_prefill";
  if (need_init()) return 1;
  if (dec == nullptr || tokens == nullptr) return fail("%s: null argument", kName);
  if (prefill_check(dec, kName, n, pos)) return 1;
  for (int i = 0; i < n; ++i)
    if (tokens[i] < 0 || tokens[i] >= dec->cfg.nvocab)
      return fail("%s: token %d at %d out of range (vocab %d)", kName, tokens[i], i,
                  dec->cfg.nvocab);
  if (prefill_stage(dec, kName, n)) return 1;
  PF_CHECK("tokens H2D",
           hipMemcpyAsync(dec->pf_tok, tokens, (size_t)n * 4, hipMemcpyHostToDevice, g.stream));
  perf_enter(kPhasePrefill);
  return prefill_run(dec, kName, n, pos, tokens[n - 1], true, false, logits, next);
}

int gemma_hip_decoder_prefill_rows(gemma_hip_decoder *dec, const float *x, int n, int pos,
                                   int mask, float *logits, int *next) {
  static const char *kName = "gemma_hip_decoder_prefill_rows";
  if (need_init()) return 1;
  if (dec == nullptr || x == nullptr) return fail("%s: null argument", kName);
  if (prefill_check(dec, kName, n, pos) || prefill_stage(dec, kName, n)) return 1;
  PF_CHECK("rows copy", hipMemcpyAsync(dec->pf_x, x, (size_t)n * dec->cfg.dim * 4,
                                       hipMemcpyDefault, g.stream));
  // text rows belong to the prefill phase, image soft tokens (the dense
  // pass of forward_gemma_image) to the vision phase
  perf_enter(mask != 0 ? kPhasePrefill : kPhaseVision);
  return prefill_run(dec, kName, n, pos, 0, false, mask == 0, logits, next);
}

int gemma_hip_decoder_set_attention(gemma_hip_decoder *dec, int mode) {
  if (dec == nullptr) return fail("gemma_hip_decoder_set_attention: null argument");
  if (mode != GEMMA_HIP_ATTN_F64 && mode != GEMMA_HIP_ATTN_F32)
    return fail("gemma_hip_decoder_set_attention: unknown mode %d", mode);
  dec->attn_f32 = mode == GEMMA_HIP_ATTN_F32;
  return 0;
}

const float *gemma_hip_decoder_logits(const gemma_hip_decoder *dec) {
  return dec != nullptr ? dec->logits : nullptr;
}

}  // extern "C"

// ---- vision tower ----------------------------------------------------------

struct gemma_hip_vision {
  gemma_hip_vision_config cfg{};
  int npatch = 0, ppi = 0, ksize = 0, hdim = 0;
  bool attn_f32 = true;  // attention on the fp32 matrix cores (gemma_hip_vision_set_attention)
  bool quant = true;     // int8 projections; false: an fp32 ('U') model
  struct Layer {
    const int8_t *w[6];  // wq wk wv wo w1 w2, device
    const float *s[6];
    const float *wf[6];  // the same, fp32 ('U'), device
    float *bqkv, *bo, *b1, *b2, *n1, *n1b, *n2, *n2b;  // device copies
  };
  std::vector<Layer> layers;
  const int8_t *pos_q = nullptr, *proj = nullptr;
  const float *pos_s = nullptr, *proj_s = nullptr;
  const float *pos_f = nullptr, *proj_f = nullptr;  // fp32 ('U')
  float *pe = nullptr, *pe_b = nullptr, *post_n = nullptr, *post_nb = nullptr, *norm = nullptr;
  char *mem = nullptr;  // parameters and activations
  float *img = nullptr, *patches = nullptr, *x = nullptr, *y = nullptr, *qkv = nullptr;
  float *att = nullptr, *hbuf = nullptr, *hln = nullptr, *out = nullptr, *as = nullptr;
  int8_t *a8 = nullptr;
};

namespace {

void vision_free(gemma_hip_vision *v) {
  if (v == nullptr) return;
  if (v->mem != nullptr) (void)hipFree(v->mem);
  delete v;
}

// forward_vision (gemma.c:4394-4725) on `st`; the image is already in v->img
hipError_t vision_enqueue_f32(gemma_hip_vision *v, hipStream_t st);

hipError_t vision_enqueue(gemma_hip_vision *v, hipStream_t st) {
  if (!v->quant) return vision_enqueue_f32(v, st);
  const gemma_hip_vision_config &c = v->cfg;
  const int n = v->npatch, dim = c.dim, mlp = c.mlp_dim;
  hipError_t e;
  auto gemm = [&](float *dst, int dstr, const int8_t *w, const float *ws, int m, int nout,
                  int k) {
    return GH_OP(kOpGemmInt8,
                 gh::launch_gemm_i8(dst, dstr, 0, w, k, ws, v->a8, k, v->as, m, nout, k, g.info, st));
  };
  // patch embedding + position embedding (4411-4468)
  // the patch GEMM (the a9 path: fp32 matrix cores; fp64 in the verification
  // mode) with the bias, clamp and position embedding in its epilogue
  gh::F32Epilogue pe{};
  pe.bias = v->pe_b;
  pe.clamp = true;
  pe.pos_q = v->pos_q;
  pe.pos_s = v->pos_s;
  const int kdim = 3 * c.psize * c.psize;
  if ((e = GH_OP(kOpGemmFpx, [&] {
         const hipError_t ei = gh::launch_im2col(v->patches, v->img, c.img_px, c.psize, st);
         if (ei != hipSuccess) return ei;
         return gh::launch_gemm_f32(v->x, dim, v->pe, kdim, v->patches, kdim, n, dim, kdim, pe,
                                    g.info, st, !v->attn_f32);
       }())) != hipSuccess)
    return e;
  for (int l = 0; l < c.nl; ++l) {
    const auto &L = v->layers[l];
    // residual of the previous layer's MLP (fc2 bias), first layer norm (4474-4484)
    const gh::VisLn n1{v->x, l > 0 ? v->y : nullptr, l > 0 ? v->layers[l - 1].b2 : nullptr,
                       L.n1, L.n1b, v->a8, v->as, nullptr, dim, c.eps};
    if ((e = GH_OP(kOpLayernorm, gh::launch_vis_ln_rows(n1, n, st))) != hipSuccess) return e;
    // q, k, v (4487-4511); their biases are added inside the attention
    const gh::GemmSegs qkv{{L.w[0], L.w[1], L.w[2]}, {L.s[0], L.s[1], L.s[2]},
                           {dim, 2 * dim, 3 * dim}, 3};
    if ((e = GH_OP(kOpGemmInt8, gh::launch_gemm_i8_segs(v->qkv, 3 * dim, qkv, v->a8, dim,
                                                        v->as, n, dim, g.info, st))) != hipSuccess)
      return e;
    const gh::VisAttn at{v->qkv, 3 * dim, L.bqkv, v->att, n, c.n_heads, dim,
                         1.0f / sqrtf((float)v->hdim)};
    if ((e = GH_OP(kOpSoftmax, gh::launch_vis_attention(at, v->hdim, v->attn_f32, st))) !=
        hipSuccess)
      return e;
    // o (4563-4573), then its bias, the residual and the second layer norm
    if ((e = GH_OP(kOpQuantizeAct, gh::launch_quantize(v->a8, v->as, v->att, dim, n, dim,
                                                       st))) != hipSuccess ||
        (e = gemm(v->y, dim, L.w[3], L.s[3], n, dim, dim)) != hipSuccess)
      return e;
    const gh::VisLn n2{v->x, v->y, L.bo, L.n2, L.n2b, v->a8, v->as, nullptr, dim, c.eps};
    if ((e = GH_OP(kOpLayernorm, gh::launch_vis_ln_rows(n2, n, st))) != hipSuccess) return e;
    // The GELU kernel reads fc2's weights after its rows, as the decoder's
    // prefill does for down: the tower's 27 layers hold more weights than the
    // Infinity Cache, so each layer's come from HBM.  Measured at 896 px,
    // five alternating runs each on one box: 19.47 -> 19.24 ms per image
    // (the same read of fc1's weights in the layer norm in front of fc1 was
    // slower).
    gh::WarmRegions w_fc2{};
    if (n >= kWarmRows) w_fc2 = {{L.w[5]}, {(size_t)mlp * dim}, 1};
    // fc1, bias + GELU, fc2 (4604-4644)
    if ((e = gemm(v->hbuf, mlp, L.w[4], L.s[4], n, mlp, dim)) != hipSuccess ||
        (e = GH_OP(kOpGelu, gh::launch_vis_gelu_quant(v->hbuf, L.b1, n, mlp, v->a8, v->as,
                                                      w_fc2, st))) != hipSuccess ||
        (e = gemm(v->y, dim, L.w[5], L.s[5], n, dim, mlp)) != hipSuccess)
      return e;
  }
  // last residual, post layer norm (4660-4668), pooling + RMSNorm (4673-4704),
  // projection (4708-4721)
  const gh::VisLn pn{v->x, v->y, v->layers[c.nl - 1].b2, v->post_n, v->post_nb, nullptr,
                     nullptr, v->hln, dim, c.eps};
  if ((e = GH_OP(kOpLayernorm, gh::launch_vis_ln_rows(pn, n, st))) != hipSuccess) return e;
  const gh::VisPool po{v->hln, v->norm, v->a8, v->as, dim, v->ppi, v->ksize, c.eps};
  if ((e = GH_OP(kOpRmsnorm, gh::launch_vis_pool(po, c.img_tok, st))) != hipSuccess) return e;
  return gemm(v->out, c.text_dim, v->proj, v->proj_s, c.img_tok, c.text_dim, dim);
}

// The fp32 ('U') tower: forward_vision's !quant branches (gemma.c:4454, 4488,
// 4562, 4604, 4626, 4709): the fp32 position embedding in the patch GEMM's
// epilogue, the layer norms and the pooling store fp32 rows, the projections
// are fp32 matrix-core GEMMs (fp64 in the verification mode, as the patch
// GEMM), the fc1 bias + GELU its own launch.
hipError_t vision_enqueue_f32(gemma_hip_vision *v, hipStream_t st) {
  const gemma_hip_vision_config &c = v->cfg;
  const int n = v->npatch, dim = c.dim, mlp = c.mlp_dim;
  const bool f64 = !v->attn_f32;
  hipError_t e;
  auto gemm = [&](float *dst, int dstr, const float *w, int m, int nout, const float *src,
                  int sstr, int k) {
    return GH_OP(kOpGemmFpx, gh::launch_gemm_f32(dst, dstr, w, k, src, sstr, m, nout, k,
                                                 gh::F32Epilogue{}, g.info, st, f64));
  };
  gh::F32Epilogue pe{};
  pe.bias = v->pe_b;
  pe.clamp = true;
  pe.pos_f = v->pos_f;
  const int kdim = 3 * c.psize * c.psize;
  if ((e = GH_OP(kOpGemmFpx, [&] {
         const hipError_t ei = gh::launch_im2col(v->patches, v->img, c.img_px, c.psize, st);
         if (ei != hipSuccess) return ei;
         return gh::launch_gemm_f32(v->x, dim, v->pe, kdim, v->patches, kdim, n, dim, kdim, pe,
                                    g.info, st, f64);
       }())) != hipSuccess)
    return e;
  for (int l = 0; l < c.nl; ++l) {
    const auto &L = v->layers[l];
    const gh::VisLn n1{v->x, l > 0 ? v->y : nullptr, l > 0 ? v->layers[l - 1].b2 : nullptr,
                       L.n1, L.n1b, nullptr, nullptr, v->hln, dim, c.eps};
    if ((e = GH_OP(kOpLayernorm, gh::launch_vis_ln_rows(n1, n, st))) != hipSuccess) return e;
    const gh::F32Segs qkv{{L.wf[0], L.wf[1], L.wf[2]}, {dim, 2 * dim, 3 * dim}, 3};
    if ((e = GH_OP(kOpGemmFpx, gh::launch_gemm_f32_segs(v->qkv, 3 * dim, qkv, dim, v->hln, dim,
                                                        n, dim, gh::F32Epilogue{}, g.info, st,
                                                        f64))) != hipSuccess)
      return e;
    const gh::VisAttn at{v->qkv, 3 * dim, L.bqkv, v->att, n, c.n_heads, dim,
                         1.0f / sqrtf((float)v->hdim)};
    if ((e = GH_OP(kOpSoftmax, gh::launch_vis_attention(at, v->hdim, v->attn_f32, st))) !=
        hipSuccess)
      return e;
    if ((e = gemm(v->y, dim, L.wf[3], n, dim, v->att, dim, dim)) != hipSuccess) return e;
    const gh::VisLn n2{v->x, v->y, L.bo, L.n2, L.n2b, nullptr, nullptr, v->hln, dim, c.eps};
    if ((e = GH_OP(kOpLayernorm, gh::launch_vis_ln_rows(n2, n, st))) != hipSuccess) return e;
    if ((e = gemm(v->hbuf, mlp, L.wf[4], n, mlp, v->hln, dim, dim)) != hipSuccess ||
        (e = GH_OP(kOpGelu, gh::launch_vis_bias_gelu(v->hbuf, L.b1, n, mlp, st))) !=
            hipSuccess ||
        (e = gemm(v->y, dim, L.wf[5], n, dim, v->hbuf, mlp, mlp)) != hipSuccess)
      return e;
  }
  const gh::VisLn pn{v->x, v->y, v->layers[c.nl - 1].b2, v->post_n, v->post_nb, nullptr,
                     nullptr, v->hln, dim, c.eps};
  if ((e = GH_OP(kOpLayernorm, gh::launch_vis_ln_rows(pn, n, st))) != hipSuccess) return e;
  gh::VisPool po{v->hln, v->norm, nullptr, nullptr, dim, v->ppi, v->ksize, c.eps, v->att};
  if ((e = GH_OP(kOpRmsnorm, gh::launch_vis_pool(po, c.img_tok, st))) != hipSuccess) return e;
  return gemm(v->out, c.text_dim, v->proj_f, c.img_tok, c.text_dim, v->att, dim, dim);
}

#undef GH_OP

}  // namespace

extern "C" {

}  // extern "C"

namespace {

// One encoder layer's tensors as a create entry point passes them.
struct VisLayerSrc {
  const void *w[6];  // wq wk wv wo w1 w2: int8 (with s) or fp32
  const float *s[6];
  const float *b[6];  // bq bk bv bo b1 b2
  const float *n[4];  // n1 n1_b n2 n2_b
};

// gemma_hip_vision_create(_f32): quant selects int8 projections, position
// embedding and projection (with their row scales) or fp32 ones.
gemma_hip_vision *vision_build(const char *name, const gemma_hip_vision_config *cfg,
                               const VisLayerSrc *layers, bool quant, const float *pe,
                               const float *pe_b, const void *pos, const float *pos_s,
                               const float *post_n, const float *post_nb, const float *norm,
                               const void *proj, const float *proj_s) {
  if (cfg == nullptr || layers == nullptr || pe == nullptr || pe_b == nullptr ||
      pos == nullptr || (quant && (pos_s == nullptr || proj_s == nullptr)) ||
      post_n == nullptr || post_nb == nullptr || norm == nullptr || proj == nullptr) {
    fail("%s: null argument", name);
    return nullptr;
  }
  const gemma_hip_vision_config c = *cfg;
  const int hdim = c.n_heads > 0 ? c.dim / c.n_heads : 0;
  const int ppi = c.psize > 0 ? c.img_px / c.psize : 0;
  int side = 0;
  while (side * side < c.img_tok) ++side;
  if (c.nl <= 0 || c.n_heads <= 0 || c.dim <= 0 || c.dim % 16 != 0 || c.dim > 6144 ||
      c.dim % c.n_heads != 0 ||
      (hdim != 16 && hdim != 32 && hdim != 64 && hdim != 72 && hdim != 128) ||
      c.mlp_dim <= 0 || c.mlp_dim % 16 != 0 || c.mlp_dim > 4 * 1024 * gh::kPfMaxNpt ||
      c.psize <= 0 || c.img_px <= 0 || c.img_px % c.psize != 0 || c.img_tok <= 0 ||
      side * side != c.img_tok || ppi % side != 0 || c.text_dim <= 0 || c.text_dim % 16 != 0) {
    fail("%s: unsupported config (nl=%d heads=%d dim=%d mlp=%d img=%d "
         "patch=%d img_tok=%d text_dim=%d)", name, c.nl, c.n_heads, c.dim, c.mlp_dim, c.img_px,
         c.psize, c.img_tok, c.text_dim);
    return nullptr;
  }
  gemma_hip_vision *v = new gemma_hip_vision();
  v->cfg = c;
  v->quant = quant;
  v->hdim = hdim;
  v->ppi = ppi;
  v->npatch = ppi * ppi;
  v->ksize = ppi / side;
  const size_t dim = c.dim, mlp = c.mlp_dim, n = v->npatch, kpe = 3 * (size_t)c.psize * c.psize;
  auto weight = [&](const void *host, size_t bytes, const char *what, const void **out) {
    const char *p = resolve(host, bytes);
    if (p == nullptr) return fail("%s: %s is not registered", name, what);
    if ((uintptr_t)p % 16 != 0) return fail("%s: %s is not 16-byte aligned on the device", name, what);
    *out = p;
    return 0;
  };
  const void *ptr = nullptr;
  const size_t wbytes = quant ? 1 : 4;  // bytes per weight
  v->layers.resize(c.nl);
  for (int l = 0; l < c.nl; ++l) {
    const VisLayerSrc &src = layers[l];
    const size_t rows[6] = {dim, dim, dim, dim, mlp, dim};
    const size_t cols[6] = {dim, dim, dim, dim, dim, mlp};
    static const char *names[6] = {"wq", "wk", "wv", "wo", "w1", "w2"};
    for (int t = 0; t < 6; ++t) {
      if (weight(src.w[t], rows[t] * cols[t] * wbytes, names[t], &ptr)) {
        vision_free(v);
        return nullptr;
      }
      if (!quant) {
        v->layers[l].wf[t] = (const float *)ptr;
        continue;
      }
      v->layers[l].w[t] = (const int8_t *)ptr;
      if (weight(src.s[t], rows[t] * 4, names[t], &ptr)) { vision_free(v); return nullptr; }
      v->layers[l].s[t] = (const float *)ptr;
    }
    bool have = true;
    for (int t = 0; t < 6; ++t) have = have && src.b[t] != nullptr;
    for (int t = 0; t < 4; ++t) have = have && src.n[t] != nullptr;
    if (!have) {
      fail("%s: layer %d lacks a bias or norm weight", name, l);
      vision_free(v);
      return nullptr;
    }
  }
  if (weight(pos, n * dim * wbytes, "pos_emb", &ptr)) { vision_free(v); return nullptr; }
  if (quant) {
    v->pos_q = (const int8_t *)ptr;
    if (weight(pos_s, n * 4, "pos_emb scales", &ptr)) { vision_free(v); return nullptr; }
    v->pos_s = (const float *)ptr;
  } else {
    v->pos_f = (const float *)ptr;
  }
  if (weight(proj, (size_t)c.text_dim * dim * wbytes, "proj", &ptr)) {
    vision_free(v);
    return nullptr;
  }
  if (quant) {
    v->proj = (const int8_t *)ptr;
    if (weight(proj_s, (size_t)c.text_dim * 4, "proj scales", &ptr)) {
      vision_free(v);
      return nullptr;
    }
    v->proj_s = (const float *)ptr;
  } else {
    v->proj_f = (const float *)ptr;
  }
  // one device allocation: copied parameters, then the activations
  Carver cv;
  const size_t per_layer = 3 * dim + dim + mlp + dim + 4 * dim;  // bqkv bo b1 b2 n1 n1b n2 n2b
  const size_t o_par = cv.take((kpe * dim + dim + 3 * dim + per_layer * c.nl) * 4);
  const size_t o_img = cv.take((size_t)c.img_px * c.img_px * 3 * 4),
               o_pat = cv.take(n * kpe * 4), o_x = cv.take(n * dim * 4),
               o_y = cv.take(n * dim * 4), o_qkv = cv.take(n * 3 * dim * 4),
               o_att = cv.take(n * dim * 4), o_h = cv.take(n * mlp * 4),
               o_hln = cv.take(n * dim * 4), o_out = cv.take((size_t)c.img_tok * c.text_dim * 4),
               o_a8 = cv.take(n * std::max(dim, mlp)), o_as = cv.take(n * 4);
  hipError_t e = hipMalloc((void **)&v->mem, cv.used);
  if (e != hipSuccess) {
    hip_fail(name, e);
    vision_free(v);
    return nullptr;
  }
  char *m = v->mem;
  std::vector<float> host;
  host.reserve((kpe * dim + dim + 3 * dim + per_layer * c.nl));
  auto put = [&](const float *src, size_t len) {
    float *at = (float *)(m + o_par) + host.size();
    host.insert(host.end(), src, src + len);
    return at;
  };
  v->pe = put(pe, kpe * dim);
  v->pe_b = put(pe_b, dim);
  v->post_n = put(post_n, dim);
  v->post_nb = put(post_nb, dim);
  v->norm = put(norm, dim);
  for (int l = 0; l < c.nl; ++l) {
    const VisLayerSrc &src = layers[l];
    auto &L = v->layers[l];
    L.bqkv = put(src.b[0], dim);
    put(src.b[1], dim);
    put(src.b[2], dim);
    L.bo = put(src.b[3], dim);
    L.b1 = put(src.b[4], mlp);
    L.b2 = put(src.b[5], dim);
    L.n1 = put(src.n[0], dim);
    L.n1b = put(src.n[1], dim);
    L.n2 = put(src.n[2], dim);
    L.n2b = put(src.n[3], dim);
  }
  e = hipMemcpy(m + o_par, host.data(), host.size() * 4, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    hip_fail(name, e);
    vision_free(v);
    return nullptr;
  }
  v->img = (float *)(m + o_img);
  v->patches = (float *)(m + o_pat);
  v->x = (float *)(m + o_x);
  v->y = (float *)(m + o_y);
  v->qkv = (float *)(m + o_qkv);
  v->att = (float *)(m + o_att);
  v->hbuf = (float *)(m + o_h);
  v->hln = (float *)(m + o_hln);
  v->out = (float *)(m + o_out);
  v->a8 = (int8_t *)(m + o_a8);
  v->as = (float *)(m + o_as);
  return v;
}

}  // namespace

extern "C" {

gemma_hip_vision *gemma_hip_vision_create(const gemma_hip_vision_config *cfg,
                                          const gemma_hip_vision_layer *layers,
                                          const float *pe, const float *pe_b,
                                          const int8_t *pos_q, const float *pos_s,
                                          const float *post_n, const float *post_nb,
                                          const float *norm, const int8_t *proj,
                                          const float *proj_s) {
  static const char *kName = "gemma_hip_vision_create";
  if (need_init()) return nullptr;
  if (cfg == nullptr || layers == nullptr || cfg->nl <= 0) {
    fail("%s: null argument", kName);
    return nullptr;
  }
  std::vector<VisLayerSrc> src(cfg->nl);
  for (int l = 0; l < cfg->nl; ++l) {
    const gemma_hip_vision_layer &a = layers[l];
    src[l] = VisLayerSrc{{a.wq, a.wk, a.wv, a.wo, a.w1, a.w2},
                         {a.wq_s, a.wk_s, a.wv_s, a.wo_s, a.w1_s, a.w2_s},
                         {a.bq, a.bk, a.bv, a.bo, a.b1, a.b2},
                         {a.n1, a.n1_b, a.n2, a.n2_b}};
  }
  return vision_build(kName, cfg, src.data(), true, pe, pe_b, pos_q, pos_s, post_n, post_nb,
                      norm, proj, proj_s);
}

gemma_hip_vision *gemma_hip_vision_create_f32(const gemma_hip_vision_config *cfg,
                                              const gemma_hip_vision_layer_f32 *layers,
                                              const float *pe, const float *pe_b,
                                              const float *pos, const float *post_n,
                                              const float *post_nb, const float *norm,
                                              const float *proj) {
  static const char *kName = "gemma_hip_vision_create_f32";
  if (need_init()) return nullptr;
  if (cfg == nullptr || layers == nullptr || cfg->nl <= 0) {
    fail("%s: null argument", kName);
    return nullptr;
  }
  std::vector<VisLayerSrc> src(cfg->nl);
  for (int l = 0; l < cfg->nl; ++l) {
    const gemma_hip_vision_layer_f32 &a = layers[l];
    src[l] = VisLayerSrc{{a.wq, a.wk, a.wv, a.wo, a.w1, a.w2},
                         {},
                         {a.bq, a.bk, a.bv, a.bo, a.b1, a.b2},
                         {a.n1, a.n1_b, a.n2, a.n2_b}};
  }
  return vision_build(kName, cfg, src.data(), false, pe, pe_b, pos, nullptr, post_n, post_nb,
                      norm, proj, nullptr);
}

void gemma_hip_vision_destroy(gemma_hip_vision *vis) {
  if (vis == nullptr) return;
  if (g.ready) (void)hipStreamSynchronize(g.stream);
  vision_free(vis);
}

int gemma_hip_vision_forward(gemma_hip_vision *vis, const float *img, float *out) {
  if (need_init()) return 1;
  if (vis == nullptr || img == nullptr || out == nullptr)
    return fail("gemma_hip_vision_forward: null argument");
  const gemma_hip_vision_config &c = vis->cfg;
  GH_CHECK("gemma_hip_vision_forward: sync", hipStreamSynchronize(g.stream));
  GH_CHECK("gemma_hip_vision_forward: image H2D",
           hipMemcpyAsync(vis->img, img, (size_t)c.img_px * c.img_px * 3 * 4,
                          hipMemcpyHostToDevice, g.stream));
  perf_enter(kPhaseVision);
  GH_CHECK("gemma_hip_vision_forward: launch", vision_enqueue(vis, g.stream));
  GH_CHECK("gemma_hip_vision_forward: D2H",
           hipMemcpyAsync(out, vis->out, (size_t)c.img_tok * c.text_dim * 4,
                          hipMemcpyDeviceToHost, g.stream));
  GH_CHECK("gemma_hip_vision_forward: sync", hipStreamSynchronize(g.stream));
  return 0;
}

int gemma_hip_vision_set_attention(gemma_hip_vision *vis, int mode) {
  if (vis == nullptr) return fail("gemma_hip_vision_set_attention: null argument");
  if (mode != GEMMA_HIP_ATTN_F64 && mode != GEMMA_HIP_ATTN_F32)
    return fail("gemma_hip_vision_set_attention: unknown mode %d", mode);
  vis->attn_f32 = mode == GEMMA_HIP_ATTN_F32;
  return 0;
}

int gemma_hip_gemma_image(gemma_hip_decoder *dec, gemma_hip_vision *vis, const float *img,
                          int *pos, float *logits, int *next) {
  static const char *kName = "gemma_hip_gemma_image";
  if (need_init()) return 1;
  if (dec == nullptr || vis == nullptr || img == nullptr || pos == nullptr)
    return fail("%s: null argument", kName);
  const gemma_hip_vision_config &c = vis->cfg;
  if (c.text_dim != dec->cfg.dim)
    return fail("%s: the tower projects to %d, the decoder is %d wide", kName, c.text_dim,
                dec->cfg.dim);
  if (prefill_check(dec, kName, c.img_tok, *pos) || prefill_stage(dec, kName, c.img_tok))
    return 1;
  PF_CHECK("image H2D", hipMemcpyAsync(vis->img, img, (size_t)c.img_px * c.img_px * 3 * 4,
                                       hipMemcpyHostToDevice, g.stream));
  perf_enter(kPhaseVision);
  PF_CHECK("vision", vision_enqueue(vis, g.stream));
  PF_CHECK("soft tokens", hipMemcpyAsync(dec->pf_x, vis->out, (size_t)c.img_tok * c.text_dim * 4,
                                         hipMemcpyDeviceToDevice, g.stream));
  if (prefill_run(dec, kName, c.img_tok, *pos, 0, false, true, logits, next)) return 1;
  *pos += c.img_tok;
  return 0;
}

}  // extern "C"
