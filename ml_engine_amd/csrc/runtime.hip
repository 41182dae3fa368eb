// Runtime part of the C ABI: errors, device memory, streams, arena, probe, fill.
#include "common.hpp"
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <atomic>
#include <mutex>
#include <string>
#include <vector>

namespace mle {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_error(hipError_t e, const char* where) {
  if (e == hipErrorOutOfMemory) {
    size_t fr = 0, tot = 0;
    (void)hipGetLastError();
    (void)hipMemGetInfo(&fr, &tot);
    return set_error(MLE_ERR_OOM, "%s: %s (device free %zu MB of %zu MB)", where, hipGetErrorString(e), fr >> 20,
                     tot >> 20);
  }
  return set_error(MLE_ERR_HIP, "%s: %s", where, hipGetErrorString(e));
}

int check_launch(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_error(e, kernel);
  return MLE_OK;
}

// ---- probe ---------------------------------------------------------------
// One record per probed call: the start/stop event pair of every kernel the
// call launched (each pair rides in its kernel's dispatch packet, so the
// measurement puts nothing else on the stream), and the call's flop and
// bytes.
struct ProbeRec {
  std::vector<std::pair<hipEvent_t, hipEvent_t>> ev;
  double flop, bytes;
};
static std::mutex g_probe_mu;
static std::string g_probe_kernel;
static std::vector<ProbeRec> g_probe_recs;
static std::vector<hipEvent_t> g_event_pool;
// The call being probed on this thread (launches made inside it take events).
static thread_local ProbeRec* t_open = nullptr;

static hipEvent_t take_event() {
  if (!g_event_pool.empty()) {
    hipEvent_t e = g_event_pool.back();
    g_event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  // Agent-scope completion only: a system-scope fence at each record would
  // write L2 back and stall the stream around every probed kernel.
  if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) return nullptr;
  return e;
}

// Set while a family is armed: an unarmed probe costs every launch one relaxed
// atomic load, no lock and no string compare.
static std::atomic<bool> g_probe_on{false};

// Armed families, as ",name1,name2," so a membership test is one search.
bool probe_armed(const char* kernel) {
  if (!g_probe_on.load(std::memory_order_relaxed)) return false;
  std::lock_guard<std::mutex> lk(g_probe_mu);
  const std::string key = std::string(",") + kernel + ",";
  return g_probe_kernel.find(key) != std::string::npos;
}

void probe_begin(hipStream_t) {
  delete t_open;
  t_open = new ProbeRec{{}, 0.0, 0.0};
}

bool probe_events(hipEvent_t* a, hipEvent_t* b) {
  *a = *b = nullptr;
  if (!t_open) return false;
  std::lock_guard<std::mutex> lk(g_probe_mu);
  hipEvent_t x = take_event();
  hipEvent_t y = x ? take_event() : nullptr;
  if (!y) {
    if (x) g_event_pool.push_back(x);
    return false;
  }
  t_open->ev.push_back({x, y});
  *a = x;
  *b = y;
  return true;
}

void probe_end(hipStream_t, double flop, double bytes) {
  ProbeRec* r = t_open;
  t_open = nullptr;
  if (!r) return;
  r->flop = flop;
  r->bytes = bytes;
  std::lock_guard<std::mutex> lk(g_probe_mu);
  if (!r->ev.empty()) g_probe_recs.push_back(std::move(*r));
  delete r;
}

// ---- scalar read-back ------------------------------------------------------
constexpr int kMaxDevices = 64;
static std::mutex g_slot_mu[kMaxDevices];
static ScalarSlot* g_slot[kMaxDevices] = {};
static unsigned g_slot_seq[kMaxDevices] = {};

__global__ void publish_scalar_kernel(const unsigned* src, ScalarSlot* slot, unsigned seq) {
  publish_scalar(slot, *src, seq);
}

int scalar_read_begin(ScalarRead& r, const char* who) {
  int dev = 0;
  MLE_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return set_error(MLE_ERR_INVALID, "%s: device %d out of range", who, dev);
  r.lock = std::unique_lock<std::mutex>(g_slot_mu[dev]);
  ScalarSlot*& slot = g_slot[dev];
  if (!slot) {
    void* p = nullptr;
    MLE_HIP(hipHostMalloc(&p, sizeof(ScalarSlot), hipHostMallocCoherent));
    slot = static_cast<ScalarSlot*>(p);
    slot->seq = 0;
    slot->bits = 0;
  }
  r.slot = slot;
  r.seq = ++g_slot_seq[dev];
  return MLE_OK;
}

int scalar_read_finish(hipStream_t s, ScalarRead& r, float* dst, const char* who) {
  // Under graph capture the publishing kernel is recorded, not run: each
  // replay publishes the value, which mle_scalar_last reads after a
  // synchronisation.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  MLE_HIP(hipStreamIsCapturing(s, &cap));
  if (cap != hipStreamCaptureStatusNone) return MLE_OK;
  // The stream is asked every 256 spins: a stream that completed or failed
  // without the value having landed ends the wait.
  ScalarSlot* slot = r.slot;
  for (unsigned long spins = 1;; ++spins) {
    if (__atomic_load_n(&slot->seq, __ATOMIC_ACQUIRE) == r.seq) break;
    if ((spins & 255) == 0) {
      const hipError_t q = hipStreamQuery(s);
      if (q == hipSuccess) {
        if (__atomic_load_n(&slot->seq, __ATOMIC_ACQUIRE) == r.seq) break;
        return set_error(MLE_ERR_HIP, "%s: the stream drained without publishing the value", who);
      }
      if (q != hipErrorNotReady) return hip_error(q, who);
    }
    __builtin_ia32_pause();
  }
  const unsigned bits = __atomic_load_n(&slot->bits, __ATOMIC_ACQUIRE);
  memcpy(dst, &bits, sizeof(float));
  return MLE_OK;
}

}  // namespace mle

using namespace mle;

// ---- arena -----------------------------------------------------------------
struct mle_arena_s {
  char* base;
  size_t cap;
  size_t used;
};

extern "C" {

const char* mle_last_error(void) { return g_last_error.c_str(); }

const char* mle_version(void) { return "mle_hip 0.1 gfx950"; }

int mle_init(int device) {
  int n = 0;
  MLE_HIP(hipGetDeviceCount(&n));
  MLE_CHECK_ARG(device >= 0 && device < n, "mle_init: device %d out of range (%d devices)", device, n);
  MLE_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  MLE_HIP(hipGetDeviceProperties(&prop, device));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return set_error(MLE_ERR_UNSUPPORTED, "mle_init: device %d is %s; this library is built for gfx950", device,
                     prop.gcnArchName);
  return optim_scratch_setup();
}

int mle_device_alloc(void** ptr, size_t bytes) {
  MLE_CHECK_ARG(ptr != nullptr, "mle_device_alloc: null out pointer");
  *ptr = nullptr;
  if (bytes == 0) bytes = 256;
  hipError_t e = hipMalloc(ptr, bytes);
  if (e != hipSuccess) {
    *ptr = nullptr;
    return hip_error(e, "mle_device_alloc");
  }
  return MLE_OK;
}

int mle_device_free(void* ptr) {
  if (ptr) MLE_HIP(hipFree(ptr));
  return MLE_OK;
}

int mle_memcpy_h2d(void* dst, const void* src, size_t bytes, mle_stream stream) {
  if (bytes == 0) return MLE_OK;
  MLE_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)));
  MLE_HIP(hipStreamSynchronize(as_stream(stream)));
  return MLE_OK;
}

int mle_memcpy_d2h(void* dst, const void* src, size_t bytes, mle_stream stream) {
  if (bytes == 0) return MLE_OK;
  MLE_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)));
  MLE_HIP(hipStreamSynchronize(as_stream(stream)));
  return MLE_OK;
}

int mle_read_scalar(mle_stream stream, const float* src, float* dst) {
  MLE_CHECK_ARG(src != nullptr && dst != nullptr, "mle_read_scalar: null pointer");
  ScalarRead r;
  int rc = scalar_read_begin(r, "mle_read_scalar");
  if (rc) return rc;
  hipStream_t s = as_stream(stream);
  publish_scalar_kernel<<<1, 1, 0, s>>>(reinterpret_cast<const unsigned*>(src), r.slot, r.seq);
  MLE_HIP(hipGetLastError());
  return scalar_read_finish(s, r, dst, "mle_read_scalar");
}

int mle_scalar_last(float* dst) {
  MLE_CHECK_ARG(dst != nullptr, "mle_scalar_last: null pointer");
  int dev = 0;
  MLE_HIP(hipGetDevice(&dev));
  MLE_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "mle_scalar_last: device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_slot_mu[dev]);
  MLE_CHECK_ARG(g_slot[dev] != nullptr, "mle_scalar_last: no value was published on device %d", dev);
  const unsigned bits = __atomic_load_n(&g_slot[dev]->bits, __ATOMIC_ACQUIRE);
  memcpy(dst, &bits, sizeof(float));
  return MLE_OK;
}

int mle_scalar_state(float* value, unsigned* published, unsigned* issued) {
  int dev = 0;
  MLE_HIP(hipGetDevice(&dev));
  MLE_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "mle_scalar_state: device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_slot_mu[dev]);
  const ScalarSlot* slot = g_slot[dev];
  const unsigned bits = slot ? __atomic_load_n(&slot->bits, __ATOMIC_ACQUIRE) : 0u;
  if (value) memcpy(value, &bits, sizeof(float));
  if (published) *published = slot ? __atomic_load_n(&slot->seq, __ATOMIC_ACQUIRE) : 0u;
  if (issued) *issued = g_slot_seq[dev];
  return MLE_OK;
}

int mle_scalar_clear(void) {
  int dev = 0;
  MLE_HIP(hipGetDevice(&dev));
  MLE_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "mle_scalar_clear: device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_slot_mu[dev]);
  if (g_slot[dev]) __atomic_store_n(&g_slot[dev]->seq, 0u, __ATOMIC_RELEASE);
  return MLE_OK;
}

int mle_scalar_expect(mle_stream stream, unsigned seq, float* dst) {
  MLE_CHECK_ARG(dst != nullptr && seq != 0, "mle_scalar_expect: bad argument");
  int dev = 0;
  MLE_HIP(hipGetDevice(&dev));
  MLE_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "mle_scalar_expect: device %d out of range", dev);
  std::unique_lock<std::mutex> lk(g_slot_mu[dev]);
  ScalarSlot* slot = g_slot[dev];
  MLE_CHECK_ARG(slot != nullptr, "mle_scalar_expect: no value was published on device %d", dev);
  hipStream_t s = as_stream(stream);
  // As scalar_read_finish: the stream is asked every 256 spins, and one that
  // drained without this number published ends the wait.
  for (unsigned long spins = 1;; ++spins) {
    if (__atomic_load_n(&slot->seq, __ATOMIC_ACQUIRE) == seq) break;
    if ((spins & 255) == 0) {
      const hipError_t q = hipStreamQuery(s);
      if (q == hipSuccess) {
        if (__atomic_load_n(&slot->seq, __ATOMIC_ACQUIRE) == seq) break;
        return set_error(MLE_ERR_INVALID, "mle_scalar_expect: the stream drained without publishing %u", seq);
      }
      if (q != hipErrorNotReady) return hip_error(q, "mle_scalar_expect");
    }
    __builtin_ia32_pause();
  }
  const unsigned bits = __atomic_load_n(&slot->bits, __ATOMIC_ACQUIRE);
  memcpy(dst, &bits, sizeof(float));
  return MLE_OK;
}

// ---- graphs ----------------------------------------------------------------
struct mle_graph_s {
  hipGraph_t graph;
  hipGraphExec_t exec;
};

int mle_graph_capture_begin(mle_stream stream) {
  MLE_CHECK_ARG(stream != nullptr, "mle_graph_capture_begin: capture needs a created stream");
  MLE_HIP(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeRelaxed));
  return MLE_OK;
}

int mle_graph_capture_end(mle_stream stream, mle_graph* out) {
  MLE_CHECK_ARG(stream != nullptr && out != nullptr, "mle_graph_capture_end: bad argument");
  *out = nullptr;
  hipGraph_t g = nullptr;
  MLE_HIP(hipStreamEndCapture(as_stream(stream), &g));
  hipGraphExec_t e = nullptr;
  const hipError_t err = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
  if (err != hipSuccess) {
    (void)hipGraphDestroy(g);
    return hip_error(err, "mle_graph_capture_end: instantiate");
  }
  *out = new mle_graph_s{g, e};
  return MLE_OK;
}

int mle_graph_launch(mle_graph graph, mle_stream stream) {
  MLE_CHECK_ARG(graph != nullptr, "mle_graph_launch: null graph");
  MLE_HIP(hipGraphLaunch(graph->exec, as_stream(stream)));
  return MLE_OK;
}

int mle_graph_destroy(mle_graph graph) {
  if (!graph) return MLE_OK;
  hipError_t e1 = hipGraphExecDestroy(graph->exec), e2 = hipGraphDestroy(graph->graph);
  delete graph;
  if (e1 != hipSuccess) return hip_error(e1, "mle_graph_destroy");
  if (e2 != hipSuccess) return hip_error(e2, "mle_graph_destroy");
  return MLE_OK;
}

int mle_memcpy_d2d(void* dst, const void* src, size_t bytes, mle_stream stream) {
  if (bytes == 0) return MLE_OK;
  MLE_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
  return MLE_OK;
}

int mle_stream_create(mle_stream* stream) {
  MLE_CHECK_ARG(stream != nullptr, "mle_stream_create: null out pointer");
  hipStream_t s = nullptr;
  MLE_HIP(hipStreamCreate(&s));  // default priority, as required on this hardware pool
  *stream = reinterpret_cast<mle_stream>(s);
  return MLE_OK;
}

int mle_stream_destroy(mle_stream stream) {
  if (stream) MLE_HIP(hipStreamDestroy(as_stream(stream)));
  return MLE_OK;
}

int mle_stream_sync(mle_stream stream) {
  MLE_HIP(hipStreamSynchronize(as_stream(stream)));
  MLE_HIP(hipGetLastError());
  return MLE_OK;
}

int mle_arena_create(size_t bytes, mle_arena* arena) {
  MLE_CHECK_ARG(arena != nullptr, "mle_arena_create: null out pointer");
  *arena = nullptr;
  bytes = (bytes + 255) & ~size_t(255);
  if (bytes == 0) bytes = 256;
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) return hip_error(e, "mle_arena_create");
  *arena = new mle_arena_s{static_cast<char*>(p), bytes, 0};
  return MLE_OK;
}

int mle_arena_alloc(mle_arena arena, size_t bytes, void** ptr) {
  MLE_CHECK_ARG(arena && ptr, "mle_arena_alloc: null argument");
  size_t need = (bytes + 255) & ~size_t(255);
  if (need == 0) need = 256;
  if (arena->used + need > arena->cap)
    return set_error(MLE_ERR_OOM, "mle_arena_alloc: %zu bytes requested, %zu of %zu used", bytes, arena->used,
                     arena->cap);
  *ptr = arena->base + arena->used;
  arena->used += need;
  return MLE_OK;
}

int mle_arena_reset(mle_arena arena) {
  MLE_CHECK_ARG(arena, "mle_arena_reset: null arena");
  arena->used = 0;
  return MLE_OK;
}

int mle_arena_destroy(mle_arena arena) {
  if (!arena) return MLE_OK;
  hipError_t e = hipFree(arena->base);
  delete arena;
  if (e != hipSuccess) return hip_error(e, "mle_arena_destroy");
  return MLE_OK;
}

size_t mle_arena_used(mle_arena arena) { return arena ? arena->used : 0; }
size_t mle_arena_capacity(mle_arena arena) { return arena ? arena->cap : 0; }

int mle_probe_arm(const char* kernel) {
  std::lock_guard<std::mutex> lk(g_probe_mu);
  for (auto& r : g_probe_recs)
    for (auto& e : r.ev) {
      g_event_pool.push_back(e.first);
      g_event_pool.push_back(e.second);
    }
  g_probe_recs.clear();
  const bool on = kernel && kernel[0];
  g_probe_kernel = on ? std::string(",") + kernel + "," : std::string();
  g_probe_on.store(on, std::memory_order_relaxed);
  return MLE_OK;
}

struct mle_event_s {
  hipEvent_t e;
};

int mle_event_create(mle_event* ev) {
  MLE_CHECK_ARG(ev != nullptr, "mle_event_create: null out pointer");
  *ev = nullptr;
  hipEvent_t e = nullptr;
  MLE_HIP(hipEventCreate(&e));
  *ev = new mle_event_s{e};
  return MLE_OK;
}

int mle_event_record(mle_event ev, mle_stream stream) {
  MLE_CHECK_ARG(ev != nullptr, "mle_event_record: null event");
  MLE_HIP(hipEventRecord(ev->e, as_stream(stream)));
  return MLE_OK;
}

int mle_event_elapsed_ms(mle_event start, mle_event stop, float* ms) {
  MLE_CHECK_ARG(start && stop && ms, "mle_event_elapsed_ms: null argument");
  MLE_HIP(hipEventSynchronize(stop->e));
  MLE_HIP(hipEventElapsedTime(ms, start->e, stop->e));
  return MLE_OK;
}

int mle_event_destroy(mle_event ev) {
  if (!ev) return MLE_OK;
  const hipError_t e = hipEventDestroy(ev->e);
  delete ev;
  if (e != hipSuccess) return hip_error(e, "mle_event_destroy");
  return MLE_OK;
}

int mle_probe_read(int* launches, double* total_ms, double* total_flop, double* total_bytes) {
  std::lock_guard<std::mutex> lk(g_probe_mu);
  double ms = 0, fl = 0, by = 0;
  for (auto& r : g_probe_recs) {
    for (auto& e : r.ev) {
      MLE_HIP(hipEventSynchronize(e.second));
      float t = 0;
      MLE_HIP(hipEventElapsedTime(&t, e.first, e.second));
      ms += t;
    }
    fl += r.flop;
    by += r.bytes;
  }
  if (launches) *launches = (int)g_probe_recs.size();
  if (total_ms) *total_ms = ms;
  if (total_flop) *total_flop = fl;
  if (total_bytes) *total_bytes = by;
  return MLE_OK;
}

}  // extern "C"
