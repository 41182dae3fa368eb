// Shared helpers for the gfx950 kernels behind include/mle_hip.h.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include <stddef.h>
#include <mutex>
#include <string>
#include "../../include/mle_hip.h"

typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace mle {

// ---- host-side error reporting -------------------------------------------
int set_error(int code, const char* fmt, ...);
int hip_error(hipError_t e, const char* where);
// Checks the launch that was just enqueued.
int check_launch(const char* kernel);

// ---- launch probe ---------------------------------------------------------
// Returns true when `kernel` is the armed probe family; then the caller wraps
// its launches in probe_begin / probe_end (ProbeScope), and each kernel it
// launches with mle::launch carries a start/stop event pair in its dispatch.
bool probe_armed(const char* kernel);
void probe_begin(hipStream_t s);
void probe_end(hipStream_t s, double flop, double bytes);
// Inside a probed call on this thread: two events for the next launch.
bool probe_events(hipEvent_t* a, hipEvent_t* b);

struct ProbeScope {
  bool on;
  hipStream_t s;
  double flop, bytes;
  ProbeScope(const char* k, hipStream_t st, double f, double b) : on(probe_armed(k)), s(st), flop(f), bytes(b) {
    if (on) {  // not while the stream records a graph: its events would join the graph
      hipStreamCaptureStatus c = hipStreamCaptureStatusNone;
      on = hipStreamIsCapturing(s, &c) == hipSuccess && c == hipStreamCaptureStatusNone;
    }
    if (on) probe_begin(s);
  }
  ~ProbeScope() {
    if (on) probe_end(s, flop, bytes);
  }
};

// Launches k<<<grid, block, shmem, s>>>(args...).  Inside a probed call the
// kernel is launched with hipExtLaunchKernelGGL and the probe's events, which
// time the kernel itself: no marker packet joins the stream, so the stream
// runs as it does unprobed.
template <typename... KArgs, typename... Args>
inline void launch(void (*k)(KArgs...), dim3 grid, dim3 block, uint32_t shmem, hipStream_t s, Args... args) {
  hipEvent_t a, b;
  if (probe_events(&a, &b)) hipExtLaunchKernelGGL(k, grid, block, shmem, s, a, b, 0u, args...);
  else k<<<grid, block, shmem, s>>>(args...);
}

// Per-device set-up of the allocation-free optimizer entry point (optim.hip);
// mle_init calls it with the device current.
int optim_scratch_setup();

// ---- scalar read-back -----------------------------------------------------
// One pinned, host-coherent slot per device: the value's bits and the
// sequence number of the read that wrote them.
struct ScalarSlot {
  unsigned seq;
  unsigned bits;
};
// A host read of a device scalar (mle_read_scalar): scalar_read_begin locks
// the current device's slot (held until the ScalarRead goes) and picks the
// sequence number that the publishing kernel writes with the value;
// scalar_read_finish waits for it, or returns at once under graph capture,
// where each replay publishes.
struct ScalarRead {
  ScalarSlot* slot = nullptr;
  unsigned seq = 0;
  std::unique_lock<std::mutex> lock;
};
int scalar_read_begin(ScalarRead& r, const char* who);
int scalar_read_finish(hipStream_t s, ScalarRead& r, float* dst, const char* who);
// Device side of a read: the value's bits, then the sequence number (system
// scope, release), so the host never sees the number before the value.
__device__ __forceinline__ void publish_scalar(ScalarSlot* slot, unsigned bits, unsigned seq) {
  __hip_atomic_store(&slot->bits, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  __hip_atomic_store(&slot->seq, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

inline hipStream_t as_stream(mle_stream s) { return reinterpret_cast<hipStream_t>(s); }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Grid size for grid-stride streaming kernels: enough waves to cover HBM
// latency on 256 CUs, a function of n only (so reductions stay deterministic).
inline unsigned stream_grid(size_t work_items, unsigned block, unsigned cap = 4096) {
  size_t g = (work_items + block - 1) / block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (unsigned)g;
}

}  // namespace mle

#define MLE_CHECK_ARG(cond, ...)                                    \
  do {                                                              \
    if (!(cond)) return ::mle::set_error(MLE_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define MLE_HIP(call)                                        \
  do {                                                       \
    hipError_t e_ = (call);                                  \
    if (e_ != hipSuccess) return ::mle::hip_error(e_, #call); \
  } while (0)

// ---- device-side reductions (wave64) --------------------------------------
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Block-wide sum for blockDim.x == NT (multiple of 64).  `red` must hold NT/64
// values.  Every thread receives the total; the summation order is fixed.
template <int NT, typename T>
__device__ __forceinline__ T block_sum(T v, T* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  T t = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) t += red[w];
  return t;
}

template <int NT>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) t = fmaxf(t, red[w]);
  return t;
}
