// Optimizer: global gradient norm (SumSquared + Sqrt_Scale), clip, and the
// Adam / AdamW update, optionally fused into one bandwidth-bound pass that reads
// g / s on the fly (Engine/kernels.cu:1486-1534, 1763-1773; Includes/kernels.h:293-300).
//
// The reference sums squares with thread 0 of every 512-thread block looping
// serially and then a CAS loop on one double (SumSquared / atomicAddDouble).
// Here every lane accumulates float4 loads in double, waves reduce with
// shuffles, and one block adds the per-block partials in a fixed order, so the
// norm is bit-reproducible.
#include "common.hpp"
#include <math.h>

#include <algorithm>
#include <atomic>
#include <mutex>

using namespace mle;

namespace {

constexpr int NT = 256;
constexpr unsigned kPartCap = 8192;

__device__ __forceinline__ f32x4 ld4(const float* p, size_t i) { return *reinterpret_cast<const f32x4*>(p + i); }
__device__ __forceinline__ void st4(float* p, size_t i, f32x4 v) { *reinterpret_cast<f32x4*>(p + i) = v; }

// Range r sums the contiguous span [r * per, (r + 1) * per) of float4 groups
// (VEC) or floats, so each workgroup streams one span of memory (the DRAM
// pages it opens are read through; strided grids across the whole array ran
// 14 % slower).  Eight 16-byte loads are in flight per lane, each feeding its
// own accumulator; the order of the additions is fixed by (n, grid), and the
// partial of range r is stored at part[r].
//
// Cache placement for the update that follows: workgroup b takes range
// grid - 1 - b, so the array is read from the top down, and ranges that start
// below `keep` units are read with ordinary (cache-allocating) loads, the rest
// with non-temporal ones.  The update then reads the array from the bottom
// up, and its first kSqKeepBytes of gradient reads are served by the 256 MiB
// Infinity Cache.  On 100 M floats (C2): update 468 -> 426 us, this pass
// 67 -> 75 us, the step 0.540 -> 0.507 ms.  Which workgroup takes which range
// changes neither the sums nor their order.
constexpr int SQ_U = 8;
constexpr size_t kSqKeepBytes = size_t(256) << 20;

template <bool KEEP>
__device__ __forceinline__ f32x4 sq_load4(const f32x4* p) {
  return KEEP ? *p : __builtin_nontemporal_load(p);
}

template <bool VEC, bool KEEP>
__device__ __forceinline__ double sqnorm_range(const float* __restrict__ g, size_t n, size_t per, unsigned r,
                                               bool& bad) {
  double acc[SQ_U];
#pragma unroll
  for (int u = 0; u < SQ_U; ++u) acc[u] = 0.0;
  const size_t units = VEC ? n / 4 : n;
  const size_t b0 = (size_t)r * per, b1 = b0 + per < units ? b0 + per : units;
  size_t i = b0 + threadIdx.x;
  if (VEC) {
    const f32x4* g4 = reinterpret_cast<const f32x4*>(g);
    for (; i + (SQ_U - 1) * NT < b1; i += SQ_U * NT) {
      f32x4 v[SQ_U];
#pragma unroll
      for (int u = 0; u < SQ_U; ++u) v[u] = sq_load4<KEEP>(g4 + i + u * NT);
#pragma unroll
      for (int u = 0; u < SQ_U; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const double d = (double)v[u][j];
          acc[u] += d * d;
          bad |= !isfinite(v[u][j]);
        }
    }
    for (; i < b1; i += NT) {
      const f32x4 v = sq_load4<KEEP>(g4 + i);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const double d = (double)v[j];
        acc[0] += d * d;
        bad |= !isfinite(v[j]);
      }
    }
    // the n % 4 tail, by the last range
    if (r == gridDim.x - 1 && threadIdx.x < n - units * 4) {
      const float x = g[units * 4 + threadIdx.x];
      acc[1] += (double)x * (double)x;
      bad |= !isfinite(x);
    }
  } else {
    for (; i < b1; i += NT) {
      const float x = g[i];
      acc[0] += (double)x * (double)x;
      bad |= !isfinite(x);
    }
  }
  double t = 0.0;
#pragma unroll
  for (int u = 0; u < SQ_U; ++u) t += acc[u];
  return t;
}

template <bool VEC>
__global__ __launch_bounds__(NT) void sqnorm_partial(const float* __restrict__ g, size_t n, size_t per,
                                                     double* __restrict__ part, int* __restrict__ nonfinite,
                                                     size_t keep) {
  __shared__ double red[NT / 64];
  const unsigned r = gridDim.x - 1 - blockIdx.x;
  bool bad = false;
  double t = (size_t)r * per < keep ? sqnorm_range<VEC, true>(g, n, per, r, bad)
                                    : sqnorm_range<VEC, false>(g, n, per, r, bad);
  t = block_sum<NT>(t, red);
  if (threadIdx.x == 0) part[r] = t;
  if (bad && nonfinite) nonfinite[0] = 1;
}

// Launch shape of the partial pass: `per` units (float4 groups when VEC,
// else floats) per workgroup, a multiple of NT, and the grid that covers n
// with at most kPartCap workgroups (100 M floats: 8139 workgroups of 3072
// float4 groups, 12 per lane).
struct SqnormShape {
  unsigned grid;
  size_t per;
};
inline SqnormShape sqnorm_shape(size_t n, bool vec) {
  const size_t units = vec ? n / 4 : n;
  size_t blocks = (units + (size_t)NT * SQ_U - 1) / ((size_t)NT * SQ_U);
  blocks = std::min<size_t>(std::max<size_t>(blocks, 1), kPartCap);
  size_t per = (units + blocks - 1) / blocks;
  per = std::max<size_t>((per + NT - 1) / NT * NT, NT);
  const size_t grid = std::max<size_t>((units + per - 1) / per, 1);
  return {(unsigned)grid, per};
}

// accum[0] (+)= sum(part).  With do_scale, then s = sqrt(accum);
// s = s > 1 ? s*scale : scale (Sqrt_Scale type 0), skipped when accum is NaN.
constexpr int FIN_NT = 1024;
static_assert(kPartCap % FIN_NT == 0, "the finishing launch reads kPartCap / FIN_NT partials per lane");
__global__ __launch_bounds__(FIN_NT) void sqnorm_finish(const double* __restrict__ part, unsigned nparts,
                                                        double* __restrict__ accum, int add_existing, int do_scale,
                                                        double scale, double* __restrict__ copy_out) {
  __shared__ double red[FIN_NT / 64];
  // Up to kPartCap / FIN_NT = 8 partials per lane, all loads issued before
  // the first add (a loop would wait out one memory latency per partial).
  constexpr int PER = kPartCap / FIN_NT;
  double v[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const unsigned i = threadIdx.x + (unsigned)j * FIN_NT;
    v[j] = i < nparts ? part[i] : 0.0;
  }
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < PER; ++j) acc += v[j];
  acc = block_sum<FIN_NT>(acc, red);
  if (threadIdx.x == 0) {
    double v = add_existing ? accum[0] + acc : acc;
    if (do_scale && v == v) {
      const double cur = sqrt(v);
      v = (cur > 1.0) ? cur * scale : scale;
    }
    accum[0] = v;
    if (copy_out) copy_out[0] = v;
  }
}

__global__ void sqrt_scale_kernel(double* s, double scale) {
  const double x = s[0];
  if (x == x) {
    const double cur = sqrt(x);
    s[0] = (cur > 1.0) ? cur * scale : scale;
  }
}

struct AdamArgs {
  float* p;
  const float* g;
  float* m;
  float* v;
  size_t n;
  float lr, b1, b2, eps, wd;
  double omb1, omb2;  // 1.0 - b (double, as the reference's (1.0 - b1) literal)
  double r1, r2;      // 1 / (1 - b^t): the bias corrections, applied in double
  const double* clip; // g is read as g / (float)clip[0] when set
};

// One element of AdamUpdate / AdamWUpdate (Engine/kernels.cu:1508-1534).
template <bool ADAMW>
__device__ __forceinline__ void adam_elem(const AdamArgs& a, float& p, float g, float& m, float& v, float sf,
                                          bool clip) {
  if (clip) g = g / sf;
  m = (float)((double)(a.b1 * m) + a.omb1 * (double)g);
  v = (float)((double)(a.b2 * v) + (a.omb2 * (double)g) * (double)g);
  // The reference divides the promoted moment by (1 - b^t) in double; a
  // multiply by the double reciprocal rounds to the same float except when
  // the quotient lies within ~1 double ulp of a float rounding boundary.
  const float m_hat = (float)((double)m * a.r1);
  const float v_hat = (float)((double)v * a.r2);
  const float vs = sqrtf(v_hat);
  if (ADAMW) p -= a.lr * ((m_hat / (vs + a.eps)) + a.wd * p);
  else p -= a.lr * m_hat / (vs + a.eps);
}

// Vector path: one float4 of each of p, g, m, v per thread in 1024-thread
// blocks (no grid-stride loop), non-temporal loads and stores -- the stream is
// touched once.  Measured fastest on MI355X for this 4-read / 3-write pattern.
constexpr int ADAM_NT = 1024;

template <bool ADAMW, bool CLIP>
__global__ __launch_bounds__(ADAM_NT) void adam_vec_kernel(AdamArgs a) {
  const float sf = CLIP ? (float)a.clip[0] : 1.0f;
  const size_t n4 = a.n / 4;
  const size_t i = (size_t)blockIdx.x * ADAM_NT + threadIdx.x;
  if (i < n4) {
    f32x4* p4 = reinterpret_cast<f32x4*>(a.p) + i;
    f32x4* m4 = reinterpret_cast<f32x4*>(a.m) + i;
    f32x4* v4 = reinterpret_cast<f32x4*>(a.v) + i;
    f32x4 p = __builtin_nontemporal_load(p4);
    const f32x4 g = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(a.g) + i);
    f32x4 m = __builtin_nontemporal_load(m4);
    f32x4 v = __builtin_nontemporal_load(v4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float pj = p[j], mj = m[j], vj = v[j];
      adam_elem<ADAMW>(a, pj, g[j], mj, vj, sf, CLIP);
      p[j] = pj;
      m[j] = mj;
      v[j] = vj;
    }
    __builtin_nontemporal_store(p, p4);
    __builtin_nontemporal_store(m, m4);
    __builtin_nontemporal_store(v, v4);
  }
  // the n % 4 tail, by the first threads of the last block
  const size_t e = n4 * 4 + threadIdx.x;
  if (blockIdx.x == gridDim.x - 1 && e < a.n) {
    float pj = a.p[e], mj = a.m[e], vj = a.v[e];
    adam_elem<ADAMW>(a, pj, a.g[e], mj, vj, sf, CLIP);
    a.p[e] = pj;
    a.m[e] = mj;
    a.v[e] = vj;
  }
}

// Scalar path for operands that are not 16-byte aligned.
template <bool ADAMW, bool CLIP>
__global__ __launch_bounds__(NT) void adam_kernel(AdamArgs a) {
  const float sf = CLIP ? (float)a.clip[0] : 1.0f;
  const size_t stride = (size_t)gridDim.x * NT;
  for (size_t e = (size_t)blockIdx.x * NT + threadIdx.x; e < a.n; e += stride) {
    float pj = a.p[e], mj = a.m[e], vj = a.v[e];
    adam_elem<ADAMW>(a, pj, a.g[e], mj, vj, sf, CLIP);
    a.p[e] = pj;
    a.m[e] = mj;
    a.v[e] = vj;
  }
}

template <bool ADAMW, bool CLIP>
void launch_adam(hipStream_t s, const AdamArgs& a, bool vec) {
  if (vec) {
    const size_t blocks = std::max<size_t>(1, (a.n / 4 + ADAM_NT - 1) / ADAM_NT);
    mle::launch(adam_vec_kernel<ADAMW, CLIP>, (unsigned)blocks, ADAM_NT, 0, s, a);
  } else {
    mle::launch(adam_kernel<ADAMW, CLIP>, stream_grid(a.n, NT, 8192), NT, 0, s, a);
  }
}

int launch_update(hipStream_t s, float* p, const float* g, float* m, float* v, size_t n, int t, float lr, float b1,
                  float b2, float eps, float wd, int adamw, const double* clip) {
  AdamArgs a;
  a.p = p;
  a.g = g;
  a.m = m;
  a.v = v;
  a.n = n;
  a.lr = lr;
  a.b1 = b1;
  a.b2 = b2;
  a.eps = eps;
  a.wd = wd;
  a.omb1 = 1.0 - (double)b1;
  a.omb2 = 1.0 - (double)b2;
  double c1, c2;
  if (adamw) {  // pow in double (AdamWUpdate)
    c1 = 1.0 - pow((double)b1, (double)t);
    c2 = 1.0 - pow((double)b2, (double)t);
  } else {  // powf (AdamUpdate)
    c1 = 1.0 - (double)powf(b1, (float)t);
    c2 = 1.0 - (double)powf(b2, (float)t);
  }
  a.r1 = 1.0 / c1;
  a.r2 = 1.0 / c2;
  a.clip = clip;
  const bool vec = aligned16(p) && aligned16(g) && aligned16(m) && aligned16(v);
  const double bytes = 28.0 * (double)n;
  ProbeScope probe("adam_update", s, 0.0, bytes);
  if (adamw) {
    if (clip) launch_adam<true, true>(s, a, vec);
    else launch_adam<true, false>(s, a, vec);
  } else {
    if (clip) launch_adam<false, true>(s, a, vec);
    else launch_adam<false, false>(s, a, vec);
  }
  return check_launch("mle_adam_update");
}

// Workspace slots the partial pass needs: its larger grid of the two layouts
// (the pointer's alignment picks one at launch).
unsigned sqnorm_grid(size_t n) { return std::max(sqnorm_shape(n, false).grid, sqnorm_shape(n, true).grid); }

void launch_sqnorm_partial(hipStream_t s, const float* g, size_t n, double* part, int* nonfinite, unsigned& grid) {
  const bool vec = aligned16(g);
  const SqnormShape sh = sqnorm_shape(n, vec);
  grid = sh.grid;
  const size_t keep = kSqKeepBytes / (vec ? 16 : 4);  // in the pass's units
  if (vec) mle::launch(sqnorm_partial<true>, sh.grid, NT, 0, s, g, n, sh.per, part, nonfinite, keep);
  else mle::launch(sqnorm_partial<false>, sh.grid, NT, 0, s, g, n, sh.per, part, nonfinite, keep);
}

}  // namespace

extern "C" {

size_t mle_sqnorm_ws_bytes(size_t n) { return (size_t)sqnorm_grid(n) * sizeof(double); }

int mle_grad_sqnorm_ex(mle_stream stream, const float* g, size_t n, double* accum, int* nonfinite, int sqrt_scale,
                       double scale, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(accum && (n == 0 || (g && ws)), "mle_grad_sqnorm: null pointer");
  hipStream_t s = as_stream(stream);
  if (n == 0) return sqrt_scale ? mle_sqrt_scale(stream, accum, scale) : MLE_OK;
  if (ws_bytes < mle_sqnorm_ws_bytes(n)) return set_error(MLE_ERR_WORKSPACE, "mle_grad_sqnorm: workspace too small");
  double* part = static_cast<double*>(ws);
  // The probe times the whole sum: the partial pass and the launch that
  // finishes it.
  ProbeScope probe("sqnorm", s, 0.0, 4.0 * (double)n);
  unsigned grid = 0;
  launch_sqnorm_partial(s, g, n, part, nonfinite, grid);
  mle::launch(sqnorm_finish, 1, FIN_NT, 0, s, part, grid, accum, 1, sqrt_scale ? 1 : 0, scale, nullptr);
  return check_launch("mle_grad_sqnorm");
}

int mle_grad_sqnorm(mle_stream stream, const float* g, size_t n, double* accum, int* nonfinite, void* ws,
                    size_t ws_bytes) {
  return mle_grad_sqnorm_ex(stream, g, n, accum, nonfinite, 0, 1.0, ws, ws_bytes);
}

int mle_sqrt_scale(mle_stream stream, double* s, double scale) {
  MLE_CHECK_ARG(s, "mle_sqrt_scale: null pointer");
  mle::launch(sqrt_scale_kernel, 1, 1, 0, as_stream(stream), s, scale);
  return check_launch("mle_sqrt_scale");
}

int mle_adam_update(mle_stream stream, float* p, const float* g, float* m, float* v, size_t n, int t, float lr,
                    float b1, float b2, float eps, float weight_decay, int adamw, const double* clip) {
  MLE_CHECK_ARG(p && g && m && v, "mle_adam_update: null pointer");
  MLE_CHECK_ARG(t >= 1, "mle_adam_update: step t = %d must be >= 1", t);
  if (n == 0) return MLE_OK;
  return launch_update(as_stream(stream), p, g, m, v, n, t, lr, b1, b2, eps, weight_decay, adamw, clip);
}

size_t mle_adamw_clip_ws_bytes(size_t n) { return 256 + mle_sqnorm_ws_bytes(n); }

}  // extern "C"

namespace {

// accumulate -> Sqrt_Scale -> update with g / s over one span; `ws` holds s in
// its first 256 bytes and the per-block partial sums after them.  Every value
// read from ws is written earlier in the same call (each partial block writes
// its own slot, the finish kernel writes s from the partials alone), so ws
// needs no clearing between calls.
int adamw_clip(hipStream_t s, float* p, const float* g, float* m, float* v, size_t n, int t, float lr, float b1,
               float b2, float eps, float weight_decay, int adamw, double clip_scale, double* norm_out, void* ws) {
  const double* clip = nullptr;
  if (clip_scale > 0.0) {
    double* sdev = static_cast<double*>(ws);
    double* part = reinterpret_cast<double*>(static_cast<char*>(ws) + 256);
    {
      ProbeScope probe("sqnorm", s, 0.0, 4.0 * (double)n);
      unsigned grid = 0;
      launch_sqnorm_partial(s, g, n, part, nullptr, grid);
      // s = Sqrt_Scale(sum g^2) computed from zero, so nothing is cleared beforehand.
      mle::launch(sqnorm_finish, 1, FIN_NT, 0, s, part, grid, sdev, 0, 1, clip_scale, norm_out);
    }
    int rc = check_launch("adamw_clip: norm");
    if (rc) return rc;
    clip = sdev;
  }
  return launch_update(s, p, g, m, v, n, t, lr, b1, b2, eps, weight_decay, adamw, clip);
}

// ---- allocation-free variant ----------------------------------------------
// Scratch of mle_adamw_clip_fused_noalloc: the clip scale s (256 bytes) and
// at most kPartCap per-block partial sums -- the workspace mle_adamw_clip_fused
// takes, at its largest (sqnorm_grid never exceeds kPartCap).  One copy per
// GPU, alive until the process ends; every call on a GPU uses that GPU's copy.
constexpr size_t kScratchBytes = 256 + (size_t)kPartCap * sizeof(double);
static __device__ __align__(256) double scratch[kScratchBytes / sizeof(double)];

// Device address of `scratch` per device.  The host-side name `scratch` is a
// stand-in, not a device address: kernels and copies take these pointers.
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_dev[kMaxDevices];
std::mutex g_scratch_mu;

int scratch_on_current_device(void** out) {
  int dev = 0;
  MLE_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(MLE_ERR_UNSUPPORTED, "adamw scratch: device %d is beyond the %d devices supported", dev,
                     kMaxDevices);
  void* ptr = g_scratch_dev[dev].load(std::memory_order_acquire);
  if (!ptr) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    ptr = g_scratch_dev[dev].load(std::memory_order_relaxed);
    if (!ptr) {
      hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !ptr) return hip_error(e, "adamw scratch: hipGetSymbolAddress(scratch)");
      g_scratch_dev[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return MLE_OK;
}

}  // namespace

namespace mle {
// Called by mle_init with `device` current: looks up this device's scratch
// address once, so the allocation-free entry point makes no setup call later.
int optim_scratch_setup() {
  void* ptr = nullptr;
  return scratch_on_current_device(&ptr);
}
}  // namespace mle

extern "C" {

int mle_adamw_clip_fused(mle_stream stream, float* p, const float* g, float* m, float* v, size_t n, int t, float lr,
                         float b1, float b2, float eps, float weight_decay, int adamw, double clip_scale,
                         double* norm_out, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(p && g && m && v && ws, "mle_adamw_clip_fused: null pointer");
  MLE_CHECK_ARG(t >= 1, "mle_adamw_clip_fused: step t = %d must be >= 1", t);
  if (n == 0) return MLE_OK;
  if (ws_bytes < mle_adamw_clip_ws_bytes(n)) return set_error(MLE_ERR_WORKSPACE, "mle_adamw_clip_fused: workspace too small");
  int rc = adamw_clip(as_stream(stream), p, g, m, v, n, t, lr, b1, b2, eps, weight_decay, adamw, clip_scale, norm_out,
                      ws);
  if (rc) return rc;
  return check_launch("mle_adamw_clip_fused");
}

int mle_adamw_clip_fused_noalloc(mle_stream stream, float* p, const float* g, float* m, float* v, size_t n, int t,
                                 float lr, float b1, float b2, float eps, float weight_decay, int adamw,
                                 double clip_scale, double* norm_out) {
  MLE_CHECK_ARG(p && g && m && v, "mle_adamw_clip_fused_noalloc: null pointer");
  MLE_CHECK_ARG(t >= 1, "mle_adamw_clip_fused_noalloc: step t = %d must be >= 1", t);
  if (n == 0) return MLE_OK;
  const size_t need = mle_adamw_clip_ws_bytes(n);
  if (need > kScratchBytes)
    return set_error(MLE_ERR_UNSUPPORTED,
                     "mle_adamw_clip_fused_noalloc: n = %zu needs %zu bytes of scratch, the fixed scratch holds %zu", n,
                     need, kScratchBytes);
  void* ws = nullptr;
  int rc = scratch_on_current_device(&ws);
  if (rc) return rc;
  rc = adamw_clip(as_stream(stream), p, g, m, v, n, t, lr, b1, b2, eps, weight_decay, adamw, clip_scale, norm_out, ws);
  if (rc) return rc;
  return check_launch("mle_adamw_clip_fused_noalloc");
}

}  // extern "C"
