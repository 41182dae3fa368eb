// Elementwise and data-movement kernels: HBM streaming, dwordx4 where the
// operands are 16-byte aligned, grid-stride loops sized for 256 CUs.
#include "activation.hpp"
#include "common.hpp"
#include <math.h>

#include <algorithm>

using namespace mle;

namespace {

__device__ __forceinline__ f32x4 ld4(const float* p, size_t i) { return *reinterpret_cast<const f32x4*>(p + i); }
__device__ __forceinline__ void st4(float* p, size_t i, f32x4 v) { *reinterpret_cast<f32x4*>(p + i) = v; }

// Vector body over n4 groups of four; the first workgroup also takes the
// (at most three) elements from 4 * n4 to n.
template <class Op>
__global__ __launch_bounds__(256) void map4_kernel(size_t n4, size_t n, Op op) {
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) op.vec(i * 4);
  if (blockIdx.x == 0 && 4 * n4 + threadIdx.x < n) op.one(4 * n4 + threadIdx.x);
}

template <class Op>
__global__ __launch_bounds__(256) void map1_kernel(size_t begin, size_t n, Op op) {
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t i = begin + (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) op.one(i);
}

template <class Op>
int run_map(hipStream_t s, size_t n, bool vec, const Op& op, const char* name) {
  if (n == 0) return MLE_OK;
  const size_t n4 = vec ? n / 4 : 0;
  if (n4) map4_kernel<Op><<<stream_grid(n4, 256, 8192), 256, 0, s>>>(n4, n, op);
  else map1_kernel<Op><<<stream_grid(n, 256, 8192), 256, 0, s>>>(0, n, op);
  return check_launch(name);
}

// ---- ops ---------------------------------------------------------------
struct FillOp {
  float* x;
  float v;
  __device__ void one(size_t i) const { x[i] = v; }
  __device__ void vec(size_t i) const { st4(x, i, f32x4{v, v, v, v}); }
};

struct ScaleAddOp {  // z = x + scale*y
  const float* x;
  const float* y;
  float* z;
  float s;
  __device__ void one(size_t i) const { z[i] = x[i] + s * y[i]; }
  __device__ void vec(size_t i) const { st4(z, i, ld4(x, i) + s * ld4(y, i)); }
};

struct AccumOneOp {  // y += x
  const float* x;
  float* y;
  __device__ void one(size_t i) const { y[i] += x[i]; }
  __device__ void vec(size_t i) const { st4(y, i, ld4(y, i) + ld4(x, i)); }
};

struct ScaleAssignOp {  // y = (float)(scale*(double)x): AccumOp applied to y == 0
  const float* x;
  float* y;
  double s;
  __device__ void one(size_t i) const { y[i] = (float)(s * (double)x[i]); }
  __device__ void vec(size_t i) const {
    f32x4 a = ld4(x, i), b;
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = (float)(s * (double)a[j]);
    st4(y, i, b);
  }
};

// ya (+)= x and yb (+)= x in one pass over x.  The sums are float adds and the
// assignments copies, which is what AccumOneOp and ScaleAssignOp give at scale 1.
template <bool ACC_A, bool ACC_B>
struct Accum2Op {
  const float* x;
  float* ya;
  float* yb;
  __device__ void one(size_t i) const {
    const float v = x[i];
    ya[i] = ACC_A ? ya[i] + v : v;
    yb[i] = ACC_B ? yb[i] + v : v;
  }
  __device__ void vec(size_t i) const {
    // every load before the first store (a load after a store waits for it)
    const f32x4 v = ld4(x, i);
    const f32x4 a = ACC_A ? ld4(ya, i) : v, b = ACC_B ? ld4(yb, i) : v;
    st4(ya, i, ACC_A ? a + v : v);
    st4(yb, i, ACC_B ? b + v : v);
  }
};

// z = a + b and y = act(z): the Add forward (x + 1 * y, the same sum) and
// the activation after it in one pass.
template <int K>
struct AddActOp {
  const float* a;
  const float* b;
  float* z;
  float* y;
  __device__ void one(size_t i) const {
    const float v = a[i] + b[i];
    z[i] = v;
    y[i] = act_f<K>(v);
  }
  __device__ void vec(size_t i) const {
    const f32x4 v = ld4(a, i) + ld4(b, i);
    st4(z, i, v);
    f32x4 w;
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = act_f<K>(v[j]);
    st4(y, i, w);
  }
};

// dz (+)= act'(z) * da (the activation's backward into the Add before it),
// then ga (+)= dz and gb (+)= dz (the Add's backward), in one pass: the steps
// of ActBwdOp then Accum2Op, so the same bits.
template <int K>
struct ActBwdAddOp {
  const float* z;
  const float* da;
  float* dz;
  float* ga;
  float* gb;
  bool acc_z, acc_a, acc_b;
  __device__ void one(size_t i) const {
#pragma clang fp contract(off)
    const float v = act_df<K>(z[i]) * da[i];
    const float d = acc_z ? dz[i] + v : v;
    dz[i] = d;
    ga[i] = acc_a ? ga[i] + d : d;
    gb[i] = acc_b ? gb[i] + d : d;
  }
  __device__ void vec(size_t i) const {
#pragma clang fp contract(off)
    // every load before the first store (a load after a store waits for it)
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    const f32x4 x = ld4(z, i), g = ld4(da, i);
    const f32x4 oz = acc_z ? ld4(dz, i) : z4, oa = acc_a ? ld4(ga, i) : z4, ob = acc_b ? ld4(gb, i) : z4;
    f32x4 d;
#pragma unroll
    for (int j = 0; j < 4; ++j) d[j] = act_df<K>(x[j]) * g[j];
    if (acc_z) d = oz + d;
    st4(dz, i, d);
    st4(ga, i, acc_a ? oa + d : d);
    st4(gb, i, acc_b ? ob + d : d);
  }
};

struct AccumOp {  // y = (float)((double)y + scale*(double)x)
  const float* x;
  float* y;
  double s;
  __device__ void one(size_t i) const { y[i] = (float)((double)y[i] + s * (double)x[i]); }
  __device__ void vec(size_t i) const {
    f32x4 a = ld4(x, i), b = ld4(y, i);
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = (float)((double)b[j] + s * (double)a[j]);
    st4(y, i, b);
  }
};

struct ScaleWriteOp {
  const float* x;
  float* y;
  float s;
  __device__ void one(size_t i) const { y[i] = s * x[i]; }
  __device__ void vec(size_t i) const { st4(y, i, s * ld4(x, i)); }
};

struct ScaleInplaceOp {
  float* x;
  float f;
  int div;
  __device__ void one(size_t i) const { x[i] = div ? x[i] / f : x[i] * f; }
  __device__ void vec(size_t i) const {
    f32x4 a = ld4(x, i);
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = div ? a[j] / f : a[j] * f;
    st4(x, i, a);
  }
};

struct ScaleDevOp {
  float* x;
  const double* s;
  int div;
  __device__ void one(size_t i) const {
    const float f = (float)s[0];
    x[i] = div ? x[i] / f : x[i] * f;
  }
  __device__ void vec(size_t i) const {
    const float f = (float)s[0];
    f32x4 a = ld4(x, i);
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = div ? a[j] / f : a[j] * f;
    st4(x, i, a);
  }
};

struct BiasRowsOp {  // y[r, c] += b[c]
  float* y;
  const float* b;
  int cols;
  __device__ void one(size_t i) const { y[i] += b[i % cols]; }
  __device__ void vec(size_t i) const { st4(y, i, ld4(y, i) + ld4(b, i % cols)); }
};

struct ChanAddOp {  // y = x + b[(i / hw) % C]
  const float* x;
  const float* b;
  float* y;
  size_t hw;
  int C;
  __device__ void one(size_t i) const { y[i] = x[i] + b[(i / hw) % C]; }
  __device__ void vec(size_t i) const { st4(y, i, ld4(x, i) + b[(i / hw) % C]); }
};

template <int K>
struct ActFwdOp {
  const float* x;
  float* y;
  __device__ void one(size_t i) const { y[i] = act_f<K>(x[i]); }
  __device__ void vec(size_t i) const {
    f32x4 a = ld4(x, i);
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = act_f<K>(a[j]);
    st4(y, i, a);
  }
};

template <int K>
struct ActBwdOp {  // dx (+)= dy * f'(x); acc = false assigns (dx is not read)
  const float* x;
  const float* dy;
  float* dx;
  bool acc;
  // The product is rounded before the add (never contracted into an fma), so
  // the normalisation kernels that form this gradient in their own pass
  // (mle_norm_bwd_act) give the same bits.
  __device__ void one(size_t i) const {
#pragma clang fp contract(off)
    const float v = act_df<K>(x[i]) * dy[i];
    dx[i] = acc ? dx[i] + v : v;
  }
  __device__ void vec(size_t i) const {
#pragma clang fp contract(off)
    f32x4 a = ld4(x, i), g = ld4(dy, i), d;
#pragma unroll
    for (int j = 0; j < 4; ++j) d[j] = act_df<K>(a[j]) * g[j];
    st4(dx, i, acc ? ld4(dx, i) + d : d);
  }
};

// ---- layout / encodings -----------------------------------------------------
__global__ __launch_bounds__(256) void headify_kernel(const float* __restrict__ in, float* __restrict__ out, int B,
                                                      int H, int S, int D, int flag) {
  const size_t total = (size_t)B * H * S * D;
  const size_t stride = (size_t)gridDim.x * 256;
  const size_t E = (size_t)H * D;
  for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += stride) {
    const size_t d = idx % D;
    const size_t s = (idx / D) % S;
    const size_t h = (idx / ((size_t)D * S)) % H;
    const size_t b = idx / ((size_t)D * S * H);
    const size_t flat = b * (S * E) + s * E + h * D + d;  // idx is the headified index
    if (flag == 0) out[idx] = in[flat];
    else if (flag == 1) out[flat] += in[idx];
    else if (flag == 2) out[flat] = in[idx];
    else out[idx] += in[flat];
  }
}

// Same mapping moving 4 consecutive head_dim elements per thread (head_dim % 4 == 0).
__global__ __launch_bounds__(256) void headify4_kernel(const float* __restrict__ in, float* __restrict__ out, int B,
                                                       int H, int S, int D, int flag) {
  const int D4 = D / 4;
  const size_t total4 = (size_t)B * H * S * D4;
  const size_t stride = (size_t)gridDim.x * 256;
  const size_t E = (size_t)H * D;
  for (size_t i4 = (size_t)blockIdx.x * 256 + threadIdx.x; i4 < total4; i4 += stride) {
    const size_t d = (i4 % D4) * 4;
    const size_t s = (i4 / D4) % S;
    const size_t h = (i4 / ((size_t)D4 * S)) % H;
    const size_t b = i4 / ((size_t)D4 * S * H);
    const size_t idx = i4 * 4;
    const size_t flat = b * (S * E) + s * E + h * D + d;
    if (flag == 0) *reinterpret_cast<f32x4*>(out + idx) = ld4(in, flat);
    else if (flag == 1) st4(out, flat, ld4(out, flat) + ld4(in, idx));
    else if (flag == 2) st4(out, flat, ld4(in, idx));
    else st4(out, idx, ld4(out, idx) + ld4(in, flat));
  }
}

// Each thread evaluates the encoding of one (position, dim) once -- in double,
// as MatPEncoding does -- and applies it to every batch item.
__global__ __launch_bounds__(256) void matpe_kernel(const float* __restrict__ x, float* __restrict__ y, int batch,
                                                    int rows, int cols, int start) {
  const size_t plane = (size_t)rows * cols;
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t g = (size_t)blockIdx.x * 256 + threadIdx.x; g < plane; g += stride) {
    const int pos = (int)(g / cols) + start;
    const int dim = (int)(g % cols);
    const int i = dim / 2;
    const double expo = (2.0 * i) / cols;
    const double freq = 1.0 / pow(10000.0, expo);
    const double ang = (double)pos * freq;
    const float pe = (dim % 2 == 0) ? (float)sin(ang) : (float)cos(ang);
    for (int b = 0; b < batch; ++b) y[b * plane + g] = x[b * plane + g] + pe;
  }
}

// The encoding MatPEncoding adds, one value per (position, dim), by the same
// double-precision formula as matpe_kernel: computed once, then added by
// add_bcast_kernel for every batch item and every step.
__global__ __launch_bounds__(256) void pe_table_kernel(float* __restrict__ pe, int rows, int cols, int start) {
  const size_t plane = (size_t)rows * cols;
  const size_t g = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= plane) return;
  const int pos = (int)(g / cols) + start;
  const int dim = (int)(g % cols);
  const int i = dim / 2;
  const double expo = (2.0 * i) / cols;
  const double freq = 1.0 / pow(10000.0, expo);
  const double ang = (double)pos * freq;
  pe[g] = (dim % 2 == 0) ? (float)sin(ang) : (float)cos(ang);
}

// y[b, i] = x[b, i] + t[i] over batch items of n floats: blockIdx.y is the item.
template <bool VEC>
__global__ __launch_bounds__(256) void add_bcast_kernel(const float* __restrict__ x, const float* __restrict__ t,
                                                        float* __restrict__ y, size_t n) {
  const size_t off = (size_t)blockIdx.y * n;
  const size_t stride = (size_t)gridDim.x * 256;
  if (VEC) {
    for (size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4; i < n; i += stride * 4)
      st4(y + off, i, ld4(x + off, i) + ld4(t, i));
  } else {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) y[off + i] = x[off + i] + t[i];
  }
}

__global__ void tpe_kernel(float* __restrict__ y, int t, int dim) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= dim) return;
  const int half = dim / 2;
  const int fi = (g < half) ? g : g - half;
  const double expo = -(double)fi * log(10000.0) / (half - 1);
  const double ang = (double)t * exp(expo);
  y[g] = (g < half) ? (float)cos(ang) : (float)sin(ang);
}

template <int K>
int act_fwd_t(hipStream_t s, const float* x, float* y, size_t n) {
  return run_map(s, n, aligned16(x) && aligned16(y), ActFwdOp<K>{x, y}, "mle_act_fwd");
}
template <int K>
int act_bwd_t(hipStream_t s, const float* x, const float* dy, float* dx, size_t n, bool acc) {
  return run_map(s, n, aligned16(x) && aligned16(dy) && aligned16(dx), ActBwdOp<K>{x, dy, dx, acc}, "mle_act_bwd");
}

}  // namespace

extern "C" {

int mle_fill(mle_stream stream, float* x, float value, size_t n) {
  if (n == 0) return MLE_OK;
  MLE_CHECK_ARG(x, "mle_fill: null pointer");
  return run_map(as_stream(stream), n, aligned16(x), FillOp{x, value}, "mle_fill");
}

int mle_scale_add(mle_stream stream, const float* x, const float* y, float* z, float scale, size_t n) {
  if (n == 0) return MLE_OK;
  MLE_CHECK_ARG(x && y && z, "mle_scale_add: null pointer");
  return run_map(as_stream(stream), n, aligned16(x) && aligned16(y) && aligned16(z), ScaleAddOp{x, y, z, scale},
                 "mle_scale_add");
}

int mle_accumulate(mle_stream stream, const float* x, float* y, double scale, size_t n) {
  if (n == 0) return MLE_OK;
  MLE_CHECK_ARG(x && y, "mle_accumulate: null pointer");
  const bool v = aligned16(x) && aligned16(y);
  // With scale == 1 the double sum of two floats rounds to the float sum.
  if (scale == 1.0) return run_map(as_stream(stream), n, v, AccumOneOp{x, y}, "mle_accumulate");
  return run_map(as_stream(stream), n, v, AccumOp{x, y, scale}, "mle_accumulate");
}

int mle_accumulate2(mle_stream stream, const float* x, float* ya, int acc_a, float* yb, int acc_b, size_t n) {
  if (n == 0) return MLE_OK;
  MLE_CHECK_ARG(x && ya && yb, "mle_accumulate2: null pointer");
  MLE_CHECK_ARG(ya != yb, "mle_accumulate2: the two destinations must differ");
  const hipStream_t s = as_stream(stream);
  const bool v = aligned16(x) && aligned16(ya) && aligned16(yb);
  if (acc_a && acc_b) return run_map(s, n, v, Accum2Op<true, true>{x, ya, yb}, "mle_accumulate2");
  if (acc_a) return run_map(s, n, v, Accum2Op<true, false>{x, ya, yb}, "mle_accumulate2");
  if (acc_b) return run_map(s, n, v, Accum2Op<false, true>{x, ya, yb}, "mle_accumulate2");
  return run_map(s, n, v, Accum2Op<false, false>{x, ya, yb}, "mle_accumulate2");
}

int mle_add_act_fwd(mle_stream stream, const float* a, const float* b, float* z, float* y, int kind, size_t n) {
  if (n == 0) return MLE_OK;
  MLE_CHECK_ARG(a && b && z && y, "mle_add_act_fwd: null pointer");
  const hipStream_t s = as_stream(stream);
  const bool v = aligned16(a) && aligned16(b) && aligned16(z) && aligned16(y);
  switch (kind) {
    case MLE_RELU: return run_map(s, n, v, AddActOp<MLE_RELU>{a, b, z, y}, "mle_add_act_fwd");
    case MLE_GELU: return run_map(s, n, v, AddActOp<MLE_GELU>{a, b, z, y}, "mle_add_act_fwd");
    case MLE_SILU: return run_map(s, n, v, AddActOp<MLE_SILU>{a, b, z, y}, "mle_add_act_fwd");
    case MLE_TANH: return run_map(s, n, v, AddActOp<MLE_TANH>{a, b, z, y}, "mle_add_act_fwd");
    case MLE_SIGMOID: return run_map(s, n, v, AddActOp<MLE_SIGMOID>{a, b, z, y}, "mle_add_act_fwd");
    case MLE_LEAKY_RELU: return run_map(s, n, v, AddActOp<MLE_LEAKY_RELU>{a, b, z, y}, "mle_add_act_fwd");
    default: return set_error(MLE_ERR_INVALID, "mle_add_act_fwd: unknown activation %d", kind);
  }
}

int mle_act_bwd_add(mle_stream stream, const float* z, const float* da, int kind, float* dz, int accumulate_dz,
                    float* ga, int acc_a, float* gb, int acc_b, size_t n) {
  if (n == 0) return MLE_OK;
  MLE_CHECK_ARG(z && da && dz && ga && gb, "mle_act_bwd_add: null pointer");
  MLE_CHECK_ARG(ga != gb && ga != dz && gb != dz, "mle_act_bwd_add: the three gradients must differ");
  const hipStream_t s = as_stream(stream);
  const bool v = aligned16(z) && aligned16(da) && aligned16(dz) && aligned16(ga) && aligned16(gb);
  const bool az = accumulate_dz != 0, aa = acc_a != 0, ab = acc_b != 0;
  switch (kind) {
    case MLE_RELU: return run_map(s, n, v, ActBwdAddOp<MLE_RELU>{z, da, dz, ga, gb, az, aa, ab}, "mle_act_bwd_add");
    case MLE_GELU: return run_map(s, n, v, ActBwdAddOp<MLE_GELU>{z, da, dz, ga, gb, az, aa, ab}, "mle_act_bwd_add");
    case MLE_SILU: return run_map(s, n, v, ActBwdAddOp<MLE_SILU>{z, da, dz, ga, gb, az, aa, ab}, "mle_act_bwd_add");
    case MLE_TANH: return run_map(s, n, v, ActBwdAddOp<MLE_TANH>{z, da, dz, ga, gb, az, aa, ab}, "mle_act_bwd_add");
    case MLE_SIGMOID:
      return run_map(s, n, v, ActBwdAddOp<MLE_SIGMOID>{z, da, dz, ga, gb, az, aa, ab}, "mle_act_bwd_add");
    case MLE_LEAKY_RELU:
      return run_map(s, n, v, ActBwdAddOp<MLE_LEAKY_RELU>{z, da, dz, ga, gb, az, aa, ab}, "mle_act_bwd_add");
    default: return set_error(MLE_ERR_INVALID, "mle_act_bwd_add: unknown activation %d", kind);
  }
}

int mle_scale_assign(mle_stream stream, const float* x, float* y, double scale, size_t n) {
  if (n == 0) return MLE_OK;
  MLE_CHECK_ARG(x && y, "mle_scale_assign: null pointer");
  return run_map(as_stream(stream), n, aligned16(x) && aligned16(y), ScaleAssignOp{x, y, scale}, "mle_scale_assign");
}

int mle_scale_write(mle_stream stream, const float* x, float* y, float scale, size_t n) {
  if (n == 0) return MLE_OK;
  MLE_CHECK_ARG(x && y, "mle_scale_write: null pointer");
  return run_map(as_stream(stream), n, aligned16(x) && aligned16(y), ScaleWriteOp{x, y, scale}, "mle_scale_write");
}

int mle_scale_inplace(mle_stream stream, float* x, float factor, int divide, size_t n) {
  if (n == 0) return MLE_OK;
  MLE_CHECK_ARG(x, "mle_scale_inplace: null pointer");
  return run_map(as_stream(stream), n, aligned16(x), ScaleInplaceOp{x, factor, divide}, "mle_scale_inplace");
}

int mle_scale_by_device(mle_stream stream, float* x, const double* s, int divide, size_t n) {
  if (n == 0) return MLE_OK;
  MLE_CHECK_ARG(x && s, "mle_scale_by_device: null pointer");
  return run_map(as_stream(stream), n, aligned16(x), ScaleDevOp{x, s, divide}, "mle_scale_by_device");
}

int mle_bias_add_rows(mle_stream stream, float* y, const float* b, size_t rows, int cols) {
  MLE_CHECK_ARG(y && b && cols > 0, "mle_bias_add_rows: bad argument");
  const size_t n = rows * (size_t)cols;
  return run_map(as_stream(stream), n, aligned16(y) && aligned16(b) && (cols % 4 == 0), BiasRowsOp{y, b, cols},
                 "mle_bias_add_rows");
}

int mle_broadcast_channel_add(mle_stream stream, const float* x, const float* b, float* y, int batch, int channels,
                              size_t hw) {
  MLE_CHECK_ARG(x && b && y && channels > 0 && hw > 0, "mle_broadcast_channel_add: bad argument");
  const size_t n = (size_t)batch * channels * hw;
  return run_map(as_stream(stream), n, aligned16(x) && aligned16(y) && (hw % 4 == 0), ChanAddOp{x, b, y, hw, channels},
                 "mle_broadcast_channel_add");
}

int mle_headify(mle_stream stream, const float* in, float* out, int batch, int heads, int seq, int head_dim,
                int flag) {
  MLE_CHECK_ARG(in && out && flag >= 0 && flag <= 3, "mle_headify: bad argument");
  const size_t total = (size_t)batch * heads * seq * head_dim;
  if (total == 0) return MLE_OK;
  if (head_dim % 4 == 0 && aligned16(in) && aligned16(out))
    headify4_kernel<<<stream_grid(total / 4, 256, 8192), 256, 0, as_stream(stream)>>>(in, out, batch, heads, seq,
                                                                                      head_dim, flag);
  else
    headify_kernel<<<stream_grid(total, 256, 8192), 256, 0, as_stream(stream)>>>(in, out, batch, heads, seq, head_dim,
                                                                                 flag);
  return check_launch("mle_headify");
}

int mle_matpe(mle_stream stream, const float* x, float* y, int batch, int rows, int cols, int start_idx) {
  MLE_CHECK_ARG(x && y && rows > 0 && cols > 0, "mle_matpe: bad argument");
  const size_t total = (size_t)batch * rows * cols;
  if (total == 0) return MLE_OK;
  matpe_kernel<<<stream_grid((size_t)rows * cols, 256, 8192), 256, 0, as_stream(stream)>>>(x, y, batch, rows, cols,
                                                                                         start_idx);
  return check_launch("mle_matpe");
}

int mle_matpe_table(mle_stream stream, float* pe, int rows, int cols, int start_idx) {
  MLE_CHECK_ARG(pe && rows > 0 && cols > 0, "mle_matpe_table: bad argument");
  const size_t plane = (size_t)rows * cols;
  pe_table_kernel<<<(unsigned)((plane + 255) / 256), 256, 0, as_stream(stream)>>>(pe, rows, cols, start_idx);
  return check_launch("mle_matpe_table");
}

int mle_add_broadcast(mle_stream stream, const float* x, const float* t, float* y, int batch, size_t n) {
  MLE_CHECK_ARG(x && t && y && batch >= 0 && batch <= 65535, "mle_add_broadcast: bad argument");
  if (n == 0 || batch == 0) return MLE_OK;
  const bool vec = n % 4 == 0 && aligned16(x) && aligned16(t) && aligned16(y);
  const size_t items = vec ? n / 4 : n;
  const unsigned gx = (unsigned)std::min<size_t>((items + 255) / 256, std::max<size_t>(1, 8192 / (size_t)batch));
  const dim3 grid(gx, (unsigned)batch);
  if (vec) add_bcast_kernel<true><<<grid, 256, 0, as_stream(stream)>>>(x, t, y, n);
  else add_bcast_kernel<false><<<grid, 256, 0, as_stream(stream)>>>(x, t, y, n);
  return check_launch("mle_add_broadcast");
}

int mle_timestep_pe(mle_stream stream, float* y, int t, int dim) {
  MLE_CHECK_ARG(y && dim > 2, "mle_timestep_pe: bad argument");
  tpe_kernel<<<(dim + 255) / 256, 256, 0, as_stream(stream)>>>(y, t, dim);
  return check_launch("mle_timestep_pe");
}

int mle_act_fwd(mle_stream stream, int kind, const float* x, float* y, size_t n) {
  if (n == 0) return MLE_OK;
  MLE_CHECK_ARG(x && y, "mle_act_fwd: null pointer");
  hipStream_t s = as_stream(stream);
  switch (kind) {
    case MLE_RELU: return act_fwd_t<MLE_RELU>(s, x, y, n);
    case MLE_GELU: return act_fwd_t<MLE_GELU>(s, x, y, n);
    case MLE_SILU: return act_fwd_t<MLE_SILU>(s, x, y, n);
    case MLE_TANH: return act_fwd_t<MLE_TANH>(s, x, y, n);
    case MLE_SIGMOID: return act_fwd_t<MLE_SIGMOID>(s, x, y, n);
    case MLE_LEAKY_RELU: return act_fwd_t<MLE_LEAKY_RELU>(s, x, y, n);
  }
  return set_error(MLE_ERR_INVALID, "mle_act_fwd: unknown kind %d", kind);
}

int mle_act_bwd(mle_stream stream, int kind, const float* x, const float* dy, float* dx, size_t n, int accumulate) {
  if (n == 0) return MLE_OK;
  MLE_CHECK_ARG(x && dy && dx, "mle_act_bwd: null pointer");
  hipStream_t s = as_stream(stream);
  switch (kind) {
    case MLE_RELU: return act_bwd_t<MLE_RELU>(s, x, dy, dx, n, accumulate != 0);
    case MLE_GELU: return act_bwd_t<MLE_GELU>(s, x, dy, dx, n, accumulate != 0);
    case MLE_SILU: return act_bwd_t<MLE_SILU>(s, x, dy, dx, n, accumulate != 0);
    case MLE_TANH: return act_bwd_t<MLE_TANH>(s, x, dy, dx, n, accumulate != 0);
    case MLE_SIGMOID: return act_bwd_t<MLE_SIGMOID>(s, x, dy, dx, n, accumulate != 0);
    case MLE_LEAKY_RELU: return act_bwd_t<MLE_LEAKY_RELU>(s, x, dy, dx, n, accumulate != 0);
  }
  return set_error(MLE_ERR_INVALID, "mle_act_bwd: unknown kind %d", kind);
}

}  // extern "C"
