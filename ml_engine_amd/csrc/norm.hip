// LayerNorm (whole-sample statistics), GroupNorm / InstanceNorm and BatchNorm
// forward/backward with gamma = 1, beta = 0 (Engine/engine.cu:3080-3347), and
// the reference's RMSNorm (an L2 normalisation along rows or columns,
// Engine/engine.cu:2613-2648).
//
// A group (one batch item for LayerNorm, one (batch, group) for GroupNorm) is
// a contiguous span of N = (C/G)*HW floats in NCHW.  A BatchNorm group is one
// channel across the batch: `batch` segments of HW floats, C*HW apart.  The reference reduces a
// group with a single 512-thread block (LayerMean/LayerStd, GroupMean/GroupStd,
// Engine/kernels.cu:541-763), i.e. 32 blocks for the transformer LayerNorm.
// Here each group is split into chunks of CH floats so every CU gets work:
//   pass 1: per chunk (mean, M2) from registers -> workspace (double)
//   pass 2: each chunk's workgroup combines its group's chunk partials in a
//           fixed order (Chan et al. pairwise update) and normalises.
// The backward uses the same split for sum(dy) and sum(dy*y).
#include "common.hpp"

using namespace mle;

namespace {

constexpr int NT = 256;
constexpr int VPT = 16;          // floats per thread per chunk
constexpr int CH = NT * VPT;     // 4096 floats per chunk

struct NormShape {
  size_t N;        // elements per group
  int nchunk;      // chunks per group
  int groups_tot;  // groups in the launch
  // Segmented groups (SEG kernels): element e of group g sits at
  // g * group_stride + (e / seg) * seg_stride + e % seg.
  uint32_t seg;
  size_t seg_stride, group_stride;
};

// Offset of element e of group g.  Contiguous groups: g * N + e.
template <bool SEG>
__device__ __forceinline__ size_t at(const NormShape& sh, int g, size_t e) {
  if (!SEG) return (size_t)g * sh.N + e;
  const uint32_t e32 = (uint32_t)e;  // N < 2^32 on this path (checked on the host)
  return (size_t)g * sh.group_stride + (size_t)(e32 / sh.seg) * sh.seg_stride + e32 % sh.seg;
}

template <bool SEG>
__device__ __forceinline__ void load_chunk(const float* __restrict__ src, const NormShape& sh, int g, size_t c0,
                                           float (&v)[VPT], int& cnt) {
  cnt = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const size_t e = c0 + threadIdx.x + (size_t)i * NT;
    v[i] = (e < sh.N) ? src[at<SEG>(sh, g, e)] : 0.f;
    cnt += (e < sh.N) ? 1 : 0;
  }
}

template <bool SEG>
__global__ __launch_bounds__(NT) void norm_stats_partial(const float* __restrict__ x, NormShape sh,
                                                         double* __restrict__ part) {
  __shared__ double red[NT / 64];
  const int g = blockIdx.y, ck = blockIdx.x;
  const size_t c0 = (size_t)ck * CH;
  float v[VPT];
  int cnt;
  load_chunk<SEG>(x, sh, g, c0, v, cnt);
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) s += v[i];
  s = block_sum<NT>(s, red);
  const size_t n_c = (sh.N - c0 < (size_t)CH) ? sh.N - c0 : (size_t)CH;
  const double mean = s / (double)n_c;
  double m2 = 0.0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const double d = (double)v[i] - mean;
    if (c0 + threadIdx.x + (size_t)i * NT < sh.N) m2 += d * d;
  }
  m2 = block_sum<NT>(m2, red);
  if (threadIdx.x == 0) {
    double* p = part + ((size_t)g * sh.nchunk + ck) * 2;
    p[0] = mean;
    p[1] = m2;
  }
}

// Fixed-order combination of the chunk partials of group g.
__device__ __forceinline__ void combine_stats(const double* __restrict__ part, const NormShape& sh, int g, double& mean,
                                              double& m2) {
  const double* p = part + (size_t)g * sh.nchunk * 2;
  double n_a = 0, mu = 0, M = 0;
  for (int c = 0; c < sh.nchunk; ++c) {
    const size_t c0 = (size_t)c * CH;
    const double n_b = (double)((sh.N - c0 < (size_t)CH) ? sh.N - c0 : (size_t)CH);
    const double mu_b = p[2 * c], M_b = p[2 * c + 1];
    const double n = n_a + n_b;
    const double d = mu_b - mu;
    mu += d * (n_b / n);
    M += M_b + d * d * (n_a * n_b / n);
    n_a = n;
  }
  mean = mu;
  m2 = M;
}

template <bool SEG>
__global__ __launch_bounds__(NT) void norm_apply(const float* __restrict__ x, float* __restrict__ y,
                                                 float* __restrict__ stats, NormShape sh, const double* __restrict__ part,
                                                 float eps) {
  const int g = blockIdx.y, ck = blockIdx.x;
  double mean_d, m2_d;
  combine_stats(part, sh, g, mean_d, m2_d);
  const float mean = (float)mean_d, ssd = (float)m2_d;
  const float r = rsqrtf((1.0f / (float)sh.N) * ssd + eps);  // LNorm/GNorm (Engine/kernels.cu:794-834)
  if (ck == 0 && threadIdx.x == 0) {
    stats[2 * g] = mean;
    stats[2 * g + 1] = ssd;
  }
  const size_t c0 = (size_t)ck * CH;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const size_t e = c0 + threadIdx.x + (size_t)i * NT;
    if (e < sh.N) {
      const size_t o = at<SEG>(sh, g, e);
      y[o] = (x[o] - mean) * r;
    }
  }
}

template <bool SEG>
__global__ __launch_bounds__(NT) void norm_bwd_partial(const float* __restrict__ y, const float* __restrict__ dy,
                                                       NormShape sh, double* __restrict__ part) {
  __shared__ double red[NT / 64];
  const int g = blockIdx.y, ck = blockIdx.x;
  const size_t c0 = (size_t)ck * CH;
  double sg = 0.0, sgy = 0.0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const size_t e = c0 + threadIdx.x + (size_t)i * NT;
    if (e < sh.N) {
      const size_t o = at<SEG>(sh, g, e);
      const float gv = dy[o];
      sg += gv;
      sgy += (double)(gv * y[o]);
    }
  }
  sg = block_sum<NT>(sg, red);
  sgy = block_sum<NT>(sgy, red);
  if (threadIdx.x == 0) {
    double* p = part + ((size_t)g * sh.nchunk + ck) * 2;
    p[0] = sg;
    p[1] = sgy;
  }
}

// dx (+)= r (dy - sum(dy)/N - y sum(dy*y)/N)  (LayerBackward/GroupBackward,
// Engine/kernels.cu:849-896); acc = 0 assigns.  `quirk_hw` != 0 reproduces
// LayerBackward for channels > 1: only elements e < batch*hw receive a
// gradient, with group e / hw (the others are left alone, or set to 0 when
// assigning, which is what adding nothing to a cleared gradient gives).
template <bool SEG>
__global__ __launch_bounds__(NT) void norm_bwd_apply(const float* __restrict__ y, const float* __restrict__ dy,
                                                     float* __restrict__ dx, const float* __restrict__ stats,
                                                     NormShape sh, const double* __restrict__ part, float eps,
                                                     size_t quirk_hw, int acc) {
  const int g = blockIdx.y, ck = blockIdx.x;
  const size_t c0 = (size_t)ck * CH;
  const float fN = (float)(int)sh.N;
  auto group_terms = [&](int gs, float& sg, float& sgy, float& r) {
    const double* p = part + (size_t)gs * sh.nchunk * 2;
    double sgd = 0.0, sgyd = 0.0;
    for (int c = 0; c < sh.nchunk; ++c) {
      sgd += p[2 * c];
      sgyd += p[2 * c + 1];
    }
    sg = (float)sgd;
    sgy = (float)sgyd;
    r = rsqrtf(stats[2 * gs + 1] / fN + eps);
  };
  float sg, sgy, r;
  group_terms(g, sg, sgy, r);
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const size_t e = c0 + threadIdx.x + (size_t)i * NT;
    if (e >= sh.N) continue;
    const size_t idx = at<SEG>(sh, g, e);
    if (!SEG && quirk_hw) {
      if (idx >= (size_t)sh.groups_tot * quirk_hw) {
        if (!acc) dx[idx] = 0.f;
        continue;
      }
      group_terms((int)(idx / quirk_hw), sg, sgy, r);
    }
    const float v = r * (dy[idx] - (sg / fN) - y[idx] * (sgy / fN));
    dx[idx] = acc ? dx[idx] + v : v;
  }
}

int shape_of(int batch, int channels, size_t hw, int groups, NormShape& sh) {
  if (batch <= 0 || channels <= 0 || hw == 0 || groups <= 0 || channels % groups != 0)
    return set_error(MLE_ERR_INVALID, "norm: bad shape batch %d channels %d hw %zu groups %d", batch, channels, hw,
                     groups);
  sh.N = (size_t)(channels / groups) * hw;
  sh.nchunk = (int)((sh.N + CH - 1) / CH);
  sh.groups_tot = batch * groups;
  sh.seg = 0;
  sh.seg_stride = sh.group_stride = 0;
  if (sh.groups_tot > 65535) return set_error(MLE_ERR_UNSUPPORTED, "norm: %d groups > 65535", sh.groups_tot);
  return MLE_OK;
}

// BatchNorm: one group per channel, `batch` segments of hw floats.
int bn_shape_of(int batch, int channels, size_t hw, NormShape& sh) {
  if (batch <= 0 || channels <= 0 || hw == 0)
    return set_error(MLE_ERR_INVALID, "batchnorm: bad shape batch %d channels %d hw %zu", batch, channels, hw);
  sh.N = (size_t)batch * hw;
  if (sh.N > 0xffffffffull || hw > 0xffffffffull)
    return set_error(MLE_ERR_UNSUPPORTED, "batchnorm: %zu elements per channel >= 2^32", sh.N);
  sh.nchunk = (int)((sh.N + CH - 1) / CH);
  sh.groups_tot = channels;
  sh.seg = (uint32_t)hw;
  sh.seg_stride = (size_t)channels * hw;
  sh.group_stride = hw;
  if (channels > 65535) return set_error(MLE_ERR_UNSUPPORTED, "batchnorm: %d channels > 65535", channels);
  return MLE_OK;
}

// RMSNorm.  A line is a row (type 0: `len` = cols contiguous floats) or a
// column (type 1: `len` = rows floats, cols apart).  norms[line] =
// sqrtf(sum x^2) (SumSquaredSqrtCols / SumSquaredSqrtRows, Engine/kernels.cu:
// 2246-2277), y = x / norm (Scale_arr, Engine/kernels.cu:2058-2071).
// Rows: one workgroup per line, sums in double with a fixed-order block
// reduction.  Columns: one thread per column, walking the rows, so a wave
// reads 64 consecutive floats of each row.
__global__ __launch_bounds__(NT) void rms_row_fwd(const float* __restrict__ x, float* __restrict__ y,
                                                  float* __restrict__ norms, int cols) {
  __shared__ double red[NT / 64];
  const size_t base = (size_t)blockIdx.x * cols;
  double s = 0.0;
  for (int i = threadIdx.x; i < cols; i += NT) {
    const float v = x[base + i];
    s += (double)v * (double)v;
  }
  s = block_sum<NT>(s, red);
  const float n = sqrtf((float)s);
  if (threadIdx.x == 0) norms[blockIdx.x] = n;
  for (int i = threadIdx.x; i < cols; i += NT) y[base + i] = x[base + i] / n;
}

__global__ __launch_bounds__(NT) void rms_col_fwd(const float* __restrict__ x, float* __restrict__ y,
                                                  float* __restrict__ norms, int rows, int cols) {
  const int c = blockIdx.x * NT + threadIdx.x;
  if (c >= cols) return;
  const size_t base = (size_t)blockIdx.y * rows * cols + c;
  double s = 0.0;
  for (int r = 0; r < rows; ++r) {
    const float v = x[base + (size_t)r * cols];
    s += (double)v * (double)v;
  }
  const float n = sqrtf((float)s);
  norms[(size_t)blockIdx.y * cols + c] = n;
  for (int r = 0; r < rows; ++r) y[base + (size_t)r * cols] = x[base + (size_t)r * cols] / n;
}

// dx (+)= (dy - y <dy, y>) / norm along the line (Accumulate_rmsnorm_kernel,
// Engine/kernels.cu:2073-2105); acc = 0 assigns.
__global__ __launch_bounds__(NT) void rms_row_bwd(const float* __restrict__ y, const float* __restrict__ dy,
                                                  const float* __restrict__ norms, float* __restrict__ dx, int cols,
                                                  int acc) {
  __shared__ double red[NT / 64];
  const size_t base = (size_t)blockIdx.x * cols;
  double s = 0.0;
  for (int i = threadIdx.x; i < cols; i += NT) s += (double)dy[base + i] * (double)y[base + i];
  s = block_sum<NT>(s, red);
  const float d = (float)s, inv = 1.0f / norms[blockIdx.x];
  for (int i = threadIdx.x; i < cols; i += NT) {
    const float v = (dy[base + i] - y[base + i] * d) * inv;
    dx[base + i] = acc ? dx[base + i] + v : v;
  }
}

__global__ __launch_bounds__(NT) void rms_col_bwd(const float* __restrict__ y, const float* __restrict__ dy,
                                                  const float* __restrict__ norms, float* __restrict__ dx, int rows,
                                                  int cols, int acc) {
  const int c = blockIdx.x * NT + threadIdx.x;
  if (c >= cols) return;
  const size_t base = (size_t)blockIdx.y * rows * cols + c;
  double s = 0.0;
  for (int r = 0; r < rows; ++r) s += (double)dy[base + (size_t)r * cols] * (double)y[base + (size_t)r * cols];
  const float d = (float)s, inv = 1.0f / norms[(size_t)blockIdx.y * cols + c];
  for (int r = 0; r < rows; ++r) {
    const size_t o = base + (size_t)r * cols;
    const float v = (dy[o] - y[o] * d) * inv;
    dx[o] = acc ? dx[o] + v : v;
  }
}

int rms_check(int bc, int rows, int cols, int type) {
  if (bc <= 0 || rows <= 0 || cols <= 0 || (type != 0 && type != 1))
    return set_error(MLE_ERR_INVALID, "rmsnorm: bad shape bc %d rows %d cols %d type %d", bc, rows, cols, type);
  if (type == 0 && (long long)bc * rows > 0x7fffffffLL)
    return set_error(MLE_ERR_UNSUPPORTED, "rmsnorm: too many rows");
  if (type == 1 && bc > 65535) return set_error(MLE_ERR_UNSUPPORTED, "rmsnorm: bc %d > 65535", bc);
  return MLE_OK;
}

}  // namespace

extern "C" {

size_t mle_norm_ws_bytes(int batch, int channels, size_t hw, int groups) {
  NormShape sh;
  if (shape_of(batch, channels, hw, groups, sh) != MLE_OK) return 0;
  return (size_t)sh.groups_tot * sh.nchunk * 2 * sizeof(double);
}

int mle_norm_fwd(mle_stream stream, const float* x, float* y, float* stats, int batch, int channels, size_t hw,
                 int groups, float eps, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(x && y && stats && ws, "mle_norm_fwd: null pointer");
  NormShape sh;
  int rc = shape_of(batch, channels, hw, groups, sh);
  if (rc) return rc;
  if (ws_bytes < mle_norm_ws_bytes(batch, channels, hw, groups))
    return set_error(MLE_ERR_WORKSPACE, "mle_norm_fwd: workspace too small");
  hipStream_t s = as_stream(stream);
  dim3 grid(sh.nchunk, sh.groups_tot);
  double* part = static_cast<double*>(ws);
  norm_stats_partial<false><<<grid, NT, 0, s>>>(x, sh, part);
  norm_apply<false><<<grid, NT, 0, s>>>(x, y, stats, sh, part, eps);
  return check_launch("mle_norm_fwd");
}

int mle_norm_bwd(mle_stream stream, const float* y, const float* dy, float* dx, const float* stats, int batch,
                 int channels, size_t hw, int groups, float eps, int reference_layout, void* ws, size_t ws_bytes,
                 int accumulate) {
  MLE_CHECK_ARG(y && dy && dx && stats && ws, "mle_norm_bwd: null pointer");
  NormShape sh;
  int rc = shape_of(batch, channels, hw, groups, sh);
  if (rc) return rc;
  if (ws_bytes < mle_norm_ws_bytes(batch, channels, hw, groups))
    return set_error(MLE_ERR_WORKSPACE, "mle_norm_bwd: workspace too small");
  hipStream_t s = as_stream(stream);
  dim3 grid(sh.nchunk, sh.groups_tot);
  double* part = static_cast<double*>(ws);
  const size_t quirk = (reference_layout && groups == 1 && channels > 1) ? hw : 0;
  norm_bwd_partial<false><<<grid, NT, 0, s>>>(y, dy, sh, part);
  norm_bwd_apply<false><<<grid, NT, 0, s>>>(y, dy, dx, stats, sh, part, eps, quirk, accumulate);
  return check_launch("mle_norm_bwd");
}

size_t mle_batchnorm_ws_bytes(int batch, int channels, size_t hw) {
  NormShape sh;
  if (bn_shape_of(batch, channels, hw, sh) != MLE_OK) return 0;
  return (size_t)sh.groups_tot * sh.nchunk * 2 * sizeof(double);
}

int mle_batchnorm_fwd(mle_stream stream, const float* x, float* y, float* stats, int batch, int channels, size_t hw,
                      float eps, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(x && y && stats && ws, "mle_batchnorm_fwd: null pointer");
  NormShape sh;
  int rc = bn_shape_of(batch, channels, hw, sh);
  if (rc) return rc;
  if (ws_bytes < mle_batchnorm_ws_bytes(batch, channels, hw))
    return set_error(MLE_ERR_WORKSPACE, "mle_batchnorm_fwd: workspace too small");
  hipStream_t s = as_stream(stream);
  dim3 grid(sh.nchunk, sh.groups_tot);
  double* part = static_cast<double*>(ws);
  norm_stats_partial<true><<<grid, NT, 0, s>>>(x, sh, part);
  norm_apply<true><<<grid, NT, 0, s>>>(x, y, stats, sh, part, eps);
  return check_launch("mle_batchnorm_fwd");
}

int mle_batchnorm_bwd(mle_stream stream, const float* y, const float* dy, float* dx, const float* stats, int batch,
                      int channels, size_t hw, float eps, void* ws, size_t ws_bytes, int accumulate) {
  MLE_CHECK_ARG(y && dy && dx && stats && ws, "mle_batchnorm_bwd: null pointer");
  NormShape sh;
  int rc = bn_shape_of(batch, channels, hw, sh);
  if (rc) return rc;
  if (ws_bytes < mle_batchnorm_ws_bytes(batch, channels, hw))
    return set_error(MLE_ERR_WORKSPACE, "mle_batchnorm_bwd: workspace too small");
  hipStream_t s = as_stream(stream);
  dim3 grid(sh.nchunk, sh.groups_tot);
  double* part = static_cast<double*>(ws);
  norm_bwd_partial<true><<<grid, NT, 0, s>>>(y, dy, sh, part);
  norm_bwd_apply<true><<<grid, NT, 0, s>>>(y, dy, dx, stats, sh, part, eps, 0, accumulate);
  return check_launch("mle_batchnorm_bwd");
}

int mle_rmsnorm_fwd(mle_stream stream, const float* x, float* y, float* norms, int bc, int rows, int cols, int type) {
  MLE_CHECK_ARG(x && y && norms, "mle_rmsnorm_fwd: null pointer");
  int rc = rms_check(bc, rows, cols, type);
  if (rc) return rc;
  hipStream_t s = as_stream(stream);
  if (type == 0) rms_row_fwd<<<(unsigned)((long long)bc * rows), NT, 0, s>>>(x, y, norms, cols);
  else rms_col_fwd<<<dim3((cols + NT - 1) / NT, bc), NT, 0, s>>>(x, y, norms, rows, cols);
  return check_launch("mle_rmsnorm_fwd");
}

int mle_rmsnorm_bwd(mle_stream stream, const float* y, const float* dy, const float* norms, float* dx, int bc, int rows,
                    int cols, int type, int accumulate) {
  MLE_CHECK_ARG(y && dy && norms && dx, "mle_rmsnorm_bwd: null pointer");
  int rc = rms_check(bc, rows, cols, type);
  if (rc) return rc;
  hipStream_t s = as_stream(stream);
  if (type == 0) rms_row_bwd<<<(unsigned)((long long)bc * rows), NT, 0, s>>>(y, dy, norms, dx, cols, accumulate);
  else rms_col_bwd<<<dim3((cols + NT - 1) / NT, bc), NT, 0, s>>>(y, dy, norms, dx, rows, cols, accumulate);
  return check_launch("mle_rmsnorm_bwd");
}

}  // extern "C"
