// LayerNorm (whole-sample statistics) and GroupNorm forward/backward with
// gamma = 1, beta = 0 (Engine/engine.cu:3080-3146, 3212-3282).
//
// A group (one batch item for LayerNorm, one (batch, group) for GroupNorm) is
// a contiguous span of N = (C/G)*HW floats in NCHW.  The reference reduces a
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
  int groups_tot;  // batch * groups
};

__device__ __forceinline__ void load_chunk(const float* __restrict__ src, size_t N, size_t c0, float (&v)[VPT],
                                           int& cnt) {
  cnt = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const size_t e = c0 + threadIdx.x + (size_t)i * NT;
    v[i] = (e < N) ? src[e] : 0.f;
    cnt += (e < N) ? 1 : 0;
  }
}

__global__ __launch_bounds__(NT) void norm_stats_partial(const float* __restrict__ x, NormShape sh,
                                                         double* __restrict__ part) {
  __shared__ double red[NT / 64];
  const int g = blockIdx.y, ck = blockIdx.x;
  const float* xg = x + (size_t)g * sh.N;
  const size_t c0 = (size_t)ck * CH;
  float v[VPT];
  int cnt;
  load_chunk(xg, sh.N, c0, v, cnt);
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
  const size_t off = (size_t)g * sh.N, c0 = (size_t)ck * CH;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const size_t e = c0 + threadIdx.x + (size_t)i * NT;
    if (e < sh.N) y[off + e] = (x[off + e] - mean) * r;
  }
}

__global__ __launch_bounds__(NT) void norm_bwd_partial(const float* __restrict__ y, const float* __restrict__ dy,
                                                       NormShape sh, double* __restrict__ part) {
  __shared__ double red[NT / 64];
  const int g = blockIdx.y, ck = blockIdx.x;
  const size_t off = (size_t)g * sh.N, c0 = (size_t)ck * CH;
  double sg = 0.0, sgy = 0.0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const size_t e = c0 + threadIdx.x + (size_t)i * NT;
    if (e < sh.N) {
      const float gv = dy[off + e];
      sg += gv;
      sgy += (double)(gv * y[off + e]);
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
__global__ __launch_bounds__(NT) void norm_bwd_apply(const float* __restrict__ y, const float* __restrict__ dy,
                                                     float* __restrict__ dx, const float* __restrict__ stats,
                                                     NormShape sh, const double* __restrict__ part, float eps,
                                                     size_t quirk_hw, int acc) {
  const int g = blockIdx.y, ck = blockIdx.x;
  const size_t off = (size_t)g * sh.N, c0 = (size_t)ck * CH;
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
    const size_t idx = off + e;
    if (quirk_hw) {
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
  if (sh.groups_tot > 65535) return set_error(MLE_ERR_UNSUPPORTED, "norm: %d groups > 65535", sh.groups_tot);
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
  norm_stats_partial<<<grid, NT, 0, s>>>(x, sh, part);
  norm_apply<<<grid, NT, 0, s>>>(x, y, stats, sh, part, eps);
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
  norm_bwd_partial<<<grid, NT, 0, s>>>(y, dy, sh, part);
  norm_bwd_apply<<<grid, NT, 0, s>>>(y, dy, dx, stats, sh, part, eps, quirk, accumulate);
  return check_launch("mle_norm_bwd");
}

}  // extern "C"
