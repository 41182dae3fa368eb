// NCHW / OIHW convolution as implicit GEMM on fp32 MFMA (the tile machinery of
// gemm_core.hpp).  Replaces the scalar direct loops of CV2D, CV2D_GradInput and
// GV2D (Engine/kernels.cu:985-1089), whose weight gradient runs one thread per
// weight over B*OH*OW serial products.
//
//   forward : C[co][(b,oh,ow)]  = W[co][(ci,kh,kw)] * im2col(X)[(ci,kh,kw)][(b,oh,ow)]
//   dgrad   : C[ci][(b,ih,iw)] += W^T[ci][(co,kh,kw)] * col2im-gather(dY)[(co,kh,kw)][(b,ih,iw)]
//   wgrad   : C[co][(ci,kh,kw)] = dY[co][(b,oh,ow)] * im2col(X)^T[(b,oh,ow)][(ci,kh,kw)]
// wgrad splits its long K = B*OH*OW across workgroups; the partial tiles land
// in the workspace and one pass adds them in split order (assign semantics).
#include "gemm_core.hpp"

using namespace mle;
using namespace gemm;

namespace {

struct ConvGeom {
  int n, cin, h, w, cout, kh, kw, pad, stride, oh, ow;
};

// Each operand functor returns the GEMM element or 0 outside the problem.
struct FwdOps {
  const float* x;
  const float* wt;
  const float* bias;
  float* y;
  ConvGeom g;
  int M, N, K;
  __device__ float a(int m, int k) const { return (m < M && k < K) ? wt[(size_t)m * K + k] : 0.f; }
  __device__ float b(int k, int n) const {
    if (k >= K || n >= N) return 0.f;
    const int khw = g.kh * g.kw;
    const int ci = k / khw, r = k - ci * khw, kh = r / g.kw, kw = r - kh * g.kw;
    const int ohw = g.oh * g.ow;
    const int bb = n / ohw, pix = n - bb * ohw, oh = pix / g.ow, ow = pix - oh * g.ow;
    const int ih = oh * g.stride - g.pad + kh, iw = ow * g.stride - g.pad + kw;
    if (ih < 0 || ih >= g.h || iw < 0 || iw >= g.w) return 0.f;
    return x[(((size_t)bb * g.cin + ci) * g.h + ih) * g.w + iw];
  }
  __device__ void store(int m, int n, float v, int) const {
    const int ohw = g.oh * g.ow;
    const int bb = n / ohw, pix = n - bb * ohw;
    y[((size_t)bb * g.cout + m) * ohw + pix] = bias ? v + bias[m] : v;
  }
};

struct DgradOps {
  const float* dy;
  const float* wt;
  float* dx;
  ConvGeom g;
  int M, N, K;
  __device__ float a(int m, int k) const {
    if (m >= M || k >= K) return 0.f;
    const int khw = g.kh * g.kw;
    const int co = k / khw, r = k - co * khw;
    return wt[((size_t)co * g.cin + m) * khw + r];
  }
  __device__ float b(int k, int n) const {
    if (k >= K || n >= N) return 0.f;
    const int khw = g.kh * g.kw;
    const int co = k / khw, r = k - co * khw, kh = r / g.kw, kw = r - kh * g.kw;
    const int hw = g.h * g.w;
    const int bb = n / hw, pix = n - bb * hw, ih = pix / g.w, iw = pix - ih * g.w;
    const int nr = ih + g.pad - kh, nc = iw + g.pad - kw;
    if (nr < 0 || nc < 0 || nr % g.stride != 0 || nc % g.stride != 0) return 0.f;
    const int oy = nr / g.stride, ox = nc / g.stride;
    if (oy >= g.oh || ox >= g.ow) return 0.f;
    return dy[(((size_t)bb * g.cout + co) * g.oh + oy) * g.ow + ox];
  }
  __device__ void store(int m, int n, float v, int) const {
    const int hw = g.h * g.w;
    const int bb = n / hw, pix = n - bb * hw;
    dx[((size_t)bb * g.cin + m) * hw + pix] += v;
  }
};

struct WgradOps {
  const float* x;
  const float* dy;
  float* part;  // [splits][M*N]
  ConvGeom g;
  int M, N, K;
  __device__ float a(int m, int k) const {
    if (m >= M || k >= K) return 0.f;
    const int ohw = g.oh * g.ow;
    const int bb = k / ohw, pix = k - bb * ohw;
    return dy[((size_t)bb * g.cout + m) * ohw + pix];
  }
  __device__ float b(int k, int n) const {
    if (k >= K || n >= N) return 0.f;
    const int khw = g.kh * g.kw;
    const int ci = n / khw, r = n - ci * khw, kh = r / g.kw, kw = r - kh * g.kw;
    const int ohw = g.oh * g.ow;
    const int bb = k / ohw, pix = k - bb * ohw, oh = pix / g.ow, ow = pix - oh * g.ow;
    const int ih = oh * g.stride - g.pad + kh, iw = ow * g.stride - g.pad + kw;
    if (ih < 0 || ih >= g.h || iw < 0 || iw >= g.w) return 0.f;
    return x[(((size_t)bb * g.cin + ci) * g.h + ih) * g.w + iw];
  }
  __device__ void store(int m, int n, float v, int split) const { part[(size_t)split * M * N + (size_t)m * N + n] = v; }
};

// B_KC selects the B tile layout: false = [BK][BN] (threads walk n), true =
// [BN][BK] (threads walk k); chosen per operand so consecutive lanes read
// consecutive addresses.  blockIdx.z is the K split.
template <class Ops, bool B_KC>
__global__ __launch_bounds__(NT, 2) void igemm_kernel(Ops op, int kchunk) {
  constexpr int ASZ = a_tile_floats<false>();
  constexpr int BSZ = b_tile_floats<B_KC>();
  __shared__ __attribute__((aligned(16))) float smem[2 * (ASZ + BSZ)];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, q = lane >> 4, wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int kbeg = blockIdx.z * kchunk;
  const int kend = min(op.K, kbeg + kchunk);

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};

  float ra[16], rb[16];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int f = tid + NT * i;
      const int am = f / BK, ak = f % BK;  // A tile [BM][BK]
      ra[i] = (k0 + ak < kend) ? op.a(m0 + am, k0 + ak) : 0.f;
      if (B_KC) {
        const int bn = f / BK, bk = f % BK;
        rb[i] = (k0 + bk < kend) ? op.b(k0 + bk, n0 + bn) : 0.f;
      } else {
        const int bk = f / BN, bn = f % BN;
        rb[i] = (k0 + bk < kend) ? op.b(k0 + bk, n0 + bn) : 0.f;
      }
    }
  };
  auto store = [&](int buf) {
    float* As = smem + buf * ASZ;
    float* Bs = smem + 2 * ASZ + buf * BSZ;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int f = tid + NT * i;
      As[(f / BK) * LDK + (f % BK)] = ra[i];
      if (B_KC) Bs[(f / BK) * LDK + (f % BK)] = rb[i];
      else Bs[(f / BN) * LDMN + (f % BN)] = rb[i];
    }
  };

  const int nk = (kend > kbeg) ? (kend - kbeg + BK - 1) / BK : 0;
  if (nk > 0) {
    load(kbeg);
    store(0);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) load(kbeg + (kt + 1) * BK);
    mma_stage<false, B_KC>(smem + cur * ASZ, smem + 2 * ASZ + cur * BSZ, acc, wm, wn, lr, q);
    if (more) store(cur ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int col = n0 + acc_col(wn, n, lr);
      if (col >= op.N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + acc_row(wm, i, q, r);
        if (row < op.M) op.store(row, col, acc[i][n][r], blockIdx.z);
      }
    }
}

__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ part, int splits, size_t mn,
                                                           float* __restrict__ out) {
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < mn; i += stride) {
    float acc = 0.f;
    for (int s = 0; s < splits; ++s) acc += part[(size_t)s * mn + i];
    out[i] = acc;
  }
}

int geom(int n, int cin, int h, int w, int cout, int kh, int kw, int pad, int stride, ConvGeom& g) {
  if (n <= 0 || cin <= 0 || h <= 0 || w <= 0 || cout <= 0 || kh <= 0 || kw <= 0 || pad < 0 || stride <= 0)
    return set_error(MLE_ERR_INVALID, "conv2d: bad geometry");
  g = ConvGeom{n, cin, h, w, cout, kh, kw, pad, stride, (2 * pad + h - kh) / stride + 1, (2 * pad + w - kw) / stride + 1};
  if (g.oh <= 0 || g.ow <= 0) return set_error(MLE_ERR_INVALID, "conv2d: empty output");
  const double big = (double)n * (cin > cout ? cin : cout) * (double)h * w;
  const double bigo = (double)n * cout * (double)g.oh * g.ow;
  if (big >= 2147483647.0 || bigo >= 2147483647.0)
    return set_error(MLE_ERR_UNSUPPORTED, "conv2d: tensor exceeds 2^31 elements");
  return MLE_OK;
}

// K split for wgrad: aim for >= ~512 workgroups, chunks of whole BK slices.
int wgrad_splits(const ConvGeom& g, int& kchunk) {
  const int M = g.cout, N = g.cin * g.kh * g.kw, K = g.n * g.oh * g.ow;
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  int splits = (512 + tiles - 1) / tiles;
  const int max_splits = (K + 511) / 512;  // keep at least 512 of K per split
  if (splits > max_splits) splits = max_splits;
  if (splits < 1) splits = 1;
  if (splits > 65535) splits = 65535;
  kchunk = (K + splits - 1) / splits;
  kchunk = ((kchunk + BK - 1) / BK) * BK;
  splits = (K + kchunk - 1) / kchunk;
  return splits;
}

}  // namespace

extern "C" {

int mle_conv2d_fwd(mle_stream stream, const float* x, const float* w, const float* b, float* y, int n, int cin, int h,
                   int w_in, int cout, int kh, int kw, int pad, int stride) {
  MLE_CHECK_ARG(x && w && y, "mle_conv2d_fwd: null pointer");
  ConvGeom g;
  int rc = geom(n, cin, h, w_in, cout, kh, kw, pad, stride, g);
  if (rc) return rc;
  FwdOps op{x, w, b, y, g, cout, n * g.oh * g.ow, cin * kh * kw};
  dim3 grid((op.N + BN - 1) / BN, (op.M + BM - 1) / BM, 1);
  hipStream_t s = as_stream(stream);
  ProbeScope probe("conv_fwd", s, 2.0 * op.M * (double)op.N * op.K, 0.0);
  igemm_kernel<FwdOps, false><<<grid, NT, 0, s>>>(op, op.K);
  return check_launch("mle_conv2d_fwd");
}

int mle_conv2d_dgrad(mle_stream stream, const float* dy, const float* w, float* dx, int n, int cin, int h, int w_in,
                     int cout, int kh, int kw, int pad, int stride) {
  MLE_CHECK_ARG(dy && w && dx, "mle_conv2d_dgrad: null pointer");
  ConvGeom g;
  int rc = geom(n, cin, h, w_in, cout, kh, kw, pad, stride, g);
  if (rc) return rc;
  DgradOps op{dy, w, dx, g, cin, n * h * w_in, cout * kh * kw};
  dim3 grid((op.N + BN - 1) / BN, (op.M + BM - 1) / BM, 1);
  hipStream_t s = as_stream(stream);
  ProbeScope probe("conv_dgrad", s, 2.0 * op.M * (double)op.N * op.K, 0.0);
  igemm_kernel<DgradOps, false><<<grid, NT, 0, s>>>(op, op.K);
  return check_launch("mle_conv2d_dgrad");
}

size_t mle_conv2d_wgrad_ws_bytes(int n, int cin, int h, int w_in, int cout, int kh, int kw, int pad, int stride) {
  ConvGeom g;
  if (geom(n, cin, h, w_in, cout, kh, kw, pad, stride, g) != MLE_OK) return 0;
  int kchunk;
  const int splits = wgrad_splits(g, kchunk);
  return (size_t)splits * cout * cin * kh * kw * sizeof(float);
}

int mle_conv2d_wgrad(mle_stream stream, const float* x, const float* dy, float* dw, int n, int cin, int h, int w_in,
                     int cout, int kh, int kw, int pad, int stride, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(x && dy && dw && ws, "mle_conv2d_wgrad: null pointer");
  ConvGeom g;
  int rc = geom(n, cin, h, w_in, cout, kh, kw, pad, stride, g);
  if (rc) return rc;
  int kchunk;
  const int splits = wgrad_splits(g, kchunk);
  if (ws_bytes < mle_conv2d_wgrad_ws_bytes(n, cin, h, w_in, cout, kh, kw, pad, stride))
    return set_error(MLE_ERR_WORKSPACE, "mle_conv2d_wgrad: workspace too small");
  WgradOps op{x, dy, static_cast<float*>(ws), g, cout, cin * kh * kw, n * g.oh * g.ow};
  dim3 grid((op.N + BN - 1) / BN, (op.M + BM - 1) / BM, splits);
  hipStream_t s = as_stream(stream);
  {
    ProbeScope probe("conv_wgrad", s, 2.0 * op.M * (double)op.N * op.K, 0.0);
    igemm_kernel<WgradOps, true><<<grid, NT, 0, s>>>(op, kchunk);
  }
  const size_t mn = (size_t)op.M * op.N;
  split_reduce_kernel<<<stream_grid(mn, 256, 4096), 256, 0, s>>>(static_cast<float*>(ws), splits, mn, dw);
  return check_launch("mle_conv2d_wgrad");
}

}  // extern "C"
