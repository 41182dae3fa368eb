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
  int acc;
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
    float* d = dx + ((size_t)bb * g.cin + m) * hw + pix;
    *d = acc ? *d + v : v;
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

// out = sum_s part[s] in split order; float4 per thread when possible, with the
// loads of four splits issued together.
template <bool VEC>
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ part, int splits, size_t mn,
                                                           float* __restrict__ out) {
  constexpr int W = VEC ? 4 : 1;
  const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * W;
  if (i >= mn) return;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  int s = 0;
  for (; s + 4 <= splits; s += 4) {
    f32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (VEC) v[u] = *reinterpret_cast<const f32x4*>(part + (size_t)(s + u) * mn + i);
      else v[u][0] = part[(size_t)(s + u) * mn + i];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc += v[u];
  }
  for (; s < splits; ++s) {
    if (VEC) acc += *reinterpret_cast<const f32x4*>(part + (size_t)s * mn + i);
    else acc[0] += part[(size_t)s * mn + i];
  }
  if (VEC) *reinterpret_cast<f32x4*>(out + i) = acc;
  else out[i] = acc[0];
}

// ---------------------------------------------------------------------------
// Fast path: stride 1, filter KH x KW known at compile time (3x3 and 1x1).
// Same 128 x 128 x 32 MFMA tiles; what changes is the operand gather:
//  * every filter-tap decode (k -> channel, kh, kw) divides by constants;
//  * a thread's output pixel (forward / dgrad) or input pixel (wgrad) is
//    decoded once per tile or once per K stage, not once per element;
//  * reads go through raw buffer resources: a tap that falls in the zero
//    padding, or past the tile, gets an offset beyond the extent and the
//    hardware returns 0, so the K loop has no branches;
//  * the epilogue stages each wave's block in LDS and writes 16-byte rows.
// Requirements (checked on the host, else the generic kernel runs): every
// tensor below 2 GiB, pixel counts and K multiples of 4 (float4 never
// straddles an image), 16-byte aligned outputs.
enum ConvKind { CONV_FWD = 0, CONV_DGRAD = 1, CONV_WGRAD = 2 };
constexpr uint32_t kOOB = 0x80000000u;

struct FastConv {
  const float* src;   // gathered operand: x (fwd, wgrad) or dy (dgrad)
  const float* wa;    // A operand: weights (fwd, dgrad) or dy (wgrad)
  const float* bias;  // fwd only (nullable)
  float* out;         // y (fwd, assign), dx (dgrad, accumulate), partials (wgrad)
  uint32_t src_bytes, wa_bytes;
  int M, N, K, kchunk;
  // gathered tensor: channels, spatial size; output-pixel grid (pixels of C's n)
  int sc, sh, sw, shw;
  int ph, pw, phw;
  int pad;
  int cout, cin;  // for the A / output index maps
  int acc;        // dgrad: 1 accumulates into dx, 0 assigns
};

__device__ __forceinline__ float buf_ld1(__amdgpu_buffer_rsrc_t r, uint32_t off_bytes) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off_bytes, 0, 0));
}
__device__ __forceinline__ f32x4 buf_ld4(__amdgpu_buffer_rsrc_t r, uint32_t off_bytes) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off_bytes, 0, 0));
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const float* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, (int)bytes, 0x00020000);
}

template <int KIND, int KH, int KW>
__global__ __launch_bounds__(NT, 2) void conv_fast_kernel(FastConv c) {
  constexpr int KHW = KH * KW;
  constexpr bool B_KC = KIND == CONV_WGRAD;
  constexpr int ASZ = a_tile_floats<false>();
  constexpr int BSZ = b_tile_floats<B_KC>();
  __shared__ __attribute__((aligned(16))) float smem[2 * (ASZ + BSZ)];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, q = lane >> 4, wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int kbeg = blockIdx.z * c.kchunk;
  const int kend = min(c.K, kbeg + c.kchunk);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(c.src, c.src_bytes);
  const __amdgpu_buffer_rsrc_t ra_rs = make_rsrc(c.wa, c.wa_bytes);

  // Per-thread output pixel of the B gather (fwd / dgrad): fixed for the tile.
  int g_base = 0, g_y0 = 0, g_x0 = 0;
  bool g_nok = false;
  if (KIND != CONV_WGRAD) {
    const int n = n0 + (tid & 127);
    g_nok = n < c.N;
    const int b = n / c.phw, pix = n - b * c.phw, py = pix / c.pw, px = pix - py * c.pw;
    g_base = b * c.sc * c.shw;
    g_y0 = KIND == CONV_FWD ? py - c.pad : py + c.pad;
    g_x0 = KIND == CONV_FWD ? px - c.pad : px + c.pad;
  }

  f32x4 ra4[4];
  float ra1[16], rb[16];
  auto load = [&](int k0) {
    // ---- A ----
    if (KIND == CONV_FWD) {  // W [cout][K], k-contiguous float4
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int f = tid + NT * i, row = m0 + (f >> 3), k = k0 + (f & 7) * 4;
        const bool ok = (row < c.M) & (k < kend);
        ra4[i] = buf_ld4(ra_rs, ok ? (uint32_t)(row * c.K + k) * 4u : kOOB);
      }
    } else if (KIND == CONV_DGRAD) {  // A[ci][(co,r)] = W[co][ci][r]
      const int k = k0 + (tid & 31);
      const int co = k / KHW, r = k - co * KHW;
      const bool kok = k < kend;
      const uint32_t kb = (uint32_t)(co * c.cin * KHW + r);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = m0 + (tid >> 5) + 8 * i;
        const bool ok = kok & (row < c.M);
        ra1[i] = buf_ld1(ra_rs, ok ? (kb + (uint32_t)(row * KHW)) * 4u : kOOB);
      }
    } else {  // WGRAD: A[co][pixel] = dy[b][co][pix], float4 along pixels
      const int b0 = k0 / c.phw, p0 = k0 - b0 * c.phw;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int f = tid + NT * i, row = m0 + (f >> 3), kk = (f & 7) * 4;
        int pix = p0 + kk, b = b0;
        if (pix >= c.phw) {
          pix -= c.phw;
          ++b;
        }
        const bool ok = (row < c.M) & (k0 + kk < kend);
        ra4[i] = buf_ld4(ra_rs, ok ? (uint32_t)((b * c.cout + row) * c.phw + pix) * 4u : kOOB);
      }
    }
    // ---- B ----
    if (KIND != CONV_WGRAD) {  // B[(ch,kh,kw)][pixel], n-contiguous
      const int kq = tid >> 7;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int k = k0 + kq + 2 * i;
        const int ch = k / KHW, r = k - ch * KHW, kh = r / KW, kw = r - kh * KW;
        const int sy = KIND == CONV_FWD ? g_y0 + kh : g_y0 - kh;
        const int sx = KIND == CONV_FWD ? g_x0 + kw : g_x0 - kw;
        const bool ok = g_nok & (k < kend) & ((unsigned)sy < (unsigned)c.sh) & ((unsigned)sx < (unsigned)c.sw);
        rb[i] = buf_ld1(rs, ok ? (uint32_t)(g_base + ch * c.shw + sy * c.sw + sx) * 4u : kOOB);
      }
    } else {  // WGRAD: B[pixel][(ci,kh,kw)] = x[b][ci][py - pad + kh][px - pad + kw], k-contiguous
      const int k = k0 + (tid & 31);
      const int b0 = k0 / c.phw;
      int pix = k0 - b0 * c.phw + (tid & 31), b = b0;
      if (pix >= c.phw) {
        pix -= c.phw;
        ++b;
      }
      const int py = pix / c.pw, px = pix - py * c.pw;
      const bool kok = k < kend;
      const int base = b * c.sc * c.shw;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int n = n0 + (tid >> 5) + 8 * i;
        const int ch = n / KHW, r = n - ch * KHW, kh = r / KW, kw = r - kh * KW;
        const int sy = py - c.pad + kh, sx = px - c.pad + kw;
        const bool ok = kok & (n < c.N) & ((unsigned)sy < (unsigned)c.sh) & ((unsigned)sx < (unsigned)c.sw);
        rb[i] = buf_ld1(rs, ok ? (uint32_t)(base + ch * c.shw + sy * c.sw + sx) * 4u : kOOB);
      }
    }
  };
  auto store = [&](int buf) {
    float* As = smem + buf * ASZ;
    float* Bs = smem + 2 * ASZ + buf * BSZ;
    if (KIND == CONV_DGRAD) {
#pragma unroll
      for (int i = 0; i < 16; ++i) As[((tid >> 5) + 8 * i) * LDK + (tid & 31)] = ra1[i];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int f = tid + NT * i;
        *reinterpret_cast<f32x4*>(As + (f >> 3) * LDK + (f & 7) * 4) = ra4[i];
      }
    }
    if (KIND != CONV_WGRAD) {
#pragma unroll
      for (int i = 0; i < 16; ++i) Bs[((tid >> 7) + 2 * i) * LDMN + (tid & 127)] = rb[i];
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) Bs[((tid >> 5) + 8 * i) * LDK + (tid & 31)] = rb[i];
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
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

  // Epilogue: each wave's 64 x 64 block through LDS, 32 rows at a time; a lane
  // writes 4 consecutive columns (pixels, or weight taps for wgrad).
  constexpr int EPI = 68;
  float* T = smem + wave * (32 * EPI);
#pragma unroll
  for (int half = 0; half < 2; ++half) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int i = half * 2 + ii;
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) T[(ii * 16 + 4 * q + r) * EPI + n * 16 + lr] = acc[i][n][r];
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int rr = it * 4 + (lane >> 4), cc = (lane & 15) * 4;
      const int row = m0 + wm * 64 + half * 32 + rr, col = n0 + wn * 64 + cc;
      if (row < c.M && col < c.N) {
        f32x4 v = *reinterpret_cast<const f32x4*>(T + rr * EPI + cc);
        if (KIND == CONV_WGRAD) {
          *reinterpret_cast<f32x4*>(c.out + (size_t)blockIdx.z * c.M * c.N + (size_t)row * c.N + col) = v;
        } else {
          const int b = col / c.phw, pix = col - b * c.phw;
          const int oc = KIND == CONV_FWD ? c.cout : c.cin;
          f32x4* dst = reinterpret_cast<f32x4*>(c.out + ((size_t)b * oc + row) * c.phw + pix);
          if (KIND == CONV_FWD) {
            if (c.bias) v += c.bias[row];
          } else if (c.acc) {
            v += *dst;
          }
          *dst = v;
        }
      }
    }
    __syncthreads();
  }
}

bool fits_2g(double elems) { return elems * 4.0 < 2147483647.0; }
bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <int KIND>
void launch_fast(hipStream_t s, const FastConv& c, int kh, int splits) {
  dim3 grid((c.N + BN - 1) / BN, (c.M + BM - 1) / BM, splits);
  if (kh == 3) conv_fast_kernel<KIND, 3, 3><<<grid, NT, 0, s>>>(c);
  else conv_fast_kernel<KIND, 1, 1><<<grid, NT, 0, s>>>(c);
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

bool fast_filter(const ConvGeom& g) {
  return g.stride == 1 && ((g.kh == 3 && g.kw == 3) || (g.kh == 1 && g.kw == 1));
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
  hipStream_t s = as_stream(stream);
  ProbeScope probe("conv_fwd", s, 2.0 * op.M * (double)op.N * op.K, 0.0);
  const int ohw = g.oh * g.ow;
  if (fast_filter(g) && ohw % 4 == 0 && op.K % 4 == 0 && a16(y) && fits_2g((double)n * cin * h * w_in) &&
      fits_2g((double)n * cout * ohw) && fits_2g((double)cout * op.K)) {
    FastConv c{x, w, b, y, (uint32_t)((size_t)n * cin * h * w_in * 4), (uint32_t)((size_t)cout * op.K * 4),
               op.M, op.N, op.K, op.K, cin, h, w_in, h * w_in, g.oh, g.ow, ohw, pad, cout, cin, 0};
    launch_fast<CONV_FWD>(s, c, kh, 1);
  } else {
    dim3 grid((op.N + BN - 1) / BN, (op.M + BM - 1) / BM, 1);
    igemm_kernel<FwdOps, false><<<grid, NT, 0, s>>>(op, op.K);
  }
  return check_launch("mle_conv2d_fwd");
}

int mle_conv2d_dgrad(mle_stream stream, const float* dy, const float* w, float* dx, int n, int cin, int h, int w_in,
                     int cout, int kh, int kw, int pad, int stride, int accumulate) {
  MLE_CHECK_ARG(dy && w && dx, "mle_conv2d_dgrad: null pointer");
  ConvGeom g;
  int rc = geom(n, cin, h, w_in, cout, kh, kw, pad, stride, g);
  if (rc) return rc;
  DgradOps op{dy, w, dx, g, cin, n * h * w_in, cout * kh * kw, accumulate != 0};
  hipStream_t s = as_stream(stream);
  ProbeScope probe("conv_dgrad", s, 2.0 * op.M * (double)op.N * op.K, 0.0);
  const int hw = h * w_in;
  if (fast_filter(g) && hw % 4 == 0 && a16(dx) && fits_2g((double)n * cin * hw) &&
      fits_2g((double)n * cout * g.oh * g.ow) && fits_2g((double)cout * cin * kh * kw)) {
    FastConv c{dy, w, nullptr, dx, (uint32_t)((size_t)n * cout * g.oh * g.ow * 4),
               (uint32_t)((size_t)cout * cin * kh * kw * 4), op.M, op.N, op.K, op.K, cout, g.oh, g.ow, g.oh * g.ow,
               h, w_in, hw, pad, cout, cin, accumulate != 0};
    launch_fast<CONV_DGRAD>(s, c, kh, 1);
  } else {
    dim3 grid((op.N + BN - 1) / BN, (op.M + BM - 1) / BM, 1);
    igemm_kernel<DgradOps, false><<<grid, NT, 0, s>>>(op, op.K);
  }
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
  hipStream_t s = as_stream(stream);
  {
    ProbeScope probe("conv_wgrad", s, 2.0 * op.M * (double)op.N * op.K, 0.0);
    const int ohw = g.oh * g.ow;
    if (fast_filter(g) && ohw % 4 == 0 && ohw >= BK && op.N % 4 == 0 && a16(ws) &&
        fits_2g((double)n * cin * h * w_in) && fits_2g((double)n * cout * ohw)) {
      FastConv c{x, dy, nullptr, static_cast<float*>(ws), (uint32_t)((size_t)n * cin * h * w_in * 4),
                 (uint32_t)((size_t)n * cout * ohw * 4), op.M, op.N, op.K, kchunk, cin, h, w_in, h * w_in,
                 g.oh, g.ow, ohw, pad, cout, cin, 0};
      launch_fast<CONV_WGRAD>(s, c, kh, splits);
    } else {
      dim3 grid((op.N + BN - 1) / BN, (op.M + BM - 1) / BM, splits);
      igemm_kernel<WgradOps, true><<<grid, NT, 0, s>>>(op, kchunk);
    }
  }
  const size_t mn = (size_t)op.M * op.N;
  if (mn % 4 == 0 && aligned16(ws) && aligned16(dw))
    split_reduce_kernel<true><<<(unsigned)((mn / 4 + 255) / 256), 256, 0, s>>>(static_cast<float*>(ws), splits, mn, dw);
  else
    split_reduce_kernel<false><<<(unsigned)((mn + 255) / 256), 256, 0, s>>>(static_cast<float*>(ws), splits, mn, dw);
  return check_launch("mle_conv2d_wgrad");
}

}  // extern "C"
