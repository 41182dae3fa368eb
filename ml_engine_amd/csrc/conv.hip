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

#include <algorithm>

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

// out = sum over s of part[s].  A workgroup covers 64 columns (float4 each
// when possible) with four split groups: thread (column, g) adds splits
// g, g + 4, g + 8, ... in order, and the four group sums are added in group
// order through LDS, so the result does not depend on timing.  Four waves
// per 64 columns keep enough loads in flight for the few-hundred-KB outputs
// of a weight gradient.
// Workgroups from `nmain` on reduce a second, small array the same way (the
// bias partials of a weight gradient) and add the sums into out2 (acc2 = 1)
// or assign them (0).
template <bool VEC>
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ part, int splits, size_t mn,
                                                           float* __restrict__ out, unsigned nmain,
                                                           const float* __restrict__ part2, int n2,
                                                           float* __restrict__ out2, int acc2) {
  constexpr int W = VEC ? 4 : 1;
  __shared__ f32x4 grp[4][64];
  const bool second = blockIdx.x >= nmain;
  const float* P = second ? part2 : part;
  const size_t n = second ? (size_t)n2 : mn;
  const size_t blk = second ? blockIdx.x - nmain : blockIdx.x;
  const int col = threadIdx.x & 63, sg = threadIdx.x >> 6;
  const size_t i = (blk * 64 + col) * W;
  const bool live = i < n;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (live) {
    int s = sg;
    for (; s + 12 < splits; s += 16) {
      f32x4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (VEC) v[u] = *reinterpret_cast<const f32x4*>(P + (size_t)(s + 4 * u) * n + i);
        else v[u] = f32x4{P[(size_t)(s + 4 * u) * n + i], 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) acc += v[u];
    }
    for (; s < splits; s += 4) {
      if (VEC) acc += *reinterpret_cast<const f32x4*>(P + (size_t)s * n + i);
      else acc[0] += P[(size_t)s * n + i];
    }
  }
  grp[sg][col] = acc;
  __syncthreads();
  if (sg != 0 || !live) return;
  const f32x4 r = ((grp[0][col] + grp[1][col]) + grp[2][col]) + grp[3][col];
  if (second) {
    if (VEC) *reinterpret_cast<f32x4*>(out2 + i) = acc2 ? *reinterpret_cast<const f32x4*>(out2 + i) + r : r;
    else out2[i] = acc2 ? out2[i] + r[0] : r[0];
  } else {
    if (VEC) *reinterpret_cast<f32x4*>(out + i) = r;
    else out[i] = r[0];
  }
}

// out = sum of the splits of part; with n2 > 0 also out2 (+)= sum of the
// splits of part2 (acc2: 1 adds, 0 assigns; the same launch).
void launch_split_reduce(hipStream_t s, const float* part, int splits, size_t mn, float* out,
                         const float* part2 = nullptr, int n2 = 0, float* out2 = nullptr, int acc2 = 1) {
  const bool vec = mn % 4 == 0 && aligned16(part) && aligned16(out) &&
                   (n2 == 0 || (n2 % 4 == 0 && aligned16(part2) && aligned16(out2)));
  const size_t w = vec ? 4 : 1;
  const unsigned nmain = (unsigned)((mn / w + 63) / 64);
  const unsigned nb2 = n2 > 0 ? (unsigned)(((size_t)n2 / w + 63) / 64) : 0u;
  if (vec)
    mle::launch(split_reduce_kernel<true>, nmain + nb2, 256, 0, s, part, splits, mn, out, nmain, part2, n2, out2, acc2);
  else
    mle::launch(split_reduce_kernel<false>, nmain + nb2, 256, 0, s, part, splits, mn, out, nmain, part2, n2, out2, acc2);
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

// ---------------------------------------------------------------------------
constexpr int kC3U = 2, kC3D = 4;  // 3 x 3 direct kernels: channel quads per stage, stages in flight

// Register-direct 3 x 3 convolution, stride 1, pad 1 (output grid = input
// grid): forward and input gradient with no LDS in the K loop.
//
//   C[m][pixel] = sum over (c, kh, kw) of A(m, c, kh, kw) * S[c][pixel + shift(kh, kw)]
//   forward: S = x,  m = output channel, A = w[m][c][kh][kw], shift (kh - 1, kw - 1)
//   dgrad:   S = dy, m = input channel,  A = w[c][m][kh][kw], shift (1 - kh, 1 - kw)
//
// Each wave owns a 64 x 64 block of C (64 channels x 64 pixels) as 4 x 4 MFMA
// blocks of 16 x 16.  Lane (lr, q) owns pixels g .. g + 3 (g = the wave's
// first pixel + 4 lr) and feeds channel c0 + q to every MFMA step: its B
// operand for block n is S at pixel g + n, so one float4 of S serves the four
// blocks, and each (block i, r) of the result is one 16-byte store.  The K
// loop walks (kh, channel); the three kw taps are three MFMA steps sharing
// that float4: the column shifts by -1 and +1 take the edge element of the
// neighbouring lane with a DPP row shift (a DPP row is the 16 lanes of one q
// group, 64 consecutive pixels), and the three taps' weights arrive in one
// dwordx3 load (w[..][..][kh][0..2] is contiguous).  The tap that falls in
// the padding of column 0 or W - 1 reads zero.  When 64 is not a multiple of
// W, lanes 0 and 15 of a DPP row can need a pixel owned by another wave; they
// load that element themselves (HALO).  A row shift out of the image, a pixel
// past the batch or a row past M reads at kOOB and gets 0; stores there are
// dropped by the buffer range check.
struct Conv3Args {
  const float* src;   // S [batch][cs][h][w]
  const float* wt;    // [cout][cin][3][3]
  const float* bias;  // forward only, nullable
  float* out;         // [batch][M][h][w]
  uint32_t src_bytes, wt_bytes, out_bytes;
  int M, cs, h, w, hw, npix;
  int a_rs, a_cs;  // weight offset (floats) per row m and per source channel c
  int acc;         // dgrad: 1 accumulates into out
  int tiles_m, tiles;
};

typedef float f32x3 __attribute__((ext_vector_type(3)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float lane_from_left(float v) {  // lane i gets lane i - 1 of its DPP row, 0 at lane 0
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x111, 0xF, 0xF, true));
}
__device__ __forceinline__ float lane_from_right(float v) {  // lane i gets lane i + 1, 0 at lane 15
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x101, 0xF, 0xF, true));
}

// Finish a wave's 64 x 64 block of a forward / input-gradient convolution
// (pixels g .. g + 3 of image b at p for lane (lr, q)): with KS > 1 the
// waves ks > 0 hand their partial blocks to wave ks = 0 through LDS
// (lane-major, so each write and read is conflict free), which adds them in
// ks order; then (i, r), row m0 + 16 i + 4 q + r, is one 16-byte store, plus
// the bias (forward) or the previous value (accumulating input gradient).
template <bool DG, int WM, int WN, int KS>
__device__ __forceinline__ void conv_block_out(f32x4 (&acc)[4][4], const Conv3Args& c, int m0, int lane, int wave,
                                               int ks, bool gok, int b, int p) {
  const int q = lane >> 4;
  if (KS > 1) {
    __shared__ float red[KS > 1 ? (KS - 1) * WM * WN * 64 * 64 : 1];
    const int blk = wave % (WM * WN);
    if (ks > 0) {
      float* dst = red + ((ks - 1) * WM * WN + blk) * 64 * 64 + lane;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r) dst[((i * 4 + n) * 4 + r) * 64] = acc[i][n][r];
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int k = 1; k < KS; ++k) {
      const float* src = red + ((k - 1) * WM * WN + blk) * 64 * 64 + lane;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][n][r] += src[((i * 4 + n) * 4 + r) * 64];
    }
  }
  // Every bias or previous value is loaded before the first store: the
  // vector memory counter also counts stores, so a load between two stores
  // would make the second wait for the first to complete.
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(c.out, c.out_bytes);
  uint32_t off[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + 16 * i + 4 * q + r;
      off[i][r] = gok && row < c.M ? (uint32_t)((b * c.M + row) * c.hw + p) * 4u : kOOB;
    }
  auto put = [&](int i, int r, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), ro, (int)off[i][r], 0, 0);
  };
  if (!DG) {
    // Rows past M read 0 (and store nowhere).
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(c.bias, c.bias ? (uint32_t)c.M * 4u : 0u);
    float bv[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) bv[i][r] = buf_ld1(rb, (uint32_t)(m0 + 16 * i + 4 * q + r) * 4u);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        f32x4 v = {acc[i][0][r], acc[i][1][r], acc[i][2][r], acc[i][3][r]};
        if (c.bias) v += bv[i][r];
        put(i, r, v);
      }
  } else if (c.acc) {
    f32x4 old[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) old[i][r] = buf_ld4(ro, off[i][r]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        f32x4 v = {acc[i][0][r], acc[i][1][r], acc[i][2][r], acc[i][3][r]};
        put(i, r, v + old[i][r]);
      }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) put(i, r, f32x4{acc[i][0][r], acc[i][1][r], acc[i][2][r], acc[i][3][r]});
  }
}

template <bool DG, int KS, int D>
__device__ __forceinline__ void conv1_kloop(f32x4 (&acc)[4][4], const Conv3Args& c, int m0, int lr, int q, int ks,
                                            bool gok, int b, int p);

// One 64 WM x 64 WN tile of a 3 x 3 convolution: L is the workgroup's index
// among this product's workgroups (its XCD is L % 8).  EXTRA (input
// gradient only): after the 3 x 3 stages the same accumulators also take the
// input gradient of a 1 x 1 convolution of the same input (c1: its output
// gradient and weights), so one tile writes dx = dgrad3 + dgrad1.
template <bool DG, bool HALO, int WM, int WN, int KS, int U, int D, bool EXTRA = false>
__device__ __forceinline__ void conv3_direct_body(const Conv3Args& c, const Conv3Args& c1, int L) {
  constexpr int SG = DG ? -1 : 1;  // shift of tap t is SG * (t - 1)
  constexpr int CPS = 4 * U;       // channels per stage
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 15, q = lane >> 4;
  const int wm = wave % WM, wn = (wave / WM) % WN, ks = wave / (WM * WN);
  // Workgroup -> tile: consecutive tiles on one XCD (workgroups are dealt to
  // the 8 XCDs round robin), so neighbouring pixel tiles share its L2.
  const int xq = c.tiles / 8, xr = c.tiles % 8, xc = L % 8;
  const int item = xc * xq + min(xc, xr) + L / 8;
  const int tm = item % c.tiles_m, tn = item / c.tiles_m;
  const int m0 = (tm * WM + wm) * 64;
  const int g = (tn * WN + wn) * 64 + 4 * lr;
  const bool gok = g < c.npix;
  const int b = g / c.hw, p = g - b * c.hw, py = p / c.w, px = p - py * c.w;
  const bool lpad = px == 0, rpad = px + 4 == c.w;
  bool rok[3];
#pragma unroll
  for (int t = 0; t < 3; ++t) rok[t] = gok && (unsigned)(py + SG * (t - 1)) < (unsigned)c.h;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(c.src, c.src_bytes);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(c.wt, c.wt_bytes);
  const uint32_t b_base = (uint32_t)((b * c.cs + q) * c.hw + p) * 4u;
  uint32_t a_base[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = m0 + 16 * i + lr;
    a_base[i] = row < c.M ? (uint32_t)(row * c.a_rs + q * c.a_cs) * 4u : kOOB;
  }
  const int spk = c.cs / CPS;  // stages per tap row
  // KS waves share each 64 x 64 block, splitting its stages: wave ks runs
  // [k0, k1) and the partial sums meet in LDS at the end.
  const int nks = (3 * spk + KS - 1) / KS;
  const int k0 = ks * nks, k1 = min(3 * spk, k0 + nks);

  // Stage kt: tap row t, channels cb .. cb + CPS - 1.  Stages fetched past
  // the end (up to D - 1) stay in bounds of the 32-bit offsets (the host
  // checks the extents) and are never consumed.
  auto load = [&](int kt, f32x3(&fa)[U][4], f32x4(&fb)[U], float(&fh)[U]) {
    const int t = (kt >= spk) + (kt >= 2 * spk);
    const int cb = (kt - t * spk) * CPS;
    const bool ok = t == 0 ? rok[0] : (t == 1 ? rok[1] : rok[2]);
    const int rsh = SG * (t - 1) * c.w;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t da = (uint32_t)((cb + 4 * u) * c.a_cs + 3 * t) * 4u;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        fa[u][i] = __builtin_bit_cast(f32x3, __builtin_amdgcn_raw_buffer_load_b96(ra, (int)(a_base[i] + da), 0, 0));
      const uint32_t off = b_base + (uint32_t)((cb + 4 * u) * c.hw + rsh) * 4u;
      fb[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(ok ? off : kOOB), 0, 0));
      if (HALO) {
        const uint32_t ho = lr == 0 ? (lpad ? kOOB : off - 4u) : (lr == 15 ? (rpad ? kOOB : off + 16u) : kOOB);
        fh[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(ok ? ho : kOOB), 0, 0));
      }
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto mfma = [&](const f32x3(&fa)[U][4], const f32x4(&fb)[U], const float(&fh)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const f32x4 v = fb[u];
      float lf = lane_from_left(v[3]), rt = lane_from_right(v[0]);
      if (HALO) {
        lf = lr == 0 ? fh[u] : lf;
        rt = lr == 15 ? fh[u] : rt;
      }
      lf = lpad ? 0.f : lf;
      rt = rpad ? 0.f : rt;
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const int d = SG * (j - 1);
        float bv[4];
#pragma unroll
        for (int n = 0; n < 4; ++n) bv[n] = d == 0 ? v[n] : (d < 0 ? (n == 0 ? lf : v[n - 1]) : (n == 3 ? rt : v[n + 1]));
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int n = 0; n < 4; ++n)
            acc[i][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[u][i][j], bv[n], acc[i][n], 0, 0, 0);
      }
    }
  };

  // Stage s lives in register set s % D; loads run D - 1 stages ahead.
  f32x3 fa[D][U][4];
  f32x4 fb[D][U];
  float fh[D][U];
#pragma unroll
  for (int s = 0; s < D - 1; ++s) load(k0 + s, fa[s], fb[s], fh[s]);
  int kt = k0;
  for (; kt + D - 1 < k1; kt += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      load(kt + s + D - 1, fa[(s + D - 1) % D], fb[(s + D - 1) % D], fh[(s + D - 1) % D]);
      __builtin_amdgcn_sched_barrier(0);
      mfma(fa[s], fb[s], fh[s]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int s = 0; s < D - 1; ++s)
    if (kt + s < k1) mfma(fa[s], fb[s], fh[s]);
  if (EXTRA) conv1_kloop<true, KS, 4>(acc, c1, m0, lr, q, ks, gok, b, p);

  conv_block_out<DG, WM, WN, KS>(acc, c, m0, lane, wave, ks, gok, b, p);
}

template <bool DG, bool HALO, int WM, int WN, int KS, int U, int D>
__global__ __launch_bounds__(64 * WM * WN * KS, 2) void conv3_direct_kernel(Conv3Args c) {
  conv3_direct_body<DG, HALO, WM, WN, KS, U, D>(c, c, blockIdx.x);
}

// Register-direct 1 x 1 convolution (stride 1, pad 0), forward and input
// gradient: C[m][pixel] = sum_c A(m, c) S[c][pixel] with A = w[m][c]
// (forward) or w[c][m] (dgrad).  The same blocks, pixel ownership and
// epilogue as the 3 x 3 kernel; a stage is 16 channels, lane group q feeding
// channels c0 + 4 q .. c0 + 4 q + 3 to the four MFMA steps: the forward's
// weights are one float4 per 16-row block (the dgrad's, strided by cin, four
// dwords), S one float4 of pixels per channel.  cs % 4 == 0, so a group's
// four channels are all inside or all past cs.
// The K loop of the 1 x 1 kernel: channels of c.src (16 per stage, the
// stages split over KS waves) into acc, for the wave's rows m0 .. m0 + 63
// and the lane's pixels g .. g + 3 (g = image b, position p).
template <bool DG, int KS, int D>
__device__ __forceinline__ void conv1_kloop(f32x4 (&acc)[4][4], const Conv3Args& c, int m0, int lr, int q, int ks,
                                            bool gok, int b, int p) {
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(c.src, c.src_bytes);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(c.wt, c.wt_bytes);
  const uint32_t b_base = (uint32_t)((b * c.cs + 4 * q) * c.hw + p) * 4u;
  uint32_t a_base[4];
  bool a_ok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = m0 + 16 * i + lr;
    a_ok[i] = row < c.M;
    a_base[i] = (uint32_t)(row * c.a_rs + 4 * q * c.a_cs) * 4u;
  }
  const int nst = (c.cs + 15) / 16;
  const int nks = (nst + KS - 1) / KS;
  const int k0 = ks * nks, k1 = min(nst, k0 + nks);

  auto load = [&](int kt, f32x4(&fa)[4], f32x4(&fb)[4]) {
    const bool cok = kt * 16 + 4 * q < c.cs;
    uint32_t ao[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ao[i] = (cok & a_ok[i]) ? a_base[i] + (uint32_t)(kt * 16 * c.a_cs) * 4u : kOOB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (!DG) {
        fa[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, (int)ao[i], 0, 0));
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
          fa[i][u] = __builtin_bit_cast(
              float, __builtin_amdgcn_raw_buffer_load_b32(ra, (int)(ao[i] + (uint32_t)(u * c.a_cs) * 4u), 0, 0));
      }
    }
    const uint32_t bo = (cok & gok) ? b_base + (uint32_t)(kt * 16 * c.hw) * 4u : kOOB;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      fb[u] = __builtin_bit_cast(f32x4,
                                 __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(bo + (uint32_t)(u * c.hw) * 4u), 0, 0));
  };
  auto mfma = [&](const f32x4(&fa)[4], const f32x4(&fb)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int n = 0; n < 4; ++n)
          acc[i][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i][u], fb[u][n], acc[i][n], 0, 0, 0);
  };

  f32x4 fa[D][4], fb[D][4];
#pragma unroll
  for (int s = 0; s < D - 1; ++s) load(k0 + s, fa[s], fb[s]);
  int kt = k0;
  for (; kt + D - 1 < k1; kt += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      load(kt + s + D - 1, fa[(s + D - 1) % D], fb[(s + D - 1) % D]);
      __builtin_amdgcn_sched_barrier(0);
      mfma(fa[s], fb[s]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int s = 0; s < D - 1; ++s)
    if (kt + s < k1) mfma(fa[s], fb[s]);
}

// Register-direct 1 x 1 tile (see above); L is the workgroup's index among
// this product's workgroups.
template <bool DG, int WM, int WN, int KS, int D>
__device__ __forceinline__ void conv1_direct_body(const Conv3Args& c, int L) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 15, q = lane >> 4;
  const int wm = wave % WM, wn = (wave / WM) % WN, ks = wave / (WM * WN);
  const int xq = c.tiles / 8, xr = c.tiles % 8, xc = L % 8;
  const int item = xc * xq + min(xc, xr) + L / 8;
  const int tm = item % c.tiles_m, tn = item / c.tiles_m;
  const int m0 = (tm * WM + wm) * 64;
  const int g = (tn * WN + wn) * 64 + 4 * lr;
  const bool gok = g < c.npix;
  const int b = g / c.hw, p = g - b * c.hw;

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nst = (c.cs + 15) / 16;
  if (!DG && KS == 1 && nst <= D) {
    // Forward with every stage resident at once (cs <= 16 D): the 16-row
    // blocks finish one at a time, so a block's stores drain while the next
    // block's products run instead of all stores waiting for the last product.
    // Each sum takes the stages and channels in the order of the K loop and
    // adds the bias last, as conv_block_out does: the same bits.
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(c.src, c.src_bytes);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(c.wt, c.wt_bytes);
    const uint32_t b_base = (uint32_t)((b * c.cs + 4 * q) * c.hw + p) * 4u;
    f32x4 fa[D][4], fb[D][4];
#pragma unroll
    for (int s = 0; s < D; ++s) {
      const bool cok = s < nst && s * 16 + 4 * q < c.cs;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = m0 + 16 * i + lr;
        const uint32_t ao = (cok && row < c.M) ? (uint32_t)(row * c.a_rs + (s * 16 + 4 * q) * c.a_cs) * 4u : kOOB;
        fa[s][i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, (int)ao, 0, 0));
      }
      const uint32_t bo = (cok & gok) ? b_base + (uint32_t)(s * 16 * c.hw) * 4u : kOOB;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        fb[s][u] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(bo + (uint32_t)(u * c.hw) * 4u), 0, 0));
    }
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(c.bias, c.bias ? (uint32_t)c.M * 4u : 0u);
    float bv[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) bv[i][r] = buf_ld1(rb, (uint32_t)(m0 + 16 * i + 4 * q + r) * 4u);
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(c.out, c.out_bytes);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int s = 0; s < D; ++s)
        if (s < nst)
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int n = 0; n < 4; ++n)
              acc[i][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[s][i][u], fb[s][u][n], acc[i][n], 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + 16 * i + 4 * q + r;
        const bool ok = gok && row < c.M;
        const uint32_t off = ok ? (uint32_t)((b * c.M + row) * c.hw + p) * 4u : kOOB;
        f32x4 v = {acc[i][0][r], acc[i][1][r], acc[i][2][r], acc[i][3][r]};
        if (c.bias) v += bv[i][r];
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), ro, (int)off, 0, 0);
      }
    }
    return;
  }
  conv1_kloop<DG, KS, D>(acc, c, m0, lr, q, ks, gok, b, p);
  conv_block_out<DG, WM, WN, KS>(acc, c, m0, lane, wave, ks, gok, b, p);
}

template <bool DG, int WM, int WN, int KS, int D>
__global__ __launch_bounds__(64 * WM * WN * KS, 2) void conv1_direct_kernel(Conv3Args c) {
  conv1_direct_body<DG, WM, WN, KS, D>(c, blockIdx.x);
}

// Forward of a 3 x 3 (pad 1) and a 1 x 1 (pad 0) convolution of the same x
// (a residual block's first convolution and its skip) in one grid: the 1 x 1
// tiles first, then the 3 x 3 tiles, each product with its own XCD-aware
// tile order.  Measured on the C5 shapes (16 x 64 -> 128 x 64 x 64):
// 100.4 us against 109.4 us for the two launches.  The 3 x 3 tiles first ran
// 104.5 us, each workgroup's 3 x 3 tile followed by the same pixels' 1 x 1
// tile 103.6 us, and the two products alternating across the XCDs 154.7 us
// (the 3 x 3 tiles slow down when they do not run in lockstep with their
// neighbours).
template <bool HALO, int WM3, int WM1>
__global__ __launch_bounds__(256, 2) void conv_pair_fwd_kernel(Conv3Args a, Conv3Args b) {
  const int L = blockIdx.x;
  if (L < b.tiles)
    conv1_direct_body<false, WM1, 2, WM1 == 1 ? 2 : 1, 4>(b, L);
  else
    conv3_direct_body<false, HALO, WM3, 2, WM3 == 1 ? 2 : 1, kC3U, kC3D>(a, a, L - b.tiles);
}

// Input gradient of the same pair: dx (+)= dgrad3(dy3) + dgrad1(dy1), the
// 1 x 1 product as extra stages of each 3 x 3 tile.
template <bool HALO, int WM>
__global__ __launch_bounds__(256, 2) void conv_pair_dgrad_kernel(Conv3Args a, Conv3Args b) {
  conv3_direct_body<true, HALO, WM, 2, WM == 1 ? 2 : 1, kC3U, kC3D, true>(a, b, blockIdx.x);
}

// ---------------------------------------------------------------------------
// Register-direct 3 x 3 weight gradient, stride 1, pad 1:
//   dW[co][ci][kh][kw] = sum over pixels p of dy[co][p] * x[ci][p + (kh - 1, kw - 1)]
// as C[co][(ci, kh, kw)] with K = the batch's pixels, split across workgroups
// (each split writes its partial C; a second pass adds them in split order).
// Lane (lr, q) of a wave owns one (ci, kh) pair (16 pairs per wave) and its
// three kw taps are the wave's three MFMA column blocks, so a wave's block is
// 64 output channels x 48 columns.  Per 16-pixel stage lane group q feeds
// pixels P .. P + 3 (P = stage start + 4 q) to the four MFMA steps: dy as one
// aligned float4 per 16-row block, x of its (ci, kh) row as one aligned
// float4 plus the two neighbours x[P - 1] and x[P + 4], from which the three
// taps' operands are picked in registers.  A neighbour in the column padding,
// a row shift out of the image, a pixel past the split, a pair past cin * 3
// or a row past cout reads at kOOB and gets 0.  The lane's pixel position
// advances by 16 per stage with at most one row and one image carry (W >= 16).
struct Wgrad3Args {
  const float* x;   // [n][cin][h][w]
  const float* dy;  // [n][cout][h][w]
  float* out;       // one split: dW [cout][cin * 9]; else partials [splits][cout][cin * 9]
  uint32_t x_bytes, dy_bytes, out_bytes;
  int cout, cin, h, w, hw, npix;
  int chunk;  // pixels per split, a multiple of 16
  int tiles_m, tiles, items;
  // Bias gradient from the dy rows the kernel already loads (sum over the
  // pixels per output channel), taken by the waves of the first column block:
  // db_mode 1 adds into db (one split), 3 assigns it; 2 writes the split's
  // partial sums to bpart[split][cout].
  float* db;
  float* bpart;
  int db_mode;
};

// Per lane, the dy row sums of stage `fa` (block i: four pixels of row
// m0 + 16 i + lr), added pairwise.
__device__ __forceinline__ void bias_stage(float (&bs)[4], const f32x4 (&fa)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) bs[i] += (fa[i][0] + fa[i][1]) + (fa[i][2] + fa[i][3]);
}

// Combine the four lane groups' row sums (q order fixed by the xor tree) and
// store them: lane (lr, q = 0) owns rows m0 + 16 i + lr.
__device__ __forceinline__ void bias_store(const Wgrad3Args& c, float (&bs)[4], int m0, int split, int lr, int q) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float v = bs[i];
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    const int co = m0 + 16 * i + lr;
    if (q == 0 && co < c.cout) {
      if (c.db_mode == 1) c.db[co] += v;
      else if (c.db_mode == 3) c.db[co] = v;
      else c.bpart[(size_t)split * c.cout + co] = v;
    }
  }
}

template <int WM, int D>
__global__ __launch_bounds__(256, 2) void conv3_wgrad_kernel(Wgrad3Args c) {
  constexpr int WN = 4 / WM;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 15, q = lane >> 4;
  const int wm = wave % WM, wn = wave / WM;
  // Workgroup -> (tile, split): consecutive items on one XCD, tiles of one
  // split adjacent (they read the same dy and x pixels).
  const int L = blockIdx.x, xq = c.items / 8, xr = c.items % 8, xc = L % 8;
  const int item = xc * xq + min(xc, xr) + L / 8;
  const int tile = item % c.tiles, split = item / c.tiles;
  const int tm = tile % c.tiles_m, tn = tile / c.tiles_m;
  const int m0 = (tm * WM + wm) * 64;
  const int pair = (tn * WN + wn) * 16 + lr;
  const bool pok = pair < 3 * c.cin;
  const int ci = pair / 3, kh = pair - 3 * ci;
  const int kbeg = split * c.chunk, kend = min(c.npix, kbeg + c.chunk);
  const int nk = (kend - kbeg + 15) / 16;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(c.x, c.x_bytes);
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(c.dy, c.dy_bytes);
  uint32_t a_row[4];
  bool a_ok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int co = m0 + 16 * i + lr;
    a_ok[i] = co < c.cout;
    a_row[i] = (uint32_t)(co * c.hw) * 4u;
  }
  const uint32_t x_lane = (uint32_t)(ci * c.hw + (kh - 1) * c.w) * 4u;  // modulo 2^32
  // Load cursor: the next stage's pixel P of this lane, its column px and row
  // py, and its pixel byte offsets in dy and x (without the channel part).
  // Advancing 16 pixels adds 64 bytes, plus the rest of an image's channel
  // planes when P crosses into the next image; W >= 16, so at most one row
  // and one image carry.  Only adds and selects: no multiplies in the loop.
  int P = kbeg + 4 * q;
  int py, px;
  uint32_t dpix, xpix;
  {
    const int b = P / c.hw, pp = P - b * c.hw;
    py = pp / c.w;
    px = pp - py * c.w;
    dpix = (uint32_t)(b * c.cout * c.hw + pp) * 4u;
    xpix = (uint32_t)(b * c.cin * c.hw + pp) * 4u;
  }
  const uint32_t d_img = (uint32_t)((c.cout - 1) * c.hw) * 4u, x_img = (uint32_t)((c.cin - 1) * c.hw) * 4u;

  auto load = [&](f32x4(&fa)[4], f32x4& fb, float& fl, float& fr) {
    const bool pix = P < kend;
    const bool rowok = (unsigned)(py + kh - 1) < (unsigned)c.h;
    // Offsets are selected (bitwise conditions, no short circuit) so the
    // loads stay unconditional.
    uint32_t ao[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ao[i] = (pix & a_ok[i]) ? a_row[i] + dpix : kOOB;
    const bool ok = pix & rowok & pok;
    const uint32_t xo = x_lane + xpix;
    const uint32_t xc = ok ? xo : kOOB;
    const uint32_t xl = (ok & (px != 0)) ? xo - 4u : kOOB;
    const uint32_t xr = (ok & (px + 4 != c.w)) ? xo + 16u : kOOB;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      fa[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rd, (int)ao[i], 0, 0));
    fb = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)xc, 0, 0));
    fl = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, (int)xl, 0, 0));
    fr = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, (int)xr, 0, 0));
    P += 16;
    px += 16;
    dpix += 64u;
    xpix += 64u;
    const bool cx = px >= c.w;
    px = cx ? px - c.w : px;
    py += cx ? 1 : 0;
    const bool cy = py >= c.h;
    py = cy ? 0 : py;
    dpix += cy ? d_img : 0u;
    xpix += cy ? x_img : 0u;
  };

  f32x4 acc[4][3];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 3; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};

  const bool do_b = c.db_mode != 0 && tn == 0 && wn == 0;
  float bs[4] = {0.f, 0.f, 0.f, 0.f};
  auto mfma = [&](const f32x4(&fa)[4], const f32x4& v, float fl, float fr) {
    if (do_b) bias_stage(bs, fa);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float b0 = j == 0 ? fl : v[j - 1];
      const float b2 = j == 3 ? fr : v[j + 1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[i][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i][j], b0, acc[i][0], 0, 0, 0);
        acc[i][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i][j], v[j], acc[i][1], 0, 0, 0);
        acc[i][2] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i][j], b2, acc[i][2], 0, 0, 0);
      }
    }
  };

  f32x4 fa[D][4], fb[D];
  float fl[D], fr[D];
#pragma unroll
  for (int s = 0; s < D - 1; ++s) load(fa[s], fb[s], fl[s], fr[s]);
  int kt = 0;
  for (; kt + D - 1 < nk; kt += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      const int ls = (s + D - 1) % D;
      load(fa[ls], fb[ls], fl[ls], fr[ls]);
      __builtin_amdgcn_sched_barrier(0);
      mfma(fa[s], fb[s], fl[s], fr[s]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int s = 0; s < D - 1; ++s)
    if (kt + s < nk) mfma(fa[s], fb[s], fl[s], fr[s]);

  if (do_b) bias_store(c, bs, m0, split, lr, q);
  // (i, r) is row m0 + 16 i + 4 q + r, columns 3 pair .. 3 pair + 2.
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(c.out, c.out_bytes);
  const int ncol = 9 * c.cin;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + 16 * i + 4 * q + r;
      const bool ok = pok && row < c.cout;
      const uint32_t off = ok ? (uint32_t)(((split * c.cout + row) * ncol) + 3 * pair) * 4u : kOOB;
      const f32x3 v = {acc[i][0][r], acc[i][1][r], acc[i][2][r]};
      __builtin_amdgcn_raw_buffer_store_b96(__builtin_bit_cast(__attribute__((ext_vector_type(3))) unsigned, v), ro,
                                            (int)off, 0, 0);
    }
}

// Register-direct 1 x 1 weight gradient (stride 1, pad 0):
//   dW[co][ci] = sum over pixels p of dy[co][p] * x[ci][p]
// with the pixel splits, stages and dy loads of the 3 x 3 kernel.  Lane
// (lr, q) owns the four columns ci0 .. ci0 + 3 (ci0 = the wave's first
// column + 4 lr) as the four MFMA column blocks: one aligned float4 of x per
// column per stage, and a 16-byte store per (block i, r).  The lane's pixel
// advances 16 per stage with at most one image carry (H * W >= 16).  The
// four waves are WM x WN blocks of 64 x 64 times KS = 4 / (WM WN) shares of
// the split's stages (the host sizes WN to cin, so no wave computes columns
// past cin); shares ks > 0 hand their blocks and bias sums to share 0
// through LDS, which adds them in ks order.
template <int WM, int WN, int D>
__global__ __launch_bounds__(256, 2) void conv1_wgrad_kernel(Wgrad3Args c) {
  constexpr int KS = 4 / (WM * WN);
  static_assert(WM * WN * KS == 4, "four waves");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 15, q = lane >> 4;
  const int wm = wave % WM, wn = (wave / WM) % WN, ks = wave / (WM * WN);
  const int L = blockIdx.x, xq = c.items / 8, xr = c.items % 8, xc = L % 8;
  const int item = xc * xq + min(xc, xr) + L / 8;
  const int tile = item % c.tiles, split = item / c.tiles;
  const int tm = tile % c.tiles_m, tn = tile / c.tiles_m;
  const int m0 = (tm * WM + wm) * 64;
  const int ci0 = (tn * WN + wn) * 64 + 4 * lr;
  const bool cok = ci0 < c.cin;  // cin % 4 == 0: all four columns or none
  // Share ks: pixels [kbeg, kend) of the split, whole 16-pixel stages.
  const int sbeg = split * c.chunk, send = min(c.npix, sbeg + c.chunk);
  const int nks = ((send - sbeg + 15) / 16 + KS - 1) / KS;
  const int kbeg = min(send, sbeg + ks * nks * 16), kend = min(send, kbeg + nks * 16);
  const int nk = (kend - kbeg + 15) / 16;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(c.x, c.x_bytes);
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(c.dy, c.dy_bytes);
  uint32_t a_row[4];
  bool a_ok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int co = m0 + 16 * i + lr;
    a_ok[i] = co < c.cout;
    a_row[i] = (uint32_t)(co * c.hw) * 4u;
  }
  const uint32_t x_lane = (uint32_t)(ci0 * c.hw) * 4u;
  int P = kbeg + 4 * q, pp;
  uint32_t dpix, xpix;
  {
    const int b = P / c.hw;
    pp = P - b * c.hw;
    dpix = (uint32_t)(b * c.cout * c.hw + pp) * 4u;
    xpix = (uint32_t)(b * c.cin * c.hw + pp) * 4u;
  }
  const uint32_t d_img = (uint32_t)((c.cout - 1) * c.hw) * 4u, x_img = (uint32_t)((c.cin - 1) * c.hw) * 4u;
  const uint32_t x_ch = (uint32_t)c.hw * 4u;

  auto load = [&](f32x4(&fa)[4], f32x4(&fb)[4]) {
    const bool pix = P < kend;
    uint32_t ao[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ao[i] = (pix & a_ok[i]) ? a_row[i] + dpix : kOOB;
    const uint32_t xo = (pix & cok) ? x_lane + xpix : kOOB;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      fa[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rd, (int)ao[i], 0, 0));
#pragma unroll
    for (int n = 0; n < 4; ++n)
      fb[n] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(xo + n * x_ch), 0, 0));
    P += 16;
    pp += 16;
    dpix += 64u;
    xpix += 64u;
    const bool cy = pp >= c.hw;
    pp = cy ? pp - c.hw : pp;
    dpix += cy ? d_img : 0u;
    xpix += cy ? x_img : 0u;
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bool do_b = c.db_mode != 0 && tn == 0 && wn == 0;
  float bs[4] = {0.f, 0.f, 0.f, 0.f};
  auto mfma = [&](const f32x4(&fa)[4], const f32x4(&fb)[4]) {
    if (do_b) bias_stage(bs, fa);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int n = 0; n < 4; ++n)
          acc[i][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i][j], fb[n][j], acc[i][n], 0, 0, 0);
  };

  f32x4 fa[D][4], fb[D][4];
#pragma unroll
  for (int s = 0; s < D - 1; ++s) load(fa[s], fb[s]);
  int kt = 0;
  for (; kt + D - 1 < nk; kt += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      const int ls = (s + D - 1) % D;
      load(fa[ls], fb[ls]);
      __builtin_amdgcn_sched_barrier(0);
      mfma(fa[s], fb[s]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int s = 0; s < D - 1; ++s)
    if (kt + s < nk) mfma(fa[s], fb[s]);

  if (KS > 1) {
    constexpr int RW = 64 * 64 + 4 * 64;  // a wave's block, then its bias sums
    __shared__ float red[KS > 1 ? (KS - 1) * WM * WN * RW : 1];
    const int blk = wave % (WM * WN);
    if (ks > 0) {
      float* dst = red + ((ks - 1) * WM * WN + blk) * RW + lane;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r) dst[((i * 4 + n) * 4 + r) * 64] = acc[i][n][r];
      if (do_b)
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[(64 + i) * 64] = bs[i];
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll 1
    for (int k = 1; k < KS; ++k) {
      const float* src = red + ((k - 1) * WM * WN + blk) * RW + lane;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][n][r] += src[((i * 4 + n) * 4 + r) * 64];
      if (do_b)
#pragma unroll
        for (int i = 0; i < 4; ++i) bs[i] += src[(64 + i) * 64];
    }
  }
  if (do_b) bias_store(c, bs, m0, split, lr, q);
  // (i, r) is row m0 + 16 i + 4 q + r, columns ci0 .. ci0 + 3.
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(c.out, c.out_bytes);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + 16 * i + 4 * q + r;
      const bool ok = cok && row < c.cout;
      const uint32_t off = ok ? (uint32_t)((split * c.cout + row) * c.cin + ci0) * 4u : kOOB;
      const f32x4 v = {acc[i][0][r], acc[i][1][r], acc[i][2][r], acc[i][3][r]};
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), ro, (int)off, 0, 0);
    }
}

bool fits_2g(double elems) { return elems * 4.0 < 2147483647.0; }
bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }


// 64-row blocks (M <= 64) split each block's stages over two waves, so the
// grid still holds two waves per SIMD.
template <bool DG, bool HALO, int WM>
void launch_conv3(hipStream_t s, const Conv3Args& c) {
  constexpr int KS = WM == 1 ? 2 : 1;
  mle::launch(conv3_direct_kernel<DG, HALO, WM, 2, KS, kC3U, kC3D>, c.tiles, 64 * WM * 2 * KS, 0, s, c);
}

template <bool DG, int WM>
void launch_conv1(hipStream_t s, const Conv3Args& c) {
  constexpr int KS = WM == 1 ? 2 : 1;
  mle::launch(conv1_direct_kernel<DG, WM, 2, KS, 4>, c.tiles, 64 * WM * 2 * KS, 0, s, c);
}

// Arguments of the register-direct kernels for a 3 x 3 (stride 1, pad 1) or
// 1 x 1 (stride 1, pad 0) forward (dg = 0: src = x, M = cout) or input
// gradient (dg = 1: src = dy, M = cin).  Returns false when the shape is
// outside what the kernels assume; k3 tells which filter, wm the row blocks
// per workgroup, halo whether 64 pixels span a partial image row.
bool direct_args(bool dg, const ConvGeom& g, const float* src, const float* wt, const float* bias, float* out,
                 int acc, Conv3Args& c, bool& k3, int& wm, bool& halo) {
  k3 = g.kh == 3 && g.kw == 3 && g.pad == 1 && g.stride == 1 && g.w % 4 == 0;
  const bool k1 = g.kh == 1 && g.kw == 1 && g.pad == 0 && g.stride == 1 && (g.h * g.w) % 4 == 0;
  if (!k3 && !k1) return false;
  const int M = dg ? g.cin : g.cout, cs = dg ? g.cout : g.cin;
  if (cs % (k3 ? 4 * kC3U : 4) != 0 || !a16(out)) return false;
  const double hw = (double)g.h * g.w;
  const int taps = g.kh * g.kw;
  // 32-bit byte offsets: tensors below 2 GiB, weights below 1 GiB (an
  // out-of-range row's kOOB offset plus a weight offset must not wrap).
  if ((double)g.n * cs * hw * 4.0 >= 2147483647.0 || (double)g.n * M * hw * 4.0 >= 2147483647.0 ||
      (double)g.cout * g.cin * taps * 4.0 >= 1073741824.0)
    return false;
  c = Conv3Args{};
  c.src = src;
  c.wt = wt;
  c.bias = dg ? nullptr : bias;
  c.out = out;
  c.src_bytes = (uint32_t)((size_t)g.n * cs * g.h * g.w * 4);
  c.wt_bytes = (uint32_t)((size_t)g.cout * g.cin * taps * 4);
  c.out_bytes = (uint32_t)((size_t)g.n * M * g.h * g.w * 4);
  c.M = M;
  c.cs = cs;
  c.h = g.h;
  c.w = g.w;
  c.hw = g.h * g.w;
  c.npix = g.n * c.hw;
  c.a_rs = dg ? taps : g.cin * taps;
  c.a_cs = dg ? g.cin * taps : taps;
  c.acc = acc;
  wm = M <= 64 ? 1 : 2;
  c.tiles_m = (M + 64 * wm - 1) / (64 * wm);
  c.tiles = c.tiles_m * ((c.npix + 127) / 128);
  halo = k3 && 64 % g.w != 0;
  return true;
}

// Register-direct path for one convolution (see direct_args).  Returns false,
// launching nothing, when the shape is outside what the kernels assume.
bool conv_direct(hipStream_t s, bool dg, const ConvGeom& g, const float* src, const float* wt, const float* bias,
                 float* out, int acc) {
  Conv3Args c;
  bool k3, halo;
  int wm;
  if (!direct_args(dg, g, src, wt, bias, out, acc, c, k3, wm, halo)) return false;
  if (!k3) {
    if (dg) wm == 1 ? launch_conv1<true, 1>(s, c) : launch_conv1<true, 2>(s, c);
    else wm == 1 ? launch_conv1<false, 1>(s, c) : launch_conv1<false, 2>(s, c);
    return true;
  }
  if (dg) {
    if (halo) wm == 1 ? launch_conv3<true, true, 1>(s, c) : launch_conv3<true, true, 2>(s, c);
    else wm == 1 ? launch_conv3<true, false, 1>(s, c) : launch_conv3<true, false, 2>(s, c);
  } else {
    if (halo) wm == 1 ? launch_conv3<false, true, 1>(s, c) : launch_conv3<false, true, 2>(s, c);
    else wm == 1 ? launch_conv3<false, false, 1>(s, c) : launch_conv3<false, false, 2>(s, c);
  }
  return true;
}

int geom(int n, int cin, int h, int w, int cout, int kh, int kw, int pad, int stride, ConvGeom& g);

// The geometries of a 3 x 3 (pad 1) and a 1 x 1 (pad 0) convolution, stride
// 1, of one input [n][cin][h][w], with cout3 and cout1 output channels.
bool pair_geoms(int n, int cin, int h, int w, int cout3, int cout1, ConvGeom& g3, ConvGeom& g1) {
  if (geom(n, cin, h, w, cout3, 3, 3, 1, 1, g3) != MLE_OK) return false;
  if (geom(n, cin, h, w, cout1, 1, 1, 0, 1, g1) != MLE_OK) return false;
  return true;
}

template <bool HALO>
void launch_pair_fwd(hipStream_t s, const Conv3Args& a, int wma, const Conv3Args& b, int wmb) {
  const unsigned grid = (unsigned)(a.tiles + b.tiles);
  if (wma == 1) {
    if (wmb == 1) mle::launch(conv_pair_fwd_kernel<HALO, 1, 1>, grid, 256, 0, s, a, b);
    else mle::launch(conv_pair_fwd_kernel<HALO, 1, 2>, grid, 256, 0, s, a, b);
  } else {
    if (wmb == 1) mle::launch(conv_pair_fwd_kernel<HALO, 2, 1>, grid, 256, 0, s, a, b);
    else mle::launch(conv_pair_fwd_kernel<HALO, 2, 2>, grid, 256, 0, s, a, b);
  }
}

template <int KIND>
void launch_fast(hipStream_t s, const FastConv& c, int kh, int splits) {
  dim3 grid((c.N + BN - 1) / BN, (c.M + BM - 1) / BM, splits);
  if (kh == 3) mle::launch(conv_fast_kernel<KIND, 3, 3>, grid, NT, 0, s, c);
  else mle::launch(conv_fast_kernel<KIND, 1, 1>, grid, NT, 0, s, c);
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

// Workgroups of `kernel` (256 threads) resident at once on the current
// device (per-CU occupancy x CUs), cached per device in `cache`.
template <class K>
int resident_wgs(K kernel, int (&cache)[64]) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 768;
  int& v = cache[dev];
  if (v <= 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, 0) != hipSuccess || per_cu <= 0) per_cu = 2;
    v = per_cu * cus;
  }
  return v;
}

// Workgroups of the weight-gradient kernel for (taps, wm, wn) resident at
// once (3 x 256 on MI355X for the 3 x 3 kernel).  One full round of resident
// workgroups measured fastest: at 512 workgroups on 768 slots some CUs hold
// 1 and others 3 (54 % of fp32 MFMA for the C5 weight gradients), at 768
// every CU holds 3 (77 %), at 1024 the last 256 run as a tail (62 %).
int wgrad_slots(int taps, int wm, int wn) {
  static int c3[2][64], c1[5][64];
  if (taps == 9)
    return wm == 1 ? resident_wgs(conv3_wgrad_kernel<1, 3>, c3[0]) : resident_wgs(conv3_wgrad_kernel<2, 3>, c3[1]);
  if (wm == 1)
    return wn == 4 ? resident_wgs(conv1_wgrad_kernel<1, 4, 4>, c1[0])
                   : (wn == 2 ? resident_wgs(conv1_wgrad_kernel<1, 2, 4>, c1[1])
                              : resident_wgs(conv1_wgrad_kernel<1, 1, 4>, c1[2]));
  return wn == 2 ? resident_wgs(conv1_wgrad_kernel<2, 2, 4>, c1[3]) : resident_wgs(conv1_wgrad_kernel<2, 1, 4>, c1[4]);
}

// Register-direct weight gradient plan: 3 x 3 (stride 1, pad 1, W >= 16)
// in 128 x 96 tiles of C (64 x 192 when cout <= 64), or 1 x 1 (stride 1,
// pad 0, cin % 4 == 0, H * W >= 16) in 64 wm x 64 wn tiles (wm = 1 when
// cout <= 64, else 2; wn the smallest power of two up to 4 / wm whose
// columns cover cin, the remaining waves sharing the pixels); the pixels
// split so that tiles x splits fills one round of resident workgroups, each
// split a whole number of 16-pixel stages and at least 256 pixels.  Returns
// false when the shape is outside what the kernels assume.
bool wgrad_plan(const ConvGeom& g, Wgrad3Args& c, int& taps, int& wm, int& wn) {
  const bool k3 = g.kh == 3 && g.kw == 3 && g.pad == 1 && g.stride == 1 && g.w % 4 == 0 && g.w >= 16;
  const bool k1 = g.kh == 1 && g.kw == 1 && g.pad == 0 && g.stride == 1 && (g.h * g.w) % 4 == 0 &&
                  g.h * g.w >= 16 && g.cin % 4 == 0;
  if (!k3 && !k1) return false;
  taps = k3 ? 9 : 1;
  const double hw = (double)g.h * g.w;
  if ((double)g.n * g.cin * hw * 4.0 >= 2147483647.0 || (double)g.n * g.cout * hw * 4.0 >= 2147483647.0) return false;
  c = Wgrad3Args{};
  c.cout = g.cout;
  c.cin = g.cin;
  c.h = g.h;
  c.w = g.w;
  c.hw = g.h * g.w;
  c.npix = g.n * c.hw;
  wm = g.cout <= 64 ? 1 : 2;
  wn = 4 / wm;
  if (k1)
    while (wn > 1 && 64 * (wn / 2) >= g.cin) wn /= 2;
  c.tiles_m = (g.cout + 64 * wm - 1) / (64 * wm);
  c.tiles = c.tiles_m * (k3 ? (3 * g.cin + 16 * wn - 1) / (16 * wn) : (g.cin + 64 * wn - 1) / (64 * wn));
  const int slots = wgrad_slots(taps, wm, wn);
  int splits = std::max(1, slots / c.tiles);
  // At least 256 pixels per split: the C5 1 x 1 weight gradient (65536
  // pixels) ran 25.1 us with 256-pixel splits and 32.6 us with 128 or fewer,
  // where the partials' reduce grows faster than the kernel shrinks.
  const int max_splits = (c.npix + 255) / 256;
  splits = std::max(1, std::min(splits, max_splits));
  c.chunk = ((c.npix + splits - 1) / splits + 15) / 16 * 16;
  splits = (c.npix + c.chunk - 1) / c.chunk;
  c.items = c.tiles * splits;
  if ((double)splits * g.cout * g.cin * taps * 4.0 >= 2147483647.0) return false;
  c.x_bytes = (uint32_t)((size_t)g.n * g.cin * c.hw * 4);
  c.dy_bytes = (uint32_t)((size_t)g.n * g.cout * c.hw * 4);
  c.out_bytes = (uint32_t)((size_t)splits * g.cout * g.cin * taps * 4);
  return true;
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
  if (conv_direct(s, false, g, x, w, b, y, 0)) {
  } else if (fast_filter(g) && ohw % 4 == 0 && op.K % 4 == 0 && a16(y) && fits_2g((double)n * cin * h * w_in) &&
      fits_2g((double)n * cout * ohw) && fits_2g((double)cout * op.K)) {
    FastConv c{x, w, b, y, (uint32_t)((size_t)n * cin * h * w_in * 4), (uint32_t)((size_t)cout * op.K * 4),
               op.M, op.N, op.K, op.K, cin, h, w_in, h * w_in, g.oh, g.ow, ohw, pad, cout, cin, 0};
    launch_fast<CONV_FWD>(s, c, kh, 1);
  } else {
    dim3 grid((op.N + BN - 1) / BN, (op.M + BM - 1) / BM, 1);
    mle::launch(igemm_kernel<FwdOps, false>, grid, NT, 0, s, op, op.K);
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
  if (conv_direct(s, true, g, dy, w, nullptr, dx, accumulate != 0)) {
  } else if (fast_filter(g) && hw % 4 == 0 && a16(dx) && fits_2g((double)n * cin * hw) &&
      fits_2g((double)n * cout * g.oh * g.ow) && fits_2g((double)cout * cin * kh * kw)) {
    FastConv c{dy, w, nullptr, dx, (uint32_t)((size_t)n * cout * g.oh * g.ow * 4),
               (uint32_t)((size_t)cout * cin * kh * kw * 4), op.M, op.N, op.K, op.K, cout, g.oh, g.ow, g.oh * g.ow,
               h, w_in, hw, pad, cout, cin, accumulate != 0};
    launch_fast<CONV_DGRAD>(s, c, kh, 1);
  } else {
    dim3 grid((op.N + BN - 1) / BN, (op.M + BM - 1) / BM, 1);
    mle::launch(igemm_kernel<DgradOps, false>, grid, NT, 0, s, op, op.K);
  }
  return check_launch("mle_conv2d_dgrad");
}

size_t mle_conv2d_wgrad_ws_bytes(int n, int cin, int h, int w_in, int cout, int kh, int kw, int pad, int stride) {
  ConvGeom g;
  if (geom(n, cin, h, w_in, cout, kh, kw, pad, stride, g) != MLE_OK) return 0;
  Wgrad3Args c3;
  int taps, wm, wn;
  // Split partials of dW, then (mle_conv2d_wgrad_bias) those of db.
  if (wgrad_plan(g, c3, taps, wm, wn))
    return c3.items > c3.tiles ? (size_t)c3.out_bytes + (size_t)(c3.items / c3.tiles) * cout * sizeof(float) : 0;
  int kchunk;
  const int splits = wgrad_splits(g, kchunk);
  return (size_t)splits * cout * cin * kh * kw * sizeof(float);
}

int mle_conv2d_wgrad(mle_stream stream, const float* x, const float* dy, float* dw, int n, int cin, int h, int w_in,
                     int cout, int kh, int kw, int pad, int stride, void* ws, size_t ws_bytes) {
  return mle_conv2d_wgrad_bias(stream, x, dy, dw, nullptr, 1, n, cin, h, w_in, cout, kh, kw, pad, stride, ws,
                               ws_bytes);
}

int mle_conv2d_wgrad_bias(mle_stream stream, const float* x, const float* dy, float* dw, float* db, int accumulate_db,
                          int n, int cin, int h, int w_in, int cout, int kh, int kw, int pad, int stride, void* ws,
                          size_t ws_bytes) {
  MLE_CHECK_ARG(x && dy && dw, "mle_conv2d_wgrad: null pointer");
  ConvGeom g;
  int rc = geom(n, cin, h, w_in, cout, kh, kw, pad, stride, g);
  if (rc) return rc;
  const size_t need = mle_conv2d_wgrad_ws_bytes(n, cin, h, w_in, cout, kh, kw, pad, stride);
  if (ws_bytes < need || (need > 0 && !ws)) return set_error(MLE_ERR_WORKSPACE, "mle_conv2d_wgrad: workspace too small");
  hipStream_t s = as_stream(stream);
  const double flop = 2.0 * cout * (double)cin * kh * kw * (double)n * g.oh * g.ow;
  Wgrad3Args c3;
  int taps, wm, wn;
  if (wgrad_plan(g, c3, taps, wm, wn)) {
    const int splits = c3.items / c3.tiles;
    c3.x = x;
    c3.dy = dy;
    c3.out = splits > 1 ? static_cast<float*>(ws) : dw;
    if (splits == 1) c3.out_bytes = (uint32_t)((size_t)cout * cin * taps * 4);
    const size_t mn = (size_t)cout * cin * taps;
    float* bpart = splits > 1 ? static_cast<float*>(ws) + (size_t)splits * mn : nullptr;
    c3.db = db;
    c3.bpart = bpart;
    c3.db_mode = db ? (splits > 1 ? 2 : (accumulate_db ? 1 : 3)) : 0;
    {
      ProbeScope probe("conv_wgrad", s, flop, 0.0);
      if (taps == 9) {
        if (wm == 1) mle::launch(conv3_wgrad_kernel<1, 3>, c3.items, 256, 0, s, c3);
        else mle::launch(conv3_wgrad_kernel<2, 3>, c3.items, 256, 0, s, c3);
      } else if (wm == 1) {
        if (wn == 4) mle::launch(conv1_wgrad_kernel<1, 4, 4>, c3.items, 256, 0, s, c3);
        else if (wn == 2) mle::launch(conv1_wgrad_kernel<1, 2, 4>, c3.items, 256, 0, s, c3);
        else mle::launch(conv1_wgrad_kernel<1, 1, 4>, c3.items, 256, 0, s, c3);
      } else {
        if (wn == 2) mle::launch(conv1_wgrad_kernel<2, 2, 4>, c3.items, 256, 0, s, c3);
        else mle::launch(conv1_wgrad_kernel<2, 1, 4>, c3.items, 256, 0, s, c3);
      }
      // The reduce that completes dW and db is part of the probed family.
      if (splits > 1)
        launch_split_reduce(s, static_cast<const float*>(ws), splits, mn, dw, bpart, db ? cout : 0, db,
                            accumulate_db);
    }
    return check_launch("mle_conv2d_wgrad");
  }
  int kchunk;
  const int splits = wgrad_splits(g, kchunk);
  WgradOps op{x, dy, static_cast<float*>(ws), g, cout, cin * kh * kw, n * g.oh * g.ow};
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
      mle::launch(igemm_kernel<WgradOps, true>, grid, NT, 0, s, op, kchunk);
    }
    launch_split_reduce(s, static_cast<const float*>(ws), splits, (size_t)op.M * op.N, dw);
  }
  rc = check_launch("mle_conv2d_wgrad");
  if (rc != MLE_OK || !db) return rc;
  // Other filters: the bias gradient by its own channel sum.
  if (!accumulate_db) {
    rc = mle_fill(stream, db, 0.0f, (size_t)cout);
    if (rc != MLE_OK) return rc;
  }
  return mle_channel_sum(stream, dy, n, cout, (size_t)g.oh * g.ow, cout, db);
}


// ---- a 3 x 3 and a 1 x 1 convolution of one input, in one launch ----------
// (a residual block's first convolution and its skip; both stride 1)

// Arguments of both products for the paired forward (dg = 0) or input
// gradient (dg = 1); false when either is outside the direct kernels.
static bool pair_args(bool dg, int n, int cin, int h, int w, int cout3, int cout1, const float* s3, const float* w3,
                      const float* b3, float* o3, const float* s1, const float* w1, const float* b1, float* o1,
                      int acc, Conv3Args& a, Conv3Args& b, int& wma, int& wmb, bool& halo) {
  ConvGeom g3, g1;
  if (!pair_geoms(n, cin, h, w, cout3, cout1, g3, g1)) return false;
  bool k3a, k3b, hb;
  if (!direct_args(dg, g3, s3, w3, b3, o3, acc, a, k3a, wma, halo) || !k3a) return false;
  if (!direct_args(dg, g1, s1, w1, b1, o1, acc, b, k3b, wmb, hb) || k3b) return false;
  return true;
}

int mle_conv2d_pair_supported(int n, int cin, int h, int w, int cout3, int cout1) {
  Conv3Args a, b;
  int wma, wmb;
  bool halo;
  float* const al = reinterpret_cast<float*>(256);  // any 16-byte aligned address: only the shapes are checked
  const bool fwd = pair_args(false, n, cin, h, w, cout3, cout1, al, al, nullptr, al, al, al, nullptr, al, 0, a, b, wma,
                             wmb, halo);
  const bool dg = pair_args(true, n, cin, h, w, cout3, cout1, al, al, nullptr, al, al, al, nullptr, al, 0, a, b, wma,
                            wmb, halo);
  return fwd && dg ? 1 : 0;
}

int mle_conv2d_pair_fwd(mle_stream stream, const float* x, int n, int cin, int h, int w, const float* w3,
                        const float* b3, float* y3, int cout3, const float* w1, const float* b1, float* y1, int cout1) {
  MLE_CHECK_ARG(x && w3 && y3 && w1 && y1, "mle_conv2d_pair_fwd: null pointer");
  Conv3Args a, b;
  int wma, wmb;
  bool halo;
  if (!pair_args(false, n, cin, h, w, cout3, cout1, x, w3, b3, y3, x, w1, b1, y1, 0, a, b, wma, wmb, halo))
    return set_error(MLE_ERR_UNSUPPORTED, "mle_conv2d_pair_fwd: shape outside the direct kernels");
  hipStream_t s = as_stream(stream);
  const double flop = 2.0 * (double)n * h * w * cin * (9.0 * cout3 + cout1);
  ProbeScope probe("conv_fwd", s, flop, 0.0);
  if (halo) launch_pair_fwd<true>(s, a, wma, b, wmb);
  else launch_pair_fwd<false>(s, a, wma, b, wmb);
  return check_launch("mle_conv2d_pair_fwd");
}

int mle_conv2d_pair_dgrad(mle_stream stream, float* dx, int accumulate, int n, int cin, int h, int w,
                          const float* dy3, const float* w3, int cout3, const float* dy1, const float* w1, int cout1) {
  MLE_CHECK_ARG(dx && dy3 && w3 && dy1 && w1, "mle_conv2d_pair_dgrad: null pointer");
  Conv3Args a, b;
  int wma, wmb;
  bool halo;
  if (!pair_args(true, n, cin, h, w, cout3, cout1, dy3, w3, nullptr, dx, dy1, w1, nullptr, dx, accumulate != 0, a, b,
                 wma, wmb, halo))
    return set_error(MLE_ERR_UNSUPPORTED, "mle_conv2d_pair_dgrad: shape outside the direct kernels");
  hipStream_t s = as_stream(stream);
  const double flop = 2.0 * (double)n * h * w * cin * (9.0 * cout3 + cout1);
  ProbeScope probe("conv_dgrad", s, flop, 0.0);
  auto k = halo ? (wma == 1 ? conv_pair_dgrad_kernel<true, 1> : conv_pair_dgrad_kernel<true, 2>)
                : (wma == 1 ? conv_pair_dgrad_kernel<false, 1> : conv_pair_dgrad_kernel<false, 2>);
  mle::launch(k, (unsigned)a.tiles, 256, 0, s, a, b);
  return check_launch("mle_conv2d_pair_dgrad");
}

}  // extern "C"
