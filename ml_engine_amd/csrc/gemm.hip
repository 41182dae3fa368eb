// mle_gemm: batched / broadcast fp32 GEMM on MFMA with an optional fused
// column sum of op(B) (the Linear bias gradient).  Replaces the 32 x 32
// scalar-FMA tiles and atomicAdd epilogues of bcmm / bcmmABT / bcmmATB / bcmmT
// (Engine/kernels.cu:387-539): every C element is written by exactly one lane,
// so results are deterministic.
#include "gemm_core.hpp"

#include <algorithm>

using namespace mle;
using namespace gemm;

namespace {

struct GemmArgs {
  const float* A;
  const float* B;
  float* C;
  float* colsum;
  int64_t lda, ldb, ldc, sa, sb, sc;
  int M, N, K;
  float alpha, beta;
  // split-K: blockIdx.z = batch item * splits + split; each split covers
  // kchunk of K and writes its raw tile to part (and its column sums to
  // part_cs); split_reduce_kernel combines them in split order.
  int splits, kchunk;
  float* part;
  float* part_cs;
  const float* bias;  // nullable: C[r, c] += bias[c] after alpha/beta
};

// Load 4 consecutive elements base[r*ld + c .. c+3] with bounds (R rows, Cc cols).
template <bool VEC>
__device__ __forceinline__ f32x4 ld_guard(const float* __restrict__ base, int64_t ld, int r, int c, int R, int Cc) {
  f32x4 v = {0.f, 0.f, 0.f, 0.f};
  if (r < R) {
    const float* p = base + (int64_t)r * ld + c;
    if (VEC && c + 3 < Cc) {
      v = *reinterpret_cast<const f32x4*>(p);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c + j < Cc) v[j] = p[j];
    }
  }
  return v;
}

// Branch-free operand reads through a raw buffer resource: lanes outside the
// matrix use an offset beyond the resource's extent and the hardware range
// check returns zeros (buffer_load_dwordx4 ... offen).  Used when every
// operand extent is below 2 GiB and the contiguous bound is a multiple of 4,
// so a float4 is either wholly inside or wholly outside.
constexpr uint32_t kBufOOB = 0x80000000u;
constexpr int kBufWord3 = 0x00020000;  // gfx9-family raw buffer descriptor word 3

struct BufOperand {
  __amdgpu_buffer_rsrc_t rsrc;
  int64_t ld;
  __device__ BufOperand(const float* base, int64_t ld_, uint32_t bytes)
      : rsrc(__builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)bytes, kBufWord3)), ld(ld_) {}
  __device__ __forceinline__ f32x4 load(int r, int c, int R, int Cc) const {
    const bool ok = (r < R) & (c < Cc);
    const uint32_t off = ok ? (uint32_t)(((int64_t)r * ld + c) * 4) : kBufOOB;
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)off, 0, 0));
  }
};

// Global -> registers for one stage.  Tiles are 4096 floats = 1024 float4,
// four per thread.  A_MC == trans_a (A stored K x M); B_KC == trans_b.
// `kend` bounds K for this workgroup's split.
template <bool A_MC, bool VEC>
__device__ __forceinline__ void load_a(const GemmArgs& g, const float* A, int m0, int k0, int kend, int tid,
                                       f32x4 (&r)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = tid + NT * i;
    if (!A_MC) r[i] = ld_guard<VEC>(A, g.lda, m0 + (f >> 3), k0 + (f & 7) * 4, g.M, kend);
    else r[i] = ld_guard<VEC>(A, g.lda, k0 + (f >> 5), m0 + (f & 31) * 4, kend, g.M);
  }
}
template <bool B_KC, bool VEC>
__device__ __forceinline__ void load_b(const GemmArgs& g, const float* B, int n0, int k0, int kend, int tid,
                                       f32x4 (&r)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = tid + NT * i;
    if (B_KC) r[i] = ld_guard<VEC>(B, g.ldb, n0 + (f >> 3), k0 + (f & 7) * 4, g.N, kend);
    else r[i] = ld_guard<VEC>(B, g.ldb, k0 + (f >> 5), n0 + (f & 31) * 4, kend, g.N);
  }
}
template <bool A_MC>
__device__ __forceinline__ void load_a_buf(const GemmArgs& g, const BufOperand& A, int m0, int k0, int kend, int tid,
                                           f32x4 (&r)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = tid + NT * i;
    if (!A_MC) r[i] = A.load(m0 + (f >> 3), k0 + (f & 7) * 4, g.M, kend);
    else r[i] = A.load(k0 + (f >> 5), m0 + (f & 31) * 4, kend, g.M);
  }
}
template <bool B_KC>
__device__ __forceinline__ void load_b_buf(const GemmArgs& g, const BufOperand& B, int n0, int k0, int kend, int tid,
                                           f32x4 (&r)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = tid + NT * i;
    if (B_KC) r[i] = B.load(n0 + (f >> 3), k0 + (f & 7) * 4, g.N, kend);
    else r[i] = B.load(k0 + (f >> 5), n0 + (f & 31) * 4, kend, g.N);
  }
}

// Row stride of the epilogue staging tile (32 x 64 per wave, 16-byte aligned rows).
constexpr int EPI_LD = 68;

// Registers -> LDS (same element mapping as the loads).
template <bool KC>
__device__ __forceinline__ void store_tile(float* S, int tid, const f32x4 (&r)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = tid + NT * i;
    if (KC) *reinterpret_cast<f32x4*>(S + (f >> 3) * LDK + (f & 7) * 4) = r[i];
    else *reinterpret_cast<f32x4*>(S + (f >> 5) * LDMN + (f & 31) * 4) = r[i];
  }
}

// VEC: 0 = guarded scalar loads, 1 = guarded float4 loads, 2 = buffer loads.
template <int TA, int TB, int VEC, bool COLSUM>
__global__ __launch_bounds__(NT, 2) void gemm_kernel(GemmArgs g) {
  constexpr bool A_MC = TA != 0;
  constexpr bool B_KC = TB != 0;
  constexpr int ASZ = a_tile_floats<A_MC>();
  constexpr int BSZ = b_tile_floats<B_KC>();
  __shared__ __attribute__((aligned(16))) float smem[2 * (ASZ + BSZ)];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, q = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int64_t z = blockIdx.z / g.splits;
  const int split = blockIdx.z % g.splits;
  const float* A = g.A + z * g.sa;
  const float* B = g.B + z * g.sb;
  float* C = g.C + z * g.sc;
  const int kbeg = split * g.kchunk;
  const int kend = min(g.K, kbeg + g.kchunk);
  const uint32_t a_bytes = (uint32_t)(((int64_t)((A_MC ? g.K : g.M) - 1) * g.lda + (A_MC ? g.M : g.K)) * 4);
  const uint32_t b_bytes = (uint32_t)(((int64_t)((B_KC ? g.N : g.K) - 1) * g.ldb + (B_KC ? g.K : g.N)) * 4);
  const BufOperand Ab(A, g.lda, a_bytes), Bb(B, g.ldb, b_bytes);
  auto load_stage = [&](int k0, f32x4(&ra_)[4], f32x4(&rb_)[4]) {
    if (VEC == 2) {
      load_a_buf<A_MC>(g, Ab, m0, k0, kend, tid, ra_);
      load_b_buf<B_KC>(g, Bb, n0, k0, kend, tid, rb_);
    } else {
      load_a<A_MC, VEC == 1>(g, A, m0, k0, kend, tid, ra_);
      load_b<B_KC, VEC == 1>(g, B, n0, k0, kend, tid, rb_);
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};

  const bool do_cs = COLSUM && blockIdx.y == 0;
  float csum = 0.f;
  const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
  f32x4 ra[4], rb[4];
  if (nk > 0) {
    load_stage(kbeg, ra, rb);
    store_tile<!A_MC>(smem, tid, ra);
    store_tile<B_KC>(smem + 2 * ASZ, tid, rb);
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const float* As = smem + cur * ASZ;
    const float* Bs = smem + 2 * ASZ + cur * BSZ;
    const bool more = kt + 1 < nk;
    if (more) load_stage(kbeg + (kt + 1) * BK, ra, rb);
    mma_stage<A_MC, B_KC>(As, Bs, acc, wm, wn, lr, q);
    if (do_cs) {
      const int c = tid & 127, h = tid >> 7;
#pragma unroll
      for (int k = 0; k < 16; ++k) csum += B_KC ? Bs[c * LDK + h * 16 + k] : Bs[(h * 16 + k) * LDMN + c];
    }
    if (more) {
      store_tile<!A_MC>(smem + (cur ^ 1) * ASZ, tid, ra);
      store_tile<B_KC>(smem + 2 * ASZ + (cur ^ 1) * BSZ, tid, rb);
    }
    __syncthreads();
  }

  const float alpha = g.alpha, beta = g.beta;
  const bool split_mode = g.splits > 1;
  float* P = split_mode ? g.part + (int64_t)blockIdx.z * g.M * g.N : nullptr;
  if (VEC == 2 && (g.N & 3) == 0 && (g.ldc & 3) == 0 && ((reinterpret_cast<uintptr_t>(C) & 15) == 0)) {
    // Stage each wave's 64 x 64 block through LDS, 32 rows at a time, and
    // write rows back with 16-byte stores (a wave covers 4 full 256-byte row
    // segments per instruction instead of 16 x 64-byte pieces).
    float* T = smem + wave * (32 * EPI_LD);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
#pragma unroll
      for (int ii = 0; ii < 2; ++ii) {
        const int i = half * 2 + ii;
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r) T[(ii * 16 + 4 * q + r) * EPI_LD + n * 16 + lr] = acc[i][n][r];
      }
      __syncthreads();
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int rr = it * 4 + (lane >> 4);  // 0..31
        const int cc = (lane & 15) * 4;       // 0..60
        const int row = m0 + wm * 64 + half * 32 + rr;
        const int col = n0 + wn * 64 + cc;
        if (row < g.M && col < g.N) {
          f32x4 v = *reinterpret_cast<const f32x4*>(T + rr * EPI_LD + cc);
          if (split_mode) {
            *reinterpret_cast<f32x4*>(P + (int64_t)row * g.N + col) = v;
          } else {
            float* p = C + (int64_t)row * g.ldc + col;
            v = alpha * v;
            if (beta != 0.f) v += beta * *reinterpret_cast<const f32x4*>(p);
            if (g.bias) v += *reinterpret_cast<const f32x4*>(g.bias + col);
            *reinterpret_cast<f32x4*>(p) = v;
          }
        }
      }
      __syncthreads();
    }
  } else {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int col = n0 + acc_col(wn, n, lr);
      if (col >= g.N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + acc_row(wm, i, q, r);
        if (row < g.M) {
          if (split_mode) {
            P[(int64_t)row * g.N + col] = acc[i][n][r];
          } else {
            float* p = C + (int64_t)row * g.ldc + col;
            float v = alpha * acc[i][n][r];
            if (beta != 0.f) v += beta * *p;
            if (g.bias) v += g.bias[col];
            *p = v;
          }
        }
      }
    }
  }

  if (do_cs) {
    // smem is free after the final barrier of the K loop.
    smem[tid] = csum;
    __syncthreads();
    if (tid < 128 && n0 + tid < g.N) {
      const float cs = smem[tid] + smem[tid + 128];
      if (split_mode) g.part_cs[(int64_t)split * g.N + n0 + tid] = cs;
      else g.colsum[n0 + tid] += cs;
    }
  }
}

// C = alpha * sum_s part[s] + beta * C and colsum += sum_s part_cs[s], in split
// order.  Grid: x over column groups of W (4 with VEC, else 1) columns, y over
// rows (looping when M > 65535), z over batch items -- no integer division.
// Loads of four splits are issued together; the additions keep split order.
template <bool VEC>
__global__ __launch_bounds__(256) void split_reduce_kernel(GemmArgs g) {
  constexpr int W = VEC ? 4 : 1;
  const int col = (blockIdx.x * 256 + threadIdx.x) * W;
  const int64_t mn = (int64_t)g.M * g.N;
  const int64_t b = blockIdx.z;
  if (col < g.N) {
    for (int row = blockIdx.y; row < g.M; row += gridDim.y) {
      const float* p = g.part + b * g.splits * mn + (int64_t)row * g.N + col;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      int sp = 0;
      for (; sp + 4 <= g.splits; sp += 4) {
        f32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (VEC) v[u] = *reinterpret_cast<const f32x4*>(p + (sp + u) * mn);
          else v[u][0] = p[(sp + u) * mn];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) acc += v[u];
      }
      for (; sp < g.splits; ++sp) {
        if (VEC) acc += *reinterpret_cast<const f32x4*>(p + sp * mn);
        else acc[0] += p[sp * mn];
      }
      float* c = g.C + b * g.sc + (int64_t)row * g.ldc + col;
      if (VEC) {
        f32x4 v = g.alpha * acc;
        if (g.beta != 0.f) v += g.beta * *reinterpret_cast<const f32x4*>(c);
        if (g.bias) v += *reinterpret_cast<const f32x4*>(g.bias + col);
        *reinterpret_cast<f32x4*>(c) = v;
      } else {
        float v = g.alpha * acc[0];
        if (g.beta != 0.f) v += g.beta * *c;
        if (g.bias) v += g.bias[col];
        *c = v;
      }
    }
    if (g.colsum && blockIdx.y == 0 && b == 0) {
#pragma unroll
      for (int j = 0; j < W; ++j) {
        float acc = 0.f;
        for (int sp = 0; sp < g.splits; ++sp) acc += g.part_cs[(int64_t)sp * g.N + col + j];
        g.colsum[col + j] += acc;
      }
    }
  }
}

// Split count: a function of the shape only.  Splits are used when the tile
// grid leaves most of the 256 CUs idle and K is long enough to share.
int choose_splits(int M, int N, int K, int batch, int& kchunk) {
  kchunk = K;
  const long long tiles = (long long)((M + BM - 1) / BM) * ((N + BN - 1) / BN) * batch;
  // Measured on MI355X: with ~256 tiles a split only pays off for long K.
  if (tiles >= 384 || (tiles >= 128 && K < 4096)) return 1;
  int s = (int)((768 + tiles - 1) / tiles);
  const int smax = K / 256;
  if (s > smax) s = smax;
  if (s < 2) return 1;
  kchunk = (K + s - 1) / s;
  kchunk = ((kchunk + BK - 1) / BK) * BK;
  s = (K + kchunk - 1) / kchunk;
  if ((long long)s * batch > 65535) return 1;
  return s;
}

template <int TA, int TB>
void launch_t(hipStream_t s, const GemmArgs& g, dim3 grid, int vec, bool cs) {
  if (vec == 2) {
    if (cs) gemm_kernel<TA, TB, 2, true><<<grid, NT, 0, s>>>(g);
    else gemm_kernel<TA, TB, 2, false><<<grid, NT, 0, s>>>(g);
  } else if (vec == 1) {
    if (cs) gemm_kernel<TA, TB, 1, true><<<grid, NT, 0, s>>>(g);
    else gemm_kernel<TA, TB, 1, false><<<grid, NT, 0, s>>>(g);
  } else {
    if (cs) gemm_kernel<TA, TB, 0, true><<<grid, NT, 0, s>>>(g);
    else gemm_kernel<TA, TB, 0, false><<<grid, NT, 0, s>>>(g);
  }
}

// Bytes spanned by one batch item of an operand stored rows x cols with leading dimension ld.
double extent_bytes(int rows, int cols, int64_t ld) { return ((double)(rows - 1) * (double)ld + cols) * 4.0; }

}  // namespace

static int gemm_impl(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A,
                     int64_t lda, int64_t stride_a, const float* B, int64_t ldb, int64_t stride_b, float beta, float* C,
                     int64_t ldc, int64_t stride_c, int batch, float* colsum, const float* bias, void* ws,
                     size_t ws_bytes) {
  MLE_CHECK_ARG(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "mle_gemm: negative size");
  if (M == 0 || N == 0 || batch == 0) return MLE_OK;
  MLE_CHECK_ARG(C != nullptr && (K == 0 || (A != nullptr && B != nullptr)), "mle_gemm: null operand");
  MLE_CHECK_ARG(ldc >= N, "mle_gemm: ldc %lld < N %d", (long long)ldc, N);
  MLE_CHECK_ARG(lda >= (trans_a ? M : K) && ldb >= (trans_b ? K : N), "mle_gemm: leading dimension too small");
  MLE_CHECK_ARG(colsum == nullptr || batch == 1, "mle_gemm: fused colsum needs batch == 1");
  MLE_CHECK_ARG((M + BM - 1) / BM <= 65535 && batch <= 65535, "mle_gemm: grid too large (M %d, batch %d)", M, batch);
  GemmArgs g{A, B, C, colsum, lda, ldb, ldc, stride_a, stride_b, stride_c, M, N, K, alpha, beta, 1, K, nullptr, nullptr,
             bias};
  int kchunk = K;
  const int splits = ws ? choose_splits(M, N, K, batch, kchunk) : 1;
  if (splits > 1) {
    const size_t need = mle_gemm_ws_bytes(M, N, K, batch);
    if (ws_bytes >= need) {
      g.splits = splits;
      g.kchunk = kchunk;
      g.part = static_cast<float*>(ws);
      g.part_cs = g.part + (size_t)splits * batch * M * N;
    }
  }
  const bool v4 = (lda % 4 == 0) && (ldb % 4 == 0) && (stride_a % 4 == 0) && (stride_b % 4 == 0) &&
                  aligned16(A) && aligned16(B);
  // Buffer loads need the contiguous bound of each operand to be a multiple of
  // 4 and every extent addressable with a 31-bit byte offset.
  const int a_rows = trans_a ? K : M, a_cols = trans_a ? M : K;
  const int b_rows = trans_b ? N : K, b_cols = trans_b ? K : N;
  const bool buf = v4 && a_cols % 4 == 0 && b_cols % 4 == 0 && K > 0 &&
                   extent_bytes(a_rows, a_cols, lda) < 2147483648.0 - 64 &&
                   extent_bytes(b_rows, b_cols, ldb) < 2147483648.0 - 64;
  const int vec = buf ? 2 : (v4 ? 1 : 0);
  const bool cs = colsum != nullptr;
  dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM, batch * g.splits);
  hipStream_t s = as_stream(stream);
  static const char* names[4] = {"gemm_nn", "gemm_nt", "gemm_tn", "gemm_tt"};
  const int which = (trans_a ? 2 : 0) + (trans_b ? 1 : 0);
  const double flop = 2.0 * M * (double)N * K * batch;
  const double bytes = 4.0 * batch * ((double)M * K + (double)K * N + (double)M * N * (beta != 0.f ? 2 : 1));
  {
    ProbeScope probe(names[which], s, flop, bytes);
    switch (which) {
      case 0: launch_t<0, 0>(s, g, grid, vec, cs); break;
      case 1: launch_t<0, 1>(s, g, grid, vec, cs); break;
      case 2: launch_t<1, 0>(s, g, grid, vec, cs); break;
      default: launch_t<1, 1>(s, g, grid, vec, cs); break;
    }
    if (g.splits > 1) {
      const bool rv = N % 4 == 0 && ldc % 4 == 0 && stride_c % 4 == 0 && aligned16(C) && aligned16(g.part) &&
                      (!bias || aligned16(bias));
      const int w = rv ? 4 : 1;
      dim3 rgrid((unsigned)((N / w + 255) / 256), (unsigned)std::min(M, 65535), (unsigned)batch);
      if (rv) split_reduce_kernel<true><<<rgrid, 256, 0, s>>>(g);
      else split_reduce_kernel<false><<<rgrid, 256, 0, s>>>(g);
    }
  }
  return check_launch(names[which]);
}

extern "C" {

size_t mle_gemm_ws_bytes(int M, int N, int K, int batch) {
  int kchunk;
  const int splits = choose_splits(M, N, K, batch, kchunk);
  if (splits <= 1) return 0;
  return ((size_t)splits * batch * M * N + (size_t)splits * N) * sizeof(float);
}

int mle_gemm(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A,
             int64_t lda, int64_t stride_a, const float* B, int64_t ldb, int64_t stride_b, float beta, float* C,
             int64_t ldc, int64_t stride_c, int batch, float* colsum) {
  return gemm_impl(stream, trans_a, trans_b, M, N, K, alpha, A, lda, stride_a, B, ldb, stride_b, beta, C, ldc,
                   stride_c, batch, colsum, nullptr, nullptr, 0);
}

int mle_gemm_ex(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A,
                int64_t lda, int64_t stride_a, const float* B, int64_t ldb, int64_t stride_b, float beta, float* C,
                int64_t ldc, int64_t stride_c, int batch, float* colsum, const float* bias, void* ws,
                size_t ws_bytes) {
  return gemm_impl(stream, trans_a, trans_b, M, N, K, alpha, A, lda, stride_a, B, ldb, stride_b, beta, C, ldc,
                   stride_c, batch, colsum, bias, ws, ws_bytes);
}

}  // extern "C"
