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

// Global -> registers for one stage.  A tile is TM x BK (TM/32 float4 per
// thread), a B tile BK x TN.  A_MC == trans_a (A stored K x M); B_KC ==
// trans_b.  `kend` bounds K for this workgroup's split.  k-contiguous tiles
// give each row 8 float4 (BK = 32); m/n-contiguous ones TM/4 per k row.
template <bool MC, int T>
__device__ __forceinline__ void tile_coord(int f, int& r, int& c) {
  if (!MC) {  // [T][BK]: r = row along M/N, c = k
    r = f >> 3;
    c = (f & 7) * 4;
  } else {  // [BK][T]: r = k, c = along M/N
    r = f / (T / 4);
    c = (f % (T / 4)) * 4;
  }
}

template <bool A_MC, int VEC, int TM>
__device__ __forceinline__ void load_a(const GemmArgs& g, const float* A, const BufOperand& Ab, int m0, int k0,
                                       int kend, int tid, f32x4 (&r)[TM / 32]) {
#pragma unroll
  for (int i = 0; i < TM / 32; ++i) {
    int a, b;
    tile_coord<A_MC, TM>(tid + NT * i, a, b);
    if (!A_MC) r[i] = VEC == 2 ? Ab.load(m0 + a, k0 + b, g.M, kend) : ld_guard<VEC == 1>(A, g.lda, m0 + a, k0 + b, g.M, kend);
    else r[i] = VEC == 2 ? Ab.load(k0 + a, m0 + b, kend, g.M) : ld_guard<VEC == 1>(A, g.lda, k0 + a, m0 + b, kend, g.M);
  }
}
template <bool B_KC, int VEC, int TN>
__device__ __forceinline__ void load_b(const GemmArgs& g, const float* B, const BufOperand& Bb, int n0, int k0,
                                       int kend, int tid, f32x4 (&r)[TN / 32]) {
#pragma unroll
  for (int i = 0; i < TN / 32; ++i) {
    int a, b;
    tile_coord<!B_KC, TN>(tid + NT * i, a, b);
    if (B_KC) r[i] = VEC == 2 ? Bb.load(n0 + a, k0 + b, g.N, kend) : ld_guard<VEC == 1>(B, g.ldb, n0 + a, k0 + b, g.N, kend);
    else r[i] = VEC == 2 ? Bb.load(k0 + a, n0 + b, kend, g.N) : ld_guard<VEC == 1>(B, g.ldb, k0 + a, n0 + b, kend, g.N);
  }
}

// Registers -> LDS (same element mapping as the loads).  KC: k-contiguous.
template <bool KC, int T>
__device__ __forceinline__ void store_tile(float* S, int tid, const f32x4 (&r)[T / 32]) {
#pragma unroll
  for (int i = 0; i < T / 32; ++i) {
    int a, b;
    tile_coord<!KC, T>(tid + NT * i, a, b);
    *reinterpret_cast<f32x4*>(S + a * (KC ? LDK : T + PAD) + b) = r[i];
  }
}

// VEC: 0 = guarded scalar loads, 1 = guarded float4 loads, 2 = buffer loads.
// WM x WN MFMA blocks per wave: the workgroup tile is (32 WM) x (32 WN).
template <int TA, int TB, int VEC, bool COLSUM, int WM, int WN>
__global__ __launch_bounds__(NT, 2) void gemm_kernel(GemmArgs g) {
  constexpr bool A_MC = TA != 0;
  constexpr bool B_KC = TB != 0;
  constexpr int TM = 32 * WM, TN = 32 * WN;
  constexpr int ASZ = a_tile_floats<A_MC, TM>();
  constexpr int BSZ = b_tile_floats<B_KC, TN>();
  constexpr int EPI_LD = 16 * WN + 4;  // epilogue staging row stride (16-byte aligned rows)
  static_assert(4 * 32 * EPI_LD <= 2 * (ASZ + BSZ), "epilogue staging does not fit");
  __shared__ __attribute__((aligned(16))) float smem[2 * (ASZ + BSZ)];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, q = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.y * TM, n0 = blockIdx.x * TN;
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

  f32x4 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int n = 0; n < WN; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};

  const bool do_cs = COLSUM && blockIdx.y == 0;
  constexpr int CS_T = NT / TN;  // threads per column of the column sum
  float csum = 0.f;
  const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
  f32x4 ra[TM / 32], rb[TN / 32];
  if (nk > 0) {
    load_a<A_MC, VEC, TM>(g, A, Ab, m0, kbeg, kend, tid, ra);
    load_b<B_KC, VEC, TN>(g, B, Bb, n0, kbeg, kend, tid, rb);
    store_tile<!A_MC, TM>(smem, tid, ra);
    store_tile<B_KC, TN>(smem + 2 * ASZ, tid, rb);
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const float* As = smem + cur * ASZ;
    const float* Bs = smem + 2 * ASZ + cur * BSZ;
    const bool more = kt + 1 < nk;
    if (more) {
      load_a<A_MC, VEC, TM>(g, A, Ab, m0, kbeg + (kt + 1) * BK, kend, tid, ra);
      load_b<B_KC, VEC, TN>(g, B, Bb, n0, kbeg + (kt + 1) * BK, kend, tid, rb);
    }
    mma_stage<A_MC, B_KC, WM, WN>(As, Bs, acc, wm, wn, lr, q);
    if (do_cs) {
      const int c = tid % TN, h = tid / TN;
#pragma unroll
      for (int k = 0; k < BK / CS_T; ++k) {
        const int kk = h * (BK / CS_T) + k;
        csum += B_KC ? Bs[c * LDK + kk] : Bs[kk * (TN + PAD) + c];
      }
    }
    if (more) {
      store_tile<!A_MC, TM>(smem + (cur ^ 1) * ASZ, tid, ra);
      store_tile<B_KC, TN>(smem + 2 * ASZ + (cur ^ 1) * BSZ, tid, rb);
    }
    __syncthreads();
  }

  const float alpha = g.alpha, beta = g.beta;
  const bool split_mode = g.splits > 1;
  float* P = split_mode ? g.part + (int64_t)blockIdx.z * g.M * g.N : nullptr;
  if (VEC == 2 && (g.N & 3) == 0 && (g.ldc & 3) == 0 && ((reinterpret_cast<uintptr_t>(C) & 15) == 0)) {
    // Stage each wave's (16 WM) x (16 WN) block through LDS, 32 rows at a
    // time, and write rows back with 16-byte stores.
    constexpr int F4_ROW = 4 * WN;          // float4 per staged row
    constexpr int ROWS_PASS = 64 / F4_ROW;  // rows a wave writes per pass
    float* T = smem + wave * (32 * EPI_LD);
#pragma unroll
    for (int half = 0; half < WM / 2; ++half) {
#pragma unroll
      for (int ii = 0; ii < 2; ++ii) {
        const int i = half * 2 + ii;
#pragma unroll
        for (int n = 0; n < WN; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r) T[(ii * 16 + 4 * q + r) * EPI_LD + n * 16 + lr] = acc[i][n][r];
      }
      __syncthreads();
#pragma unroll
      for (int it = 0; it < 32 / ROWS_PASS; ++it) {
        const int rr = it * ROWS_PASS + lane / F4_ROW;
        const int cc = (lane % F4_ROW) * 4;
        const int row = m0 + wm * 16 * WM + half * 32 + rr;
        const int col = n0 + wn * 16 * WN + cc;
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
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int n = 0; n < WN; ++n) {
        const int col = n0 + acc_col<WN>(wn, n, lr);
        if (col >= g.N) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + acc_row<WM>(wm, i, q, r);
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
    if (tid < TN && n0 + tid < g.N) {
      float cs = 0.f;
#pragma unroll
      for (int h = 0; h < CS_T; ++h) cs += smem[tid + h * TN];
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

// Workgroup tile: 128 x 128 unless a side is <= 64 (the 64-wide variants waste
// nothing there) or the 128 x 128 grid would leave CUs idle and K is too short
// for split-K to fill them (half-width tiles double the workgroups; measured
// on MI355X, for K >= 4096 full tiles plus split-K are faster).  A function of
// the shape only, as mle_gemm_ws_bytes needs.
struct Tile {
  int wm, wn;  // MFMA blocks per wave along M / N
  int tm() const { return 32 * wm; }
  int tn() const { return 32 * wn; }
};

Tile choose_tile(int M, int N, int K, int batch) {
  (void)K;
  if (M <= 64 && N <= 64) return {2, 2};
  if (N <= 64) return {4, 2};
  if (M <= 64) return {2, 4};
  const long long t128 = (long long)((M + 127) / 128) * ((N + 127) / 128) * batch;
  if (t128 >= 512 || K >= 4096) return {4, 4};
  return N >= M ? Tile{2, 4} : Tile{4, 2};
}

// Split count: a function of the shape only.  Splits are used when the tile
// grid leaves most of the 256 CUs idle and K is long enough to share.
int choose_splits(int M, int N, int K, int batch, int& kchunk) {
  kchunk = K;
  const Tile t = choose_tile(M, N, K, batch);
  const long long tiles = (long long)((M + t.tm() - 1) / t.tm()) * ((N + t.tn() - 1) / t.tn()) * batch;
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

template <int TA, int TB, int WM, int WN>
void launch_t(hipStream_t s, const GemmArgs& g, dim3 grid, int vec, bool cs) {
  if (vec == 2) {
    if (cs) gemm_kernel<TA, TB, 2, true, WM, WN><<<grid, NT, 0, s>>>(g);
    else gemm_kernel<TA, TB, 2, false, WM, WN><<<grid, NT, 0, s>>>(g);
  } else if (vec == 1) {
    if (cs) gemm_kernel<TA, TB, 1, true, WM, WN><<<grid, NT, 0, s>>>(g);
    else gemm_kernel<TA, TB, 1, false, WM, WN><<<grid, NT, 0, s>>>(g);
  } else {
    if (cs) gemm_kernel<TA, TB, 0, true, WM, WN><<<grid, NT, 0, s>>>(g);
    else gemm_kernel<TA, TB, 0, false, WM, WN><<<grid, NT, 0, s>>>(g);
  }
}

template <int TA, int TB>
void launch_tile(hipStream_t s, const GemmArgs& g, Tile t, dim3 grid, int vec, bool cs) {
  if (t.wm == 4 && t.wn == 4) launch_t<TA, TB, 4, 4>(s, g, grid, vec, cs);
  else if (t.wm == 4) launch_t<TA, TB, 4, 2>(s, g, grid, vec, cs);
  else if (t.wn == 4) launch_t<TA, TB, 2, 4>(s, g, grid, vec, cs);
  else launch_t<TA, TB, 2, 2>(s, g, grid, vec, cs);
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
  const Tile tile = choose_tile(M, N, K, batch);
  MLE_CHECK_ARG((M + tile.tm() - 1) / tile.tm() <= 65535 && batch <= 65535, "mle_gemm: grid too large (M %d, batch %d)",
                M, batch);
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
  dim3 grid((N + tile.tn() - 1) / tile.tn(), (M + tile.tm() - 1) / tile.tm(), batch * g.splits);
  hipStream_t s = as_stream(stream);
  static const char* names[4] = {"gemm_nn", "gemm_nt", "gemm_tn", "gemm_tt"};
  const int which = (trans_a ? 2 : 0) + (trans_b ? 1 : 0);
  const double flop = 2.0 * M * (double)N * K * batch;
  const double bytes = 4.0 * batch * ((double)M * K + (double)K * N + (double)M * N * (beta != 0.f ? 2 : 1));
  {
    ProbeScope probe(names[which], s, flop, bytes);
    switch (which) {
      case 0: launch_tile<0, 0>(s, g, tile, grid, vec, cs); break;
      case 1: launch_tile<0, 1>(s, g, tile, grid, vec, cs); break;
      case 2: launch_tile<1, 0>(s, g, tile, grid, vec, cs); break;
      default: launch_tile<1, 1>(s, g, tile, grid, vec, cs); break;
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
