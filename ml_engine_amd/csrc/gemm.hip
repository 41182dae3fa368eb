// mle_gemm: batched / broadcast fp32 GEMM on MFMA with an optional fused
// column sum of op(B) (the Linear bias gradient).  Replaces the 32 x 32
// scalar-FMA tiles and atomicAdd epilogues of bcmm / bcmmABT / bcmmATB / bcmmT
// (Engine/kernels.cu:387-539): every C element is written by exactly one lane,
// so results are deterministic.
#include "gemm_core.hpp"

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

// Global -> registers for one stage.  Tiles are 4096 floats = 1024 float4,
// four per thread.  A_MC == trans_a (A stored K x M); B_KC == trans_b.
template <bool A_MC, bool VEC>
__device__ __forceinline__ void load_a(const GemmArgs& g, const float* A, int m0, int k0, int tid, f32x4 (&r)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = tid + NT * i;
    if (!A_MC) r[i] = ld_guard<VEC>(A, g.lda, m0 + (f >> 3), k0 + (f & 7) * 4, g.M, g.K);
    else r[i] = ld_guard<VEC>(A, g.lda, k0 + (f >> 5), m0 + (f & 31) * 4, g.K, g.M);
  }
}
template <bool B_KC, bool VEC>
__device__ __forceinline__ void load_b(const GemmArgs& g, const float* B, int n0, int k0, int tid, f32x4 (&r)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = tid + NT * i;
    if (B_KC) r[i] = ld_guard<VEC>(B, g.ldb, n0 + (f >> 3), k0 + (f & 7) * 4, g.N, g.K);
    else r[i] = ld_guard<VEC>(B, g.ldb, k0 + (f >> 5), n0 + (f & 31) * 4, g.K, g.N);
  }
}
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

template <int TA, int TB, bool VEC, bool COLSUM>
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
  const int64_t z = blockIdx.z;
  const float* A = g.A + z * g.sa;
  const float* B = g.B + z * g.sb;
  float* C = g.C + z * g.sc;

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};

  const bool do_cs = COLSUM && blockIdx.y == 0;
  float csum = 0.f;
  const int nk = (g.K + BK - 1) / BK;
  f32x4 ra[4], rb[4];
  if (nk > 0) {
    load_a<A_MC, VEC>(g, A, m0, 0, tid, ra);
    load_b<B_KC, VEC>(g, B, n0, 0, tid, rb);
    store_tile<!A_MC>(smem, tid, ra);
    store_tile<B_KC>(smem + 2 * ASZ, tid, rb);
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const float* As = smem + cur * ASZ;
    const float* Bs = smem + 2 * ASZ + cur * BSZ;
    const bool more = kt + 1 < nk;
    if (more) {
      load_a<A_MC, VEC>(g, A, m0, (kt + 1) * BK, tid, ra);
      load_b<B_KC, VEC>(g, B, n0, (kt + 1) * BK, tid, rb);
    }
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
          float* p = C + (int64_t)row * g.ldc + col;
          float v = alpha * acc[i][n][r];
          if (beta != 0.f) v += beta * *p;
          *p = v;
        }
      }
    }

  if (do_cs) {
    // smem is free after the final barrier of the K loop.
    smem[tid] = csum;
    __syncthreads();
    if (tid < 128 && n0 + tid < g.N) g.colsum[n0 + tid] += smem[tid] + smem[tid + 128];
  }
}

template <int TA, int TB>
void launch_t(hipStream_t s, const GemmArgs& g, dim3 grid, bool vec, bool cs) {
  if (vec) {
    if (cs) gemm_kernel<TA, TB, true, true><<<grid, NT, 0, s>>>(g);
    else gemm_kernel<TA, TB, true, false><<<grid, NT, 0, s>>>(g);
  } else {
    if (cs) gemm_kernel<TA, TB, false, true><<<grid, NT, 0, s>>>(g);
    else gemm_kernel<TA, TB, false, false><<<grid, NT, 0, s>>>(g);
  }
}

}  // namespace

extern "C" int mle_gemm(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha,
                        const float* A, int64_t lda, int64_t stride_a, const float* B, int64_t ldb,
                        int64_t stride_b, float beta, float* C, int64_t ldc, int64_t stride_c, int batch,
                        float* colsum) {
  MLE_CHECK_ARG(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "mle_gemm: negative size");
  if (M == 0 || N == 0 || batch == 0) return MLE_OK;
  MLE_CHECK_ARG(C != nullptr && (K == 0 || (A != nullptr && B != nullptr)), "mle_gemm: null operand");
  MLE_CHECK_ARG(ldc >= N, "mle_gemm: ldc %lld < N %d", (long long)ldc, N);
  MLE_CHECK_ARG(lda >= (trans_a ? M : K) && ldb >= (trans_b ? K : N), "mle_gemm: leading dimension too small");
  MLE_CHECK_ARG(colsum == nullptr || batch == 1, "mle_gemm: fused colsum needs batch == 1");
  MLE_CHECK_ARG((N + BN - 1) / BN <= 2147483647 && (M + BM - 1) / BM <= 65535 && batch <= 65535,
                "mle_gemm: grid too large (M %d, batch %d)", M, batch);
  GemmArgs g{A, B, C, colsum, lda, ldb, ldc, stride_a, stride_b, stride_c, M, N, K, alpha, beta};
  const bool vec = (lda % 4 == 0) && (ldb % 4 == 0) && (stride_a % 4 == 0) && (stride_b % 4 == 0) &&
                   aligned16(A) && aligned16(B);
  const bool cs = colsum != nullptr;
  dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM, batch);
  hipStream_t s = as_stream(stream);
  static const char* names[4] = {"gemm_nn", "gemm_nt", "gemm_tn", "gemm_tt"};
  const int which = (trans_a ? 2 : 0) + (trans_b ? 1 : 0);
  const double flop = 2.0 * M * (double)N * K * batch;
  const double bytes = 4.0 * batch * ((double)M * K + (double)K * N + (double)M * N * (beta != 0.f ? 2 : 1));
  ProbeScope probe(names[which], s, flop, bytes);
  switch (which) {
    case 0: launch_t<0, 0>(s, g, grid, vec, cs); break;
    case 1: launch_t<0, 1>(s, g, grid, vec, cs); break;
    case 2: launch_t<1, 0>(s, g, grid, vec, cs); break;
    default: launch_t<1, 1>(s, g, grid, vec, cs); break;
  }
  return check_launch(names[which]);
}
