// mle_gemm: batched / broadcast fp32 GEMM on MFMA with an optional fused
// column sum of op(B) (the Linear bias gradient).  Replaces the 32 x 32
// scalar-FMA tiles and atomicAdd epilogues of bcmm / bcmmABT / bcmmATB / bcmmT
// (Engine/kernels.cu:387-539): every C element is written by exactly one lane,
// so results are deterministic.
#include "activation.hpp"
#include "gemm_core.hpp"

#include <float.h>

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
  // Two-level batch: item z = zo * inner + zi sits at zo * s + zi * s2 of
  // each operand (inner == 1: one stride).  Lets per-head products address
  // the heads of a [batch, seq, heads * dim] tensor in place.
  int inner;
  int64_t sa2, sb2, sc2;
  // Per batch item bias and column-sum strides (0: shared).
  int64_t sbias, scs;
  // Sum of products: when grouped, split s multiplies A + s*gsa by B + s*gsb
  // over the whole K (the splits are the terms), and the reduce adds them in
  // term order.
  int grouped;
  int64_t gsa, gsb;
  // Sum of products folded into K (register-direct kernel, one split): stage
  // kt of the K loop reads term kt / (K / KD) of A + t*gsa and B + t*gsb.
  int kterms;
  // Row statistics of C (persistent kernel): for row r and 64-column block b,
  // rowpart[r * rp_ld + 2 b] = max over the block, [.. + 1] = sum of
  // exp(C - max).  nullptr: none.
  float* rowpart;
  int64_t rp_ld;
  // Activation epilogues (persistent kernel, C's layout): forward writes
  // act_y = act(C); backward writes act_dx (+)= C * act'(act_x).
  float* act_y;
  const float* act_x;
  float* act_dx;
  int act_acc;
  // 1 + an activation kind: the split reduce also writes act_y = act(C) in
  // C's layout (0: not).
  int act_red;
  // Column sums: 0 adds them into colsum (the default), 1 assigns (colsum is
  // logically zero).
  int cs_assign;
  // 1 + an activation kind: the small-product kernels (simple, K-split) also
  // write act_dx (+)= act'(act_x) * C in C's layout, act_acc choosing add or
  // assign (0: not).
  int act_bwd;
};

// colsum[i] (+)= v as GemmArgs::cs_assign says.
__device__ __forceinline__ void put_colsum(const GemmArgs& g, int64_t i, float v) {
  g.colsum[i] = g.cs_assign ? v : g.colsum[i] + v;
}

// Epilogue modes of the persistent kernel.
constexpr int kEpiPlain = 0, kEpiRowstats = 1, kEpiActFwd = 2, kEpiActBwd = 3;

__device__ __forceinline__ int64_t batch_off(int64_t z, const GemmArgs& g, int64_t s, int64_t s2) {
  if (g.inner == 1) return z * s;
  return (z / g.inner) * s + (z % g.inner) * s2;
}

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

// Global -> registers for one stage.  A tile is TM x KD (TM*KD/1024 float4
// per thread), a B tile KD x TN.  A_MC == trans_a (A stored K x M); B_KC ==
// trans_b.  `kend` bounds K for this workgroup's split.  k-contiguous tiles
// give each row KD/4 float4; m/n-contiguous ones T/4 per k row.
template <bool MC, int T, int KD>
__device__ __forceinline__ void tile_coord(int f, int& r, int& c) {
  if (!MC) {  // [T][KD]: r = row along M/N, c = k
    r = f / (KD / 4);
    c = (f % (KD / 4)) * 4;
  } else {  // [KD][T]: r = k, c = along M/N
    r = f / (T / 4);
    c = (f % (T / 4)) * 4;
  }
}

template <bool A_MC, int VEC, int TM, int KD>
__device__ __forceinline__ void load_a(const GemmArgs& g, const float* A, const BufOperand& Ab, int m0, int k0,
                                       int kend, int tid, f32x4 (&r)[TM * KD / 1024]) {
#pragma unroll
  for (int i = 0; i < TM * KD / 1024; ++i) {
    int a, b;
    tile_coord<A_MC, TM, KD>(tid + NT * i, a, b);
    if (!A_MC) r[i] = VEC == 2 ? Ab.load(m0 + a, k0 + b, g.M, kend) : ld_guard<VEC == 1>(A, g.lda, m0 + a, k0 + b, g.M, kend);
    else r[i] = VEC == 2 ? Ab.load(k0 + a, m0 + b, kend, g.M) : ld_guard<VEC == 1>(A, g.lda, k0 + a, m0 + b, kend, g.M);
  }
}
template <bool B_KC, int VEC, int TN, int KD>
__device__ __forceinline__ void load_b(const GemmArgs& g, const float* B, const BufOperand& Bb, int n0, int k0,
                                       int kend, int tid, f32x4 (&r)[TN * KD / 1024]) {
#pragma unroll
  for (int i = 0; i < TN * KD / 1024; ++i) {
    int a, b;
    tile_coord<!B_KC, TN, KD>(tid + NT * i, a, b);
    if (B_KC) r[i] = VEC == 2 ? Bb.load(n0 + a, k0 + b, g.N, kend) : ld_guard<VEC == 1>(B, g.ldb, n0 + a, k0 + b, g.N, kend);
    else r[i] = VEC == 2 ? Bb.load(k0 + a, n0 + b, kend, g.N) : ld_guard<VEC == 1>(B, g.ldb, k0 + a, n0 + b, kend, g.N);
  }
}

// Registers -> LDS (same element mapping as the loads).  KC: k-contiguous.
template <bool KC, int T, int KD>
__device__ __forceinline__ void store_tile(float* S, int tid, const f32x4 (&r)[T * KD / 1024]) {
#pragma unroll
  for (int i = 0; i < T * KD / 1024; ++i) {
    int a, b;
    tile_coord<!KC, T, KD>(tid + NT * i, a, b);
    *reinterpret_cast<f32x4*>(S + a * (KC ? KD + PAD : T + PAD) + b) = r[i];
  }
}

// Tile order.  Workgroups are handed to the 8 XCDs round-robin (linear id
// L on XCD L % 8), and each XCD has its own L2.  XCD x therefore gets the
// contiguous logical range [x*T/8, (x+1)*T/8) of the T tiles, walked in
// groups of 8 tile-rows with the columns inside a group, so the workgroups
// resident on one XCD share a few A row-panels and B column-panels.  A
// bijection on [0, T): every tile is still computed by exactly one workgroup.
constexpr int kXcds = 8, kGroupRows = 8;
__device__ __forceinline__ void tile_of(int gx, int gy, int& tm, int& tn) {
  const int T = gx * gy;
  const int L = blockIdx.x + gx * blockIdx.y;
  const int q = T / kXcds, r = T % kXcds, x = L % kXcds;
  const int logical = x * q + min(x, r) + L / kXcds;
  const int per_group = kGroupRows * gx;
  const int first_m = (logical / per_group) * kGroupRows;
  const int rows = min(gy - first_m, kGroupRows);
  const int in_group = logical % per_group;
  tm = first_m + in_group % rows;
  tn = in_group / rows;
}

// VEC: 0 = guarded scalar loads, 1 = guarded float4 loads, 2 = buffer loads.
// WM x WN MFMA blocks per wave: the workgroup tile is (32 WM) x (32 WN).
template <int TA, int TB, int VEC, bool COLSUM, int WM, int WN, int KD>
__global__ __launch_bounds__(NT, KD == 16 ? 3 : 2) void gemm_kernel(GemmArgs g) {
  constexpr bool A_MC = TA != 0;
  constexpr bool B_KC = TB != 0;
  constexpr int TM = 32 * WM, TN = 32 * WN;
  constexpr int ASZ = a_tile_floats<A_MC, TM, KD>();
  constexpr int BSZ = b_tile_floats<B_KC, TN, KD>();
  constexpr int EPI_LD = 16 * WN + 4;  // epilogue staging row stride (16-byte aligned rows)
  constexpr int SMEM = 2 * (ASZ + BSZ) > 4 * 32 * EPI_LD ? 2 * (ASZ + BSZ) : 4 * 32 * EPI_LD;
  __shared__ __attribute__((aligned(16))) float smem[SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, q = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;
  int tm, tn;
  tile_of(gridDim.x, gridDim.y, tm, tn);
  const int m0 = tm * TM, n0 = tn * TN;
  const int64_t z = blockIdx.z / g.splits;
  const int split = blockIdx.z % g.splits;
  const float* A = g.A + batch_off(z, g, g.sa, g.sa2) + (g.grouped ? split * g.gsa : 0);
  const float* B = g.B + batch_off(z, g, g.sb, g.sb2) + (g.grouped ? split * g.gsb : 0);
  float* C = g.C + batch_off(z, g, g.sc, g.sc2);
  const int kbeg = g.grouped ? 0 : split * g.kchunk;
  const int kend = g.grouped ? g.K : min(g.K, kbeg + g.kchunk);
  const uint32_t a_bytes = (uint32_t)(((int64_t)((A_MC ? g.K : g.M) - 1) * g.lda + (A_MC ? g.M : g.K)) * 4);
  const uint32_t b_bytes = (uint32_t)(((int64_t)((B_KC ? g.N : g.K) - 1) * g.ldb + (B_KC ? g.K : g.N)) * 4);
  const BufOperand Ab(A, g.lda, a_bytes), Bb(B, g.ldb, b_bytes);

  f32x4 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int n = 0; n < WN; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};

  const bool do_cs = COLSUM && tm == 0;
  constexpr int CS_T = NT / TN;  // threads per column of the column sum
  float csum = 0.f;
  const int nk = kend > kbeg ? (kend - kbeg + KD - 1) / KD : 0;
  f32x4 ra[TM * KD / 1024], rb[TN * KD / 1024];
  if (nk > 0) {
    load_a<A_MC, VEC, TM, KD>(g, A, Ab, m0, kbeg, kend, tid, ra);
    load_b<B_KC, VEC, TN, KD>(g, B, Bb, n0, kbeg, kend, tid, rb);
    store_tile<!A_MC, TM, KD>(smem, tid, ra);
    store_tile<B_KC, TN, KD>(smem + 2 * ASZ, tid, rb);
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const float* As = smem + cur * ASZ;
    const float* Bs = smem + 2 * ASZ + cur * BSZ;
    const bool more = kt + 1 < nk;
    if (more) {
      load_a<A_MC, VEC, TM, KD>(g, A, Ab, m0, kbeg + (kt + 1) * KD, kend, tid, ra);
      load_b<B_KC, VEC, TN, KD>(g, B, Bb, n0, kbeg + (kt + 1) * KD, kend, tid, rb);
    }
    mma_stage<A_MC, B_KC, WM, WN, KD>(As, Bs, acc, wm, wn, lr, q);
    if (do_cs) {
      const int c = tid % TN, h = tid / TN;
#pragma unroll
      for (int k = 0; k < KD / CS_T; ++k) {
        const int kk = h * (KD / CS_T) + k;
        csum += B_KC ? Bs[c * (KD + PAD) + kk] : Bs[kk * (TN + PAD) + c];
      }
    }
    if (more) {
      store_tile<!A_MC, TM, KD>(smem + (cur ^ 1) * ASZ, tid, ra);
      store_tile<B_KC, TN, KD>(smem + 2 * ASZ + (cur ^ 1) * BSZ, tid, rb);
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
            if (g.bias) v += *reinterpret_cast<const f32x4*>(g.bias + z * g.sbias + col);
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
              if (g.bias) v += g.bias[z * g.sbias + col];
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
      if (split_mode) g.part_cs[(int64_t)blockIdx.z * g.N + n0 + tid] = cs;
      else put_colsum(g, z * g.scs + n0 + tid, cs);
    }
  }
}

// Register-direct variant for 128 x 128 tiles: no LDS and no barrier.  Each
// lane loads its own MFMA fragments from global memory with 16-byte reads,
// D - 1 K stages (KD deep each) ahead of the MFMAs, through D register sets.
// Within a stage, lane group q = lane / 16 feeds k = (KD/4) q + j to MFMA
// step j (j < KD/4); A and B use the same k permutation, so the contraction
// is unchanged.
//  * an operand stored k-contiguous gives lane (lr, q) KD/4 consecutive k
//    values of one row (column) in KD/16 loads per 16-row block; with KD = 32
//    the four lane groups cover a full 128-byte line of each row per stage;
//  * an operand stored m- (or n-) contiguous is read along m instead: one
//    load of 4 consecutive rows at k = (KD/4) q + j holds that lane's values
//    for all four blocks (one load per MFMA step j).
// Rows and columns inside the wave's 64 x 64 block are permuted so that
// every lane ends with 4 consecutive C columns per row: block n, lane column
// c is column 4c + n for both B layouts, and block i, accumulator row d is
// row 4d + i (A m-contiguous) or 16i + d (A k-contiguous).  The epilogue
// therefore writes 16-byte row segments straight from the accumulators.
// A wave issues KD/4 loads per operand per stage; the two waves that share a
// row (column) panel hit the same lines, which the L1 serves.
// One 128 x 128 tile (tm, tn) of batch item / split bz of the register-direct
// kernel; shared by gemm_direct_kernel and gemm_pair_kernel.
template <int TA, int TB, bool COLSUM, int KD, int D, bool TERMS>
__device__ __forceinline__ void direct_tile(const GemmArgs& g, int tm, int tn, int bz) {
  constexpr bool A_MC = TA != 0;
  constexpr bool B_KC = TB != 0;
  constexpr int TM = 128, TN = 128;
  constexpr int S = KD / 4;   // MFMA steps (and loads per operand) per stage
  constexpr int H = KD / 16;  // loads per 16-row block of a k-contiguous operand
  static_assert(D >= 2 && (KD == 16 || KD == 32), "unsupported stage shape");

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, q = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = tm * TM + wm * 64, n0 = tn * TN + wn * 64;  // this wave's 64 x 64 block
  const int64_t z = bz / g.splits;
  const int split = bz % g.splits;
  const float* A = g.A + batch_off(z, g, g.sa, g.sa2) + (g.grouped ? split * g.gsa : 0);
  const float* B = g.B + batch_off(z, g, g.sb, g.sb2) + (g.grouped ? split * g.gsb : 0);
  float* C = g.C + batch_off(z, g, g.sc, g.sc2);
  const int kbeg = g.grouped ? 0 : split * g.kchunk;
  const int kend = g.grouped ? g.K : min(g.K, kbeg + g.kchunk);
  // With TERMS the resources span every term (the host checks the extent).
  const int64_t a_terms = TERMS ? (int64_t)(g.kterms - 1) * g.gsa : 0;
  const int64_t b_terms = TERMS ? (int64_t)(g.kterms - 1) * g.gsb : 0;
  const uint32_t a_bytes =
      (uint32_t)((a_terms + (int64_t)((A_MC ? g.K : g.M) - 1) * g.lda + (A_MC ? g.M : g.K)) * 4);
  const uint32_t b_bytes =
      (uint32_t)((b_terms + (int64_t)((B_KC ? g.N : g.K) - 1) * g.ldb + (B_KC ? g.K : g.N)) * 4);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(A), (short)0, (int)a_bytes, kBufWord3);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(B), (short)0, (int)b_bytes, kBufWord3);
  const int nkt = kend > kbeg ? (kend - kbeg + KD - 1) / KD : 0;  // stages per term
  const int nk = TERMS ? g.kterms * nkt : nkt;

  // Byte offsets at k = kbeg of the S loads per operand, and the per-stage
  // advance.  K and the split's chunk are multiples of KD (checked on the
  // host), so every stage is full.  A row (column) outside the matrix starts
  // at kBufOOB, past the buffer's extent; the hardware range check returns
  // zeros for it, and its products only reach C rows (columns) that are never
  // stored.  Stages fetched past the end of K (up to D - 1) are never
  // consumed; a buffer load never faults, whatever its offset.
  const int kq = kbeg + S * q;  // first k of this lane group
  uint32_t a_off[S], b_off[S];
#pragma unroll
  for (int x = 0; x < S; ++x) {
    if (!A_MC) {  // x = (block i, half h): row m0 + 16 i + lr, k = kq + 4 h
      const int row = m0 + 16 * (x / H) + lr;
      a_off[x] = row < g.M ? (uint32_t)(row * (int)g.lda + kq + 4 * (x % H)) * 4u : kBufOOB;
    } else {  // x = step j: k = kq + x, rows m0 + 4 lr .. + 3
      a_off[x] = m0 + 4 * lr < g.M ? (uint32_t)((kq + x) * (int)g.lda + m0 + 4 * lr) * 4u : kBufOOB;
    }
    if (B_KC) {  // x = (block n, half h): column n0 + 4 lr + n, k = kq + 4 h
      const int col = n0 + 4 * lr + x / H;
      b_off[x] = col < g.N ? (uint32_t)(col * (int)g.ldb + kq + 4 * (x % H)) * 4u : kBufOOB;
    } else {  // x = step j: k = kq + x, columns n0 + 4 lr .. + 3
      b_off[x] = n0 + 4 * lr < g.N ? (uint32_t)((kq + x) * (int)g.ldb + n0 + 4 * lr) * 4u : kBufOOB;
    }
  }
  const uint32_t a_step = 4u * (A_MC ? KD * (uint32_t)g.lda : KD);
  const uint32_t b_step = 4u * (B_KC ? KD : KD * (uint32_t)g.ldb);

  // Terms: stage kt is stage kt % nkt of term kt / nkt, so the offset jumps
  // by (term stride - nkt stages) at each term boundary (modulo 2^32; the
  // true offsets stay below 2^31, OOB rows included).  Stages prefetched past
  // the last term are never consumed.
  const uint32_t a_jump = TERMS ? (uint32_t)(g.gsa * 4) - (uint32_t)nkt * a_step : 0u;
  const uint32_t b_jump = TERMS ? (uint32_t)(g.gsb * 4) - (uint32_t)nkt * b_step : 0u;
  auto load = [&](int kt, f32x4(&fa)[S], f32x4(&fb)[S]) {
    uint32_t da = (uint32_t)kt * a_step, db = (uint32_t)kt * b_step;
    if (TERMS) {
      const uint32_t t = (uint32_t)min(kt / nkt, g.kterms - 1);
      da += t * a_jump;
      db += t * b_jump;
    }
#pragma unroll
    for (int x = 0; x < S; ++x) {
      fa[x] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, (int)(a_off[x] + da), 0, 0));
      fb[x] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, (int)(b_off[x] + db), 0, 0));
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bool do_cs = COLSUM && tm == 0 && wm == 0;
  float csum[4] = {0.f, 0.f, 0.f, 0.f};  // per lane: partial sums of columns 4 lr + n

  // Operand value of (block i or n, step j).
  auto av = [&](const f32x4(&fa)[S], int i, int j) { return A_MC ? fa[j][i] : fa[i * H + j / 4][j % 4]; };
  auto bv = [&](const f32x4(&fb)[S], int n, int j) { return B_KC ? fb[n * H + j / 4][j % 4] : fb[j][n]; };
  auto mfma = [&](const f32x4(&fa)[S], const f32x4(&fb)[S]) {
#pragma unroll
    for (int j = 0; j < S; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int n = 0; n < 4; ++n)
          acc[i][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(av(fa, i, j), bv(fb, n, j), acc[i][n], 0, 0, 0);
    if (do_cs) {
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int j = 0; j < S; ++j) csum[n] += bv(fb, n, j);
    }
  };

  // The epilogue's bias, loaded before the K loop so that its wait is long
  // satisfied when the stores start (loaded after the loop, it cost the
  // epilogue a memory round trip).  A column past N, or no bias, reads 0.
  const bool split_mode = g.splits > 1;
  const int col = n0 + 4 * lr;
  f32x4 b4;
  {
    const bool has_b = !split_mode && g.bias;
    const __amdgpu_buffer_rsrc_t rbias = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(has_b ? g.bias + z * g.sbias : nullptr), (short)0, has_b ? g.N * 4 : 0, kBufWord3);
    b4 = __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(rbias, (int)(col < g.N ? (uint32_t)col * 4u : kBufOOB), 0, 0));
  }

  // Stage s lives in register set s % D.  Each pass of the loop consumes D
  // stages and issues the loads D - 1 stages ahead of each.
  f32x4 fa[D][S], fb[D][S];
#pragma unroll
  for (int s = 0; s < D - 1; ++s) load(s, fa[s], fb[s]);
  int kt = 0;
  for (; kt + D - 1 < nk; kt += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      load(kt + s + D - 1, fa[(s + D - 1) % D], fb[(s + D - 1) % D]);
      __builtin_amdgcn_sched_barrier(0);
      mfma(fa[s], fb[s]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // Fewer than D stages remain, all of them already loaded (sets 0 .. D - 2).
#pragma unroll
  for (int s = 0; s < D - 1; ++s)
    if (kt + s < nk) mfma(fa[s], fb[s]);

  // Epilogue: lane (lr, q) holds C[row(i, 4q + r)][4 lr + n] in acc[i][n][r],
  // so each (i, r) is one 16-byte store of 4 consecutive columns.  N, ldc and
  // C are 16-byte aligned on this path (checked on the host).
  float* P = split_mode ? g.part + (int64_t)bz * g.M * g.N : nullptr;
  auto rmap = [&](int i, int d) { return A_MC ? 4 * d + i : 16 * i + d; };
  if (col < g.N) {
    const float alpha = g.alpha, beta = g.beta;
    // beta != 0: every previous value is loaded before the first store (the
    // vector memory counter counts stores too, so loading each one between
    // two stores made every store wait for the one before).
    f32x4 old[4][4];
    if (!split_mode && beta != 0.f) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + rmap(i, 4 * q + r);
          old[i][r] = row < g.M ? *reinterpret_cast<const f32x4*>(C + (int64_t)row * g.ldc + col)
                                : f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + rmap(i, 4 * q + r);
        if (row < g.M) {
          f32x4 v = {acc[i][0][r], acc[i][1][r], acc[i][2][r], acc[i][3][r]};
          if (split_mode) {
            *reinterpret_cast<f32x4*>(P + (int64_t)row * g.N + col) = v;
          } else {
            float* p = C + (int64_t)row * g.ldc + col;
            v = alpha * v;
            if (beta != 0.f) v += beta * old[i][r];
            *reinterpret_cast<f32x4*>(p) = v + b4;
          }
        }
      }
  }
  if (do_cs) {
    // lanes lr + 16 q hold partial sums of the same 4 columns: fixed-order
    // reduction over q, then lane q == 0 owns columns col .. col + 3.
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      float v = csum[n];
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      csum[n] = v;
    }
    if (q == 0 && col < g.N) {
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        if (split_mode) g.part_cs[(int64_t)bz * g.N + col + n] = csum[n];
        else put_colsum(g, z * g.scs + col + n, csum[n]);
      }
    }
  }
}

// Tile (tm, tn) and batch item z of work item L of a launch over `items` =
// gx * gy * batch tiles.  The same XCD-aware order as tile_of: item L runs on
// XCD L % 8 (workgroups are dispatched round-robin), XCD x owns a contiguous
// logical range, walked in groups of 8 tile-rows per batch item.  A bijection
// on [0, items).
__device__ __forceinline__ void item_tile(int L, int items, int gx, int gy, int& tm, int& tn, int& z) {
  const int q = items / kXcds, r = items % kXcds, x = L % kXcds;
  const int logical = x * q + min(x, r) + L / kXcds;
  const int T = gx * gy;
  z = logical / T;
  const int t = logical - z * T;
  const int per_group = kGroupRows * gx;
  const int grp = t / per_group;
  const int first_m = grp * kGroupRows;
  const int rows = min(gy - first_m, kGroupRows);
  const int in_group = t - grp * per_group;
  tm = first_m + in_group % rows;
  tn = in_group / rows;
}

// One tile per workgroup.  The tile and the batch item / K split come from
// the workgroup's linear id over the whole grid (x, then y, then z), so each
// XCD gets a contiguous range that stays within one split: the column tiles
// that share an A row panel share that XCD's L2 (with z walked per slice,
// every XCD read every panel of a split -- 3.6x the algorithmic bytes for a
// 2048 x 512 x 8192 weight gradient in 4 splits).
template <int TA, int TB, bool COLSUM, int KD, int D, int OCC, bool TERMS = false>
__global__ __launch_bounds__(NT, OCC) void gemm_direct_kernel(GemmArgs g) {
  int tm, tn, z;
  const int L = (int)(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z));
  item_tile(L, (int)(gridDim.x * gridDim.y * gridDim.z), gridDim.x, gridDim.y, tm, tn, z);
  direct_tile<TA, TB, COLSUM, KD, D, TERMS>(g, tm, tn, z);
}

// Persistent register-direct GEMM for grids of more 128 x 128 tiles than two
// per CU: two workgroups per CU walk work items L = blockIdx.x + j * gridDim.x.
// Each wave computes its 64 x 64 block of a tile exactly as
// gemm_direct_kernel does (same fragment loads, same MFMA order, so the same
// bits).  The operand loads run D - 1 stages ahead straight across tile
// boundaries: in the last D stages of a tile they fetch the next tile's first
// D - 1 stages (offsets selected without branches), so a new tile starts with
// its operands in registers instead of waiting for a prologue, and no
// workgroup is launched or retired per tile.  One loop with a straight-line
// body: every pass issues the same loads in the same places, so the
// compiler's load waits stay tight.  At a tile boundary the wave writes its
// block from the accumulators through a buffer resource (elements outside
// the matrix get offset kBufOOB: the store is dropped, a read returns zeros);
// those stores are issued after the next tile's first loads, so the waits
// for those loads never include them.
// Measured on MI355X against the per-tile launch of gemm_direct_kernel:
// equal or faster on every C4 shape with more than 512 tiles (LM-head
// forward 604 -> 581 us, 8192 x 2048 x 512 NT 150 -> 135 us).  A variant
// with one workgroup per CU and a fifth wave writing C from an LDS staging
// tile was slower (one compute wave per SIMD hides less load latency).
// Requires: one split, no column sum, K a positive multiple of KD * D, C
// addressable by a buffer resource, and the direct kernel's alignment
// conditions (checked on the host).
template <int TA, int TB, int KD, int D, int EPI = kEpiPlain, int ACT = 0>
__global__ __launch_bounds__(NT, 2) void gemm_stream_kernel(GemmArgs g, int gx, int gy, int items) {
  constexpr bool ROWSTATS = EPI == kEpiRowstats;
  constexpr bool A_MC = TA != 0;
  constexpr bool B_KC = TB != 0;
  constexpr int S = KD / 4;   // MFMA steps (and loads per operand) per stage
  constexpr int H = KD / 16;  // loads per 16-row block of a k-contiguous operand
  static_assert(D >= 2 && (KD == 16 || KD == 32), "unsupported stage shape");
  constexpr int kRsLd = 64 + 4;  // ROWSTATS staging row stride (floats)
  __shared__ __attribute__((aligned(16))) float rs_lds[ROWSTATS ? 4 * 64 * kRsLd : 4];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int G = gridDim.x;

  const int lr = lane & 15, q = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;
  const int nk = g.K / KD;
  const uint32_t a_bytes = (uint32_t)(((int64_t)((A_MC ? g.K : g.M) - 1) * g.lda + (A_MC ? g.M : g.K)) * 4);
  const uint32_t b_bytes = (uint32_t)(((int64_t)((B_KC ? g.N : g.K) - 1) * g.ldb + (B_KC ? g.K : g.N)) * 4);
  const uint32_t a_step = 4u * (A_MC ? KD * (uint32_t)g.lda : KD);
  const uint32_t b_step = 4u * (B_KC ? KD : KD * (uint32_t)g.ldb);
  const uint32_t c_bytes = (uint32_t)(((int64_t)(g.M - 1) * g.ldc + g.N) * 4);

  // Buffer resources and this lane's byte offsets at stage 0 of an item (the
  // direct kernel's offsets with kbeg = 0).  Past the last item the first
  // item is decoded and every offset becomes kBufOOB, so those (never
  // consumed) loads return zeros.
  auto locate = [&](int L, __amdgpu_buffer_rsrc_t& ra, __amdgpu_buffer_rsrc_t& rb, uint32_t(&ao)[S],
                    uint32_t(&bo)[S]) {
    const bool live = L < items;
    int tm, tn, z;
    item_tile(live ? L : (int)blockIdx.x, items, gx, gy, tm, tn, z);
    const float* A = g.A + batch_off(z, g, g.sa, g.sa2);
    const float* B = g.B + batch_off(z, g, g.sb, g.sb2);
    ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(A), (short)0, (int)a_bytes, kBufWord3);
    rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(B), (short)0, (int)b_bytes, kBufWord3);
    const int m0 = tm * 128 + wm * 64, n0 = tn * 128 + wn * 64;
    const int kq = S * q;
#pragma unroll
    for (int x = 0; x < S; ++x) {
      if (!A_MC) {
        const int row = m0 + 16 * (x / H) + lr;
        ao[x] = live && row < g.M ? (uint32_t)(row * (int)g.lda + kq + 4 * (x % H)) * 4u : kBufOOB;
      } else {
        ao[x] = live && m0 + 4 * lr < g.M ? (uint32_t)((kq + x) * (int)g.lda + m0 + 4 * lr) * 4u : kBufOOB;
      }
      if (B_KC) {
        const int col = n0 + 4 * lr + x / H;
        bo[x] = live && col < g.N ? (uint32_t)(col * (int)g.ldb + kq + 4 * (x % H)) * 4u : kBufOOB;
      } else {
        bo[x] = live && n0 + 4 * lr < g.N ? (uint32_t)((kq + x) * (int)g.ldb + n0 + 4 * lr) * 4u : kBufOOB;
      }
    }
  };
  __amdgpu_buffer_rsrc_t ra, rb, ra_n, rb_n;  // current and next item
  uint32_t a_off[S], b_off[S], a_nx[S], b_nx[S];
  locate(blockIdx.x, ra, rb, a_off, b_off);
  locate(blockIdx.x + G, ra_n, rb_n, a_nx, b_nx);

  // Stage ks of the current item, or stage kn of the next one when `nxt`.
  auto load = [&](bool nxt, int ks, int kn, f32x4(&fa)[S], f32x4(&fb)[S]) {
    const __amdgpu_buffer_rsrc_t xa = nxt ? ra_n : ra, xb = nxt ? rb_n : rb;
    const uint32_t da = (uint32_t)(nxt ? kn : ks) * a_step, db = (uint32_t)(nxt ? kn : ks) * b_step;
#pragma unroll
    for (int x = 0; x < S; ++x) {
      const uint32_t oa = (nxt ? a_nx[x] : a_off[x]) + da, ob = (nxt ? b_nx[x] : b_off[x]) + db;
      fa[x] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xa, (int)oa, 0, 0));
      fb[x] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xb, (int)ob, 0, 0));
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto av = [&](const f32x4(&fa)[S], int i, int j) { return A_MC ? fa[j][i] : fa[i * H + j / 4][j % 4]; };
  auto bv = [&](const f32x4(&fb)[S], int n, int j) { return B_KC ? fb[n * H + j / 4][j % 4] : fb[j][n]; };
  auto mfma = [&](const f32x4(&fa)[S], const f32x4(&fb)[S]) {
#pragma unroll
    for (int j = 0; j < S; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int n = 0; n < 4; ++n)
          acc[i][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(av(fa, i, j), bv(fb, n, j), acc[i][n], 0, 0, 0);
  };

  // Stage kt of every item lives in register set kt % D (nk is a multiple of
  // D, so each item starts at set 0).
  f32x4 fa[D][S], fb[D][S];
#pragma unroll
  for (int s = 0; s < D - 1; ++s) load(false, s, 0, fa[s], fb[s]);
  int kt = 0, c_item = blockIdx.x;
  // The epilogue's bias, loaded ahead of the item's last D stages: issued
  // before the next item's first loads, its wait in the epilogue does not
  // cover them (the vector memory counter completes in order).  A column
  // past N, or no bias, reads 0.
  f32x4 b4 = {0.f, 0.f, 0.f, 0.f};
  for (;;) {
    const bool last = kt + D == nk;  // the item's last D stages
    if (last) {
      int tm, tn, z;
      item_tile(c_item, items, gx, gy, tm, tn, z);
      const int col = tn * 128 + wn * 64 + 4 * lr;
      const __amdgpu_buffer_rsrc_t rbias = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<float*>(g.bias ? g.bias + z * g.sbias : g.bias), (short)0, g.bias ? g.N * 4 : 0, kBufWord3);
      b4 = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rbias, (int)(col < g.N ? (uint32_t)col * 4u : kBufOOB), 0, 0));
    }
#pragma unroll
    for (int s = 0; s < D; ++s) {
      const int ls = kt + s + D - 1;  // stage to fetch; past nk it is the next item's
      load(s > 0 && last, ls, ls - nk, fa[(s + D - 1) % D], fb[(s + D - 1) % D]);
      __builtin_amdgcn_sched_barrier(0);
      mfma(fa[s], fb[s]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!last) {
      kt += D;
      continue;
    }
    {
      // Epilogue: lane (lr, q) holds C[row(i, 4q + r)][4 lr + n] of the
      // wave's block in acc[i][n][r] (the direct kernel's permutation), so
      // each (i, r) is one 16-byte store of 4 consecutive columns.
      int tm, tn, z;
      item_tile(c_item, items, gx, gy, tm, tn, z);
      float* C = g.C + batch_off(z, g, g.sc, g.sc2);
      const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(C, (short)0, (int)c_bytes, kBufWord3);
      // Activation operands share C's layout (and batch offsets).
      const int64_t zc = batch_off(z, g, g.sc, g.sc2);
      __amdgpu_buffer_rsrc_t ry = rc, rx = rc, rd = rc;
      if (EPI == kEpiActFwd) ry = __builtin_amdgcn_make_buffer_rsrc(g.act_y + zc, (short)0, (int)c_bytes, kBufWord3);
      if (EPI == kEpiActBwd) {
        rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(g.act_x) + zc, (short)0, (int)c_bytes, kBufWord3);
        rd = __builtin_amdgcn_make_buffer_rsrc(g.act_dx + zc, (short)0, (int)c_bytes, kBufWord3);
      }
      const int m0 = tm * 128 + wm * 64, col = tn * 128 + wn * 64 + 4 * lr;
      const float alpha = g.alpha, beta = g.beta;
      // ROWSTATS: the wave's 64 x 64 block goes to LDS (row slot
      // d' = 16 i + 4 q + r, columns outside the matrix as -FLT_MAX), then lane
      // l reduces slot l's 64 columns to (max, sum of exp(x - max)).
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + (A_MC ? 4 * (4 * q + r) + i : 16 * i + 4 * q + r);
          const uint32_t off = row < g.M && col < g.N ? (uint32_t)(row * (int)g.ldc + col) * 4u : kBufOOB;
          f32x4 v = {acc[i][0][r], acc[i][1][r], acc[i][2][r], acc[i][3][r]};
          v = alpha * v;
          if (beta != 0.f)
            v += beta * __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, (int)off, 0, 0));
          v += b4;
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, v),
                                                 rc, (int)off, 0, 0);
          if (EPI == kEpiActFwd) {
            f32x4 y;
#pragma unroll
            for (int n = 0; n < 4; ++n) y[n] = act_f<ACT>(v[n]);
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, y), ry, (int)off, 0, 0);
          }
          if (EPI == kEpiActBwd) {
            const f32x4 xh = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0));
            f32x4 old = {0.f, 0.f, 0.f, 0.f};
            if (g.act_acc) old = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rd, (int)off, 0, 0));
            f32x4 d;  // the elementwise backward's bits: the product rounded before the add
#pragma unroll
            for (int n = 0; n < 4; ++n) d[n] = act_bwd_k<ACT>(xh[n], v[n], old[n], g.act_acc);
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, d), rd, (int)off, 0, 0);
          }
          if (ROWSTATS) {
#pragma unroll
            for (int n = 0; n < 4; ++n)
              if (col + n >= g.N) v[n] = -FLT_MAX;
            *reinterpret_cast<f32x4*>(rs_lds + (wave * 64 + 16 * i + 4 * q + r) * kRsLd + 4 * lr) = v;
          }
        }
      if (ROWSTATS) {
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const float* rp = rs_lds + (wave * 64 + lane) * kRsLd;
        f32x4 x[16];
#pragma unroll
        for (int c = 0; c < 16; ++c) x[c] = *reinterpret_cast<const f32x4*>(rp + 4 * c);
        float m = -FLT_MAX;
#pragma unroll
        for (int c = 0; c < 16; ++c) m = fmaxf(fmaxf(m, fmaxf(x[c][0], x[c][1])), fmaxf(x[c][2], x[c][3]));
        float e = 0.f;
#pragma unroll
        for (int c = 0; c < 16; ++c)
#pragma unroll
          for (int j = 0; j < 4; ++j) e += __expf(x[c][j] - m);
        const int i = lane >> 4, d = lane & 15;
        const int row = m0 + (A_MC ? 4 * d + i : 16 * i + d);
        const int c0 = tn * 128 + wn * 64;  // this wave's 64-column block
        if (row < g.M && c0 < g.N)
          *reinterpret_cast<float2*>(g.rowpart + (int64_t)row * g.rp_ld + 2 * (c0 >> 6)) = make_float2(m, e);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
    c_item += G;
    if (c_item >= items) break;
    kt = 0;
    ra = ra_n;
    rb = rb_n;
#pragma unroll
    for (int x = 0; x < S; ++x) {
      a_off[x] = a_nx[x];
      b_off[x] = b_nx[x];
    }
    locate(c_item + G, ra_n, rb_n, a_nx, b_nx);
  }
}

// Row statistics of a finished C when the GEMM did not produce them in its
// epilogue: one wave per (row, 64-column block): max and sum of exp(C - max).
__global__ __launch_bounds__(256) void rowstats_kernel(const float* __restrict__ C, int64_t ldc, int M, int N,
                                                       float* __restrict__ part, int64_t ld) {
  const int nblk = (N + 63) / 64;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= (int64_t)M * nblk) return;
  const int row = (int)(w / nblk), blk = (int)(w % nblk);
  const int lane = threadIdx.x & 63, c = blk * 64 + lane;
  const float x = c < N ? C[(int64_t)row * ldc + c] : -FLT_MAX;
  float m = x;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  float e = c < N ? expf(x - m) : 0.f;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) e += __shfl_xor(e, o, 64);
  if (lane == 0) *reinterpret_cast<float2*>(part + (int64_t)row * ld + 2 * blk) = make_float2(m, e);
}

// Two independent register-direct GEMMs in one launch, one tile per
// workgroup: workgroups [0, items0) take problem 0 and the rest problem 1,
// each tile decoded by item_tile and computed by direct_tile exactly as
// gemm_direct_kernel computes it.  A Linear layer's dX and dW products
// (Engine/engine.cu:3553-3560) usually each fill about one workgroup per CU
// with work items of equal depth; launched together they run two per CU in
// a single round.
// Problem 1 starts at workgroup start1, items0 rounded up to a multiple of 8
// (the workgroups between do nothing), so that its item L runs on XCD L % 8
// as item_tile assumes.
struct PairGrid {
  int items0, gx0, gy0;
  int items1, gx1, gy1;
  int start1;
};

template <int TA0, int TB0, bool CS0, bool T0, int TA1, int TB1, bool CS1, bool T1>
__global__ __launch_bounds__(NT, 2) void gemm_pair_kernel(GemmArgs g0, GemmArgs g1, PairGrid pg) {
  const int w = blockIdx.x;
  int tm, tn, bz;
  if (w < pg.items0) {
    item_tile(w, pg.items0, pg.gx0, pg.gy0, tm, tn, bz);
    direct_tile<TA0, TB0, CS0, 16, 3, T0>(g0, tm, tn, bz);
  } else if (w >= pg.start1) {
    item_tile(w - pg.start1, pg.items1, pg.gx1, pg.gy1, tm, tn, bz);
    direct_tile<TA1, TB1, CS1, 16, 3, T1>(g1, tm, tn, bz);
  }
}

// C = alpha * sum_s part[s] + beta * C (+ bias) and colsum (+)= sum_s
// part_cs[s], in a fixed order.  A workgroup covers 64 units -- a unit is W
// (4 with VEC, else 1) columns of one row of one batch item, numbered over
// (batch, row, column group) so every thread has one -- with four split
// groups: thread (unit, g) adds splits g, g + 4, g + 8, ... in order (four
// loads in flight), and the group sums are added in group order through LDS.
// Workgroups from `nmain` on take the column sums: one thread per (batch,
// column), splits added in order.
template <bool VEC>
__global__ __launch_bounds__(256) void split_reduce_kernel(GemmArgs g, int64_t units, unsigned nmain) {
  constexpr int W = VEC ? 4 : 1;
  __shared__ f32x4 grp[4][64];
  const int64_t mn = (int64_t)g.M * g.N;
  if (blockIdx.x >= nmain) {
    const int64_t j = (int64_t)(blockIdx.x - nmain) * 256 + threadIdx.x;
    const int batch = (int)(units / ((int64_t)g.M * (g.N / W)));
    if (j >= (int64_t)batch * g.N) return;
    const int64_t b = j / g.N, col = j - b * g.N;
    const float* p = g.part_cs + b * g.splits * (int64_t)g.N + col;
    float acc = 0.f;
    int sp = 0;
    for (; sp + 4 <= g.splits; sp += 4) {
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = p[(int64_t)(sp + u) * g.N];
#pragma unroll
      for (int u = 0; u < 4; ++u) acc += v[u];
    }
    for (; sp < g.splits; ++sp) acc += p[(int64_t)sp * g.N];
    put_colsum(g, b * g.scs + col, acc);
    return;
  }
  const int lane = threadIdx.x & 63, sg = threadIdx.x >> 6;
  const int64_t u = (int64_t)blockIdx.x * 64 + lane;
  const bool live = u < units;
  int64_t b = 0, row = 0, col = 0;
  if (live) {
    const int64_t nw = g.N / W, per = (int64_t)g.M * nw;
    b = u / per;
    const int64_t r = u - b * per;
    row = r / nw;
    col = (r - row * nw) * W;
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (live) {
    const float* p = g.part + b * g.splits * mn + row * g.N + col;
    int sp = sg;
    for (; sp + 12 < g.splits; sp += 16) {
      f32x4 v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (VEC) v[k] = *reinterpret_cast<const f32x4*>(p + (int64_t)(sp + 4 * k) * mn);
        else v[k] = f32x4{p[(int64_t)(sp + 4 * k) * mn], 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) acc += v[k];
    }
    for (; sp < g.splits; sp += 4) {
      if (VEC) acc += *reinterpret_cast<const f32x4*>(p + (int64_t)sp * mn);
      else acc[0] += p[(int64_t)sp * mn];
    }
  }
  grp[sg][lane] = acc;
  __syncthreads();
  if (sg != 0 || !live) return;
  const f32x4 r = ((grp[0][lane] + grp[1][lane]) + grp[2][lane]) + grp[3][lane];
  float* c = g.C + batch_off(b, g, g.sc, g.sc2) + row * g.ldc + col;
  const int64_t co = batch_off(b, g, g.sc, g.sc2) + row * g.ldc + col;
  if (VEC) {
    f32x4 v = g.alpha * r;
    if (g.beta != 0.f) v += g.beta * *reinterpret_cast<const f32x4*>(c);
    if (g.bias) v += *reinterpret_cast<const f32x4*>(g.bias + b * g.sbias + col);
    *reinterpret_cast<f32x4*>(c) = v;
    if (g.act_red) {
      f32x4 y;
#pragma unroll
      for (int k = 0; k < 4; ++k) y[k] = act_rt(g.act_red - 1, v[k]);
      *reinterpret_cast<f32x4*>(g.act_y + co) = y;
    }
  } else {
    float v = g.alpha * r[0];
    if (g.beta != 0.f) v += g.beta * *c;
    if (g.bias) v += g.bias[b * g.sbias + col];
    *c = v;
    if (g.act_red) g.act_y[co] = act_rt(g.act_red - 1, v);
  }
}

// 64 C elements per workgroup, one per lane, the four waves taking a quarter
// of K each and adding their partial sums in wave order: products with a tiny
// M or K (a Linear layer applied to one row, or the weight gradient of one),
// where the tile kernels would spend split-K and reduce launches on little
// work.
template <int TA, int TB>
__device__ __forceinline__ void simple_body(const GemmArgs& g, int bx, int64_t z, float (&red)[2][4][64]) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t idx = (int64_t)bx * 64 + lane;
  const bool live = idx < (int64_t)g.M * g.N;
  const int m = live ? (int)(idx / g.N) : 0, n = live ? (int)(idx % g.N) : 0;
  const int kq = (g.K + 3) / 4, k0 = w * kq, k1 = min(g.K, k0 + kq);
  const float* A = g.A + z * g.sa;
  const float* B = g.B + z * g.sb;
  float acc = 0.f, cs = 0.f;
  if (live) {
#pragma unroll 8
    for (int k = k0; k < k1; ++k) {
      const float a = TA ? A[(int64_t)k * g.lda + m] : A[(int64_t)m * g.lda + k];
      const float b = TB ? B[(int64_t)n * g.ldb + k] : B[(int64_t)k * g.ldb + n];
      acc += a * b;
      cs += b;
    }
  }
  red[0][w][lane] = acc;
  red[1][w][lane] = cs;
  __syncthreads();
  if (w != 0 || !live) return;
  acc = ((red[0][0][lane] + red[0][1][lane]) + red[0][2][lane]) + red[0][3][lane];
  float* c = g.C + z * g.sc + (int64_t)m * g.ldc + n;
  float v = g.alpha * acc;
  if (g.beta != 0.f) v += g.beta * *c;
  if (g.bias) v += g.bias[z * g.sbias + n];
  *c = v;
  if (g.act_bwd) {
    const int64_t co = z * g.sc + (int64_t)m * g.ldc + n;
    g.act_dx[co] = act_bwd_rt(g.act_bwd - 1, g.act_x[co], v, g.act_acc ? g.act_dx[co] : 0.f, g.act_acc);
  }
  if (g.colsum && m == 0)
    put_colsum(g, z * g.scs + n, ((red[1][0][lane] + red[1][1][lane]) + red[1][2][lane]) + red[1][3][lane]);
}

template <int TA, int TB>
__global__ __launch_bounds__(256) void gemm_simple_kernel(GemmArgs g) {
  __shared__ float red[2][4][64];
  simple_body<TA, TB>(g, blockIdx.x, blockIdx.y, red);
}

// A Linear layer's two small products (dX = dY W^T and dW = X^T dY with db)
// in one launch: workgroups [0, nb0) compute problem 0, the rest problem 1,
// each exactly as gemm_simple_kernel does.  One launch less per small layer
// (a C1 step is bound by the host's launch rate).
__global__ __launch_bounds__(256) void gemm_simple_pair_kernel(GemmArgs g0, GemmArgs g1, int nb0) {
  __shared__ float red[2][4][64];
  if ((int)blockIdx.x < nb0) simple_body<0, 1>(g0, blockIdx.x, blockIdx.y, red);
  else simple_body<1, 0>(g1, blockIdx.x - nb0, blockIdx.y, red);
}

// Small products with a long K (an MLP's 784-wide input layer: 64 x 256 x
// 784 and its gradients): one C tile of TT x TT per workgroup of NW waves.
// Wave w multiplies the tile's operands over its K range [w kc, (w + 1) kc)
// (whole 16-deep slabs) on MFMA, the workgroup adds the NW partial tiles in
// wave order through LDS and applies the epilogue: one launch where split K
// needs two (partials, then the reduce), and more workgroups than the
// 64-wide tiles give the same shape.  Within a 16-deep slab lane group q =
// l / 16 feeds k = 4q + e to MFMA step e (the k permutation of the tile
// kernels), so an operand stored k-contiguous is read with one 16-byte load
// per lane and slab (scattered 4-byte loads of it took twice the kernel's
// time), and one stored m- or n-contiguous with four 4-byte loads, 64
// contiguous bytes per k row.  Column sums of B (the bias gradient) come
// from the workgroups of the first tile row, in (wave, lane group) order.
template <int TT, int NW>
constexpr int ks_lds_floats() {
  return NW * TT * TT + NW * 4 * TT;
}

// Four k-consecutive elements p[0..3] of a k-contiguous operand row, zero at
// k >= k1 (k = kq + e).
__device__ __forceinline__ f32x4 ks_row4(const float* p, int kq, int k1, bool vec) {
  f32x4 v = {0.f, 0.f, 0.f, 0.f};
  if (vec && kq + 3 < k1) {
    v = *reinterpret_cast<const f32x4*>(p);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (kq + e < k1) v[e] = p[e];
  }
  return v;
}

template <int TA, int TB, int TT, int NW>
__device__ __forceinline__ void ksplit_body(const GemmArgs& g, int tx, int ty, int64_t z, int kc, float* lds) {
  constexpr int S = TT / 16;
  const int lane = threadIdx.x & 63, li = lane & 15, lq = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int m0 = ty * TT, n0 = tx * TT;
  const float* __restrict__ A = g.A + batch_off(z, g, g.sa, g.sa2);
  const float* __restrict__ B = g.B + batch_off(z, g, g.sb, g.sb2);
  // 16-byte loads along k need 16-byte aligned rows
  const bool a_vec = !TA && g.lda % 4 == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0;
  const bool b_vec = TB && g.ldb % 4 == 0 && (reinterpret_cast<uintptr_t>(B) & 15) == 0;
  const bool cs_on = g.colsum != nullptr && ty == 0;
  const int k0 = w * kc, k1 = min(g.K, k0 + kc);
  int am[S], bn[S];
  bool aok[S], bok[S];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    am[i] = m0 + 16 * i + li;
    aok[i] = am[i] < g.M;
    bn[i] = n0 + 16 * i + li;
    bok[i] = bn[i] < g.N;
  }
  f32x4 acc[S][S];
  float cs[S];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    cs[i] = 0.f;
#pragma unroll
    for (int j = 0; j < S; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // Chunks of SL slabs: every load of a chunk is issued before its products
  // (one memory latency per chunk); slabs past the wave's range are skipped
  // on a wave-uniform branch.
  constexpr int SL = 4 / S;
  for (int kb = k0; kb < k1; kb += 16 * SL) {
    f32x4 a[SL][S], b[SL][S];  // element e: MFMA step e of the slab
#pragma unroll
    for (int t = 0; t < SL; ++t)
#pragma unroll
      for (int i = 0; i < S; ++i) {
        a[t][i] = f32x4{0.f, 0.f, 0.f, 0.f};
        b[t][i] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int t = 0; t < SL; ++t) {
      const int kq = kb + 16 * t + 4 * lq;  // this lane's four k of the slab
      if (kb + 16 * t < k1) {
#pragma unroll
        for (int i = 0; i < S; ++i) {
          if (aok[i]) {
            if (TA) {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (kq + e < k1) a[t][i][e] = A[(int64_t)(kq + e) * g.lda + am[i]];
            } else {
              a[t][i] = ks_row4(A + (int64_t)am[i] * g.lda + kq, kq, k1, a_vec);
            }
          }
          if (bok[i]) {
            if (TB) {
              b[t][i] = ks_row4(B + (int64_t)bn[i] * g.ldb + kq, kq, k1, b_vec);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (kq + e < k1) b[t][i][e] = B[(int64_t)(kq + e) * g.ldb + bn[i]];
            }
          }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < SL; ++t) {
      if (kb + 16 * t >= k1) break;
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < S; ++i)
#pragma unroll
          for (int j = 0; j < S; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][i][e], b[t][j][e], acc[i][j], 0, 0, 0);
      if (cs_on)
#pragma unroll
        for (int j = 0; j < S; ++j) cs[j] += ((b[t][j][0] + b[t][j][1]) + b[t][j][2]) + b[t][j][3];
    }
  }
  // Partial tiles: result lane l holds rows 4 (l / 16) + r of column l % 16.
  float* part = lds + w * (TT * TT);
#pragma unroll
  for (int i = 0; i < S; ++i)
#pragma unroll
    for (int j = 0; j < S; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) part[(16 * i + 4 * lq + r) * TT + 16 * j + li] = acc[i][j][r];
  float* cpart = lds + NW * TT * TT;  // [wave][lane group][column]
  if (cs_on)
#pragma unroll
    for (int j = 0; j < S; ++j) cpart[(w * 4 + lq) * TT + 16 * j + li] = cs[j];
  __syncthreads();
  const int64_t cz = batch_off(z, g, g.sc, g.sc2);
  for (int o = threadIdx.x; o < TT * TT; o += 64 * NW) {
    const int m = m0 + o / TT, n = n0 + o % TT;
    if (m >= g.M || n >= g.N) continue;
    float v = lds[o];
#pragma unroll
    for (int q = 1; q < NW; ++q) v += lds[q * (TT * TT) + o];
    const int64_t co = cz + (int64_t)m * g.ldc + n;
    float y = g.alpha * v;
    if (g.beta != 0.f) y += g.beta * g.C[co];
    if (g.bias) y += g.bias[z * g.sbias + n];
    g.C[co] = y;
    if (g.act_red) g.act_y[co] = act_rt(g.act_red - 1, y);
    if (g.act_bwd)
      g.act_dx[co] = act_bwd_rt(g.act_bwd - 1, g.act_x[co], y, g.act_acc ? g.act_dx[co] : 0.f, g.act_acc);
  }
  if (cs_on && (int)threadIdx.x < TT && n0 + (int)threadIdx.x < g.N) {
    const int c = threadIdx.x;
    float t = 0.f;
    for (int q = 0; q < 4 * NW; ++q) t += cpart[q * TT + c];
    put_colsum(g, z * g.scs + n0 + c, t);
  }
}

template <int TA, int TB, int TT, int NW>
__global__ __launch_bounds__(64 * NW) void gemm_ksplit_kernel(GemmArgs g, int kc) {
  __shared__ __attribute__((aligned(16))) float lds[ks_lds_floats<TT, NW>()];
  ksplit_body<TA, TB, TT, NW>(g, blockIdx.x, blockIdx.y, blockIdx.z, kc, lds);
}

// A Linear's two backward products on the K-split kernel in one launch:
// workgroups [0, nb0) take dX = dY W^T (NT, tiles of T0, gx0 per tile row),
// the rest dW = X^T dY with db (TN, tiles of T1).
template <int T0, int T1, int NW>
__global__ __launch_bounds__(64 * NW) void gemm_ksplit_pair_kernel(GemmArgs g0, GemmArgs g1, int nb0, int gx0,
                                                                   int gx1, int kc0, int kc1) {
  constexpr int F0 = ks_lds_floats<T0, NW>(), F1 = ks_lds_floats<T1, NW>();
  __shared__ __attribute__((aligned(16))) float lds[F0 > F1 ? F0 : F1];
  const int b = blockIdx.x;
  if (b < nb0) {
    ksplit_body<0, 1, T0, NW>(g0, b % gx0, b / gx0, 0, kc0, lds);
  } else {
    const int c = b - nb0;
    ksplit_body<1, 0, T1, NW>(g1, c % gx1, c / gx1, 0, kc1, lds);
  }
}

// Workgroup tile: 128 x 128 unless a side is <= 64 (the 64-wide variants waste
// nothing there) or the 128 x 128 grid would leave CUs idle and K is too short
// for split-K to fill them (half-width tiles double the workgroups; measured
// on MI355X, for K >= 4096 full tiles plus split-K are faster).  A function of
// the shape only, as mle_gemm_ws_bytes needs.
struct Tile {
  int wm, wn;         // MFMA blocks per wave along M / N
  int kd = 32;        // K depth of a stage
  bool direct = false;  // register-direct kernel (128 x 128, no LDS in the K loop)
  int tm() const { return 32 * wm; }
  int tn() const { return 32 * wn; }
};

Tile choose_tile(int M, int N, int K, int batch) {
  (void)K;
  if (M <= 64 && N <= 64) return {2, 2};
  if (N <= 64) return {4, 2};
  if (M <= 64) return {2, 4};
  const long long t128 = (long long)((M + 127) / 128) * ((N + 127) / 128) * batch;
  if (t128 >= 192 || K >= 4096) return {4, 4, 16, true};
  return N >= M ? Tile{2, 4} : Tile{4, 2};
}

// Split count: a function of the shape only.  Splits are used when the tile
// grid leaves most of the 256 CUs idle and K is long enough to share.
int choose_splits(int M, int N, int K, int batch, int& kchunk) {
  kchunk = K;
  const Tile t = choose_tile(M, N, K, batch);
  const long long tiles = (long long)((M + t.tm() - 1) / t.tm()) * ((N + t.tn() - 1) / t.tn()) * batch;
  int s, smax;
  if (t.direct) {
    // A grid of >= 3/4 of the 256 CUs runs unsplit.  Below that, at most one
    // workgroup per CU: a few CUs running two would take twice as long as the
    // rest (measured on MI355X: 48 tiles x 8192 deep, 5 splits 113 us against
    // 176 us for 6 and 122 us for 10; 16 tiles: 16 splits best, 64 tiles: 4).
    if (tiles >= 192) return 1;
    s = tiles <= 128 ? (int)(256 / tiles) : 2;
    smax = K / 512;
  } else {
    // Measured on MI355X: with ~256 tiles a split only pays off for long K.
    // A grid of a few tiles is latency-bound (each split walks its K chunk one
    // stage after another), so it takes chunks down to one 32-deep stage: the
    // C1 MLP step went from 0.136 to 0.118 ms with 64-deep chunks, and from
    // 0.065 to 0.057 ms with 32-deep ones (K / 128 or fewer splits: slower).
    if (tiles >= 384 || (tiles >= 128 && K < 4096)) return 1;
    s = (int)((768 + tiles - 1) / tiles);
    smax = tiles <= 16 ? K / 16 : K / 256;
  }
  if (s > smax) s = smax;
  if (s < 2) return 1;
  kchunk = (K + s - 1) / s;
  kchunk = ((kchunk + 31) / 32) * 32;  // whole stages of either depth
  s = (K + kchunk - 1) / kchunk;
  if ((long long)s * batch > 65535) return 1;
  return s;
}

template <int TA, int TB, int WM, int WN, int KD>
void launch_t(hipStream_t s, const GemmArgs& g, dim3 grid, int vec, bool cs) {
  if (vec == 2) {
    if (cs) mle::launch(gemm_kernel<TA, TB, 2, true, WM, WN, KD>, grid, NT, 0, s, g);
    else mle::launch(gemm_kernel<TA, TB, 2, false, WM, WN, KD>, grid, NT, 0, s, g);
  } else if (vec == 1) {
    if (cs) mle::launch(gemm_kernel<TA, TB, 1, true, WM, WN, KD>, grid, NT, 0, s, g);
    else mle::launch(gemm_kernel<TA, TB, 1, false, WM, WN, KD>, grid, NT, 0, s, g);
  } else {
    if (cs) mle::launch(gemm_kernel<TA, TB, 0, true, WM, WN, KD>, grid, NT, 0, s, g);
    else mle::launch(gemm_kernel<TA, TB, 0, false, WM, WN, KD>, grid, NT, 0, s, g);
  }
}

// Direct kernel configuration, measured on MI355X over the C3/C4 shapes:
// 16-deep stages, 3 register sets (2 stages in flight), 2 workgroups per CU.
// Deeper prefetch (up to 8 sets at 1 workgroup per CU), 32-deep stages and
// 8-wave 256 x 128 tiles were all equal or slower: the kernel is held by the
// shader clock it sustains (~2.15 GHz under load), not by load latency.
template <int TA, int TB>
void launch_direct(hipStream_t s, const GemmArgs& g, dim3 grid, bool cs) {
  if (g.kterms > 1) mle::launch(gemm_direct_kernel<TA, TB, false, 16, 3, 2, true>, grid, NT, 0, s, g);
  else if (cs) mle::launch(gemm_direct_kernel<TA, TB, true, 16, 3, 2>, grid, NT, 0, s, g);
  else mle::launch(gemm_direct_kernel<TA, TB, false, 16, 3, 2>, grid, NT, 0, s, g);
}

// Compute units of the current device (queried once per device).
int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <int TA, int TB>
void launch_tile(hipStream_t s, const GemmArgs& g, Tile t, dim3 grid, int vec, bool cs, bool direct_ok) {
  if (t.direct && direct_ok && vec == 2 && g.K % 16 == 0 && g.kchunk % 16 == 0) {
    // More tiles than two per CU, one split, no column sum: the persistent
    // kernel (two workgroups per CU, tiles streamed without per-tile
    // prologues).
    const long long items = (long long)grid.x * grid.y * grid.z;
    const int ncu = cu_count();
    const bool c_buf = ((double)(g.M - 1) * (double)g.ldc + g.N) * 4.0 < 2147483648.0 - 64;
    if (g.splits == 1 && g.kterms == 1 && !cs && g.K >= 64 && g.K % 64 == 0 && items > 2 * ncu &&
        items < (1LL << 30) && c_buf) {
      if (g.rowpart)
        mle::launch(gemm_stream_kernel<TA, TB, 16, 4, kEpiRowstats>, dim3((unsigned)(2 * ncu)), NT, 0, s, g,
                    (int)grid.x, (int)grid.y, (int)items);
      else
        mle::launch(gemm_stream_kernel<TA, TB, 16, 4>, dim3((unsigned)(2 * ncu)), NT, 0, s, g, (int)grid.x,
                    (int)grid.y, (int)items);
    } else {
      launch_direct<TA, TB>(s, g, grid, cs);
    }
  } else if (t.wm == 4 && t.wn == 4) {
    if (t.kd == 16) launch_t<TA, TB, 4, 4, 16>(s, g, grid, vec, cs);
    else launch_t<TA, TB, 4, 4, 32>(s, g, grid, vec, cs);
  } else if (t.wm == 4) {
    launch_t<TA, TB, 4, 2, 32>(s, g, grid, vec, cs);
  } else if (t.wn == 4) {
    launch_t<TA, TB, 2, 4, 32>(s, g, grid, vec, cs);
  } else {
    launch_t<TA, TB, 2, 2, 32>(s, g, grid, vec, cs);
  }
}

// Bytes spanned by one batch item of an operand stored rows x cols with leading dimension ld.
double extent_bytes(int rows, int cols, int64_t ld) { return ((double)(rows - 1) * (double)ld + cols) * 4.0; }

}  // namespace

// A GEMM call resolved to its arguments, tile shape, grid and kernel family.
struct GemmPlan {
  GemmArgs g;
  Tile tile;
  dim3 grid;
  int vec = 0, which = 0;
  bool cs = false, direct_ok = false, empty = false;
  bool simple = false;  // gemm_simple_kernel: one thread per C element, no split
  bool ksplit = false;  // gemm_ksplit_kernel: K split over a workgroup's waves
  int ks_nw = 16;       // its waves per workgroup
  int ks_kc = 0;        // and K range per wave
  double flop = 0, bytes = 0;
};

// Products small enough for gemm_simple_kernel: M of at most 4, K of at most
// 16 or at most 4096 outputs, and at most 4 Mi multiply-adds (one batch
// level, no sum of terms).
// Measured on MI355X with the C1 MLP's products (one launch each, launch
// included): 64 x 10 x 256 4.2 us against 7.6 for split K + reduce; 64 x 256
// x 10 3.9 against 7.2; 256 x 10 x 64 4.1 against 8.4; but 784 x 256 x 64
// 8.1 against 7.0 and 64 x 784 x 256 11.4 against 8.5 on the tile kernels.
static bool simple_shape(int M, int N, int K, int batch, int inner, int terms) {
  return (M <= 4 || K <= 16 || (double)M * N * batch <= 4096.0) &&
         (double)M * N * (double)(K > 0 ? K : 1) * batch <= 4194304.0 && inner == 1 && terms <= 1 &&
         (double)M * N <= 64.0 * 2147483647.0 && batch <= 65535;
}

// Products for gemm_ksplit_kernel: at most 256 Ki outputs and no sum of
// terms, with a K long enough to share over 16 waves but short enough that
// one workgroup's products stay a few microseconds of its CU's matrix cores
// (2 K cycles per SIMD for 16-wide tiles, 8 K for 32-wide).  Tiles of 32 when
// that still gives 128 workgroups, else 16.
static int ksplit_tile(int M, int N, int batch) {
  const long long t32 = (long long)((M + 31) / 32) * ((N + 31) / 32) * batch;
  return t32 >= 128 ? 32 : 16;
}
static bool ksplit_shape(int M, int N, int K, int batch, int terms) {
  if (terms > 1 || K < 32 || (double)M * N * batch > 262144.0) return false;
  const int tt = ksplit_tile(M, N, batch);
  return K <= (tt == 16 ? 4096 : 1024) && (M + tt - 1) / tt <= 65535 && batch <= 65535;
}
// Waves per workgroup: 16 for a long K (one memory latency per 64-deep chunk
// of each wave), 4 when K <= 256 (each wave's share still fits one chunk, and
// the partial tiles to add are fewer).
static int ksplit_nw(int K) { return K <= 256 ? 4 : 16; }
// K range of one wave: whole 16-deep slabs.
static int ksplit_kc(int K, int nw) { return ((K + nw - 1) / nw + 15) / 16 * 16; }

const char* const kFamily[4] = {"gemm_nn", "gemm_nt", "gemm_tn", "gemm_tt"};

static int gemm_plan(GemmPlan& P, int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A,
                     int64_t lda, int64_t stride_a, const float* B, int64_t ldb, int64_t stride_b, float beta, float* C,
                     int64_t ldc, int64_t stride_c, int batch, float* colsum, const float* bias, void* ws,
                     size_t ws_bytes, int inner = 1, int64_t sa2 = 0, int64_t sb2 = 0, int64_t sc2 = 0,
                     int64_t sbias = 0, int64_t scs = 0, int terms = 0, int64_t gsa = 0, int64_t gsb = 0) {
  MLE_CHECK_ARG(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "mle_gemm: negative size");
  P.empty = M == 0 || N == 0 || batch == 0;
  if (P.empty) return MLE_OK;
  MLE_CHECK_ARG(C != nullptr && (K == 0 || (A != nullptr && B != nullptr)), "mle_gemm: null operand");
  MLE_CHECK_ARG(ldc >= N, "mle_gemm: ldc %lld < N %d", (long long)ldc, N);
  MLE_CHECK_ARG(lda >= (trans_a ? M : K) && ldb >= (trans_b ? K : N), "mle_gemm: leading dimension too small");
  MLE_CHECK_ARG(colsum == nullptr || batch == 1 || scs != 0, "mle_gemm: fused colsum over a batch needs a stride");
  const Tile tile = choose_tile(M, N, K, batch);
  MLE_CHECK_ARG((M + tile.tm() - 1) / tile.tm() <= 65535 && batch <= 65535, "mle_gemm: grid too large (M %d, batch %d)",
                M, batch);
  MLE_CHECK_ARG(inner >= 1 && batch % inner == 0, "mle_gemm: batch %d not a multiple of inner %d", batch, inner);
  GemmArgs g{A,    B,    C,       colsum,  lda,  ldb,    ldc,  stride_a, stride_b, stride_c, M,    N,   K,
             alpha, beta, 1,       K,       nullptr, nullptr, bias, inner,    sa2,      sb2,      sc2,      sbias, scs,
             0,     gsa,  gsb,     1,       nullptr, 0,       nullptr, nullptr, nullptr, 0};
  const bool v4 = (lda % 4 == 0) && (ldb % 4 == 0) && (stride_a % 4 == 0) && (stride_b % 4 == 0) &&
                  (sa2 % 4 == 0) && (sb2 % 4 == 0) && (gsa % 4 == 0) && (gsb % 4 == 0) && aligned16(A) &&
                  aligned16(B);
  // Buffer loads need the contiguous bound of each operand to be a multiple of
  // 4 and every extent (all terms of a sum) addressable with a 31-bit offset.
  const int a_rows = trans_a ? K : M, a_cols = trans_a ? M : K;
  const int b_rows = trans_b ? N : K, b_cols = trans_b ? K : N;
  const double t_extra = terms > 1 ? (double)(terms - 1) : 0.0;
  const bool buf = v4 && a_cols % 4 == 0 && b_cols % 4 == 0 && K > 0 &&
                   extent_bytes(a_rows, a_cols, lda) + t_extra * 4.0 * (double)gsa < 2147483648.0 - 64 &&
                   extent_bytes(b_rows, b_cols, ldb) + t_extra * 4.0 * (double)gsb < 2147483648.0 - 64;
  const int vec = buf ? 2 : (v4 ? 1 : 0);
  const bool cs = colsum != nullptr;
  // The direct kernel stores 16-byte row segments of C (and reads bias as float4).
  const bool direct_ok = N % 4 == 0 && ldc % 4 == 0 && stride_c % 4 == 0 && sc2 % 4 == 0 && aligned16(C) &&
                         (bias == nullptr || (aligned16(bias) && sbias % 4 == 0));
  if (terms > 1) {
    // Sum of `terms` products.  The workspace is part of the contract either
    // way.  On the register-direct kernel the terms extend its K loop (one
    // accumulator, terms in order, no partials); otherwise one split per
    // term, reduced in term order.
    const size_t need = ((size_t)terms * batch * M * N + (size_t)terms * batch * N) * sizeof(float);
    MLE_CHECK_ARG(ws && ws_bytes >= need, "mle_gemm_sum: workspace of %zu bytes needed", need);
    MLE_CHECK_ARG(terms * batch <= 65535, "mle_gemm_sum: too many terms");
    if (tile.direct && direct_ok && vec == 2 && K % 16 == 0 && (long long)terms * (K / 16) < (1LL << 24)) {
      g.kterms = terms;
    } else {
      g.grouped = 1;
      g.splits = terms;
      g.part = static_cast<float*>(ws);
      g.part_cs = g.part + (size_t)terms * batch * M * N;
    }
  } else {
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
  }
  if (simple_shape(M, N, K, batch, inner, terms)) {
    g.splits = 1;
    g.kchunk = K;
    g.part = g.part_cs = nullptr;
    P.simple = true;
  } else if (ksplit_shape(M, N, K, batch, terms)) {
    g.splits = 1;
    g.kchunk = K;
    g.part = g.part_cs = nullptr;
    P.ksplit = true;
    P.ks_nw = ksplit_nw(K);
    P.ks_kc = ksplit_kc(K, P.ks_nw);
  }
  P.g = g;
  P.tile = tile;
  P.grid = dim3((N + tile.tn() - 1) / tile.tn(), (M + tile.tm() - 1) / tile.tm(), batch * g.splits);
  if (P.ksplit) {
    const int tt = ksplit_tile(M, N, batch);
    P.grid = dim3((N + tt - 1) / tt, (M + tt - 1) / tt, batch);
  }
  P.vec = vec;
  P.cs = cs;
  P.direct_ok = direct_ok;
  P.which = (trans_a ? 2 : 0) + (trans_b ? 1 : 0);
  P.flop = 2.0 * M * (double)N * K * batch * (terms > 1 ? terms : 1);
  P.bytes = 4.0 * batch * ((double)M * K + (double)K * N + (double)M * N * (beta != 0.f ? 2 : 1));
  return MLE_OK;
}

static void gemm_launch_main(hipStream_t s, const GemmPlan& P) {
  if (P.simple) {
    const dim3 grid((unsigned)(((int64_t)P.g.M * P.g.N + 63) / 64), P.grid.z);
    switch (P.which) {
      case 0: mle::launch(gemm_simple_kernel<0, 0>, grid, 256, 0, s, P.g); break;
      case 1: mle::launch(gemm_simple_kernel<0, 1>, grid, 256, 0, s, P.g); break;
      case 2: mle::launch(gemm_simple_kernel<1, 0>, grid, 256, 0, s, P.g); break;
      default: mle::launch(gemm_simple_kernel<1, 1>, grid, 256, 0, s, P.g); break;
    }
    return;
  }
  if (P.ksplit) {
    const bool t32 = ksplit_tile(P.g.M, P.g.N, (int)P.grid.z) == 32;
    const int kc = P.ks_kc;
    if (P.ks_nw == 4) {
      switch (P.which * 2 + (t32 ? 1 : 0)) {
        case 0: mle::launch(gemm_ksplit_kernel<0, 0, 16, 4>, P.grid, 256, 0, s, P.g, kc); break;
        case 1: mle::launch(gemm_ksplit_kernel<0, 0, 32, 4>, P.grid, 256, 0, s, P.g, kc); break;
        case 2: mle::launch(gemm_ksplit_kernel<0, 1, 16, 4>, P.grid, 256, 0, s, P.g, kc); break;
        case 3: mle::launch(gemm_ksplit_kernel<0, 1, 32, 4>, P.grid, 256, 0, s, P.g, kc); break;
        case 4: mle::launch(gemm_ksplit_kernel<1, 0, 16, 4>, P.grid, 256, 0, s, P.g, kc); break;
        case 5: mle::launch(gemm_ksplit_kernel<1, 0, 32, 4>, P.grid, 256, 0, s, P.g, kc); break;
        case 6: mle::launch(gemm_ksplit_kernel<1, 1, 16, 4>, P.grid, 256, 0, s, P.g, kc); break;
        default: mle::launch(gemm_ksplit_kernel<1, 1, 32, 4>, P.grid, 256, 0, s, P.g, kc); break;
      }
    } else {
      switch (P.which * 2 + (t32 ? 1 : 0)) {
        case 0: mle::launch(gemm_ksplit_kernel<0, 0, 16, 16>, P.grid, 1024, 0, s, P.g, kc); break;
        case 1: mle::launch(gemm_ksplit_kernel<0, 0, 32, 16>, P.grid, 1024, 0, s, P.g, kc); break;
        case 2: mle::launch(gemm_ksplit_kernel<0, 1, 16, 16>, P.grid, 1024, 0, s, P.g, kc); break;
        case 3: mle::launch(gemm_ksplit_kernel<0, 1, 32, 16>, P.grid, 1024, 0, s, P.g, kc); break;
        case 4: mle::launch(gemm_ksplit_kernel<1, 0, 16, 16>, P.grid, 1024, 0, s, P.g, kc); break;
        case 5: mle::launch(gemm_ksplit_kernel<1, 0, 32, 16>, P.grid, 1024, 0, s, P.g, kc); break;
        case 6: mle::launch(gemm_ksplit_kernel<1, 1, 16, 16>, P.grid, 1024, 0, s, P.g, kc); break;
        default: mle::launch(gemm_ksplit_kernel<1, 1, 32, 16>, P.grid, 1024, 0, s, P.g, kc); break;
      }
    }
    return;
  }
  switch (P.which) {
    case 0: launch_tile<0, 0>(s, P.g, P.tile, P.grid, P.vec, P.cs, P.direct_ok); break;
    case 1: launch_tile<0, 1>(s, P.g, P.tile, P.grid, P.vec, P.cs, P.direct_ok); break;
    case 2: launch_tile<1, 0>(s, P.g, P.tile, P.grid, P.vec, P.cs, P.direct_ok); break;
    default: launch_tile<1, 1>(s, P.g, P.tile, P.grid, P.vec, P.cs, P.direct_ok); break;
  }
}

static void gemm_launch_reduce(hipStream_t s, const GemmPlan& P) {
  const GemmArgs& g = P.g;
  if (g.splits <= 1) return;
  const bool rv = g.N % 4 == 0 && g.ldc % 4 == 0 && g.sc % 4 == 0 && g.sc2 % 4 == 0 && aligned16(g.C) &&
                  aligned16(g.part) && (!g.bias || (aligned16(g.bias) && g.sbias % 4 == 0));
  const int w = rv ? 4 : 1;
  const int batch = (int)P.grid.z / g.splits;
  const int64_t units = (int64_t)batch * g.M * (g.N / w);
  const unsigned nmain = (unsigned)((units + 63) / 64);
  const unsigned ncs = g.colsum ? (unsigned)(((int64_t)batch * g.N + 255) / 256) : 0u;
  if (rv) mle::launch(split_reduce_kernel<true>, nmain + ncs, 256, 0, s, g, units, nmain);
  else mle::launch(split_reduce_kernel<false>, nmain + ncs, 256, 0, s, g, units, nmain);
}

// Work items of a plan that launch_tile would run on gemm_direct_kernel (one
// per workgroup), or 0 when it would pick another kernel.
static long long direct_items(const GemmPlan& P) {
  const GemmArgs& g = P.g;
  if (P.empty || P.simple || P.ksplit ||
      !(P.tile.direct && P.direct_ok && P.vec == 2 && g.K % 16 == 0 && g.kchunk % 16 == 0))
    return 0;
  const long long items = (long long)P.grid.x * P.grid.y * P.grid.z;
  const bool c_buf = ((double)(g.M - 1) * (double)g.ldc + g.N) * 4.0 < 2147483648.0 - 64;
  const bool stream = g.splits == 1 && g.kterms == 1 && !P.cs && g.K >= 64 && g.K % 64 == 0 &&
                      items > 2 * cu_count() && items < (1LL << 30) && c_buf;
  return stream ? 0 : items;
}

// True when launch_tile would run the plan on the persistent kernel.
static bool uses_stream(const GemmPlan& P) {
  const GemmArgs& g = P.g;
  if (P.empty || P.simple || P.ksplit ||
      !(P.tile.direct && P.direct_ok && P.vec == 2 && g.K % 16 == 0 && g.kchunk % 16 == 0))
    return false;
  return direct_items(P) == 0;
}

// The persistent kernel with an activation epilogue (plan already known to
// run on it).
template <int TA, int TB, int EPI>
static void launch_stream_act(hipStream_t s, const GemmPlan& P, int kind) {
  const dim3 grid((unsigned)(2 * cu_count()));
  const int gx = (int)P.grid.x, gy = (int)P.grid.y, items = (int)((long long)P.grid.x * P.grid.y * P.grid.z);
  switch (kind) {
    case MLE_RELU: mle::launch(gemm_stream_kernel<TA, TB, 16, 4, EPI, MLE_RELU>, grid, NT, 0, s, P.g, gx, gy, items); break;
    case MLE_GELU: mle::launch(gemm_stream_kernel<TA, TB, 16, 4, EPI, MLE_GELU>, grid, NT, 0, s, P.g, gx, gy, items); break;
    default: mle::launch(gemm_stream_kernel<TA, TB, 16, 4, EPI, MLE_SILU>, grid, NT, 0, s, P.g, gx, gy, items); break;
  }
}

static bool epilogue_act(int kind) { return kind == MLE_RELU || kind == MLE_GELU || kind == MLE_SILU; }

static int gemm_impl(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A,
                     int64_t lda, int64_t stride_a, const float* B, int64_t ldb, int64_t stride_b, float beta, float* C,
                     int64_t ldc, int64_t stride_c, int batch, float* colsum, const float* bias, void* ws,
                     size_t ws_bytes, int inner = 1, int64_t sa2 = 0, int64_t sb2 = 0, int64_t sc2 = 0,
                     int64_t sbias = 0, int64_t scs = 0, int terms = 0, int64_t gsa = 0, int64_t gsb = 0) {
  GemmPlan P;
  const int rc = gemm_plan(P, trans_a, trans_b, M, N, K, alpha, A, lda, stride_a, B, ldb, stride_b, beta, C, ldc,
                           stride_c, batch, colsum, bias, ws, ws_bytes, inner, sa2, sb2, sc2, sbias, scs, terms, gsa,
                           gsb);
  if (rc != MLE_OK || P.empty) return rc;
  hipStream_t s = as_stream(stream);
  {
    // The probe times the whole product: the GEMM kernel and, with split K,
    // the reduce that completes C.
    ProbeScope probe(kFamily[P.which], s, P.flop, P.bytes);
    gemm_launch_main(s, P);
    gemm_launch_reduce(s, P);
  }
  return check_launch(kFamily[P.which]);
}

extern "C" {

size_t mle_gemm_ws_bytes(int M, int N, int K, int batch) {
  int kchunk;
  const int splits = choose_splits(M, N, K, batch, kchunk);
  if (splits <= 1) return 0;
  return ((size_t)splits * batch * M * N + (size_t)splits * batch * N) * sizeof(float);
}

size_t mle_gemm_sum_ws_bytes(int M, int N, int terms) {
  if (terms <= 1) return 0;
  return ((size_t)terms * M * N + (size_t)terms * N) * sizeof(float);
}

int mle_gemm_batched_ex(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A,
                        int64_t lda, int64_t stride_a, const float* B, int64_t ldb, int64_t stride_b, float beta,
                        float* C, int64_t ldc, int64_t stride_c, int batch, float* colsum, int64_t stride_colsum,
                        const float* bias, int64_t stride_bias, void* ws, size_t ws_bytes) {
  return gemm_impl(stream, trans_a, trans_b, M, N, K, alpha, A, lda, stride_a, B, ldb, stride_b, beta, C, ldc,
                   stride_c, batch, colsum, bias, ws, ws_bytes, 1, 0, 0, 0, stride_bias, stride_colsum);
}

int mle_gemm_sum(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A,
                 int64_t lda, int64_t stride_a_term, const float* B, int64_t ldb, int64_t stride_b_term, float beta,
                 float* C, int64_t ldc, int terms, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(terms >= 1, "mle_gemm_sum: terms %d", terms);
  return gemm_impl(stream, trans_a, trans_b, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1, nullptr,
                   nullptr, ws, ws_bytes, 1, 0, 0, 0, 0, 0, terms, stride_a_term, stride_b_term);
}

int mle_gemm_rowstats(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A,
                      int64_t lda, const float* B, int64_t ldb, float beta, float* C, int64_t ldc, const float* bias,
                      float* rowpart, int64_t ldp, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(rowpart != nullptr && ldp >= 2 * (int64_t)((N + 63) / 64) && (ldp % 2) == 0 &&
                    (reinterpret_cast<uintptr_t>(rowpart) & 7) == 0,
                "mle_gemm_rowstats: rowpart needs %d float pairs per row (8-byte aligned)", (N + 63) / 64);
  GemmPlan P;
  const int rc = gemm_plan(P, trans_a, trans_b, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1, nullptr,
                           bias, ws, ws_bytes);
  if (rc != MLE_OK || P.empty) return rc;
  hipStream_t s = as_stream(stream);
  const bool fused = uses_stream(P);
  if (fused) P.g.rowpart = rowpart, P.g.rp_ld = ldp;
  {
    ProbeScope probe(kFamily[P.which], s, P.flop, P.bytes);
    gemm_launch_main(s, P);
  }
  gemm_launch_reduce(s, P);
  if (!fused) {
    const int64_t waves = (int64_t)M * ((N + 63) / 64);
    MLE_CHECK_ARG((waves + 3) / 4 <= 2147483647LL, "mle_gemm_rowstats: too many rows");
    mle::launch(rowstats_kernel, (unsigned)((waves + 3) / 4), 256, 0, s, C, ldc, M, N, rowpart, ldp);
  }
  return check_launch("mle_gemm_rowstats");
}

int mle_gemm_act_fwd(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A,
                     int64_t lda, const float* B, int64_t ldb, float beta, float* C, const float* bias, int kind,
                     float* Y, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(Y != nullptr && kind >= MLE_RELU && kind <= MLE_LEAKY_RELU, "mle_gemm_act_fwd: bad argument");
  GemmPlan P;
  int rc = gemm_plan(P, trans_a, trans_b, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, N, 0, 1, nullptr, bias, ws,
                     ws_bytes);
  if (rc != MLE_OK || P.empty) return rc;
  hipStream_t s = as_stream(stream);
  if (uses_stream(P) && P.which == 0 && epilogue_act(kind) && aligned16(Y)) {
    P.g.act_y = Y;
    {
      ProbeScope probe(kFamily[P.which], s, P.flop, P.bytes);
      launch_stream_act<0, 0, kEpiActFwd>(s, P, kind);
    }
    return check_launch("mle_gemm_act_fwd");
  }
  // Split K: the reduce that completes C writes Y too; on the K-split kernel
  // its epilogue does.
  if ((P.g.splits > 1 && aligned16(Y)) || P.ksplit) {
    P.g.act_y = Y;
    P.g.act_red = 1 + kind;
    ProbeScope probe(kFamily[P.which], s, P.flop, P.bytes);
    gemm_launch_main(s, P);
    gemm_launch_reduce(s, P);
    return check_launch("mle_gemm_act_fwd");
  }
  {
    ProbeScope probe(kFamily[P.which], s, P.flop, P.bytes);
    gemm_launch_main(s, P);
  }
  gemm_launch_reduce(s, P);
  rc = check_launch("mle_gemm_act_fwd");
  if (rc != MLE_OK) return rc;
  return mle_act_fwd(stream, kind, C, Y, (size_t)M * N);
}

int mle_gemm_act_bwd(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A,
                     int64_t lda, const float* B, int64_t ldb, float beta, float* C, int kind, const float* X,
                     float* dX, int accumulate_dx, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(X != nullptr && dX != nullptr && kind >= MLE_RELU && kind <= MLE_LEAKY_RELU,
                "mle_gemm_act_bwd: bad argument");
  GemmPlan P;
  int rc = gemm_plan(P, trans_a, trans_b, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, N, 0, 1, nullptr, nullptr,
                     ws, ws_bytes);
  if (rc != MLE_OK || P.empty) return rc;
  hipStream_t s = as_stream(stream);
  if (P.simple || P.ksplit) {  // the small-product kernels' epilogue
    P.g.act_x = X;
    P.g.act_dx = dX;
    P.g.act_acc = accumulate_dx ? 1 : 0;
    P.g.act_bwd = 1 + kind;
    {
      ProbeScope probe(kFamily[P.which], s, P.flop, P.bytes);
      gemm_launch_main(s, P);
    }
    return check_launch("mle_gemm_act_bwd");
  }
  if (uses_stream(P) && P.which == 1 && epilogue_act(kind) && aligned16(X) && aligned16(dX)) {
    P.g.act_x = X;
    P.g.act_dx = dX;
    P.g.act_acc = accumulate_dx ? 1 : 0;
    {
      ProbeScope probe(kFamily[P.which], s, P.flop, P.bytes);
      launch_stream_act<0, 1, kEpiActBwd>(s, P, kind);
    }
    return check_launch("mle_gemm_act_bwd");
  }
  {
    ProbeScope probe(kFamily[P.which], s, P.flop, P.bytes);
    gemm_launch_main(s, P);
  }
  gemm_launch_reduce(s, P);
  rc = check_launch("mle_gemm_act_bwd");
  if (rc != MLE_OK) return rc;
  return mle_act_bwd(stream, kind, X, C, dX, (size_t)M * N, accumulate_dx);
}

}  // extern "C"

// A Linear whose weight gradient is one round of unsplit register-direct
// tiles (192 to 256 tiles of 128 x 128: one workgroup, so one wave, per CU
// and SIMD) and whose input gradient has too many tiles to share a launch
// with it: the weight gradient then runs as two K splits (two workgroups per
// CU, as the input gradient runs) and a reduce.  A function of the shape
// only, as the workspace size must be (C3: 8192 x 1024 x 4096).
static bool dw_two_splits(int rows, int in, int out, int layers) {
  if (layers != 1 || rows < 4096 || rows % 32 != 0) return false;
  const Tile tw = choose_tile(in, out, rows, 1), tx = choose_tile(rows, in, out, 1);
  const long long nw = (long long)((in + 127) / 128) * ((out + 127) / 128);
  const long long nx = (long long)((rows + 127) / 128) * ((in + 127) / 128);
  return tw.direct && tx.direct && nw >= 192 && nw <= 256 && nx > 256;
}

extern "C" {

size_t mle_linear_bwd_ws_bytes(int rows, int in, int out, int layers) {
  const size_t dx = layers > 1 ? mle_gemm_sum_ws_bytes(rows, in, layers) : mle_gemm_ws_bytes(rows, in, out, 1);
  size_t dw = mle_gemm_ws_bytes(in, out, rows, layers);
  if (dw_two_splits(rows, in, out, layers))
    dw = std::max(dw, (2 * (size_t)in * out + 2 * (size_t)out) * sizeof(float));
  return std::max(dx, dw);
}

int mle_linear_bwd(mle_stream stream, int rows, int in, int out, int layers, const float* X, const float* dY,
                   int64_t stride_dy, const float* W, int64_t stride_w, float* dX, int accumulate_dx, float* dW,
                   float* db, int64_t stride_db, void* ws, size_t ws_bytes) {
  return mle_linear_bwd_ex(stream, rows, in, out, layers, X, dY, stride_dy, W, stride_w, dX, accumulate_dx, dW, db,
                           stride_db, 1, ws, ws_bytes);
}

}  // extern "C"

// Linear backward, optionally with the backward of the activation whose
// output is X' = this layer's input: act_dx (+)= act'(act_x) * dX (act_kind
// < 0: none).  On the small-product kernels the activation gradient is their
// epilogue; otherwise it is a pass after the products.
static int linear_bwd_impl(mle_stream stream, int rows, int in, int out, int layers, const float* X, const float* dY,
                           int64_t stride_dy, const float* W, int64_t stride_w, float* dX, int accumulate_dx,
                           float* dW, float* db, int64_t stride_db, int accumulate_dw, int act_kind,
                           const float* act_x, float* act_dx, int act_acc, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(rows >= 0 && in >= 0 && out >= 0 && layers >= 1, "mle_linear_bwd: bad sizes");
  MLE_CHECK_ARG(layers == 1 || (stride_dy != 0 && stride_w != 0 && (db == nullptr || stride_db != 0)),
                "mle_linear_bwd: %d layers need strides", layers);
  MLE_CHECK_ARG(ws_bytes >= mle_linear_bwd_ws_bytes(rows, in, out, layers) && (ws || ws_bytes == 0),
                "mle_linear_bwd: workspace of %zu bytes needed", mle_linear_bwd_ws_bytes(rows, in, out, layers));
  // dX (+)= sum_l dY_l W_l^T: NT, rows x in, depth out (terms over layers).
  GemmPlan P0, P1;
  int rc = gemm_plan(P0, 0, 1, rows, in, out, 1.0f, dY, out, 0, W, out, 0, accumulate_dx ? 1.0f : 0.0f, dX, in, 0, 1,
                     nullptr, nullptr, ws, ws_bytes, 1, 0, 0, 0, 0, 0, layers > 1 ? layers : 0, stride_dy, stride_w);
  if (rc != MLE_OK) return rc;
  // dW_l (+)= X^T dY_l and db_l (+)= colsum dY_l: TN, in x out, depth rows.
  rc = gemm_plan(P1, 1, 0, in, out, rows, 1.0f, X, in, 0, dY, out, stride_dy, accumulate_dw ? 1.0f : 0.0f, dW, out,
                 stride_w, layers, db, nullptr, ws, ws_bytes, 1, 0, 0, 0, 0, stride_db);
  if (rc != MLE_OK) return rc;
  P1.g.cs_assign = accumulate_dw ? 0 : 1;
  hipStream_t s = as_stream(stream);
  bool act_done = act_kind < 0 || P0.empty;
  if (!act_done && (P0.simple || P0.ksplit)) {
    P0.g.act_bwd = 1 + act_kind;
    P0.g.act_x = act_x;
    P0.g.act_dx = act_dx;
    P0.g.act_acc = act_acc ? 1 : 0;
    act_done = true;
  }
  // The activation pass when no epilogue took it.
  auto finish = [&](int code) {
    if (code != MLE_OK || act_done) return code;
    return mle_act_bwd(stream, act_kind, act_x, dX, act_dx, (size_t)rows * in, act_acc);
  };
  const int ncu = cu_count();
  if (dw_two_splits(rows, in, out, layers) && P1.g.splits == 1 && direct_items(P1) > 0 && direct_items(P1) <= ncu &&
      direct_items(P0) > ncu && P1.g.K % 32 == 0) {
    P1.g.splits = 2;
    P1.g.kchunk = P1.g.K / 2;
    P1.g.part = static_cast<float*>(ws);
    P1.g.part_cs = P1.g.part + 2 * (size_t)P1.g.M * P1.g.N;
    P1.grid.z = 2;
  }
  const long long n0 = direct_items(P0), n1 = direct_items(P1);
  // Both small (gemm_simple_kernel, one batch item): one launch.
  if (!P0.empty && !P1.empty && P0.simple && P1.simple && P0.grid.z == 1 && P1.grid.z == 1) {
    const unsigned nb0 = (unsigned)(((int64_t)P0.g.M * P0.g.N + 63) / 64);
    const unsigned nb1 = (unsigned)(((int64_t)P1.g.M * P1.g.N + 63) / 64);
    {
      ProbeScope probe("gemm_pair", s, P0.flop + P1.flop, P0.bytes + P1.bytes);
      mle::launch(gemm_simple_pair_kernel, dim3(nb0 + nb1, 1), 256, 0, s, P0.g, P1.g, (int)nb0);
    }
    return finish(check_launch("gemm_pair"));
  }
  // Both on the K-split kernel (one batch item): one launch.
  if (!P0.empty && !P1.empty && P0.ksplit && P1.ksplit && P0.grid.z == 1 && P1.grid.z == 1) {
    const int gx0 = (int)P0.grid.x, gx1 = (int)P1.grid.x;
    const int nb0 = gx0 * (int)P0.grid.y, nb1 = gx1 * (int)P1.grid.y;
    const bool w0 = ksplit_tile(P0.g.M, P0.g.N, 1) == 32, w1 = ksplit_tile(P1.g.M, P1.g.N, 1) == 32;
    // one workgroup size for both: the larger wave count, K ranges re-cut for it
    const int nw = std::max(P0.ks_nw, P1.ks_nw);
    const int kc0 = ksplit_kc(P0.g.K, nw), kc1 = ksplit_kc(P1.g.K, nw);
    auto k = nw == 4 ? (w0 ? (w1 ? gemm_ksplit_pair_kernel<32, 32, 4> : gemm_ksplit_pair_kernel<32, 16, 4>)
                           : (w1 ? gemm_ksplit_pair_kernel<16, 32, 4> : gemm_ksplit_pair_kernel<16, 16, 4>))
                     : (w0 ? (w1 ? gemm_ksplit_pair_kernel<32, 32, 16> : gemm_ksplit_pair_kernel<32, 16, 16>)
                           : (w1 ? gemm_ksplit_pair_kernel<16, 32, 16> : gemm_ksplit_pair_kernel<16, 16, 16>));
    {
      ProbeScope probe("gemm_pair", s, P0.flop + P1.flop, P0.bytes + P1.bytes);
      mle::launch(k, dim3((unsigned)(nb0 + nb1)), 64 * nw, 0, s, P0.g, P1.g, nb0, gx0, gx1, kc0, kc1);
    }
    return finish(check_launch("gemm_pair"));
  }
  // One launch when both would run on the register-direct kernel at most one
  // workgroup per CU each, and the dX product needs no workspace (the dW
  // product's split partials own it).
  if (n0 > 0 && n1 > 0 && n0 <= ncu && n1 <= ncu && P0.g.splits == 1) {
    const int start1 = (int)((n0 + 7) / 8 * 8);
    const PairGrid pg{(int)n0, (int)P0.grid.x, (int)P0.grid.y, (int)n1, (int)P1.grid.x, (int)P1.grid.y, start1};
    const dim3 grid((unsigned)(start1 + n1));
    const bool t0 = P0.g.kterms > 1;
    {
      ProbeScope probe("gemm_pair", s, P0.flop + P1.flop, P0.bytes + P1.bytes);
      auto k = t0 ? (P1.cs ? gemm_pair_kernel<0, 1, false, true, 1, 0, true, false>
                           : gemm_pair_kernel<0, 1, false, true, 1, 0, false, false>)
                  : (P1.cs ? gemm_pair_kernel<0, 1, false, false, 1, 0, true, false>
                           : gemm_pair_kernel<0, 1, false, false, 1, 0, false, false>);
      mle::launch(k, grid, NT, 0, s, P0.g, P1.g, pg);
      gemm_launch_reduce(s, P1);
    }
    return finish(check_launch("gemm_pair"));
  }
  // Otherwise one launch each, in order (they may share the workspace).  (A
  // dX on the persistent kernel writing the activation's gradient in its
  // epilogue measured slower in the C4 step than the separate pass.)
  if (!P0.empty) {
    ProbeScope probe(kFamily[P0.which], s, P0.flop, P0.bytes);
    gemm_launch_main(s, P0);
    gemm_launch_reduce(s, P0);
  }
  rc = check_launch(kFamily[P0.which]);
  if (rc != MLE_OK || P1.empty) return finish(rc);
  {
    ProbeScope probe(kFamily[P1.which], s, P1.flop, P1.bytes);
    gemm_launch_main(s, P1);
    gemm_launch_reduce(s, P1);
  }
  return finish(check_launch(kFamily[P1.which]));
}


extern "C" {

int mle_linear_bwd_ex(mle_stream stream, int rows, int in, int out, int layers, const float* X, const float* dY,
                      int64_t stride_dy, const float* W, int64_t stride_w, float* dX, int accumulate_dx, float* dW,
                      float* db, int64_t stride_db, int accumulate_dw, void* ws, size_t ws_bytes) {
  return linear_bwd_impl(stream, rows, in, out, layers, X, dY, stride_dy, W, stride_w, dX, accumulate_dx, dW, db,
                         stride_db, accumulate_dw, -1, nullptr, nullptr, 0, ws, ws_bytes);
}

int mle_linear_bwd_act(mle_stream stream, int rows, int in, int out, const float* X, const float* dY,
                       const float* W, float* dX, int accumulate_dx, float* dW, float* db, int accumulate_dw,
                       int act_kind, const float* act_x, float* act_dx, int act_accumulate, void* ws,
                       size_t ws_bytes) {
  MLE_CHECK_ARG(act_kind >= MLE_RELU && act_kind <= MLE_LEAKY_RELU && act_x != nullptr && act_dx != nullptr,
                "mle_linear_bwd_act: bad activation argument");
  MLE_CHECK_ARG(act_dx != dX && act_dx != dY && act_dx != X && act_dx != W,
                "mle_linear_bwd_act: act_dx must not alias X, dY, W or dX");
  return linear_bwd_impl(stream, rows, in, out, 1, X, dY, 0, W, 0, dX, accumulate_dx, dW, db, 0, accumulate_dw,
                         act_kind, act_x, act_dx, act_accumulate, ws, ws_bytes);
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

int mle_gemm_grid(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A,
                  int64_t lda, int64_t sa_outer, int64_t sa_inner, const float* B, int64_t ldb, int64_t sb_outer,
                  int64_t sb_inner, float beta, float* C, int64_t ldc, int64_t sc_outer, int64_t sc_inner, int outer,
                  int inner, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(outer >= 0 && inner >= 1, "mle_gemm_grid: bad batch grid %d x %d", outer, inner);
  return gemm_impl(stream, trans_a, trans_b, M, N, K, alpha, A, lda, sa_outer, B, ldb, sb_outer, beta, C, ldc,
                   sc_outer, outer * inner, nullptr, nullptr, ws, ws_bytes, inner, sa_inner, sb_inner, sc_inner);
}

}  // extern "C"
