// Fused multi-head attention with the reference's column-normalised softmax.
//
// MultiHeadAttention (Engine/transformer.cu:647-661) runs, per head h of a
// [batch, 1, seq, heads * 64] projection:
//   S = scale * Q_h K_h^T                        (BMMABT + Scale, Engine/engine.cu:2260-2314, 2523-2551)
//   P = SOFTMASK(S, type 1)                      (Engine/engine.cu:2430-2505; SoftMask, Engine/kernels.cu:2183-2235)
//   O_h = P V_h, written into head h's columns   (BMM + DeHeadify, Engine/engine.cu:2205-2258, 1166-1178)
// Type 1 normalises each column c (one key) over the rows r (queries): the
// column maximum m_c is taken over every row, the causal mask (c > r) zeroes
// exp(S - m_c) before the column sum l_c (l_c < 1e-45 counts as 1), and
// P = exp(S - m_c) / l_c.  The backward is the chain of those nodes:
//   dP = dO V^T, dV = P^T dO, dS = P (dP - D_c) with D_c = sum_r P dP over the
//   column (deriv_SoftMax, Engine/kernels.cu:2149-2181), dQ = scale dS K and
//   dK = scale dS^T Q -- or, reproducing BMMABT's gradient (Engine/engine.cu:2307),
//   bcmmT(Q, dS): scale * (dS Q)^T written row-major into the head's [seq x 64]
//   block of K's gradient.
//
// Here none of S, P, dP, dS is stored.  The column statistics (m_c, l_c) come
// from one pass over all of S; everything else recomputes its score tiles in
// registers.  Because P is normalised over the rows, D_c = <dV_c, V_c>: the
// key-block kernel finishes dV first and gets D from it.
//
//   attn_stats_kernel  (key blocks)   : m_c, l_c
//   attn_fwd_kernel    (query blocks) : O = P V
//   attn_bwd_kv_kernel (key blocks)   : dV, D (and dK = scale dS^T Q)
//   attn_bwd_q_kernel  (query blocks) : dQ = scale dS K (or the reference's dK)
//
// All products are v_mfma_f32_16x16x4f32 with operands loaded from memory in
// the MFMA lane layout.  Lane (lr, q) = (lane % 16, lane / 16).  A score tile
// in the accumulator layout holds, in lane (lr, q), rows 4q + r (r = 0..3) of
// column lr -- which is exactly the B operand layout of the next product when
// the tile's rows are that product's contraction index (step r feeds rows
// 4q + r).  The other operand of such a product is addressed with row
// 4 lr + i for MFMA block i, so it is one float4 per step along the head
// dimension, and the result's block (i, n) row 4q + r is element
// 16 q + 4 r + i of the head dimension: four blocks give one float4 store.
#include "common.hpp"

#include <float.h>

using namespace mle;

namespace {

constexpr int HD = 64;   // head dimension handled here
constexpr int NTA = 256; // four waves

struct AttnArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* dout;
  float* out;
  float* dq;
  float* dk;
  float* dv;
  float* stats;  // [slices][seq][2]: m_c, l_c
  float* dcol;   // [slices][seq]: D_c
  int heads, seq, ld;
  uint32_t bytes;  // extent of each [batch][seq][ld] tensor
  float scale;
  int acc_q, acc_k, acc_v;
};

__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
// Operand reads go through buffer resources with 32-bit element offsets (the
// host checks that every tensor is below 2 GiB), which keeps 64-bit
// addresses out of the register budget.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const float* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ f32x4 bld4(__amdgpu_buffer_rsrc_t r, uint32_t elem) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(elem * 4u), 0, 0));
}
__device__ __forceinline__ float bld1(__amdgpu_buffer_rsrc_t r, uint32_t elem) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)(elem * 4u), 0, 0));
}
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void bst4(__amdgpu_buffer_rsrc_t r, uint32_t elem, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (int)(elem * 4u), 0, 0);
}
__device__ __forceinline__ void bst1(__amdgpu_buffer_rsrc_t r, uint32_t elem, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, (int)(elem * 4u), 0, 0);
}
__device__ __forceinline__ void st4(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

struct Slice {
  int z;
  uint32_t base;  // element offset of (batch item, head) in the [batch][seq][ld] tensors
};
__device__ __forceinline__ Slice slice_of(const AttnArgs& a) {
  const int z = blockIdx.y, b = z / a.heads, h = z - b * a.heads;
  return {z, (uint32_t)b * a.seq * a.ld + (uint32_t)h * HD};
}

// Waves 1..3 hand their 64 accumulators per lane to wave 0 through LDS
// (lane-major: conflict free); wave 0 adds them in wave order.  Returns true
// in wave 0.
__device__ __forceinline__ bool reduce_waves(f32x4 (&acc)[4][4], float* red, int w, int lane) {
  if (w > 0) {
    float* dst = red + (w - 1) * 4096 + lane;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[((i * 4 + n) * 4 + r) * 64] = acc[i][n][r];
  }
  __syncthreads();
  if (w > 0) return false;
  // One 16-value group at a time, so the reads in flight stay few.
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const float* src = red + k * 4096 + lane;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][n][r] += src[((i * 4 + n) * 4 + r) * 64];
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  return true;
}

// Column statistics.  Wave w of block x owns keys k0 .. k0 + 15 (k0 = 64 x +
// 16 w) and walks all queries 64 at a time: S^T = K Q^T puts key k0 + 4q + r
// and query qc + 16 n + lr in acc[n][r].  Each lane keeps a running (max,
// masked sum) per key; the 16 lanes of a key merge at the end.
template <bool CAUSAL>
__global__ __launch_bounds__(NTA, 2) void attn_stats_kernel(AttnArgs a) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, lr = lane & 15, q = lane >> 4;
  const Slice sl = slice_of(a);
  const __amdgpu_buffer_rsrc_t Q = rsrc(a.q, a.bytes);
  const __amdgpu_buffer_rsrc_t K = rsrc(a.k, a.bytes);
  const int k0 = blockIdx.x * 64 + w * 16;
  f32x4 ka[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) ka[s] = bld4(K, sl.base + (uint32_t)(k0 + lr) * a.ld + 16 * s + 4 * q);
  float m[4], l[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m[r] = -FLT_MAX;
    l[r] = 0.f;
  }
  for (int qc = 0; qc < a.seq; qc += 64) {
    f32x4 acc[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      f32x4 qb[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) qb[s] = bld4(Q, sl.base + (uint32_t)(qc + 16 * n + lr) * a.ld + 16 * s + 4 * q);
      acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[n] = mfma4(ka[s][j], qb[s][j], acc[n]);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = k0 + 4 * q + r;
      float sv[4], cm = -FLT_MAX;
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        sv[n] = a.scale * acc[n][r];
        cm = fmaxf(cm, sv[n]);
      }
      const float mn = fmaxf(m[r], cm);
      float add = 0.f;
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const float e = __expf(sv[n] - mn);
        add += (!CAUSAL || qc + 16 * n + lr >= key) ? e : 0.f;
      }
      l[r] = l[r] * __expf(m[r] - mn) + add;
      m[r] = mn;
    }
  }
  // Merge the 16 lanes of each key (a butterfly: every lane ends with the
  // same value, each pair combined in the same order on both sides).
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      const float mo = __shfl_xor(m[r], off, 64), lo = __shfl_xor(l[r], off, 64);
      const float M = fmaxf(m[r], mo);
      l[r] = l[r] * __expf(m[r] - M) + lo * __expf(mo - M);
      m[r] = M;
    }
  if (lr == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (l[r] < 1e-45f) l[r] = 1.0f;
    float* S = a.stats + ((size_t)sl.z * a.seq + k0 + 4 * q) * 2;
    st4(S, f32x4{m[0], l[0], m[1], l[1]});
    st4(S + 4, f32x4{m[2], l[2], m[3], l[3]});
  }
}

// O = P V for 64 queries q0 .. q0 + 63; the four waves take every fourth
// 16-key chunk (with the causal mask, chunks up to the block's last query).
// Per chunk: S^T (K rows as A, the block's Q^T held in registers as B),
// P^T = exp(S - m) / l masked, then O^T += V^T P^T.
template <bool CAUSAL>
__global__ __launch_bounds__(NTA, 2) void attn_fwd_kernel(AttnArgs a) {
  __shared__ float red[3 * 4096];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, lr = lane & 15, q = lane >> 4;
  const Slice sl = slice_of(a);
  const __amdgpu_buffer_rsrc_t Q = rsrc(a.q, a.bytes);
  const __amdgpu_buffer_rsrc_t K = rsrc(a.k, a.bytes);
  const __amdgpu_buffer_rsrc_t V = rsrc(a.v, a.bytes);
  const float* ST = a.stats + (size_t)sl.z * a.seq * 2;
  const int q0 = blockIdx.x * 64;
  f32x4 qB[4][4];
#pragma unroll
  for (int n = 0; n < 4; ++n)
#pragma unroll
    for (int s = 0; s < 4; ++s) qB[n][s] = bld4(Q, sl.base + (uint32_t)(q0 + 16 * n + lr) * a.ld + 16 * s + 4 * q);
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nch = CAUSAL ? (q0 + 64) / 16 : a.seq / 16;
  for (int c = w; c < nch; c += 4) {
    const int k0 = 16 * c;
    f32x4 ka[4], va[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) ka[s] = bld4(K, sl.base + (uint32_t)(k0 + lr) * a.ld + 16 * s + 4 * q);
#pragma unroll
    for (int r = 0; r < 4; ++r) va[r] = bld4(V, sl.base + (uint32_t)(k0 + 4 * q + r) * a.ld + 4 * lr);
    const f32x4 s01 = ld4(ST + (size_t)(k0 + 4 * q) * 2), s23 = ld4(ST + (size_t)(k0 + 4 * q) * 2 + 4);
    const float mk[4] = {s01[0], s01[2], s23[0], s23[2]};
    const float il[4] = {1.0f / s01[1], 1.0f / s01[3], 1.0f / s23[1], 1.0f / s23[3]};
    f32x4 st[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      st[n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) st[n] = mfma4(ka[s][j], qB[n][s][j], st[n]);
    }
    float pt[4][4];
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool keep = !CAUSAL || q0 + 16 * n + lr >= k0 + 4 * q + r;
        pt[n][r] = __expf(a.scale * st[n][r] - mk[r]) * (keep ? il[r] : 0.f);
      }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int n = 0; n < 4; ++n) acc[i][n] = mfma4(va[r][i], pt[n][r], acc[i][n]);
  }
  if (!reduce_waves(acc, red, w, lane)) return;
  const __amdgpu_buffer_rsrc_t O = rsrc(a.out, a.bytes);
#pragma unroll
  for (int n = 0; n < 4; ++n)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      bst4(O, sl.base + (uint32_t)(q0 + 16 * n + lr) * a.ld + 16 * q + 4 * r,
           f32x4{acc[0][n][r], acc[1][n][r], acc[2][n][r], acc[3][n][r]});
}

// One 16-query chunk of the key-block kernel, processed per 16-key column
// block n (the next block's K / V rows are fetched while block n's MFMAs run,
// which keeps the register footprint at two blocks of operands): S and, with
// DP, dP for queries qc + 4q + r and keys k0 + 16n + lr; then f(n, p, dp)
// turns them into block n's B operand (P, or dS) and
// acc[i][n] += at[r][i] * b[r] accumulates the product.
template <bool CAUSAL, bool DP, class F>
__device__ __forceinline__ void kv_chunk(const AttnArgs& a, uint32_t base, __amdgpu_buffer_rsrc_t Q,
                                         __amdgpu_buffer_rsrc_t K, __amdgpu_buffer_rsrc_t V, __amdgpu_buffer_rsrc_t dO,
                                         int qc, int k0, int lr, int q, const float (&mk)[4],
                                         const float (&il)[4], const f32x4 (&at)[4], f32x4 (&acc)[4][4], F f) {
  f32x4 qa[4], oa[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    qa[s] = bld4(Q, base + (uint32_t)(qc + lr) * a.ld + 16 * s + 4 * q);
    if (DP) oa[s] = bld4(dO, base + (uint32_t)(qc + lr) * a.ld + 16 * s + 4 * q);
  }
  f32x4 kb[2][4], vb[2][4];
  auto fetch = [&](int n, f32x4(&kk)[4], f32x4(&vv)[4]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      kk[s] = bld4(K, base + (uint32_t)(k0 + 16 * n + lr) * a.ld + 16 * s + 4 * q);
      if (DP) vv[s] = bld4(V, base + (uint32_t)(k0 + 16 * n + lr) * a.ld + 16 * s + 4 * q);
    }
  };
  fetch(0, kb[0], vb[0]);
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    if (n + 1 < 4) fetch(n + 1, kb[(n + 1) & 1], vb[(n + 1) & 1]);
    __builtin_amdgcn_sched_barrier(0);
    f32x4 sa = {0.f, 0.f, 0.f, 0.f}, da = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sa = mfma4(qa[s][j], kb[n & 1][s][j], sa);
        if (DP) da = mfma4(oa[s][j], vb[n & 1][s][j], da);
      }
    float bop[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool keep = !CAUSAL || qc + 4 * q + r >= k0 + 16 * n + lr;
      const float pv = __expf(a.scale * sa[r] - mk[n]) * (keep ? il[n] : 0.f);
      bop[r] = f(n, pv, DP ? da[r] : 0.f);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i][n] = mfma4(at[r][i], bop[r], acc[i][n]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// dV (and D, and with DK the true dK) for 64 keys k0 .. k0 + 63; the waves
// take every fourth 16-query chunk (with the mask, from the block's first
// key on).  Pass 1: dV^T += dO^T P.  The block's dV is then complete: D_c =
// <dV_c, V_c> goes to LDS and to dcol.  Pass 2 (DK): dS = P (dP - D),
// dK^T += Q^T dS.
template <bool CAUSAL, bool DK>
__global__ __launch_bounds__(NTA, 2) void attn_bwd_kv_kernel(AttnArgs a) {
  __shared__ float red[3 * 4096];
  __shared__ float dsh[64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, lr = lane & 15, q = lane >> 4;
  const Slice sl = slice_of(a);
  const __amdgpu_buffer_rsrc_t Q = rsrc(a.q, a.bytes);
  const __amdgpu_buffer_rsrc_t K = rsrc(a.k, a.bytes);
  const __amdgpu_buffer_rsrc_t V = rsrc(a.v, a.bytes);
  const __amdgpu_buffer_rsrc_t dO = rsrc(a.dout, a.bytes);
  const int k0 = blockIdx.x * 64;
  float mk[4], il[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const float* sp = a.stats + ((size_t)sl.z * a.seq + k0 + 16 * n + lr) * 2;
    mk[n] = sp[0];
    il[n] = 1.0f / sp[1];
  }
  const int c0 = CAUSAL ? k0 / 16 : 0, nch = a.seq / 16;
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c = c0 + w; c < nch; c += 4) {
    const int qc = 16 * c;
    f32x4 ot[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) ot[r] = bld4(dO, sl.base + (uint32_t)(qc + 4 * q + r) * a.ld + 4 * lr);
    kv_chunk<CAUSAL, false>(a, sl.base, Q, K, V, dO, qc, k0, lr, q, mk, il, ot, acc,
                            [](int, float pv, float) { return pv; });
  }
  if (reduce_waves(acc, red, w, lane)) {
    // acc[i][n][r] = dV[k0 + 16n + lr][16q + 4r + i]
    const __amdgpu_buffer_rsrc_t dVr = rsrc(a.dv, a.bytes);
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const uint32_t row = (uint32_t)(k0 + 16 * n + lr) * a.ld;
      float part = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const f32x4 vv = bld4(V, sl.base + row + 16 * q + 4 * r);
        f32x4 g = {acc[0][n][r], acc[1][n][r], acc[2][n][r], acc[3][n][r]};
        part += g[0] * vv[0] + g[1] * vv[1] + g[2] * vv[2] + g[3] * vv[3];
        if (a.acc_v) g += bld4(dVr, sl.base + row + 16 * q + 4 * r);
        bst4(dVr, sl.base + row + 16 * q + 4 * r, g);
      }
      part += __shfl_xor(part, 16, 64);
      part += __shfl_xor(part, 32, 64);
      if (q == 0) {
        dsh[16 * n + lr] = part;
        a.dcol[(size_t)sl.z * a.seq + k0 + 16 * n + lr] = part;
      }
    }
  }
  if (!DK) return;
  __syncthreads();
  float D[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) D[n] = dsh[16 * n + lr];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c = c0 + w; c < nch; c += 4) {
    const int qc = 16 * c;
    f32x4 qt[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) qt[r] = bld4(Q, sl.base + (uint32_t)(qc + 4 * q + r) * a.ld + 4 * lr);
    kv_chunk<CAUSAL, true>(a, sl.base, Q, K, V, dO, qc, k0, lr, q, mk, il, qt, acc,
                           [&](int n, float pv, float dpv) { return pv * (dpv - D[n]); });
  }
  if (!reduce_waves(acc, red, w, lane)) return;
  const __amdgpu_buffer_rsrc_t dKr = rsrc(a.dk, a.bytes);
#pragma unroll
  for (int n = 0; n < 4; ++n)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t e = sl.base + (uint32_t)(k0 + 16 * n + lr) * a.ld + 16 * q + 4 * r;
      f32x4 g = a.scale * f32x4{acc[0][n][r], acc[1][n][r], acc[2][n][r], acc[3][n][r]};
      if (a.acc_k) g += bld4(dKr, e);
      bst4(dKr, e, g);
    }
}

// dQ for 64 queries q0 .. q0 + 63 (or, with KREF, the reference's K
// gradient bcmmT(Q, dS): the same product with Q's rows at the key positions
// in place of K, stored in the head block's row-major [64 x seq] order).  The
// waves take every fourth 16-key chunk.  Per chunk and 16-query column block
// n: S^T = K Q^T and dP^T = V dO^T, dS^T = P^T (dP^T - D), X^T += Y^T dS^T
// (Y = K or Q); block n + 1's Q / dO rows are fetched during block n.
template <bool CAUSAL, bool KREF>
__global__ __launch_bounds__(NTA, 2) void attn_bwd_q_kernel(AttnArgs a) {
  __shared__ float red[3 * 4096];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, lr = lane & 15, q = lane >> 4;
  const Slice sl = slice_of(a);
  const __amdgpu_buffer_rsrc_t Q = rsrc(a.q, a.bytes);
  const __amdgpu_buffer_rsrc_t K = rsrc(a.k, a.bytes);
  const __amdgpu_buffer_rsrc_t V = rsrc(a.v, a.bytes);
  const __amdgpu_buffer_rsrc_t dO = rsrc(a.dout, a.bytes);
  const __amdgpu_buffer_rsrc_t Y = KREF ? Q : K;
  const float* ST = a.stats + (size_t)sl.z * a.seq * 2;
  const float* DC = a.dcol + (size_t)sl.z * a.seq;
  const int q0 = blockIdx.x * 64;
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nch = CAUSAL ? (q0 + 64) / 16 : a.seq / 16;
  for (int c = w; c < nch; c += 4) {
    const int k0 = 16 * c;
    f32x4 ka[4], va[4], yt[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      ka[s] = bld4(K, sl.base + (uint32_t)(k0 + lr) * a.ld + 16 * s + 4 * q);
      va[s] = bld4(V, sl.base + (uint32_t)(k0 + lr) * a.ld + 16 * s + 4 * q);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) yt[r] = bld4(Y, sl.base + (uint32_t)(k0 + 4 * q + r) * a.ld + 4 * lr);
    const f32x4 s01 = ld4(ST + (size_t)(k0 + 4 * q) * 2), s23 = ld4(ST + (size_t)(k0 + 4 * q) * 2 + 4);
    const float mk[4] = {s01[0], s01[2], s23[0], s23[2]};
    const float il[4] = {1.0f / s01[1], 1.0f / s01[3], 1.0f / s23[1], 1.0f / s23[3]};
    const f32x4 Dk = ld4(DC + k0 + 4 * q);
    f32x4 qb[2][4], ob[2][4];
    auto fetch = [&](int n, f32x4(&qq)[4], f32x4(&oo)[4]) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        qq[s] = bld4(Q, sl.base + (uint32_t)(q0 + 16 * n + lr) * a.ld + 16 * s + 4 * q);
        oo[s] = bld4(dO, sl.base + (uint32_t)(q0 + 16 * n + lr) * a.ld + 16 * s + 4 * q);
      }
    };
    fetch(0, qb[0], ob[0]);
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      if (n + 1 < 4) fetch(n + 1, qb[(n + 1) & 1], ob[(n + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      f32x4 st = {0.f, 0.f, 0.f, 0.f}, dt = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          st = mfma4(ka[s][j], qb[n & 1][s][j], st);
          dt = mfma4(va[s][j], ob[n & 1][s][j], dt);
        }
      float ds[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool keep = !CAUSAL || q0 + 16 * n + lr >= k0 + 4 * q + r;
        const float pv = __expf(a.scale * st[r] - mk[r]) * (keep ? il[r] : 0.f);
        ds[r] = pv * (dt[r] - Dk[r]);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][n] = mfma4(yt[r][i], ds[r], acc[i][n]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (!reduce_waves(acc, red, w, lane)) return;
  // acc[i][n][r] = X^T[d = 16q + 4r + i][query q0 + 16n + lr]
  if (!KREF) {
    const __amdgpu_buffer_rsrc_t dQr = rsrc(a.dq, a.bytes);
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t e = sl.base + (uint32_t)(q0 + 16 * n + lr) * a.ld + 16 * q + 4 * r;
        f32x4 g = a.scale * f32x4{acc[0][n][r], acc[1][n][r], acc[2][n][r], acc[3][n][r]};
        if (a.acc_q) g += bld4(dQr, e);
        bst4(dQr, e, g);
      }
  } else {
    // C[d][j] lands at flat d * seq + j of the head's [seq x 64] block.
    const __amdgpu_buffer_rsrc_t dKr = rsrc(a.dk, a.bytes);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t d = 16 * q + 4 * r + i, j = q0 + 16 * n + lr;
          const uint32_t f = d * (uint32_t)a.seq + j;
          const uint32_t e = sl.base + (f / HD) * a.ld + f % HD;
          float g = a.scale * acc[i][n][r];
          if (a.acc_k) g += bld1(dKr, e);
          bst1(dKr, e, g);
        }
  }
}

bool attn_shape_ok(int batch, int heads, int seq, int head_dim, int ld) {
  return batch > 0 && heads > 0 && head_dim == HD && seq >= 64 && seq % 64 == 0 && ld % 4 == 0 &&
         ld >= heads * HD && (double)batch * heads <= 65535.0 && (double)batch * seq * ld < 2147483647.0;
}

}  // namespace

extern "C" {

size_t mle_attention_ws_bytes(int batch, int heads, int seq) {
  if (batch <= 0 || heads <= 0 || seq <= 0) return 0;
  return (size_t)batch * heads * seq * 3 * sizeof(float);
}

int mle_attention_fwd(mle_stream stream, const float* q, const float* k, const float* v, float* out, int batch,
                      int heads, int seq, int head_dim, int ld, float scale, int causal, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(q && k && v && out && ws, "mle_attention_fwd: null pointer");
  if (!attn_shape_ok(batch, heads, seq, head_dim, ld))
    return set_error(MLE_ERR_UNSUPPORTED, "mle_attention_fwd: needs head_dim 64, seq a multiple of 64, ld %% 4 == 0");
  if (ws_bytes < mle_attention_ws_bytes(batch, heads, seq))
    return set_error(MLE_ERR_WORKSPACE, "mle_attention_fwd: workspace too small");
  MLE_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) && aligned16(ws),
                "mle_attention_fwd: pointers must be 16-byte aligned");
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.stats = static_cast<float*>(ws);
  a.dcol = a.stats + (size_t)batch * heads * seq * 2;
  a.heads = heads;
  a.seq = seq;
  a.ld = ld;
  a.bytes = (uint32_t)((size_t)batch * seq * ld * sizeof(float));
  a.scale = scale;
  hipStream_t s = as_stream(stream);
  const dim3 grid(seq / 64, batch * heads);
  const double flop = 4.0 * batch * heads * (double)seq * seq * HD;  // S and P V, as the reference computes them
  ProbeScope probe("attn_fwd", s, flop, 0.0);
  if (causal) {
    attn_stats_kernel<true><<<grid, NTA, 0, s>>>(a);
    attn_fwd_kernel<true><<<grid, NTA, 0, s>>>(a);
  } else {
    attn_stats_kernel<false><<<grid, NTA, 0, s>>>(a);
    attn_fwd_kernel<false><<<grid, NTA, 0, s>>>(a);
  }
  return check_launch("mle_attention_fwd");
}

int mle_attention_bwd(mle_stream stream, const float* q, const float* k, const float* v, const float* dout, float* dq,
                      float* dk, float* dv, int batch, int heads, int seq, int head_dim, int ld, float scale,
                      int causal, int acc_q, int acc_k, int acc_v, int k_reference_grad, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(q && k && v && dout && dq && dk && dv && ws, "mle_attention_bwd: null pointer");
  if (!attn_shape_ok(batch, heads, seq, head_dim, ld))
    return set_error(MLE_ERR_UNSUPPORTED, "mle_attention_bwd: needs head_dim 64, seq a multiple of 64, ld %% 4 == 0");
  if (ws_bytes < mle_attention_ws_bytes(batch, heads, seq))
    return set_error(MLE_ERR_WORKSPACE, "mle_attention_bwd: workspace too small");
  MLE_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(dout) && aligned16(dq) && aligned16(dk) &&
                    aligned16(dv) && aligned16(ws),
                "mle_attention_bwd: pointers must be 16-byte aligned");
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.dout = dout;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.stats = static_cast<float*>(ws);
  a.dcol = a.stats + (size_t)batch * heads * seq * 2;
  a.heads = heads;
  a.seq = seq;
  a.ld = ld;
  a.bytes = (uint32_t)((size_t)batch * seq * ld * sizeof(float));
  a.scale = scale;
  a.acc_q = acc_q != 0;
  a.acc_k = acc_k != 0;
  a.acc_v = acc_v != 0;
  hipStream_t s = as_stream(stream);
  const dim3 grid(seq / 64, batch * heads);
  const double flop = 8.0 * batch * heads * (double)seq * seq * HD;  // dP, dV, dQ, dK
  ProbeScope probe("attn_bwd", s, flop, 0.0);
  const bool kref = k_reference_grad != 0;
  if (causal) {
    if (kref) attn_bwd_kv_kernel<true, false><<<grid, NTA, 0, s>>>(a);
    else attn_bwd_kv_kernel<true, true><<<grid, NTA, 0, s>>>(a);
    attn_bwd_q_kernel<true, false><<<grid, NTA, 0, s>>>(a);
    if (kref) attn_bwd_q_kernel<true, true><<<grid, NTA, 0, s>>>(a);
  } else {
    if (kref) attn_bwd_kv_kernel<false, false><<<grid, NTA, 0, s>>>(a);
    else attn_bwd_kv_kernel<false, true><<<grid, NTA, 0, s>>>(a);
    attn_bwd_q_kernel<false, false><<<grid, NTA, 0, s>>>(a);
    if (kref) attn_bwd_q_kernel<false, true><<<grid, NTA, 0, s>>>(a);
  }
  return check_launch("mle_attention_bwd");
}

}  // extern "C"
