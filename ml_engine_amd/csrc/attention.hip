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
// Here none of S, P, dP, dS is stored.  The column statistics (m_c, 1 / l_c,
// the reciprocal divided once per key) come from one pass over all of S; everything else recomputes its score tiles in
// registers.  Because P is normalised over the rows, D_c = <dV_c, V_c>: the
// key-block kernel finishes dV first and gets D from it.
//
//   attn_stats_kernel  (key blocks)   : m_c, 1 / l_c
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

#include <type_traits>

using namespace mle;

namespace {

constexpr int HD = 64;   // head dimension handled here

struct AttnArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* dout;
  float* out;
  float* dq;
  float* dk;
  float* dv;
  float* stats;  // [slices][seq][2]: m_c, 1 / l_c
  float* dcol;   // [slices][seq]: D_c
  float* kept;   // causal, seq <= 256: [slices][kept_blocks(seq)][16 keys][16 queries] of P
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
// Same with a wave-uniform part of the offset in the instruction's scalar
// offset (rows r = 0..3 of a lane's group share one address register).
__device__ __forceinline__ f32x4 bld4s(__amdgpu_buffer_rsrc_t r, uint32_t elem, uint32_t uniform_elem) {
  return __builtin_bit_cast(f32x4,
                            __builtin_amdgcn_raw_buffer_load_b128(r, (int)(elem * 4u), (int)(uniform_elem * 4u), 0));
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
// The causal slice kernels' 16x16 blocks on or below the diagonal: block
// (query block qb, key block kb), kb <= qb, at index qb (qb + 1) / 2 + kb.
__host__ __device__ constexpr size_t kept_blocks(int seq) { return (size_t)(seq / 16) * (seq / 16 + 1) / 2; }
__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

struct Slice {
  int z;
  uint32_t base;  // element offset of (batch item, head) in the [batch][seq][ld] tensors
  int pair;       // this workgroup's tile pair within the slice
};
// Slice z's kept probabilities, kept_blocks(seq) blocks of 256 floats.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t kept_rsrc(const AttnArgs& a, const Slice& sl) {
  const size_t n = kept_blocks(a.seq) * 256;
  return rsrc(a.kept + (size_t)sl.z * n, (uint32_t)(n * sizeof(float)));
}
// The grid is one-dimensional: workgroup L runs on XCD L % 8 (workgroups are
// dispatched round-robin over the XCDs).  XCD x takes a contiguous range of
// the (slice, tile pair) items, slice-major, so every workgroup of a slice
// runs on one XCD and shares its L2 copy of the slice's Q, K, V and dO rows.
// A bijection on [0, gridDim.x) for any grid size.
constexpr int kXcds = 8;
__device__ __forceinline__ Slice slice_of(const AttnArgs& a) {
  const int L = blockIdx.x, total = gridDim.x, pairs = a.seq / 64;
  const int x = L % kXcds, j = L / kXcds, per = total / kXcds, rem = total % kXcds;
  const int t = x * per + min(x, rem) + j;
  const int z = t / pairs, b = z / a.heads, h = z - b * a.heads;
  return {z, (uint32_t)b * a.seq * a.ld + (uint32_t)h * HD, t - z * pairs};
}

// Work split: every wave owns a 32-row tile of one output (32 keys of the
// statistics, 32 queries of O or dQ, 32 keys of dV / dK) and walks the whole
// contraction range for it, so no partial sums cross waves.  A workgroup is
// two waves of the same (batch item, head) slice taking tiles j and
// nb - 1 - j (nb = seq / 32): under the causal mask a query tile's work grows
// with j and a key tile's shrinks, so each workgroup gets the same total.  A
// loop over 16-row chunks keeps two register sets of chunk operands and
// fetches chunk c + 1 into one while chunk c computes from the other.
constexpr int TW = 32;      // rows of a wave's tile
constexpr int LQ = HD + 4;  // padded LDS row: the 16 rows a b128 read touches sit on distinct banks

__device__ __forceinline__ int tile_of(const AttnArgs& a, const Slice& sl, int w) {
  return w == 0 ? sl.pair : a.seq / TW - 1 - sl.pair;
}

// Chunk loop with two alternating register sets (no copies between them,
// so a chunk's loads are waited for only when that chunk is computed).  The
// optional late(c) issues chunk c's loads that are needed only at the end of
// its computation; it runs before the next chunk's prefetch, because the
// hardware counts loads in order: waiting for them then leaves the prefetch
// in flight.
struct NoLate {
  __device__ void operator()(int) const {}
};
template <class Chunk, class Fetch, class Compute, class Late = NoLate>
__device__ __forceinline__ void chunk_loop(int c0, int c1, Fetch fetch, Compute compute, Late late = NoLate{}) {
  Chunk ca, cb;
  if (c0 < c1) fetch(c0, ca);
  for (int c = c0; c < c1; c += 2) {
    late(c);
    fetch(min(c + 1, c1 - 1), cb);
    __builtin_amdgcn_sched_barrier(0);
    compute(c, ca);
    __builtin_amdgcn_sched_barrier(0);
    if (c + 1 >= c1) break;
    late(c + 1);
    fetch(min(c + 2, c1 - 1), ca);
    __builtin_amdgcn_sched_barrier(0);
    compute(c + 1, cb);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Column statistics for keys k0 .. k0 + 31 over all queries, 32 at a time:
// S^T = K Q^T puts key k0 + 16i + 4q + r and query qc + 16n + lr in
// acc[i][n][r].  Each lane keeps a running (max over all rows, masked sum)
// per key; the 16 lanes of a key merge at the end.
// KEEP_S (causal): the tile's S^T blocks on or below the diagonal (16-row
// key block kb <= query block qb) are also written to sst, 1 KB per block in
// the accumulator lane layout, at block index qb (qb + 1) / 2 + kb.
template <bool CAUSAL, bool KEEP_S = false>
__device__ __forceinline__ void stats_tile(const AttnArgs& a, const Slice& sl, int k0, float* sst = nullptr) {
  const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
  const __amdgpu_buffer_rsrc_t Q = rsrc(a.q, a.bytes);
  const __amdgpu_buffer_rsrc_t K = rsrc(a.k, a.bytes);
  f32x4 ka[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int s = 0; s < 4; ++s) ka[i][s] = bld4(K, sl.base + (uint32_t)(k0 + 16 * i + lr) * a.ld + 16 * s + 4 * q);
  float m[2][4], l[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      m[i][r] = -FLT_MAX;
      l[i][r] = 0.f;
    }
  struct Chunk {
    f32x4 qb[2][4];
  };
  auto fetch = [&](int c, Chunk& ch) {
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        ch.qb[n][s] = bld4(Q, sl.base + (uint32_t)(TW * c + 16 * n + lr) * a.ld + 16 * s + 4 * q);
  };
  auto compute = [&](int c, const Chunk& ch) {
    const int qc = TW * c;
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][n] = mfma4(ka[i][s][j], ch.qb[n][s][j], acc[i][n]);
      }
    if (KEEP_S) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int n = 0; n < 2; ++n) {
          const int kb = k0 / 16 + i, qb = 2 * c + n;
          if (kb <= qb) *reinterpret_cast<f32x4*>(sst + (qb * (qb + 1) / 2 + kb) * 256 + 4 * lane) = acc[i][n];
        }
    }
    // Under the causal mask, chunks before the tile's diagonal chunk lie
    // wholly above the diagonal: they only raise the maximum (the sum is still
    // exactly 0 there, so skipping its update changes no bit), and chunks
    // after it need no mask.
    const int diag = k0 / TW;
    auto update = [&](auto masked_tag) {
      constexpr bool MASKED = decltype(masked_tag)::value;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = k0 + 16 * i + 4 * q + r;
          const float s0 = a.scale * acc[i][0][r], s1 = a.scale * acc[i][1][r];
          const float mn = fmaxf(m[i][r], fmaxf(s0, s1));
          const float e0 = __expf(s0 - mn), e1 = __expf(s1 - mn);
          const float add = ((!MASKED || qc + lr >= key) ? e0 : 0.f) + ((!MASKED || qc + 16 + lr >= key) ? e1 : 0.f);
          l[i][r] = l[i][r] * __expf(m[i][r] - mn) + add;
          m[i][r] = mn;
        }
    };
    if (CAUSAL && c < diag) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) m[i][r] = fmaxf(m[i][r], fmaxf(a.scale * acc[i][0][r], a.scale * acc[i][1][r]));
    } else if (CAUSAL && c == diag) {
      update(std::true_type{});
    } else {
      update(std::false_type{});
    }
  };
  chunk_loop<Chunk>(0, a.seq / TW, fetch, compute);
  // Merge the 16 lanes of each key (a butterfly: every lane ends with the
  // same value, each pair combined in the same order on both sides).
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) {
        const float mo = __shfl_xor(m[i][r], off, 64), lo = __shfl_xor(l[i][r], off, 64);
        const float M = fmaxf(m[i][r], mo);
        l[i][r] = l[i][r] * __expf(m[i][r] - M) + lo * __expf(mo - M);
        m[i][r] = M;
      }
  if (lr == 0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) l[i][r] = 1.0f / (l[i][r] < 1e-45f ? 1.0f : l[i][r]);
      float* S = a.stats + ((size_t)sl.z * a.seq + k0 + 16 * i + 4 * q) * 2;
      st4(S, f32x4{m[i][0], l[i][0], m[i][1], l[i][1]});
      st4(S + 4, f32x4{m[i][2], l[i][2], m[i][3], l[i][3]});
    }
  }
}

// O = P V for queries q0 .. q0 + 31 over the 16-key chunks (with the causal
// mask, up to the tile's last query).  The tile's Q^T (the B operand of
// S^T = K Q^T) stays in registers; per chunk: S^T, P^T = exp(S - m) / l
// masked, O^T += V^T P^T.  The loop is software-pipelined: while chunk c's
// softmax (VALU) and P V products run, chunk c + 1's S^T products are
// already issued, so the matrix core has independent work while the wave
// computes exponentials.  Two register sets alternate; at step c the K rows
// of chunk c + 2 and the V rows and statistics of chunk c + 1 load into the
// set whose previous contents step c - 1 consumed.  KEEP_S: the S^T blocks
// come from sst (written by stats_tile<CAUSAL, true> over the same operands
// in the same order, so the same bits) and no K rows are loaded; the one
// block above the diagonal (the lower query block's last chunk) is never
// read, its P^T is 0 by the mask.
template <bool CAUSAL, bool KEEP_S = false>
__device__ __forceinline__ void fwd_tile(const AttnArgs& a, const Slice& sl, int q0, const float* sst = nullptr) {
  const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
  const __amdgpu_buffer_rsrc_t Q = rsrc(a.q, a.bytes);
  const __amdgpu_buffer_rsrc_t K = rsrc(a.k, a.bytes);
  const __amdgpu_buffer_rsrc_t V = rsrc(a.v, a.bytes);
  const float* ST = a.stats + (size_t)sl.z * a.seq * 2;
  f32x4 qB[2][4];
  if (!KEEP_S) {
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int s = 0; s < 4; ++s) qB[n][s] = bld4(Q, sl.base + (uint32_t)(q0 + 16 * n + lr) * a.ld + 16 * s + 4 * q);
  }
  f32x4 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 2; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  struct Chunk {
    f32x4 ka[4], va[4], s01, s23, st[2];
  };
  auto fetch_k = [&](int c, Chunk& ch) {
    if (KEEP_S) return;
#pragma unroll
    for (int s = 0; s < 4; ++s) ch.ka[s] = bld4(K, sl.base + (uint32_t)(16 * c + lr) * a.ld + 16 * s + 4 * q);
  };
  auto fetch_v = [&](int c, Chunk& ch) {
    const int k0 = 16 * c;
#pragma unroll
    for (int r = 0; r < 4; ++r) ch.va[r] = bld4s(V, sl.base + (uint32_t)(k0 + 4 * q) * a.ld + 4 * lr, (uint32_t)r * a.ld);
    ch.s01 = ld4(ST + (size_t)(k0 + 4 * q) * 2);
    ch.s23 = ld4(ST + (size_t)(k0 + 4 * q) * 2 + 4);
  };
  auto scores = [&](int c, Chunk& ch) {
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      ch.st[n] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (KEEP_S) {
        const int qb = q0 / 16 + n;
        if (c <= qb) ch.st[n] = *reinterpret_cast<const f32x4*>(sst + (qb * (qb + 1) / 2 + c) * 256 + 4 * lane);
        continue;
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) ch.st[n] = mfma4(ch.ka[s][j], qB[n][s][j], ch.st[n]);
    }
  };
  // Only the tile's last two chunks reach past the diagonal (MASK).
  auto finish = [&](auto mask_tag, int c, const Chunk& ch) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int k0 = 16 * c;
    const float mk[4] = {ch.s01[0], ch.s01[2], ch.s23[0], ch.s23[2]};
    const float il[4] = {ch.s01[1], ch.s01[3], ch.s23[1], ch.s23[3]};
    float pt[2][4];
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool keep = !MASK || q0 + 16 * n + lr >= k0 + 4 * q + r;
        pt[n][r] = keep ? __expf(a.scale * ch.st[n][r] - mk[r]) * il[r] : 0.f;
      }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int n = 0; n < 2; ++n) acc[i][n] = mfma4(ch.va[r][i], pt[n][r], acc[i][n]);
  };
  const int nc = CAUSAL ? (q0 + TW) / 16 : a.seq / 16;  // at least 2
  // cur holds chunk c's scores, V rows and statistics; nxt holds chunk c + 1's
  // K rows.  Loads past the last chunk repeat it.
  const int cm = CAUSAL ? q0 / 16 : nc;  // first chunk that needs the mask
  auto step = [&](auto mask_tag, int c, Chunk& cur, Chunk& nxt) {
    fetch_k(min(c + 2, nc - 1), cur);
    fetch_v(c + 1, nxt);
    __builtin_amdgcn_sched_barrier(0);  // loads first: they have the whole step to land
    scores(c + 1, nxt);
    finish(mask_tag, c, cur);
    // Issue order: one S^T product, then two softmax instructions, so the
    // wave keeps issuing VALU work while each product occupies the matrix core.
    if (!KEEP_S) {
#pragma unroll
      for (int k = 0; k < 24; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  Chunk X, Y;
  fetch_k(0, X);
  fetch_v(0, X);
  fetch_k(1, Y);
  scores(0, X);
  auto step_at = [&](int c, Chunk& cur, Chunk& nxt) {
    if (c >= cm) step(std::true_type{}, c, cur, nxt);
    else step(std::false_type{}, c, cur, nxt);
  };
  for (int c = 0;; c += 2) {
    if (c + 1 >= nc) {
      finish(std::integral_constant<bool, CAUSAL>{}, c, X);
      break;
    }
    step_at(c, X, Y);
    if (c + 2 >= nc) {
      finish(std::integral_constant<bool, CAUSAL>{}, c + 1, Y);
      break;
    }
    step_at(c + 1, Y, X);
  }
  const __amdgpu_buffer_rsrc_t O = rsrc(a.out, a.bytes);
#pragma unroll
  for (int n = 0; n < 2; ++n)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      bst4(O, sl.base + (uint32_t)(q0 + 16 * n + lr) * a.ld + 16 * q + 4 * r,
           f32x4{acc[0][n][r], acc[1][n][r], acc[2][n][r], acc[3][n][r]});
}

// dV, D and, with DK, the true dK for keys k0 .. k0 + 31 over the 16-query
// chunks (with the mask, from the tile's first key on).  The tile's K^T (and
// V^T) B operands stay in registers; per chunk and 16-key column block n: S
// (and dP) in the S layout (query qc + 4q + r, key k0 + 16n + lr), then
//   pass 1: dV^T += dO^T P        -> dV and D_c = <dV_c, V_c> (the wave holds
//                                    all of its keys' dV, so D needs no exchange)
//   pass 2 (DK): dS = P (dP - D), dK^T += Q^T dS.
// KEEP_P (causal): pass 1's P blocks on or below the diagonal (16-row query
// block qb >= key block kb) are also written to sst, 1 KB per block at index
// qb (qb + 1) / 2 + kb, row = query and column = key within the block.
template <bool CAUSAL, bool DK, bool KEEP_P = false>
__device__ __forceinline__ void bwd_kv_tile(const AttnArgs& a, const Slice& sl, int k0, float* sst = nullptr) {
  const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
  const __amdgpu_buffer_rsrc_t Q = rsrc(a.q, a.bytes);
  const __amdgpu_buffer_rsrc_t K = rsrc(a.k, a.bytes);
  const __amdgpu_buffer_rsrc_t V = rsrc(a.v, a.bytes);
  const __amdgpu_buffer_rsrc_t dO = rsrc(a.dout, a.bytes);
  f32x4 kB[2][4], vB[2][4];
  float mk[2], il[2];
#pragma unroll
  for (int n = 0; n < 2; ++n) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      kB[n][s] = bld4(K, sl.base + (uint32_t)(k0 + 16 * n + lr) * a.ld + 16 * s + 4 * q);
      if (DK) vB[n][s] = bld4(V, sl.base + (uint32_t)(k0 + 16 * n + lr) * a.ld + 16 * s + 4 * q);
    }
    const float* sp = a.stats + ((size_t)sl.z * a.seq + k0 + 16 * n + lr) * 2;
    mk[n] = sp[0];
    il[n] = sp[1];
  }
  f32x4 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 2; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  float D[2] = {0.f, 0.f};
  // A chunk: Q rows (S), dO rows (dP, pass 2), and the final product's A
  // operand rows in the 4 lr + i layout (dO for dV, Q for dK).
  struct Chunk {
    f32x4 qa[4], oa[4], at[4];
  };
  auto run = [&](auto pass2_tag) {
    constexpr bool P2 = decltype(pass2_tag)::value;
    auto fetch = [&](int c, Chunk& ch) {
      const int qc = 16 * c;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        ch.qa[s] = bld4(Q, sl.base + (uint32_t)(qc + lr) * a.ld + 16 * s + 4 * q);
        if (P2) ch.oa[s] = bld4(dO, sl.base + (uint32_t)(qc + lr) * a.ld + 16 * s + 4 * q);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) ch.at[r] = bld4s(P2 ? Q : dO, sl.base + (uint32_t)(qc + 4 * q) * a.ld + 4 * lr, (uint32_t)r * a.ld);
    };
    // Only the tile's first two chunks reach past the diagonal (MASK).
    auto body = [&](auto mask_tag, int c, const Chunk& ch) {
      constexpr bool MASK = decltype(mask_tag)::value;
      const int qc = 16 * c;
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        f32x4 sa = {0.f, 0.f, 0.f, 0.f}, da = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            sa = mfma4(ch.qa[s][j], kB[n][s][j], sa);
            if (P2) da = mfma4(ch.oa[s][j], vB[n][s][j], da);
          }
        float bop[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool keep = !MASK || qc + 4 * q + r >= k0 + 16 * n + lr;
          const float pv = __expf(a.scale * sa[r] - mk[n]) * (keep ? il[n] : 0.f);
          bop[r] = P2 ? pv * (da[r] - D[n]) : pv;
        }
        if (KEEP_P && !P2) {
          const int kb = k0 / 16 + n;
          if (kb <= c) {
            float* blk = sst + (c * (c + 1) / 2 + kb) * 256 + lr;
#pragma unroll
            for (int r = 0; r < 4; ++r) blk[(4 * q + r) * 16] = bop[r];
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i][n] = mfma4(ch.at[r][i], bop[r], acc[i][n]);
      }
    };
    auto compute = [&](int c, const Chunk& ch) {
      if (CAUSAL && c < k0 / 16 + 2) body(std::true_type{}, c, ch);
      else body(std::false_type{}, c, ch);
    };
    chunk_loop<Chunk>(CAUSAL ? k0 / 16 : 0, a.seq / 16, fetch, compute);
  };
  run(std::false_type{});
  // acc[i][n][r] = dV[k0 + 16n + lr][16q + 4r + i]
  const __amdgpu_buffer_rsrc_t dVr = rsrc(a.dv, a.bytes);
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    const uint32_t row = sl.base + (uint32_t)(k0 + 16 * n + lr) * a.ld;
    float part = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const f32x4 vv = bld4(V, row + 16 * q + 4 * r);
      f32x4 g = {acc[0][n][r], acc[1][n][r], acc[2][n][r], acc[3][n][r]};
      part += g[0] * vv[0] + g[1] * vv[1] + g[2] * vv[2] + g[3] * vv[3];
      if (a.acc_v) g += bld4(dVr, row + 16 * q + 4 * r);
      bst4(dVr, row + 16 * q + 4 * r, g);
    }
    part += __shfl_xor(part, 16, 64);
    part += __shfl_xor(part, 32, 64);
    D[n] = part;
    if (q == 0) a.dcol[(size_t)sl.z * a.seq + k0 + 16 * n + lr] = part;
  }
  if (!DK) return;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 2; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  run(std::true_type{});
  const __amdgpu_buffer_rsrc_t dKr = rsrc(a.dk, a.bytes);
#pragma unroll
  for (int n = 0; n < 2; ++n)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t e = sl.base + (uint32_t)(k0 + 16 * n + lr) * a.ld + 16 * q + 4 * r;
      f32x4 g = a.scale * f32x4{acc[0][n][r], acc[1][n][r], acc[2][n][r], acc[3][n][r]};
      if (a.acc_k) g += bld4(dKr, e);
      bst4(dKr, e, g);
    }
}

// dQ = scale dS K and, with KREF, the reference's K gradient bcmmT(Q, dS)
// (the same product with Q's rows at the key positions, stored in the head
// block's row-major [64 x seq] order) for queries q0 .. q0 + 31; both come
// from the same dS tiles.  The tile's Q and dO rows (the B operands of
// S^T = K Q^T and dP^T = V dO^T) are staged in the wave's own LDS region
// (qs, os: TW * LQ floats each).
// Per chunk and 16-query column block n: S^T and dP^T, dS^T = P^T (dP^T -
// D), then X^T += Y^T dS^T for Y = K (acc[.][n]) and Y = Q (acc[.][2 + n]).
//
// KEEP_P (causal): P comes from sst, written by bwd_kv_tile<CAUSAL, false,
// true> (row = query, column = key within a 16 x 16 block, so one lane's four
// keys are one 16-byte read); no S^T products, no K rows and no statistics
// are needed, and the tile's dO rows stay in registers (qs, os unused).  The
// block above the diagonal (the lower query block's last chunk) is not kept:
// its P is 0 by the mask.
template <bool CAUSAL, bool KREF, bool KEEP_P = false>
__device__ __forceinline__ void bwd_q_tile(const AttnArgs& a, const Slice& sl, int q0, float* qs, float* os,
                                           const float* sst = nullptr) {
  const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
  const __amdgpu_buffer_rsrc_t Q = rsrc(a.q, a.bytes);
  const __amdgpu_buffer_rsrc_t K = rsrc(a.k, a.bytes);
  const __amdgpu_buffer_rsrc_t V = rsrc(a.v, a.bytes);
  const __amdgpu_buffer_rsrc_t dO = rsrc(a.dout, a.bytes);
  const float* ST = a.stats + (size_t)sl.z * a.seq * 2;
  const float* DC = a.dcol + (size_t)sl.z * a.seq;
  f32x4 obr[2][4];
  if (KEEP_P) {
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int s = 0; s < 4; ++s) obr[n][s] = bld4(dO, sl.base + (uint32_t)(q0 + 16 * n + lr) * a.ld + 16 * s + 4 * q);
  } else {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = lane + 64 * u, row = idx >> 4, col = (idx & 15) * 4;
      const uint32_t e = sl.base + (uint32_t)(q0 + row) * a.ld + col;
      *reinterpret_cast<f32x4*>(qs + row * LQ + col) = bld4(Q, e);
      *reinterpret_cast<f32x4*>(os + row * LQ + col) = bld4(dO, e);
    }
    // The region is the wave's own: its writes only have to land before its reads.
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  }
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  struct Chunk {
    f32x4 ka[4], va[4];
  };
  auto fetch = [&](int c, Chunk& ch) {
    const int k0 = 16 * c;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (!KEEP_P) ch.ka[s] = bld4(K, sl.base + (uint32_t)(k0 + lr) * a.ld + 16 * s + 4 * q);
      ch.va[s] = bld4(V, sl.base + (uint32_t)(k0 + lr) * a.ld + 16 * s + 4 * q);
    }
  };
  // Chunk c's operands needed only after its S^T / dP^T products: the
  // statistics and D of its keys, and its Y rows (A of the last products).
  f32x4 yk[4], yq[4], s01, s23, dk;
  auto late = [&](int c) {
    if (!KEEP_P) {
      s01 = ld4(ST + (size_t)(16 * c + 4 * q) * 2);
      s23 = ld4(ST + (size_t)(16 * c + 4 * q) * 2 + 4);
    }
    dk = ld4(DC + 16 * c + 4 * q);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      yk[r] = bld4s(K, sl.base + (uint32_t)(16 * c + 4 * q) * a.ld + 4 * lr, (uint32_t)r * a.ld);
      if (KREF) yq[r] = bld4s(Q, sl.base + (uint32_t)(16 * c + 4 * q) * a.ld + 4 * lr, (uint32_t)r * a.ld);
    }
  };
  // Only the tile's last two chunks reach past the diagonal (MASK).
  auto body = [&](auto mask_tag, int c, const Chunk& ch) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int k0 = 16 * c;
    const float mk[4] = {s01[0], s01[2], s23[0], s23[2]};
    const float il[4] = {s01[1], s01[3], s23[1], s23[3]};
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      f32x4 qb[4], ob[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if (KEEP_P) {
          ob[s] = obr[n][s];
        } else {
          qb[s] = *reinterpret_cast<const f32x4*>(qs + (16 * n + lr) * LQ + 16 * s + 4 * q);
          ob[s] = *reinterpret_cast<const f32x4*>(os + (16 * n + lr) * LQ + 16 * s + 4 * q);
        }
      }
      f32x4 st = {0.f, 0.f, 0.f, 0.f}, dt = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (!KEEP_P) st = mfma4(ch.ka[s][j], qb[s][j], st);
          dt = mfma4(ch.va[s][j], ob[s][j], dt);
        }
      float ds[4];
      if (KEEP_P) {
        const int qb16 = q0 / 16 + n;
        f32x4 pt = {0.f, 0.f, 0.f, 0.f};
        if (c <= qb16) pt = *reinterpret_cast<const f32x4*>(sst + (qb16 * (qb16 + 1) / 2 + c) * 256 + lr * 16 + 4 * q);
#pragma unroll
        for (int r = 0; r < 4; ++r) ds[r] = pt[r] * (dt[r] - dk[r]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool keep = !MASK || q0 + 16 * n + lr >= k0 + 4 * q + r;
          ds[r] = __expf(a.scale * st[r] - mk[r]) * (keep ? il[r] : 0.f) * (dt[r] - dk[r]);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[i][n] = mfma4(yk[r][i], ds[r], acc[i][n]);
          if (KREF) acc[i][2 + n] = mfma4(yq[r][i], ds[r], acc[i][2 + n]);
        }
      __builtin_amdgcn_sched_barrier(0);  // block n + 1's LDS reads stay after block n's products
    }
  };
  auto compute = [&](int c, const Chunk& ch) {
    if (CAUSAL && c >= q0 / 16) body(std::true_type{}, c, ch);
    else body(std::false_type{}, c, ch);
  };
  chunk_loop<Chunk>(0, CAUSAL ? (q0 + TW) / 16 : a.seq / 16, fetch, compute, late);
  // acc[i][n][r] = X^T[d = 16q + 4r + i][query q0 + 16(n % 2) + lr]
  const __amdgpu_buffer_rsrc_t dQr = rsrc(a.dq, a.bytes);
#pragma unroll
  for (int n = 0; n < 2; ++n)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t e = sl.base + (uint32_t)(q0 + 16 * n + lr) * a.ld + 16 * q + 4 * r;
      f32x4 g = a.scale * f32x4{acc[0][n][r], acc[1][n][r], acc[2][n][r], acc[3][n][r]};
      if (a.acc_q) g += bld4(dQr, e);
      bst4(dQr, e, g);
    }
  if (KREF) {
    // C[d][j] lands at flat d * seq + j of the head's [seq x 64] block.
    const __amdgpu_buffer_rsrc_t dKr = rsrc(a.dk, a.bytes);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t d = 16 * q + 4 * r + i, j = q0 + 16 * n + lr;
          const uint32_t f = d * (uint32_t)a.seq + j;
          const uint32_t e = sl.base + (f / HD) * a.ld + f % HD;
          float g = a.scale * acc[i][2 + n][r];
          if (a.acc_k) g += bld1(dKr, e);
          bst1(dKr, e, g);
        }
  }
}

// ---------------------------------------------------------------------------
// Causal whole-slice passes (seq <= 256) with the scores or probabilities kept
// in LDS.  The output passes give every wave two 16-row blocks b and
// nb - 1 - b (nb = seq / 16): under the mask block b's work grows with b, so
// every wave carries nb + 1 block-chunks, and no wave is left running alone on
// its SIMD at the end (with 32-row tiles balanced only per SIMD pair, the
// heaviest wave had twice the average work).  Chunks a block does not reach
// (wholly above the diagonal, all-zero probabilities) are skipped.

// Statistics for keys k0 .. k0 + 31 in two passes.  Pass A: S^T = K Q^T over
// every query chunk (the maximum is taken over every row), each lane's running
// maximum, and the blocks on or below the diagonal written to sst as
// stats_tile<true, true> writes them.  Pass B: the wave reads its own kept
// blocks back and sums exp(S - m_c) over the unmasked queries with the final
// maximum -- one exponential per kept score, where an online sum rescales in
// every chunk.
__device__ __forceinline__ void stats_kept(const AttnArgs& a, const Slice& sl, int k0, float* sst) {
  const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
  const __amdgpu_buffer_rsrc_t Q = rsrc(a.q, a.bytes);
  const __amdgpu_buffer_rsrc_t K = rsrc(a.k, a.bytes);
  f32x4 ka[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int s = 0; s < 4; ++s) ka[i][s] = bld4(K, sl.base + (uint32_t)(k0 + 16 * i + lr) * a.ld + 16 * s + 4 * q);
  float m[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) m[i][r] = -FLT_MAX;
  struct Chunk {
    f32x4 qb[2][4];
  };
  auto fetch = [&](int c, Chunk& ch) {
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        ch.qb[n][s] = bld4(Q, sl.base + (uint32_t)(TW * c + 16 * n + lr) * a.ld + 16 * s + 4 * q);
  };
  auto compute = [&](int c, const Chunk& ch) {
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][n] = mfma4(ka[i][s][j], ch.qb[n][s][j], acc[i][n]);
      }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        const int kb = k0 / 16 + i, qb = 2 * c + n;
        if (kb <= qb) *reinterpret_cast<f32x4*>(sst + (qb * (qb + 1) / 2 + kb) * 256 + 4 * lane) = acc[i][n];
      }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) m[i][r] = fmaxf(m[i][r], fmaxf(a.scale * acc[i][0][r], a.scale * acc[i][1][r]));
  };
  chunk_loop<Chunk>(0, a.seq / TW, fetch, compute);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) m[i][r] = fmaxf(m[i][r], __shfl_xor(m[i][r], off, 64));
  // The blocks read below are this wave's own writes.
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  float l[2][4];
  const int nb = a.seq / 16;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int kb = k0 / 16 + i;
    const f32x4 d4 = *reinterpret_cast<const f32x4*>(sst + (kb * (kb + 1) / 2 + kb) * 256 + 4 * lane);
#pragma unroll
    for (int r = 0; r < 4; ++r)  // the diagonal block: query lr against key 4q + r
      l[i][r] = lr >= 4 * q + r ? __expf(a.scale * d4[r] - m[i][r]) : 0.f;
    int qb = kb + 1;
    for (; qb + 1 < nb; qb += 2) {
      const f32x4 s0 = *reinterpret_cast<const f32x4*>(sst + (qb * (qb + 1) / 2 + kb) * 256 + 4 * lane);
      const f32x4 s1 = *reinterpret_cast<const f32x4*>(sst + ((qb + 1) * (qb + 2) / 2 + kb) * 256 + 4 * lane);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        l[i][r] += __expf(a.scale * s0[r] - m[i][r]);
        l[i][r] += __expf(a.scale * s1[r] - m[i][r]);
      }
    }
    if (qb < nb) {
      const f32x4 s0 = *reinterpret_cast<const f32x4*>(sst + (qb * (qb + 1) / 2 + kb) * 256 + 4 * lane);
#pragma unroll
      for (int r = 0; r < 4; ++r) l[i][r] += __expf(a.scale * s0[r] - m[i][r]);
    }
  }
  // Sum over the 16 lanes of a key (a + b == b + a: every lane ends equal).
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) l[i][r] += __shfl_xor(l[i][r], off, 64);
  if (lr == 0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) l[i][r] = 1.0f / (l[i][r] < 1e-45f ? 1.0f : l[i][r]);
      float* S = a.stats + ((size_t)sl.z * a.seq + k0 + 16 * i + 4 * q) * 2;
      st4(S, f32x4{m[i][0], l[i][0], m[i][1], l[i][1]});
      st4(S + 4, f32x4{m[i][2], l[i][2], m[i][3], l[i][3]});
    }
  }
}

// O = P V for the 16-query blocks b0 < b1 (rows 16 b + lr), from the kept S^T
// blocks: per 16-key chunk c <= b, P^T = exp(S - m) / l (masked on the
// diagonal chunk c == b) and O^T += V^T P^T, the products of each block in the
// order fwd_tile issues them.
__device__ __forceinline__ void fwd_kept(const AttnArgs& a, const Slice& sl, int b0, int b1, const float* sst) {
  const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
  const __amdgpu_buffer_rsrc_t V = rsrc(a.v, a.bytes);
  const __amdgpu_buffer_rsrc_t PK = kept_rsrc(a, sl);
  const float* ST = a.stats + (size_t)sl.z * a.seq * 2;
  const int bk[2] = {b0, b1};
  f32x4 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 2; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  struct Chunk {
    f32x4 va[4], s01, s23, st[2];
  };
  auto fetch = [&](int c, Chunk& ch) {
    const int k0 = 16 * c;
#pragma unroll
    for (int r = 0; r < 4; ++r) ch.va[r] = bld4s(V, sl.base + (uint32_t)(k0 + 4 * q) * a.ld + 4 * lr, (uint32_t)r * a.ld);
    ch.s01 = ld4(ST + (size_t)(k0 + 4 * q) * 2);
    ch.s23 = ld4(ST + (size_t)(k0 + 4 * q) * 2 + 4);
#pragma unroll
    for (int n = 0; n < 2; ++n)
      if (c <= bk[n]) ch.st[n] = *reinterpret_cast<const f32x4*>(sst + (bk[n] * (bk[n] + 1) / 2 + c) * 256 + 4 * lane);
  };
  auto compute = [&](int c, const Chunk& ch) {
    const float mk[4] = {ch.s01[0], ch.s01[2], ch.s23[0], ch.s23[2]};
    const float il[4] = {ch.s01[1], ch.s01[3], ch.s23[1], ch.s23[3]};
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      if (c > bk[n]) continue;
      const bool diag = c == bk[n];
      float pt[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool keep = !diag || lr >= 4 * q + r;
        pt[r] = keep ? __expf(a.scale * ch.st[n][r] - mk[r]) * il[r] : 0.f;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][n] = mfma4(ch.va[r][i], pt[r], acc[i][n]);
      // P^T[key 4q + r][query lr] for the backward, whose dV-pass lane reads
      // its four queries of one key as one 16-byte load
      const uint32_t blk = (uint32_t)(bk[n] * (bk[n] + 1) / 2 + c) * 256 + lr;
#pragma unroll
      for (int r = 0; r < 4; ++r) bst1(PK, blk + (4 * q + r) * 16, pt[r]);
    }
  };
  chunk_loop<Chunk>(0, b1 + 1, fetch, compute);
  const __amdgpu_buffer_rsrc_t O = rsrc(a.out, a.bytes);
#pragma unroll
  for (int n = 0; n < 2; ++n)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      bst4(O, sl.base + (uint32_t)(16 * bk[n] + lr) * a.ld + 16 * q + 4 * r,
           f32x4{acc[0][n][r], acc[1][n][r], acc[2][n][r], acc[3][n][r]});
}

// dV for the 16-key blocks b0 < b1 (keys 16 b + lr): per query chunk c >= b,
// P from the forward's kept blocks (zero past the diagonal), copied into sst
// with the query as the row for the dQ pass, and dV^T += dO^T P; then D, and
// with DK a second pass for dS = P (dP - D) and dK^T += Q^T dS.
template <bool DK>
__device__ __forceinline__ void bwd_kv_kept(const AttnArgs& a, const Slice& sl, int b0, int b1, float* sst) {
  const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
  const __amdgpu_buffer_rsrc_t Q = rsrc(a.q, a.bytes);
  const __amdgpu_buffer_rsrc_t V = rsrc(a.v, a.bytes);
  const __amdgpu_buffer_rsrc_t dO = rsrc(a.dout, a.bytes);
  const __amdgpu_buffer_rsrc_t PK = kept_rsrc(a, sl);
  const int bk[2] = {b0, b1};
  f32x4 vB[2][4];
  if (DK) {
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int s = 0; s < 4; ++s) vB[n][s] = bld4(V, sl.base + (uint32_t)(16 * bk[n] + lr) * a.ld + 16 * s + 4 * q);
  }
  f32x4 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 2; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  float D[2] = {0.f, 0.f};
  struct Chunk {
    f32x4 oa[4], at[4], pk[2];
  };
  auto run = [&](auto pass2_tag) {
    constexpr bool P2 = decltype(pass2_tag)::value;
    auto fetch = [&](int c, Chunk& ch) {
      const int qc = 16 * c;
      if (P2) {
#pragma unroll
        for (int s = 0; s < 4; ++s) ch.oa[s] = bld4(dO, sl.base + (uint32_t)(qc + lr) * a.ld + 16 * s + 4 * q);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
        ch.at[r] = bld4s(P2 ? Q : dO, sl.base + (uint32_t)(qc + 4 * q) * a.ld + 4 * lr, (uint32_t)r * a.ld);
      // P[query 4q + r][key lr], r = 0..3: one 16-byte load per kept block
#pragma unroll
      for (int n = 0; n < 2; ++n)
        if (c >= bk[n]) ch.pk[n] = bld4(PK, (uint32_t)(c * (c + 1) / 2 + bk[n]) * 256 + 16 * lr + 4 * q);
    };
    auto compute = [&](int c, const Chunk& ch) {
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        if (c < bk[n]) continue;
        float bop[4];
        if (P2) {
          f32x4 da = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int j = 0; j < 4; ++j) da = mfma4(ch.oa[s][j], vB[n][s][j], da);
#pragma unroll
          for (int r = 0; r < 4; ++r) bop[r] = ch.pk[n][r] * (da[r] - D[n]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) bop[r] = ch.pk[n][r];
          float* blk = sst + (c * (c + 1) / 2 + bk[n]) * 256 + lr;
#pragma unroll
          for (int r = 0; r < 4; ++r) blk[(4 * q + r) * 16] = bop[r];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i][n] = mfma4(ch.at[r][i], bop[r], acc[i][n]);
      }
    };
    chunk_loop<Chunk>(b0, a.seq / 16, fetch, compute);
  };
  run(std::false_type{});
  const __amdgpu_buffer_rsrc_t dVr = rsrc(a.dv, a.bytes);
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    const uint32_t row = sl.base + (uint32_t)(16 * bk[n] + lr) * a.ld;
    float part = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const f32x4 vv = bld4(V, row + 16 * q + 4 * r);
      f32x4 g = {acc[0][n][r], acc[1][n][r], acc[2][n][r], acc[3][n][r]};
      part += g[0] * vv[0] + g[1] * vv[1] + g[2] * vv[2] + g[3] * vv[3];
      if (a.acc_v) g += bld4(dVr, row + 16 * q + 4 * r);
      bst4(dVr, row + 16 * q + 4 * r, g);
    }
    part += __shfl_xor(part, 16, 64);
    part += __shfl_xor(part, 32, 64);
    D[n] = part;
    if (q == 0) a.dcol[(size_t)sl.z * a.seq + 16 * bk[n] + lr] = part;
  }
  if (!DK) return;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 2; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  run(std::true_type{});
  const __amdgpu_buffer_rsrc_t dKr = rsrc(a.dk, a.bytes);
#pragma unroll
  for (int n = 0; n < 2; ++n)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t e = sl.base + (uint32_t)(16 * bk[n] + lr) * a.ld + 16 * q + 4 * r;
      f32x4 g = a.scale * f32x4{acc[0][n][r], acc[1][n][r], acc[2][n][r], acc[3][n][r]};
      if (a.acc_k) g += bld4(dKr, e);
      bst4(dKr, e, g);
    }
}

// bwd_q_tile<true, KREF, true> for the 16-query blocks b0 < b1: P of every
// key chunk c <= b from sst, dP^T = V dO^T, dS^T = P^T (dP^T - D), then
// dQ^T += K^T dS^T and with KREF the reference's K gradient.
template <bool KREF>
__device__ __forceinline__ void bwd_q_kept(const AttnArgs& a, const Slice& sl, int b0, int b1, const float* sst) {
  const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
  const __amdgpu_buffer_rsrc_t Q = rsrc(a.q, a.bytes);
  const __amdgpu_buffer_rsrc_t K = rsrc(a.k, a.bytes);
  const __amdgpu_buffer_rsrc_t V = rsrc(a.v, a.bytes);
  const __amdgpu_buffer_rsrc_t dO = rsrc(a.dout, a.bytes);
  const float* DC = a.dcol + (size_t)sl.z * a.seq;
  const int bk[2] = {b0, b1};
  f32x4 obr[2][4];
#pragma unroll
  for (int n = 0; n < 2; ++n)
#pragma unroll
    for (int s = 0; s < 4; ++s) obr[n][s] = bld4(dO, sl.base + (uint32_t)(16 * bk[n] + lr) * a.ld + 16 * s + 4 * q);
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  struct Chunk {
    f32x4 va[4];
  };
  auto fetch = [&](int c, Chunk& ch) {
#pragma unroll
    for (int s = 0; s < 4; ++s) ch.va[s] = bld4(V, sl.base + (uint32_t)(16 * c + lr) * a.ld + 16 * s + 4 * q);
  };
  f32x4 yk[4], yq[4], dk;
  auto late = [&](int c) {
    dk = ld4(DC + 16 * c + 4 * q);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      yk[r] = bld4s(K, sl.base + (uint32_t)(16 * c + 4 * q) * a.ld + 4 * lr, (uint32_t)r * a.ld);
      if (KREF) yq[r] = bld4s(Q, sl.base + (uint32_t)(16 * c + 4 * q) * a.ld + 4 * lr, (uint32_t)r * a.ld);
    }
  };
  auto compute = [&](int c, const Chunk& ch) {
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      if (c > bk[n]) continue;
      f32x4 dt = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) dt = mfma4(ch.va[s][j], obr[n][s][j], dt);
      const f32x4 pt = *reinterpret_cast<const f32x4*>(sst + (bk[n] * (bk[n] + 1) / 2 + c) * 256 + lr * 16 + 4 * q);
      float ds[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) ds[r] = pt[r] * (dt[r] - dk[r]);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[i][n] = mfma4(yk[r][i], ds[r], acc[i][n]);
          if (KREF) acc[i][2 + n] = mfma4(yq[r][i], ds[r], acc[i][2 + n]);
        }
      __builtin_amdgcn_sched_barrier(0);  // block n + 1's LDS reads stay after block n's products
    }
  };
  chunk_loop<Chunk>(0, b1 + 1, fetch, compute, late);
  const __amdgpu_buffer_rsrc_t dQr = rsrc(a.dq, a.bytes);
#pragma unroll
  for (int n = 0; n < 2; ++n)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t e = sl.base + (uint32_t)(16 * bk[n] + lr) * a.ld + 16 * q + 4 * r;
      f32x4 g = a.scale * f32x4{acc[0][n][r], acc[1][n][r], acc[2][n][r], acc[3][n][r]};
      if (a.acc_q) g += bld4(dQr, e);
      bst4(dQr, e, g);
    }
  if (KREF) {
    const __amdgpu_buffer_rsrc_t dKr = rsrc(a.dk, a.bytes);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t d = 16 * q + 4 * r + i, j = 16 * bk[n] + lr;
          const uint32_t f = d * (uint32_t)a.seq + j;
          const uint32_t e = sl.base + (f / HD) * a.ld + f % HD;
          float g = a.scale * acc[i][2 + n][r];
          if (a.acc_k) g += bld1(dKr, e);
          bst1(dKr, e, g);
        }
  }
}

// One wave per 32-row tile, two tiles (j and nb - 1 - j) per workgroup,
// workgroups spread over the XCDs by slice (slice_of).
template <bool CAUSAL>
__global__ __launch_bounds__(128, 2) void attn_stats_kernel(AttnArgs a) {
  const Slice sl = slice_of(a);
  stats_tile<CAUSAL>(a, sl, tile_of(a, sl, threadIdx.x >> 6) * TW);
}
template <bool CAUSAL>
__global__ __launch_bounds__(128, 2) void attn_fwd_kernel(AttnArgs a) {
  const Slice sl = slice_of(a);
  fwd_tile<CAUSAL>(a, sl, tile_of(a, sl, threadIdx.x >> 6) * TW);
}
template <bool CAUSAL, bool DK>
__global__ __launch_bounds__(128, 2) void attn_bwd_kv_kernel(AttnArgs a) {
  const Slice sl = slice_of(a);
  bwd_kv_tile<CAUSAL, DK>(a, sl, tile_of(a, sl, threadIdx.x >> 6) * TW);
}
template <bool CAUSAL, bool KREF>
__global__ __launch_bounds__(128, 2) void attn_bwd_q_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) float lds[2][2][TW * LQ];  // [wave][Q, dO][row * LQ + col]
  const Slice sl = slice_of(a);
  const int w = threadIdx.x >> 6;
  bwd_q_tile<CAUSAL, KREF>(a, sl, tile_of(a, sl, w) * TW, lds[w][0], lds[w][1]);
}

// Whole-slice kernels for seq <= 256: workgroup z runs every tile of slice z
// with one wave per tile (SW waves), the two passes of the forward (or the
// backward) separated by a workgroup barrier instead of a kernel boundary.
// Each kernel launch pays a ramp (every wave waits for its first operands
// from memory at once) and a tail (every store at the end); this pays them
// once per direction.  Under the causal mask the passes whose work grows or
// shrinks with the row index give wave w the 16-row blocks w and
// seq / 16 - 1 - w (the *_kept functions), so every wave carries the same
// work.
constexpr int SW = 8;  // waves per slice workgroup: seq / TW tiles, at most 8
__device__ __forceinline__ Slice slice_whole(const AttnArgs& a) {
  const int z = blockIdx.x, b = z / a.heads, h = z - b * a.heads;
  return {z, (uint32_t)b * a.seq * a.ld + (uint32_t)h * HD, 0};
}
// Causal: the statistics pass keeps the slice's S^T blocks on or below the
// diagonal in LDS (seq / 16 (seq / 16 + 1) / 2 blocks of 1 KB, 136 KB at seq
// 256) and the output pass reads them instead of recomputing its products;
// the output pass stores the blocks' P to a.kept for the backward.
template <bool CAUSAL>
__global__ __launch_bounds__(SW * 64, 1) void attn_fwd_slice_kernel(AttnArgs a) {
  constexpr int kBlocks = CAUSAL ? (SW * TW / 16) * (SW * TW / 16 + 1) / 2 : 1;
  __shared__ __attribute__((aligned(16))) float sst[kBlocks * 256];
  const Slice sl = slice_whole(a);
  // the wave index, read as wave-uniform so that block choices and loop bounds
  // derived from it stay in scalar registers and branch on the scalar unit
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), ntile = a.seq / TW;
  if constexpr (CAUSAL) {
    if (w < ntile) stats_kept(a, sl, w * TW, sst);
    __syncthreads();  // the slice's statistics and kept scores are written
    if (w < ntile) fwd_kept(a, sl, w, 2 * ntile - 1 - w, sst);
  } else {
    if (w < ntile) stats_tile<false>(a, sl, w * TW);
    __syncthreads();  // the slice's statistics are written
    if (w < ntile) fwd_tile<false>(a, sl, w * TW);
  }
}
// Causal: the dV pass reads the forward's P blocks from a.kept and copies
// them into LDS (136 KB at seq 256) for the dQ pass, so neither pass
// recomputes S or its exponentials; without the mask the dQ pass stages its
// Q and dO rows in LDS and recomputes.
template <bool CAUSAL, bool KREF>
__global__ __launch_bounds__(SW * 64, 1) void attn_bwd_slice_kernel(AttnArgs a) {
  constexpr int kFloats = CAUSAL ? (SW * TW / 16) * (SW * TW / 16 + 1) / 2 * 256 : SW * 2 * TW * LQ;
  __shared__ __attribute__((aligned(16))) float lds[kFloats];
  const Slice sl = slice_whole(a);
  // the wave index, read as wave-uniform so that block choices and loop bounds
  // derived from it stay in scalar registers and branch on the scalar unit
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), ntile = a.seq / TW;
  if constexpr (CAUSAL) {
    if (w < ntile) bwd_kv_kept<!KREF>(a, sl, w, 2 * ntile - 1 - w, lds);
    __syncthreads();  // D of every key of the slice and the kept P are written
    if (w < ntile) bwd_q_kept<KREF>(a, sl, w, 2 * ntile - 1 - w, lds);
  } else {
    if (w < ntile) bwd_kv_tile<false, !KREF>(a, sl, w * TW);
    __syncthreads();  // D of every key of the slice is written
    float* own = lds + w * 2 * TW * LQ;  // the wave's staging region
    if (w < ntile) bwd_q_tile<false, KREF>(a, sl, w * TW, own, own + TW * LQ);
  }
}

// Operand addressing uses 32-bit byte offsets into buffer resources whose
// extent is the tensor's byte size (AttnArgs::bytes), so every tensor must stay
// below 2 GiB in bytes, not elements.
bool attn_shape_ok(int batch, int heads, int seq, int head_dim, int ld) {
  return batch > 0 && heads > 0 && head_dim == HD && seq >= 64 && seq % 64 == 0 && ld % 4 == 0 &&
         ld >= heads * HD && (double)batch * heads <= 65535.0 &&
         (double)batch * seq * ld * sizeof(float) < 2147483648.0 - 64.0;
}

}  // namespace

extern "C" {

size_t mle_attention_ws_bytes(int batch, int heads, int seq) {
  if (batch <= 0 || heads <= 0 || seq <= 0) return 0;
  // statistics and D per key, then (seq <= 256, the slice kernels) the kept
  // probability blocks of the causal forward for the backward
  const size_t kept = seq <= SW * TW ? kept_blocks(seq) * 256 : 0;
  return (size_t)batch * heads * (seq * 3 + kept) * sizeof(float);
}

int mle_attention_fwd(mle_stream stream, const float* q, const float* k, const float* v, float* out, int batch,
                      int heads, int seq, int head_dim, int ld, float scale, int causal, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(q && k && v && out && ws, "mle_attention_fwd: null pointer");
  if (!attn_shape_ok(batch, heads, seq, head_dim, ld))
    return set_error(MLE_ERR_UNSUPPORTED,
                     "mle_attention_fwd: needs head_dim 64, seq a multiple of 64, ld %% 4 == 0 and tensors below 2 GiB");
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
  a.kept = a.dcol + (size_t)batch * heads * seq;
  a.heads = heads;
  a.seq = seq;
  a.ld = ld;
  a.bytes = (uint32_t)((size_t)batch * seq * ld * sizeof(float));
  a.scale = scale;
  hipStream_t s = as_stream(stream);
  const dim3 grid((unsigned)(seq / (2 * TW) * batch * heads));  // two 32-row tiles per workgroup
  const double flop = 4.0 * batch * heads * (double)seq * seq * HD;  // S and P V, as the reference computes them
  ProbeScope probe("attn_fwd", s, flop, 0.0);
  if (seq <= SW * TW) {
    const dim3 slices((unsigned)(batch * heads));
    if (causal) mle::launch(attn_fwd_slice_kernel<true>, slices, SW * 64, 0, s, a);
    else mle::launch(attn_fwd_slice_kernel<false>, slices, SW * 64, 0, s, a);
  } else if (causal) {
    mle::launch(attn_stats_kernel<true>, grid, 128, 0, s, a);
    mle::launch(attn_fwd_kernel<true>, grid, 128, 0, s, a);
  } else {
    mle::launch(attn_stats_kernel<false>, grid, 128, 0, s, a);
    mle::launch(attn_fwd_kernel<false>, grid, 128, 0, s, a);
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
  a.kept = a.dcol + (size_t)batch * heads * seq;
  a.heads = heads;
  a.seq = seq;
  a.ld = ld;
  a.bytes = (uint32_t)((size_t)batch * seq * ld * sizeof(float));
  a.scale = scale;
  a.acc_q = acc_q != 0;
  a.acc_k = acc_k != 0;
  a.acc_v = acc_v != 0;
  hipStream_t s = as_stream(stream);
  const dim3 grid((unsigned)(seq / (2 * TW) * batch * heads));  // two 32-row tiles per workgroup
  const double flop = 8.0 * batch * heads * (double)seq * seq * HD;  // dP, dV, dQ, dK
  ProbeScope probe("attn_bwd", s, flop, 0.0);
  const bool kref = k_reference_grad != 0;
  if (seq <= SW * TW) {
    const dim3 slices((unsigned)(batch * heads));
    if (causal) {
      if (kref) mle::launch(attn_bwd_slice_kernel<true, true>, slices, SW * 64, 0, s, a);
      else mle::launch(attn_bwd_slice_kernel<true, false>, slices, SW * 64, 0, s, a);
    } else {
      if (kref) mle::launch(attn_bwd_slice_kernel<false, true>, slices, SW * 64, 0, s, a);
      else mle::launch(attn_bwd_slice_kernel<false, false>, slices, SW * 64, 0, s, a);
    }
  } else if (causal) {
    if (kref) {
      mle::launch(attn_bwd_kv_kernel<true, false>, grid, 128, 0, s, a);
      mle::launch(attn_bwd_q_kernel<true, true>, grid, 128, 0, s, a);
    } else {
      mle::launch(attn_bwd_kv_kernel<true, true>, grid, 128, 0, s, a);
      mle::launch(attn_bwd_q_kernel<true, false>, grid, 128, 0, s, a);
    }
  } else {
    if (kref) {
      mle::launch(attn_bwd_kv_kernel<false, false>, grid, 128, 0, s, a);
      mle::launch(attn_bwd_q_kernel<false, true>, grid, 128, 0, s, a);
    } else {
      mle::launch(attn_bwd_kv_kernel<false, true>, grid, 128, 0, s, a);
      mle::launch(attn_bwd_q_kernel<false, false>, grid, 128, 0, s, a);
    }
  }
  return check_launch("mle_attention_bwd");
}

}  // extern "C"
