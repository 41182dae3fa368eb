// Integer / index paths: embedding gather, deterministic scatter-add, one-hot,
// argmax (GatherEmbeddings, KeyUpdate, OneHotEmbeddings, ArgMax:
// Engine/kernels.cu:2279-2296, 1536-1560, 2353-2366), plus the column and
// channel reductions used by bias gradients (BCompress, Channel_Squeeze1D:
// Engine/kernels.cu:1562-1584, 1734-1761).
#include "common.hpp"

#include <algorithm>
#include <limits.h>

using namespace mle;

namespace {

constexpr int NT = 256;
constexpr int SORT_CAP = 16384;  // tokens sorted per chunk in LDS (128 KB of keys)
constexpr int SORT_NT = 1024;

__global__ __launch_bounds__(NT) void gather_kernel(float* __restrict__ out, const float* __restrict__ table,
                                                    const int32_t* __restrict__ keys, int clen, int max_clen, int dim,
                                                    size_t total) {
  const size_t stride = (size_t)gridDim.x * NT;
  for (size_t g = (size_t)blockIdx.x * NT + threadIdx.x; g < total; g += stride) {
    const size_t tok = g / dim;
    const int d = (int)(g % dim);
    const size_t b = tok / clen, s = tok % clen;
    const int key = keys[b * max_clen + s];
    out[g] = (key == INT_MIN || key < 0) ? 0.0f : table[(size_t)key * dim + d];
  }
}

__global__ __launch_bounds__(NT) void gather4_kernel(float* __restrict__ out, const float* __restrict__ table,
                                                     const int32_t* __restrict__ keys, int clen, int max_clen, int dim,
                                                     size_t total4) {
  const size_t stride = (size_t)gridDim.x * NT;
  const int dim4 = dim / 4;
  for (size_t g = (size_t)blockIdx.x * NT + threadIdx.x; g < total4; g += stride) {
    const size_t tok = g / dim4;
    const int d = (int)(g % dim4) * 4;
    const size_t b = tok / clen, s = tok % clen;
    const int key = keys[b * max_clen + s];
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (!(key == INT_MIN || key < 0)) v = *reinterpret_cast<const f32x4*>(table + (size_t)key * dim + d);
    *reinterpret_cast<f32x4*>(out + tok * dim + d) = v;
  }
}

__global__ __launch_bounds__(NT) void onehot_kernel(float* __restrict__ out, const int32_t* __restrict__ keys, int clen,
                                                    int max_clen, int vocab, size_t total) {
  const size_t stride = (size_t)gridDim.x * NT;
  for (size_t g = (size_t)blockIdx.x * NT + threadIdx.x; g < total; g += stride) {
    const size_t row = g / clen, col = g % clen;
    const int key = keys[row * max_clen + col];
    if (key == INT_MIN || key < 0 || key >= vocab) continue;
    out[g * vocab + key] = 1.0f;
  }
}

// One wave per row.  Each lane keeps its first maximum (strict >), then the
// wave keeps the larger value, ties to the lower index: the first maximum of
// the row.  A NaN at index 0 makes the row's answer 0, as in the serial scan.
__global__ __launch_bounds__(64) void argmax_kernel(const float* __restrict__ x, int cols, int32_t* __restrict__ out) {
  const float* r = x + (size_t)blockIdx.x * cols;
  const int lane = threadIdx.x;
  float best = 0.f;
  int bi = INT_MAX;
  for (int c = lane; c < cols; c += 64) {
    const float v = r[c];
    if (v != v) continue;
    if (bi == INT_MAX || v > best) {
      best = v;
      bi = c;
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    const float ob = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (oi != INT_MAX && (bi == INT_MAX || ob > best || (ob == best && oi < bi))) {
      best = ob;
      bi = oi;
    }
  }
  if (lane == 0) {
    const float first = r[0];
    out[blockIdx.x] = (first != first || bi == INT_MAX) ? 0 : bi;
  }
}

// Sort (key, token) pairs of one chunk in LDS: bitonic sort of 64-bit values
// key << 32 | token.  Invalid keys sort last with key 0x7fffffff.
__global__ __launch_bounds__(SORT_NT) void sort_chunk_kernel(const int32_t* __restrict__ keys, int clen, int max_clen,
                                                             int vocab, int tok0, int count,
                                                             unsigned long long* __restrict__ sorted) {
  __shared__ unsigned long long s[SORT_CAP];
  int np = 2;
  while (np < count) np <<= 1;
  for (int i = threadIdx.x; i < np; i += SORT_NT) {
    unsigned long long v = ~0ull;
    if (i < count) {
      const int t = tok0 + i;
      const int key = keys[(size_t)(t / clen) * max_clen + (t % clen)];
      const unsigned k = (key < 0 || key >= vocab) ? 0x7fffffffu : (unsigned)key;
      v = ((unsigned long long)k << 32) | (unsigned)t;
    }
    s[i] = v;
  }
  __syncthreads();
  for (int k = 2; k <= np; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < np; i += SORT_NT) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const unsigned long long a = s[i], b = s[ixj];
          const bool up = (i & k) == 0;
          if ((a > b) == up) {
            s[i] = b;
            s[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < count; i += SORT_NT) sorted[i] = s[i];
}

// Scatter-add by row ranges: workgroup g owns table rows [g R, g R + R) and
// reads every token's key, keeping the tokens that fall in its rows.  Per chunk
// of RS_CHUNK tokens, in LDS:
//   1. a histogram over its R rows, and its exclusive scan
//   2. placement of each kept token by atomic decrement of its row's end, which
//      leaves every row's start behind (positions within a row in arrival order)
//   3. the row's tokens put in token order: each entry goes to its row start
//      plus its rank, the number of the row's entries with a smaller token index
//   4. one wave per row sums the row's gradient rows in token order and adds
//      scale * sum to the table row.
// No sort buffer and no second launch; the result does not depend on the order
// the atomics ran in.  Chunks are applied in token order.  Step 3 costs the
// row's token count per entry, which is small for a batch over a vocabulary.
__device__ __forceinline__ int key_at(const int32_t* __restrict__ keys, int t, int clen, int max_clen) {
  return clen == max_clen ? keys[t] : keys[(size_t)(t / clen) * max_clen + t % clen];
}

// Keys of tokens t0 + threadIdx.x + k NT, k < PER, into kv, every load issued
// before any is used (a load per branch would wait for each in turn).  Tokens
// past the end read the last token's key; the caller masks them.  ntok >= 1.
template <int PER, int NT>
__device__ __forceinline__ void load_keys(const int32_t* __restrict__ keys, int t0, int ntok, int clen, int max_clen,
                                          int (&kv)[PER]) {
  if (clen == max_clen) {
#pragma unroll
    for (int k = 0; k < PER; ++k) kv[k] = keys[min(t0 + (int)threadIdx.x + k * NT, ntok - 1)];
  } else {
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int t = min(t0 + (int)threadIdx.x + k * NT, ntok - 1);
      kv[k] = keys[(size_t)(t / clen) * max_clen + t % clen];
    }
  }
}

// Inclusive prefix sum over the 64 lanes of a wave in DPP steps (no LDS
// round trips): within each row of 16 lanes by shifts of 1, 2, 4 and 8 (lanes
// shifted in from outside the row add 0), then lane 15's row total into rows
// 1 and 3 and lane 31's running total into rows 2 and 3.
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return x;
}

constexpr int RS_NT = 1024;
constexpr int RS_CHUNK = 8192;  // tokens per pass (LDS: two 32 KB lists)
constexpr int RS_RMAX = 64;     // rows per workgroup
constexpr int RS_VMAX = 16384;  // vocabularies up to RS_RMAX * 256 rows use this path
template <bool VEC>
__global__ __launch_bounds__(RS_NT) void range_scatter_kernel(float* __restrict__ table, const float* __restrict__ grad,
                                                              const int32_t* __restrict__ keys, int clen, int max_clen,
                                                              int ntok, int dim, int vocab, int rows_per_wg,
                                                              float scale, int assign) {
  __shared__ int sperm[RS_CHUNK];  // (row << 16) | chunk-local token, per row in arrival order
  __shared__ int slist[RS_CHUNK];  // chunk-local tokens, per row in token order
  __shared__ int sbin[RS_RMAX];
  __shared__ int sstart[RS_RMAX + 1];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int v_lo = blockIdx.x * rows_per_wg;
  const int nrows = min(rows_per_wg, vocab - v_lo);
  if (nrows <= 0) return;
  constexpr int PER = RS_CHUNK / RS_NT;  // tokens per thread per chunk
  for (int t0 = 0; t0 < ntok; t0 += RS_CHUNK) {
    const int count = min(RS_CHUNK, ntok - t0);
    if (tid < nrows) sbin[tid] = 0;
    // this thread's tokens t0 + tid + k * RS_NT: their row within the range
    // (negative keys wrap past nrows), kept for the placement pass
    int kv[PER];
    load_keys<PER, RS_NT>(keys, t0, ntok, clen, max_clen, kv);
    unsigned rel[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) rel[k] = tid + k * RS_NT < count ? (unsigned)(kv[k] - v_lo) : 0xffffffffu;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (rel[k] < (unsigned)nrows) atomicAdd(&sbin[rel[k]], 1);
    __syncthreads();
    if (wid == 0) {
      const int c = lane < nrows ? sbin[lane] : 0;
      const int incl = wave_incl_scan(c);
      if (lane < nrows) {
        sstart[lane] = incl - c;
        sbin[lane] = incl;  // the row's end: the placement counts it down
      }
      if (lane == nrows - 1) sstart[nrows] = incl;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (rel[k] < (unsigned)nrows) sperm[atomicSub(&sbin[rel[k]], 1) - 1] = (int)(rel[k] << 16) | (tid + k * RS_NT);
    __syncthreads();
    const int kept = sstart[nrows];
    for (int p = tid; p < kept; p += RS_NT) {
      const int r = sperm[p] >> 16, i = sperm[p] & 0xffff;
      const int b = sstart[r], e = sstart[r + 1];
      int rank = 0;
      for (int q = b; q < e; ++q) rank += (sperm[q] & 0xffff) < i;
      slist[b + rank] = i;
    }
    __syncthreads();
    // assign: the first chunk writes every row of the range (rows without
    // tokens get 0) instead of adding into it.
    const bool first = assign && t0 == 0;
    for (int r = wid; r < nrows; r += RS_NT / 64) {
      const int b = sstart[r], e = sstart[r + 1];
      if (b == e && !first) continue;
      float* row = table + (size_t)(v_lo + r) * dim;
      if (VEC) {
        // a wave covers 512 floats per pass: lane l holds float4s l and l + 64,
        // and two tokens' loads are in flight before either is added
        for (int d0 = 0; d0 < dim; d0 += 512) {
          const int da = d0 + 4 * lane, db = da + 256;
          const bool ha = da < dim, hb = db < dim;
          const f32x4 z = {0.f, 0.f, 0.f, 0.f};
          f32x4 va = first || !ha ? z : *reinterpret_cast<const f32x4*>(row + da);
          f32x4 vb = first || !hb ? z : *reinterpret_cast<const f32x4*>(row + db);
          f32x4 aa = z, ab = z;
          int j = b;
          for (; j + 1 < e; j += 2) {
            const float* g0 = grad + (size_t)(t0 + slist[j]) * dim;
            const float* g1 = grad + (size_t)(t0 + slist[j + 1]) * dim;
            const f32x4 x0 = ha ? *reinterpret_cast<const f32x4*>(g0 + da) : z;
            const f32x4 y0 = hb ? *reinterpret_cast<const f32x4*>(g0 + db) : z;
            const f32x4 x1 = ha ? *reinterpret_cast<const f32x4*>(g1 + da) : z;
            const f32x4 y1 = hb ? *reinterpret_cast<const f32x4*>(g1 + db) : z;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              aa[c] += x0[c];
              ab[c] += y0[c];
              aa[c] += x1[c];
              ab[c] += y1[c];
            }
          }
          if (j < e) {
            const float* g0 = grad + (size_t)(t0 + slist[j]) * dim;
            const f32x4 x0 = ha ? *reinterpret_cast<const f32x4*>(g0 + da) : z;
            const f32x4 y0 = hb ? *reinterpret_cast<const f32x4*>(g0 + db) : z;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              aa[c] += x0[c];
              ab[c] += y0[c];
            }
          }
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            va[c] += scale * aa[c];
            vb[c] += scale * ab[c];
          }
          if (ha) *reinterpret_cast<f32x4*>(row + da) = va;
          if (hb) *reinterpret_cast<f32x4*>(row + db) = vb;
        }
      } else {
        for (int d = lane; d < dim; d += 64) {
          float acc = 0.f;
          for (int j = b; j < e; ++j) acc += grad[(size_t)(t0 + slist[j]) * dim + d];
          row[d] = (first ? 0.f : row[d]) + scale * acc;
        }
      }
    }
    __syncthreads();  // the next chunk reuses the lists
  }
}

// ---------------------------------------------------------------------------
// Token index per table row, built by the forward gather for the backward.
//
// rinfo[v] = {start, count, tok0, tok1}: the tokens whose key is v are, in
// token order, list[start .. start + count); tok0 and tok1 repeat the first two
// (-1 where absent), so a row with at most two tokens costs the backward one
// 16-byte load.  Keys outside [0, vocab) are in no row.
//
// One launch does both jobs.  Workgroups g < nix each index IX_R table rows
// [g IX_R, g IX_R + IX_R): they read every key (as the range scatter does),
// count the row's tokens and the valid tokens with smaller keys (the range's
// start in `list`, so no global counter is needed), and order each row's
// tokens by token index in LDS.  The workgroups after them gather table rows,
// two tokens per wave at a time.  The index work is latency-bound and small, so
// it runs inside the time the gather takes to stream its bytes.
constexpr int IX_NT = 1024;
constexpr int IX_R = 64;          // table rows per index workgroup (one wave's scan)
constexpr int IX_CHUNK = 8192;    // tokens per pass
// the backward restarts its sums where the range scatter starts a new chunk
static_assert(IX_CHUNK == RS_CHUNK, "per-chunk sums must match the range scatter");
constexpr int IX_VMAX = RS_VMAX;  // larger vocabularies use the scatter paths

// Exclusive scan of cnt over lanes [0, n) of wave 0: start[l] (and start[n]).
__device__ __forceinline__ void wave_starts(const int* cnt, int* start, int n, int lane) {
  const int c = lane < n ? cnt[lane] : 0;
  const int incl = wave_incl_scan(c);
  if (lane < n) start[lane] = incl - c;
  if (lane == n - 1) start[n] = incl;
}

struct IndexLds {
  int perm[IX_CHUNK];  // (row << 16) | chunk-local token, per row in arrival order
  int total[IX_R];     // tokens per row
  int start[IX_R + 1]; // row starts within the range
  int ccnt[IX_R];      // tokens per row in this chunk
  int cstart[IX_R + 1];
  int placed[IX_R];    // tokens per row in earlier chunks
  int tok[2 * IX_R];   // first two tokens per row
  int below;           // valid tokens with keys below the range
};

__device__ __forceinline__ void build_index(IndexLds& L, const int32_t* __restrict__ keys, int clen, int max_clen,
                                            int ntok, int vocab, int range, int4* __restrict__ rinfo,
                                            int32_t* __restrict__ list) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int v_lo = range * IX_R;
  const int nrows = min(IX_R, vocab - v_lo);
  constexpr int PER = IX_CHUNK / IX_NT;
  if (tid < IX_R) {
    L.total[tid] = 0;
    L.placed[tid] = 0;
    L.tok[2 * tid] = -1;
    L.tok[2 * tid + 1] = -1;
  }
  if (tid == 0) L.below = 0;
  // pass 1: tokens per row, and valid tokens below the range.  ent[k] is the
  // token's row in the range | its arrival position in the row << 8, or ~0
  // for a token outside the range; with one chunk it is kept for the placement.
  const bool one = ntok <= IX_CHUNK;
  unsigned ent[PER];
  for (int t0 = 0; t0 < ntok; t0 += IX_CHUNK) {
    int kv[PER];
    load_keys<PER, IX_NT>(keys, t0, ntok, clen, max_clen, kv);
    if (t0 == 0) __syncthreads();  // the counters above are cleared (the loads are in flight)
    int below = 0;  // the wave's count, from ballots
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const bool in = t0 + tid + k * IX_NT < ntok;
      const unsigned rel = (unsigned)(kv[k] - v_lo);
      ent[k] = in && rel < (unsigned)nrows ? rel : 0xffffffffu;
      below += __popcll(__ballot(in && (unsigned)kv[k] < (unsigned)v_lo));
    }
    // all the atomics issued before any result is used
    unsigned pos[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      pos[k] = 0;
      if (ent[k] != 0xffffffffu) pos[k] = (unsigned)atomicAdd(&L.total[ent[k]], 1);
    }
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (ent[k] != 0xffffffffu) ent[k] |= pos[k] << 8;
    if (lane == 0 && below) atomicAdd(&L.below, below);
  }
  __syncthreads();
  if (wid == 0) wave_starts(L.total, L.start, nrows, lane);
  __syncthreads();
  const int base = L.below;
  for (int t0 = 0; t0 < ntok; t0 += IX_CHUNK) {
    const int* cs = L.start;  // with one chunk, the chunk's rows are the rows
    if (!one) {
      if (tid < IX_R) L.ccnt[tid] = 0;
      int kv[PER];
      load_keys<PER, IX_NT>(keys, t0, ntok, clen, max_clen, kv);
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const unsigned rel = (unsigned)(kv[k] - v_lo);
        ent[k] = t0 + tid + k * IX_NT < ntok && rel < (unsigned)nrows ? rel : 0xffffffffu;
      }
      __syncthreads();
      unsigned pos[PER];
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        pos[k] = 0;
        if (ent[k] != 0xffffffffu) pos[k] = (unsigned)atomicAdd(&L.ccnt[ent[k]], 1);
      }
#pragma unroll
      for (int k = 0; k < PER; ++k)
        if (ent[k] != 0xffffffffu) ent[k] |= pos[k] << 8;
      __syncthreads();
      if (wid == 0) wave_starts(L.ccnt, L.cstart, nrows, lane);
      __syncthreads();
      cs = L.cstart;
    }
    // the row starts read for every slot (cs[nrows] for tokens outside the
    // range) so that the reads are all in flight before the writes
    int at[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) at[k] = cs[min(ent[k] & 0xffu, (unsigned)nrows)];
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (ent[k] != 0xffffffffu) L.perm[at[k] + (ent[k] >> 8)] = (int)((ent[k] & 0xffu) << 16) | (tid + k * IX_NT);
    __syncthreads();
    // rank of each entry among its row's entries of the chunk: the row's
    // tokens in token order (the cost is the row's count per entry)
    const int kept = cs[nrows];
    for (int p = tid; p < kept; p += IX_NT) {
      const int r = L.perm[p] >> 16, i = L.perm[p] & 0xffff;
      const int b = cs[r], e = cs[r + 1];
      int rank = 0;
      for (int q = b; q < e; ++q) rank += (L.perm[q] & 0xffff) < i;
      const int at = L.placed[r] + rank;
      list[base + L.start[r] + at] = t0 + i;
      if (at < 2) L.tok[2 * r + at] = t0 + i;
    }
    __syncthreads();
    if (!one && tid < nrows) L.placed[tid] += L.ccnt[tid];
  }
  __syncthreads();
  if (tid < nrows) rinfo[v_lo + tid] = make_int4(base + L.start[tid], L.total[tid], L.tok[2 * tid], L.tok[2 * tid + 1]);
}

// The gather side: wave w of the gather workgroups copies tokens w, w + W, ...
// IX_TPW at a time, all their loads in flight before the stores.  Keys outside
// [0, vocab) give zero rows.
constexpr int IX_TPW = 4;  // measured at 8192 x 512: 4 beats 2 and 1 (fewer waves to dispatch)
template <bool VEC>
__device__ __forceinline__ void gather_rows(float* __restrict__ out, const float* __restrict__ table,
                                            const int32_t* __restrict__ keys, int clen, int max_clen, int ntok,
                                            int dim, int vocab, int gblock, int ngblocks) {
  const int lane = threadIdx.x & 63;
  const int nw = ngblocks * (IX_NT / 64);
  for (int t = gblock * (IX_NT / 64) + (threadIdx.x >> 6); t < ntok; t += IX_TPW * nw) {
    const float* src[IX_TPW];
    bool ok[IX_TPW];
#pragma unroll
    for (int j = 0; j < IX_TPW; ++j) {
      const int u = t + j * nw;
      const int key = u < ntok ? key_at(keys, u, clen, max_clen) : -1;
      ok[j] = (unsigned)key < (unsigned)vocab;
      src[j] = table + (size_t)(ok[j] ? key : 0) * dim;
    }
    if (VEC) {
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
      for (int d0 = 0; d0 < dim; d0 += 512) {
        const int da = d0 + 4 * lane, db = da + 256;
        const bool ha = da < dim, hb = db < dim;
        f32x4 a[IX_TPW], b[IX_TPW];
#pragma unroll
        for (int j = 0; j < IX_TPW; ++j) {
          a[j] = ha && ok[j] ? *reinterpret_cast<const f32x4*>(src[j] + da) : z;
          b[j] = hb && ok[j] ? *reinterpret_cast<const f32x4*>(src[j] + db) : z;
        }
#pragma unroll
        for (int j = 0; j < IX_TPW; ++j) {
          const int u = t + j * nw;
          if (u >= ntok) break;
          float* o = out + (size_t)u * dim;
          if (ha) *reinterpret_cast<f32x4*>(o + da) = a[j];
          if (hb) *reinterpret_cast<f32x4*>(o + db) = b[j];
        }
      }
    } else {
      for (int d = lane; d < dim; d += 64) {
        float a[IX_TPW];
#pragma unroll
        for (int j = 0; j < IX_TPW; ++j) a[j] = ok[j] ? src[j][d] : 0.f;
#pragma unroll
        for (int j = 0; j < IX_TPW; ++j) {
          const int u = t + j * nw;
          if (u < ntok) out[(size_t)u * dim + d] = a[j];
        }
      }
    }
  }
}

template <bool VEC>
__global__ __launch_bounds__(IX_NT) void gather_index_kernel(float* __restrict__ out, const float* __restrict__ table,
                                                             const int32_t* __restrict__ keys, int clen, int max_clen,
                                                             int ntok, int dim, int vocab, int nix,
                                                             int4* __restrict__ rinfo, int32_t* __restrict__ list) {
  __shared__ IndexLds L;
  // the index workgroups first, so that their latency-bound chain starts at
  // once (measured: the other order is 1.9 us slower at 8192 x 512)
  if ((int)blockIdx.x < nix)
    build_index(L, keys, clen, max_clen, ntok, vocab, blockIdx.x, rinfo, list);
  else
    gather_rows<VEC>(out, table, keys, clen, max_clen, ntok, dim, vocab, blockIdx.x - nix, gridDim.x - nix);
}

// The embedding gradient from the index: one wave per table row sums the
// row's gradient rows in token order, restarting the sum at every IX_CHUNK
// boundary (v = v + sum of the chunk), which is exactly the range scatter's
// arithmetic; so the bits equal mle_embed_grad's.  assign: v starts at 0 and
// rows without tokens are written 0.
template <bool VEC>
__global__ __launch_bounds__(256) void index_grad_kernel(float* __restrict__ dtable, const float* __restrict__ grad,
                                                         const int4* __restrict__ rinfo,
                                                         const int32_t* __restrict__ list, int ntok, int dim,
                                                         int vocab, int assign) {
  const int lane = threadIdx.x & 63;
  const int v = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (v >= vocab) return;
  const int4 ri = rinfo[v];
  // An index built by the gather has 0 <= start, start + count <= ntok and
  // token ids in [0, ntok).  Anything else reads as an empty row or a zero
  // term, never as an access outside the list or the gradient.
  const int cnt = ri.x >= 0 && ri.y >= 0 && (long long)ri.x + ri.y <= ntok ? ri.y : 0;
  if (cnt == 0 && !assign) return;
  float* row = dtable + (size_t)v * dim;
  auto tok = [&](int j) { return j == 0 ? ri.z : j == 1 ? ri.w : list[ri.x + j]; };
  auto ok = [&](int t) { return (unsigned)t < (unsigned)ntok; };
  const bool one = ntok <= IX_CHUNK;
  if (VEC) {
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    for (int d0 = 0; d0 < dim; d0 += 512) {
      const int da = d0 + 4 * lane, db = da + 256;
      const bool ha = da < dim, hb = db < dim;
      f32x4 va = assign || !ha ? z : *reinterpret_cast<const f32x4*>(row + da);
      f32x4 vb = assign || !hb ? z : *reinterpret_cast<const f32x4*>(row + db);
      f32x4 aa = z, ab = z;
      int j = 0;
      if (one) {
        // two tokens' loads in flight before either is added
        for (; j + 1 < cnt; j += 2) {
          const int t0 = tok(j), t1 = tok(j + 1);
          const bool k0 = ok(t0), k1 = ok(t1);
          const float* g0 = grad + (size_t)(k0 ? t0 : 0) * dim;
          const float* g1 = grad + (size_t)(k1 ? t1 : 0) * dim;
          const f32x4 x0 = ha && k0 ? *reinterpret_cast<const f32x4*>(g0 + da) : z;
          const f32x4 y0 = hb && k0 ? *reinterpret_cast<const f32x4*>(g0 + db) : z;
          const f32x4 x1 = ha && k1 ? *reinterpret_cast<const f32x4*>(g1 + da) : z;
          const f32x4 y1 = hb && k1 ? *reinterpret_cast<const f32x4*>(g1 + db) : z;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            aa[c] += x0[c];
            ab[c] += y0[c];
            aa[c] += x1[c];
            ab[c] += y1[c];
          }
        }
      }
      int chunk = cnt > 0 ? tok(j) / IX_CHUNK : 0;
      for (; j < cnt; ++j) {
        const int t = tok(j);
        if (t / IX_CHUNK != chunk) {
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            va[c] += aa[c];
            vb[c] += ab[c];
          }
          aa = z;
          ab = z;
          chunk = t / IX_CHUNK;
        }
        const bool k0 = ok(t);
        const float* g0 = grad + (size_t)(k0 ? t : 0) * dim;
        const f32x4 x0 = ha && k0 ? *reinterpret_cast<const f32x4*>(g0 + da) : z;
        const f32x4 y0 = hb && k0 ? *reinterpret_cast<const f32x4*>(g0 + db) : z;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          aa[c] += x0[c];
          ab[c] += y0[c];
        }
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        va[c] += aa[c];
        vb[c] += ab[c];
      }
      if (ha) *reinterpret_cast<f32x4*>(row + da) = va;
      if (hb) *reinterpret_cast<f32x4*>(row + db) = vb;
    }
  } else {
    for (int d = lane; d < dim; d += 64) {
      float val = assign ? 0.f : row[d], acc = 0.f;
      int chunk = cnt > 0 ? tok(0) / IX_CHUNK : 0;
      for (int j = 0; j < cnt; ++j) {
        const int t = tok(j);
        if (t / IX_CHUNK != chunk) {
          val += acc;
          acc = 0.f;
          chunk = t / IX_CHUNK;
        }
        acc += ok(t) ? grad[(size_t)t * dim + d] : 0.f;
      }
      row[d] = val + acc;
    }
  }
}

// One wave per sorted position; the head of each run of equal keys sums the
// run's gradient rows in token order and adds scale * sum to the table row.
// Lanes cover the row in float4s when rows are 16-byte aligned.
__global__ __launch_bounds__(256) void segment_add_kernel(float* __restrict__ table, const float* __restrict__ grad,
                                                          const unsigned long long* __restrict__ sorted, int count,
                                                          int dim, float scale, int vec) {
  const int lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= count) return;
  const unsigned key = (unsigned)(sorted[i] >> 32);
  if (key == 0x7fffffffu) return;
  if (i > 0 && (unsigned)(sorted[i - 1] >> 32) == key) return;
  int end = i + 1;
  while (end < count && (unsigned)(sorted[end] >> 32) == key) ++end;
  float* row = table + (size_t)key * dim;
  if (vec) {
    for (int d = 4 * lane; d < dim; d += 256) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int j = i; j < end; ++j) {
        const size_t tok = (size_t)(unsigned)(sorted[j] & 0xffffffffu);
        const f32x4 g = *reinterpret_cast<const f32x4*>(grad + tok * dim + d);
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] += g[c];
      }
      f32x4 r = *reinterpret_cast<const f32x4*>(row + d);
#pragma unroll
      for (int c = 0; c < 4; ++c) r[c] += scale * acc[c];
      *reinterpret_cast<f32x4*>(row + d) = r;
    }
  } else {
    for (int d = lane; d < dim; d += 64) {
      float acc = 0.f;
      for (int j = i; j < end; ++j) acc += grad[(size_t)(unsigned)(sorted[j] & 0xffffffffu) * dim + d];
      row[d] += scale * acc;
    }
  }
}

// Row-centric scatter-add: each wave owns R consecutive table rows and scans
// every token's key (a chunk at a time, staged in LDS), summing the matching
// gradient rows in token order.  No sort and no atomics; used when
// vocab * tokens is moderate.  Lane l holds dims l + 64 j of each of its rows.
constexpr int ROW_CHUNK = 2048;
template <int DMAX, int R>
__global__ __launch_bounds__(256) void row_scatter_kernel(float* __restrict__ table, const float* __restrict__ grad,
                                                          const int32_t* __restrict__ keys, int clen, int max_clen,
                                                          int ntok, int dim, int vocab, float scale) {
  __shared__ int sk[ROW_CHUNK];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int v0 = (blockIdx.x * 4 + wave) * R;  // this wave's rows v0 .. v0 + R - 1
  float acc[R][DMAX];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < DMAX; ++j) acc[r][j] = 0.f;
  unsigned hit = 0;
  for (int t0 = 0; t0 < ntok; t0 += ROW_CHUNK) {
    const int cnt = min(ROW_CHUNK, ntok - t0);
    __syncthreads();
    if (clen == max_clen) {  // dense ids: token t at keys[t]
      for (int i = threadIdx.x; i < cnt; i += 256) sk[i] = keys[t0 + i];
    } else {
      for (int i = threadIdx.x; i < cnt; i += 256) {
        const int t = t0 + i;
        sk[i] = keys[(size_t)(t / clen) * max_clen + (t % clen)];
      }
    }
    __syncthreads();
    if (v0 >= vocab) continue;
    for (int c = 0; c < cnt; c += 64) {
      const int i = c + lane;
      const unsigned rel = (i < cnt) ? (unsigned)(sk[i] - v0) : 0xffffffffu;
      unsigned long long mask = __ballot(rel < (unsigned)R);
      while (mask) {  // tokens in order; the row is uniform across the wave
        const int bit = __ffsll((long long)mask) - 1;
        mask &= mask - 1;
        const int row = __shfl(sk[c + bit] - v0, 0, 64);
        const float* gr = grad + (size_t)(t0 + c + bit) * dim;
        hit |= 1u << row;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (r != row) continue;
#pragma unroll
          for (int j = 0; j < DMAX; ++j) {
            const int d = lane + 64 * j;
            if (d < dim) acc[r][j] += gr[d];
          }
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int v = v0 + r;
    if (v >= vocab || !(hit & (1u << r))) continue;
    float* tr = table + (size_t)v * dim;
#pragma unroll
    for (int j = 0; j < DMAX; ++j) {
      const int d = lane + 64 * j;
      if (d < dim) tr[d] += scale * acc[r][j];
    }
  }
}

// Incremental one-hot: clear each token's previous position, set the new one,
// remember it.  Rows belong to tokens, so tokens never touch the same element.
__global__ __launch_bounds__(256) void onehot_update_kernel(float* __restrict__ out, int32_t* __restrict__ prev,
                                                            const int32_t* __restrict__ keys, int clen, int max_clen,
                                                            int vocab, size_t total) {
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t g = (size_t)blockIdx.x * 256 + threadIdx.x; g < total; g += stride) {
    const int old = prev[g];
    if (old >= 0 && old < vocab) out[g * vocab + old] = 0.0f;
    const int key = keys[(g / clen) * max_clen + (g % clen)];
    const bool ok = !(key == INT_MIN || key < 0 || key >= vocab);
    if (ok) out[g * vocab + key] = 1.0f;
    prev[g] = ok ? key : -1;
  }
}

// out[c] (+)= sum_r x[r, c]: 64 columns per block, 16 row lanes, fixed order.
__global__ __launch_bounds__(1024) void colsum_kernel(const float* __restrict__ x, size_t rows, int cols,
                                                      float* __restrict__ out, float beta) {
  __shared__ float red[16][64];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + tx;
  float acc = 0.f;
  if (c < cols)
    for (size_t r = ty; r < rows; r += 16) acc += x[r * cols + c];
  red[ty][tx] = acc;
  __syncthreads();
  if (ty == 0 && c < cols) {
    float t = 0.f;
    for (int k = 0; k < 16; ++k) t += red[k][tx];
    out[c] = (beta != 0.f ? beta * out[c] : 0.f) + t;
  }
}

// out[c] += sum over (batch, hw) of x[b, c, :]; one 1024-thread block per
// channel.  The vector path keeps four 16-byte loads in flight per lane; the
// per-lane partials and the block reduction have a fixed order.
constexpr int CS_NT = 1024;
template <bool VEC>
__global__ __launch_bounds__(CS_NT) void channel_sum_kernel(const float* __restrict__ x, int batch, int channels,
                                                            size_t hw, float* __restrict__ out, int nreduce,
                                                            size_t out_total, int accumulate) {
  __shared__ float red[CS_NT / 64];
  const int c = blockIdx.x;
  if (c >= nreduce) {  // assign mode: the rest of `out` becomes 0
    for (size_t j = nreduce + (size_t)(c - nreduce) * CS_NT + threadIdx.x; j < out_total;
         j += (size_t)(gridDim.x - nreduce) * CS_NT)
      out[j] = 0.f;
    return;
  }
  // acc[u] takes batch items u, u + 4, ...: four loads in flight per thread.
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  const size_t cstride = (size_t)channels * hw;
  const float* base = x + (size_t)c * hw;
  int b = 0;
  if (VEC) {
    const size_t n4 = hw / 4;
    for (; b + 4 <= batch; b += 4)
      for (size_t i = threadIdx.x; i < n4; i += CS_NT) {
        f32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = reinterpret_cast<const f32x4*>(base + (size_t)(b + u) * cstride)[i];
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[u] += (v[u][0] + v[u][1]) + (v[u][2] + v[u][3]);
      }
    for (; b < batch; ++b)
      for (size_t i = threadIdx.x; i < n4; i += CS_NT) {
        const f32x4 v = reinterpret_cast<const f32x4*>(base + (size_t)b * cstride)[i];
        acc[b & 3] += (v[0] + v[1]) + (v[2] + v[3]);
      }
  } else {
    for (; b < batch; ++b)
      for (size_t i = threadIdx.x; i < hw; i += CS_NT) acc[b & 3] += base[(size_t)b * cstride + i];
  }
  const float t = block_sum<CS_NT>((acc[0] + acc[1]) + (acc[2] + acc[3]), red);
  if (threadIdx.x == 0) out[c] = accumulate ? out[c] + t : t;
}

// table (+)= scale * scatter(grad); assign: the table is logically zero (rows
// no token reaches become 0).
int embed_scatter(mle_stream stream, float* table, const float* grad, const int32_t* keys, int batch, int clen,
                  int max_clen, int dim, int vocab, float scale, int assign, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(table && grad && keys && ws && clen > 0 && max_clen >= clen && dim > 0 && vocab > 0,
                "mle_embed_scatter_add: bad argument");
  const long long ntok = (long long)batch * clen;
  MLE_CHECK_ARG(ntok < 2147483647LL, "mle_embed_scatter_add: too many tokens");
  const bool in_kernel = ntok > 0 && vocab <= RS_VMAX;  // the range kernel assigns by itself
  if (assign && !in_kernel) {
    const int rc = mle_fill(stream, table, 0.0f, (size_t)vocab * dim);
    if (rc != MLE_OK) return rc;
  }
  if (ntok == 0) return MLE_OK;
  if (ws_bytes < mle_embed_scatter_ws_bytes(batch, clen))
    return set_error(MLE_ERR_WORKSPACE, "mle_embed_scatter_add: workspace too small");
  hipStream_t s = as_stream(stream);
  unsigned long long* sorted = static_cast<unsigned long long*>(ws);
  const int vec = (dim % 4 == 0 && aligned16(table) && aligned16(grad)) ? 1 : 0;
  if (vocab <= RS_VMAX) {
    const int rows = (vocab + 511) / 512;  // <= RS_RMAX / 2: about one row per wave, at most 512 workgroups
    const unsigned grid = (unsigned)((vocab + rows - 1) / rows);
    if (vec)
      range_scatter_kernel<true><<<grid, RS_NT, 0, s>>>(table, grad, keys, clen, max_clen, (int)ntok, dim, vocab, rows,
                                                        scale, assign);
    else
      range_scatter_kernel<false><<<grid, RS_NT, 0, s>>>(table, grad, keys, clen, max_clen, (int)ntok, dim, vocab,
                                                         rows, scale, assign);
    return check_launch("mle_embed_scatter_add");
  }
  if ((double)vocab * (double)ntok <= (double)(1u << 30) && dim <= 1024) {
    // One row per wave (measured on MI355X: 2, 4 or 8 rows per wave, or 8-16
    // waves per workgroup, are equal or slower -- the key scan bounds it).
    if (dim <= 512)
      row_scatter_kernel<8, 1><<<(vocab + 3) / 4, 256, 0, s>>>(table, grad, keys, clen, max_clen, (int)ntok, dim, vocab,
                                                               scale);
    else
      row_scatter_kernel<16, 1><<<(vocab + 3) / 4, 256, 0, s>>>(table, grad, keys, clen, max_clen, (int)ntok, dim,
                                                                vocab, scale);
    return check_launch("mle_embed_scatter_add");
  }
  // Chunks of SORT_CAP tokens are applied in token order, so every table row
  // receives its updates in a fixed order.
  for (long long t0 = 0; t0 < ntok; t0 += SORT_CAP) {
    const int count = (int)((ntok - t0 < SORT_CAP) ? ntok - t0 : SORT_CAP);
    sort_chunk_kernel<<<1, SORT_NT, 0, s>>>(keys, clen, max_clen, vocab, (int)t0, count, sorted);
    segment_add_kernel<<<(count + 3) / 4, 256, 0, s>>>(table, grad, sorted, count, dim, scale, vec);
    int rc = check_launch("mle_embed_scatter_add");
    if (rc) return rc;
  }
  return MLE_OK;
}

}  // namespace

extern "C" {

int mle_embed_gather(mle_stream stream, float* out, const float* table, const int32_t* keys, int batch, int clen,
                     int max_clen, int dim) {
  MLE_CHECK_ARG(out && table && keys && clen > 0 && max_clen >= clen && dim > 0, "mle_embed_gather: bad argument");
  const size_t total = (size_t)batch * clen * dim;
  if (total == 0) return MLE_OK;
  hipStream_t s = as_stream(stream);
  if (dim % 4 == 0 && aligned16(out) && aligned16(table))
    gather4_kernel<<<stream_grid(total / 4, NT, 8192), NT, 0, s>>>(out, table, keys, clen, max_clen, dim, total / 4);
  else
    gather_kernel<<<stream_grid(total, NT, 8192), NT, 0, s>>>(out, table, keys, clen, max_clen, dim, total);
  return check_launch("mle_embed_gather");
}

size_t mle_embed_scatter_ws_bytes(int batch, int clen) {
  size_t n = (size_t)batch * clen;
  if (n > (size_t)SORT_CAP) n = SORT_CAP;
  return (n < 32 ? 32 : n) * sizeof(unsigned long long);
}

int mle_embed_scatter_add(mle_stream stream, float* table, const float* grad, const int32_t* keys, int batch, int clen,
                          int max_clen, int dim, int vocab, float scale, void* ws, size_t ws_bytes) {
  return embed_scatter(stream, table, grad, keys, batch, clen, max_clen, dim, vocab, scale, 0, ws, ws_bytes);
}

int mle_embed_grad(mle_stream stream, float* dtable, const float* grad, const int32_t* keys, int batch, int clen,
                   int max_clen, int dim, int vocab, int accumulate, void* ws, size_t ws_bytes) {
  return embed_scatter(stream, dtable, grad, keys, batch, clen, max_clen, dim, vocab, 1.0f, accumulate ? 0 : 1, ws,
                       ws_bytes);
}

size_t mle_embed_index_bytes(int batch, int clen, int vocab) {
  if (vocab <= 0 || vocab > IX_VMAX || batch < 0 || clen <= 0) return 0;
  const size_t ntok = (size_t)batch * clen;
  const size_t bytes = (size_t)vocab * sizeof(int4) + (ntok > 0 ? ntok : 1) * sizeof(int32_t);
  return (bytes + 255) & ~(size_t)255;
}

int mle_embed_gather_indexed(mle_stream stream, float* out, const float* table, const int32_t* keys, int batch,
                             int clen, int max_clen, int dim, int vocab, void* index, size_t index_bytes) {
  MLE_CHECK_ARG(out && table && keys && index && batch >= 0 && clen > 0 && max_clen >= clen && dim > 0 && vocab > 0,
                "mle_embed_gather_indexed: bad argument");
  MLE_CHECK_ARG(vocab <= IX_VMAX, "mle_embed_gather_indexed: vocabulary above 16384 rows");
  const long long ntok = (long long)batch * clen;
  MLE_CHECK_ARG(ntok < 2147483647LL, "mle_embed_gather_indexed: too many tokens");
  MLE_CHECK_ARG(aligned16(index), "mle_embed_gather_indexed: index not 16-byte aligned");
  if (index_bytes < mle_embed_index_bytes(batch, clen, vocab))
    return set_error(MLE_ERR_WORKSPACE, "mle_embed_gather_indexed: index buffer too small");
  hipStream_t s = as_stream(stream);
  int4* rinfo = static_cast<int4*>(index);
  int32_t* list = reinterpret_cast<int32_t*>(rinfo + vocab);
  const int nix = (vocab + IX_R - 1) / IX_R;
  // 16 IX_TPW tokens per gather workgroup per pass
  constexpr int per_wg = (IX_NT / 64) * IX_TPW;
  const long long ng = ntok == 0 ? 0 : std::min<long long>((ntok + per_wg - 1) / per_wg, 2048);
  const unsigned grid = (unsigned)(nix + ng);
  if (dim % 4 == 0 && aligned16(out) && aligned16(table))
    gather_index_kernel<true><<<grid, IX_NT, 0, s>>>(out, table, keys, clen, max_clen, (int)ntok, dim, vocab, nix,
                                                     rinfo, list);
  else
    gather_index_kernel<false><<<grid, IX_NT, 0, s>>>(out, table, keys, clen, max_clen, (int)ntok, dim, vocab, nix,
                                                      rinfo, list);
  return check_launch("mle_embed_gather_indexed");
}

int mle_embed_grad_indexed(mle_stream stream, float* dtable, const float* grad, const void* index, int batch, int clen,
                           int dim, int vocab, int accumulate) {
  MLE_CHECK_ARG(dtable && grad && index && batch >= 0 && clen > 0 && dim > 0 && vocab > 0,
                "mle_embed_grad_indexed: bad argument");
  MLE_CHECK_ARG(vocab <= IX_VMAX, "mle_embed_grad_indexed: vocabulary above 16384 rows");
  const long long ntok = (long long)batch * clen;
  MLE_CHECK_ARG(ntok < 2147483647LL, "mle_embed_grad_indexed: too many tokens");
  MLE_CHECK_ARG(aligned16(index), "mle_embed_grad_indexed: index not 16-byte aligned");
  hipStream_t s = as_stream(stream);
  const int4* rinfo = static_cast<const int4*>(index);
  const int32_t* list = reinterpret_cast<const int32_t*>(rinfo + vocab);
  const unsigned grid = (unsigned)((vocab + 3) / 4);
  const int assign = accumulate ? 0 : 1;
  if (dim % 4 == 0 && aligned16(dtable) && aligned16(grad))
    index_grad_kernel<true><<<grid, 256, 0, s>>>(dtable, grad, rinfo, list, (int)ntok, dim, vocab, assign);
  else
    index_grad_kernel<false><<<grid, 256, 0, s>>>(dtable, grad, rinfo, list, (int)ntok, dim, vocab, assign);
  return check_launch("mle_embed_grad_indexed");
}


int mle_onehot(mle_stream stream, float* out, const int32_t* keys, int batch, int clen, int max_clen, int vocab) {
  MLE_CHECK_ARG(out && keys && clen > 0 && max_clen >= clen && vocab > 0, "mle_onehot: bad argument");
  const size_t total = (size_t)batch * clen;
  if (total == 0) return MLE_OK;
  onehot_kernel<<<stream_grid(total, NT, 8192), NT, 0, as_stream(stream)>>>(out, keys, clen, max_clen, vocab, total);
  return check_launch("mle_onehot");
}

int mle_onehot_update(mle_stream stream, float* out, int32_t* prev_keys, const int32_t* keys, int batch, int clen,
                      int max_clen, int vocab) {
  MLE_CHECK_ARG(out && prev_keys && keys && clen > 0 && max_clen >= clen && vocab > 0, "mle_onehot_update: bad argument");
  const size_t total = (size_t)batch * clen;
  if (total == 0) return MLE_OK;
  onehot_update_kernel<<<stream_grid(total, NT, 8192), NT, 0, as_stream(stream)>>>(out, prev_keys, keys, clen, max_clen,
                                                                                   vocab, total);
  return check_launch("mle_onehot_update");
}

int mle_argmax(mle_stream stream, const float* x, int rows, int cols, int32_t* out) {
  MLE_CHECK_ARG(x && out && rows >= 0 && cols > 0, "mle_argmax: bad argument");
  if (rows == 0) return MLE_OK;
  argmax_kernel<<<rows, 64, 0, as_stream(stream)>>>(x, cols, out);
  return check_launch("mle_argmax");
}

int mle_colsum(mle_stream stream, const float* x, size_t rows, int cols, float* out, float beta) {
  MLE_CHECK_ARG(x && out && cols > 0, "mle_colsum: bad argument");
  colsum_kernel<<<(cols + 63) / 64, 1024, 0, as_stream(stream)>>>(x, rows, cols, out, beta);
  return check_launch("mle_colsum");
}

int mle_channel_sum(mle_stream stream, const float* x, int batch, int channels, size_t hw, int nreduce, float* out) {
  return mle_channel_sum_ex(stream, x, batch, channels, hw, nreduce, out, 0, 1);
}

int mle_channel_sum_ex(mle_stream stream, const float* x, int batch, int channels, size_t hw, int nreduce, float* out,
                       size_t out_total, int accumulate) {
  MLE_CHECK_ARG(x && out && channels > 0 && nreduce >= 0, "mle_channel_sum: bad argument");
  if (nreduce > channels) nreduce = channels;  // the reference would read and write out of bounds here
  MLE_CHECK_ARG(accumulate || out_total >= (size_t)nreduce, "mle_channel_sum_ex: out_total %zu < %d channels",
                out_total, nreduce);
  const size_t rest = accumulate ? 0 : out_total - (size_t)nreduce;
  const unsigned zb = (unsigned)std::min<size_t>((rest + CS_NT - 1) / CS_NT, 1024);
  const unsigned grid = (unsigned)nreduce + zb;
  if (grid == 0) return MLE_OK;
  if (hw % 4 == 0 && aligned16(x))
    channel_sum_kernel<true><<<grid, CS_NT, 0, as_stream(stream)>>>(x, batch, channels, hw, out, nreduce, out_total,
                                                                    accumulate);
  else
    channel_sum_kernel<false><<<grid, CS_NT, 0, as_stream(stream)>>>(x, batch, channels, hw, out, nreduce, out_total,
                                                                     accumulate);
  return check_launch("mle_channel_sum");
}

}  // extern "C"
