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
    unsigned rel[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int i = tid + k * RS_NT, t = t0 + i;
      rel[k] = 0xffffffffu;
      if (i < count) {
        const size_t at = clen == max_clen ? (size_t)t : (size_t)(t / clen) * max_clen + t % clen;
        rel[k] = (unsigned)(keys[at] - v_lo);
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (rel[k] < (unsigned)nrows) atomicAdd(&sbin[rel[k]], 1);
    __syncthreads();
    if (wid == 0) {
      const int c = lane < nrows ? sbin[lane] : 0;
      int incl = c;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(incl, off, 64);
        if (lane >= off) incl += y;
      }
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
        for (int d = 4 * lane; d < dim; d += 256) {
          // in flight with the gradient loads
          f32x4 v = first ? f32x4{0.f, 0.f, 0.f, 0.f} : *reinterpret_cast<const f32x4*>(row + d);
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
          for (int j = b; j < e; ++j) {
            const f32x4 g = *reinterpret_cast<const f32x4*>(grad + (size_t)(t0 + slist[j]) * dim + d);
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[c] += g[c];
          }
#pragma unroll
          for (int c = 0; c < 4; ++c) v[c] += scale * acc[c];
          *reinterpret_cast<f32x4*>(row + d) = v;
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
