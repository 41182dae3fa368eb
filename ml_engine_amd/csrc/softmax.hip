// Softmax (row / column, optional causal mask), its backward, and the
// softmax-cross-entropy and MSE losses.  One pass over HBM per direction: a
// line (row or column) is held in registers while its max and sum are reduced
// with wave64 shuffles, instead of the reference's 4 launches with one thread
// per line (SoftMax/SoftMask/deriv_softmax, Engine/kernels.cu:2003-2244).
#include "activation.hpp"
#include "common.hpp"

#include <algorithm>
#include <float.h>

using namespace mle;

namespace {

constexpr int NT = 256;
constexpr int ROW_CPT = 32;  // row kernels cache up to NT*ROW_CPT = 8192 columns
constexpr int COL_W = 64;    // column kernels: 64 columns per workgroup
constexpr int COL_RL = 4;    // ... and 4 row lanes
constexpr int COL_RPT = 64;  // ... caching up to COL_RL*COL_RPT = 256 rows

// Cross-entropy target given as token ids (the one-hot matrix OneHotEmbeddings
// would build, Engine/kernels.cu:1551-1560): row r = b*clen + s has its single
// 1 at column keys[b*max_clen + s] when that id is in [0, cols), else no 1.
// With it the row kernels store each row's (max, sum) in stats instead of the
// probabilities, and the backward recomputes p from them.
struct KeyTargets {
  const int32_t* keys;  // nullptr: dense target (or none)
  int clen, max_clen;
  float* stats;         // [rows][2] = (max, sum)
  __device__ int key(size_t line, int cols) const {
    const int k = keys[(line / clen) * max_clen + (line % clen)];
    return (k >= 0 && k < cols) ? k : -1;
  }
};

// ---------------------------------------------------------------------------
// Row softmax (type 0).  One workgroup per line of `cols` elements.  With
// `target` set, also writes this row's -sum(t log(p + 1e-27)) (double) to
// loss_part[row] (scalar_ce_kernel, Engine/kernels.cu:1818-1826).  With key
// targets the term of the one column whose t is 1 is the row's sum (the other
// terms are zeros), and y may be null.
template <bool CACHED>
__global__ __launch_bounds__(NT) void softmax_row_kernel(const float* __restrict__ x, float* __restrict__ y, int rows,
                                                         int cols, int causal, const float* __restrict__ target,
                                                         double* __restrict__ loss_part, KeyTargets kt) {
  __shared__ float redf[NT / 64];
  __shared__ double redd[NT / 64];
  const size_t line = blockIdx.x;
  const int r_in = (int)(line % rows);
  const float* xr = x + line * cols;
  float* yr = y ? y + line * cols : nullptr;
  const int lim = causal ? min(cols, r_in + 1) : cols;  // entries c > r are masked
  const int key = kt.keys ? kt.key(line, cols) : -1;
  float v[CACHED ? ROW_CPT : 1];
  float mx = -FLT_MAX;
  if (CACHED) {
#pragma unroll
    for (int i = 0; i < ROW_CPT; ++i) {
      const int c = threadIdx.x + i * NT;
      v[i] = (c < cols) ? xr[c] : -FLT_MAX;
      mx = fmaxf(mx, v[i]);
    }
  } else {
    for (int c = threadIdx.x; c < cols; c += NT) mx = fmaxf(mx, xr[c]);
  }
  mx = block_max<NT>(mx, redf);
  float sum = 0.f;
  if (CACHED) {
#pragma unroll
    for (int i = 0; i < ROW_CPT; ++i) {
      const int c = threadIdx.x + i * NT;
      v[i] = (c < lim) ? expf(v[i] - mx) : 0.f;
      sum += v[i];
    }
  } else {
    for (int c = threadIdx.x; c < lim; c += NT) sum += expf(xr[c] - mx);
  }
  sum = block_sum<NT>(sum, redf);
  if (sum < 1e-45f) sum = 1.0f;
  double lp = 0.0;
  if (CACHED) {
#pragma unroll
    for (int i = 0; i < ROW_CPT; ++i) {
      const int c = threadIdx.x + i * NT;
      if (c < cols) {
        const float p = v[i] / sum;
        if (yr) yr[c] = p;
        if (target) lp += -(double)target[line * cols + c] * log((double)p + 1e-27);
        if (c == key) lp = -log((double)p + 1e-27);
      }
    }
  } else {
    for (int c = threadIdx.x; c < cols; c += NT) {
      const float p = (c < lim) ? expf(xr[c] - mx) / sum : 0.f;
      if (yr) yr[c] = p;
      if (target) lp += -(double)target[line * cols + c] * log((double)p + 1e-27);
      if (c == key) lp = -log((double)p + 1e-27);
    }
  }
  if (target || kt.keys) {
    lp = block_sum<NT>(lp, redd);
    if (threadIdx.x == 0) loss_part[line] = lp;
  }
  if (kt.stats && threadIdx.x == 0) {
    kt.stats[2 * line] = mx;
    kt.stats[2 * line + 1] = sum;
  }
}

// Row softmax with float4 accesses (cols % 4 == 0, cols <= 4*NT*RV4).
constexpr int RV4 = 8;
__device__ __forceinline__ f32x4 ldv(const float* p, size_t i) { return *reinterpret_cast<const f32x4*>(p + i); }
__device__ __forceinline__ void stv(float* p, size_t i, f32x4 v) { *reinterpret_cast<f32x4*>(p + i) = v; }

__global__ __launch_bounds__(NT) void softmax_row4_kernel(const float* __restrict__ x, float* __restrict__ y, int rows,
                                                          int cols, int causal, const float* __restrict__ target,
                                                          double* __restrict__ loss_part, KeyTargets kt) {
  __shared__ float redf[NT / 64];
  __shared__ double redd[NT / 64];
  const size_t line = blockIdx.x;
  const int r_in = (int)(line % rows);
  const size_t base = line * cols;
  const int lim = causal ? min(cols, r_in + 1) : cols;
  const int key = kt.keys ? kt.key(line, cols) : -1;
  f32x4 v[RV4];
  float mx = -FLT_MAX;
#pragma unroll
  for (int i = 0; i < RV4; ++i) {
    const int c = (threadIdx.x + i * NT) * 4;
    v[i] = (c < cols) ? ldv(x, base + c) : f32x4{-FLT_MAX, -FLT_MAX, -FLT_MAX, -FLT_MAX};
#pragma unroll
    for (int j = 0; j < 4; ++j) mx = fmaxf(mx, v[i][j]);
  }
  mx = block_max<NT>(mx, redf);
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < RV4; ++i) {
    const int c = (threadIdx.x + i * NT) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[i][j] = (c + j < lim) ? expf(v[i][j] - mx) : 0.f;
      sum += v[i][j];
    }
  }
  sum = block_sum<NT>(sum, redf);
  if (sum < 1e-45f) sum = 1.0f;
  double lp = 0.0;
#pragma unroll
  for (int i = 0; i < RV4; ++i) {
    const int c = (threadIdx.x + i * NT) * 4;
    if (c < cols) {
      f32x4 p;
#pragma unroll
      for (int j = 0; j < 4; ++j) p[j] = v[i][j] / sum;
      if (y) stv(y, base + c, p);
      if (target) {
        const f32x4 t = ldv(target, base + c);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (t[j] != 0.f) lp += -(double)t[j] * log((double)p[j] + 1e-27);
      }
      if (key >= c && key < c + 4) lp = -log((double)p[key - c] + 1e-27);
    }
  }
  if (target || kt.keys) {
    lp = block_sum<NT>(lp, redd);
    if (threadIdx.x == 0) loss_part[line] = lp;
  }
  if (kt.stats && threadIdx.x == 0) {
    kt.stats[2 * line] = mx;
    kt.stats[2 * line + 1] = sum;
  }
}

// Cross-entropy against key targets from row statistics a GEMM epilogue
// produced (mle_gemm_rowstats): per row, the nblk (max, sum of exp) pairs of
// its 64-column blocks combine into the row's max M and sum S (the same
// quantities softmax_row4_kernel reduces from the logits), then the key's
// probability expf(x_key - M) / S gives the row's loss term.  One wave per row;
// only the key's logit is read.
__global__ __launch_bounds__(256) void xent_keys_partials_kernel(const float* __restrict__ x,
                                                                 const float* __restrict__ part, int64_t ldp, int nblk,
                                                                 int rows, int cols, KeyTargets kt,
                                                                 double* __restrict__ loss_part) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  // The key and its logit are fetched first: their two dependent loads run
  // under the partials' loads and reductions instead of after them.
  int key = -1;
  float xk = 0.f;
  if (lane == 0) {
    key = kt.key((size_t)row, cols);
    if (key >= 0) xk = x[(size_t)row * cols + key];
  }
  const float* pr = part + (size_t)row * ldp;
  float mx = -FLT_MAX, sum = 0.f;
  if (nblk <= 4 * 64) {
    // Up to four (max, sum) pairs per lane, each one 8-byte load, held for
    // both passes (the pairs are 8-byte aligned: ldp is even).
    float2 pv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int b = lane + 64 * u;
      pv[u] = b < nblk ? *reinterpret_cast<const float2*>(pr + 2 * b) : float2{-FLT_MAX, 0.f};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) mx = fmaxf(mx, pv[u].x);
    mx = wave_max(mx);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (lane + 64 * u < nblk) sum += pv[u].y * expf(pv[u].x - mx);
  } else {
    for (int b = lane; b < nblk; b += 64) mx = fmaxf(mx, pr[2 * b]);
    mx = wave_max(mx);
    for (int b = lane; b < nblk; b += 64) sum += pr[2 * b + 1] * expf(pr[2 * b] - mx);
  }
  sum = wave_sum(sum);
  if (sum < 1e-45f) sum = 1.0f;
  if (lane == 0) {
    double lp = 0.0;
    if (key >= 0) lp = -log((double)(expf(xk - mx) / sum) + 1e-27);
    loss_part[row] = lp;
    kt.stats[2 * row] = mx;
    kt.stats[2 * row + 1] = sum;
  }
}

// Row softmax backward: dx (+)= y (dy - <dy, y>); acc = 0 assigns.
template <bool CACHED>
__global__ __launch_bounds__(NT) void softmax_row_bwd_kernel(const float* __restrict__ y, const float* __restrict__ dy,
                                                             float* __restrict__ dx, int cols, int acc) {
  __shared__ float redf[NT / 64];
  const size_t line = blockIdx.x;
  const float* yr = y + line * cols;
  const float* gr = dy + line * cols;
  float* dr = dx + line * cols;
  float yv[CACHED ? ROW_CPT : 1], gv[CACHED ? ROW_CPT : 1];
  float dot = 0.f;
  if (CACHED) {
#pragma unroll
    for (int i = 0; i < ROW_CPT; ++i) {
      const int c = threadIdx.x + i * NT;
      yv[i] = (c < cols) ? yr[c] : 0.f;
      gv[i] = (c < cols) ? gr[c] : 0.f;
      dot += gv[i] * yv[i];
    }
  } else {
    for (int c = threadIdx.x; c < cols; c += NT) dot += gr[c] * yr[c];
  }
  dot = block_sum<NT>(dot, redf);
  if (CACHED) {
#pragma unroll
    for (int i = 0; i < ROW_CPT; ++i) {
      const int c = threadIdx.x + i * NT;
      if (c < cols) dr[c] = (acc ? dr[c] : 0.f) + yv[i] * (gv[i] - dot);
    }
  } else {
    for (int c = threadIdx.x; c < cols; c += NT) dr[c] = (acc ? dr[c] : 0.f) + yr[c] * (gr[c] - dot);
  }
}

// ---------------------------------------------------------------------------
// Column softmax (type 1): for each column, max / exp / sum over the rows.  A
// workgroup owns COL_W consecutive columns of one matrix; a wave reads one
// row's COL_W columns (256 contiguous bytes) per step.
template <bool CACHED>
__global__ __launch_bounds__(NT) void softmax_col_kernel(const float* __restrict__ x, float* __restrict__ y, int rows,
                                                         int cols, int causal) {
  __shared__ float red[COL_RL][COL_W];
  const int tx = threadIdx.x % COL_W, ty = threadIdx.x / COL_W;
  const int c = blockIdx.x * COL_W + tx;
  const size_t base = (size_t)blockIdx.y * rows * cols;
  const bool cv = c < cols;
  float v[CACHED ? COL_RPT : 1];
  float mx = -FLT_MAX;
  if (CACHED) {
#pragma unroll
    for (int i = 0; i < COL_RPT; ++i) {
      const int r = ty + i * COL_RL;
      v[i] = (cv && r < rows) ? x[base + (size_t)r * cols + c] : -FLT_MAX;
      mx = fmaxf(mx, v[i]);
    }
  } else if (cv) {
    for (int r = ty; r < rows; r += COL_RL) mx = fmaxf(mx, x[base + (size_t)r * cols + c]);
  }
  red[ty][tx] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0][tx], red[1][tx]), fmaxf(red[2][tx], red[3][tx]));
  __syncthreads();
  float sum = 0.f;
  if (CACHED) {
#pragma unroll
    for (int i = 0; i < COL_RPT; ++i) {
      const int r = ty + i * COL_RL;
      const bool keep = cv && r < rows && !(causal && c > r);
      v[i] = keep ? expf(v[i] - mx) : 0.f;
      sum += v[i];
    }
  } else if (cv) {
    for (int r = ty; r < rows; r += COL_RL)
      if (!(causal && c > r)) sum += expf(x[base + (size_t)r * cols + c] - mx);
  }
  red[ty][tx] = sum;
  __syncthreads();
  sum = (red[0][tx] + red[1][tx]) + (red[2][tx] + red[3][tx]);
  if (sum < 1e-45f) sum = 1.0f;
  if (!cv) return;
  if (CACHED) {
#pragma unroll
    for (int i = 0; i < COL_RPT; ++i) {
      const int r = ty + i * COL_RL;
      if (r < rows) y[base + (size_t)r * cols + c] = v[i] / sum;
    }
  } else {
    for (int r = ty; r < rows; r += COL_RL) {
      const size_t o = base + (size_t)r * cols + c;
      y[o] = (causal && c > r) ? 0.f : expf(x[o] - mx) / sum;
    }
  }
}

template <bool CACHED>
__global__ __launch_bounds__(NT) void softmax_col_bwd_kernel(const float* __restrict__ y, const float* __restrict__ dy,
                                                             float* __restrict__ dx, int rows, int cols, int acc) {
  __shared__ float red[COL_RL][COL_W];
  const int tx = threadIdx.x % COL_W, ty = threadIdx.x / COL_W;
  const int c = blockIdx.x * COL_W + tx;
  const size_t base = (size_t)blockIdx.y * rows * cols;
  const bool cv = c < cols;
  float yv[CACHED ? COL_RPT : 1], gv[CACHED ? COL_RPT : 1];
  float dot = 0.f;
  if (CACHED) {
#pragma unroll
    for (int i = 0; i < COL_RPT; ++i) {
      const int r = ty + i * COL_RL;
      const bool ok = cv && r < rows;
      yv[i] = ok ? y[base + (size_t)r * cols + c] : 0.f;
      gv[i] = ok ? dy[base + (size_t)r * cols + c] : 0.f;
      dot += gv[i] * yv[i];
    }
  } else if (cv) {
    for (int r = ty; r < rows; r += COL_RL) {
      const size_t o = base + (size_t)r * cols + c;
      dot += dy[o] * y[o];
    }
  }
  red[ty][tx] = dot;
  __syncthreads();
  dot = (red[0][tx] + red[1][tx]) + (red[2][tx] + red[3][tx]);
  if (!cv) return;
  if (CACHED) {
#pragma unroll
    for (int i = 0; i < COL_RPT; ++i) {
      const int r = ty + i * COL_RL;
      if (r < rows) {
        const size_t o = base + (size_t)r * cols + c;
        dx[o] = (acc ? dx[o] : 0.f) + yv[i] * (gv[i] - dot);
      }
    }
  } else {
    for (int r = ty; r < rows; r += COL_RL) {
      const size_t o = base + (size_t)r * cols + c;
      dx[o] = (acc ? dx[o] : 0.f) + y[o] * (dy[o] - dot);
    }
  }
}

// ---------------------------------------------------------------------------
// Column softmax, float4 lanes: a workgroup owns 64 columns; lane (tx, ty) with
// tx < 16 covers columns 4tx..4tx+3 and rows ty, ty+16, ... (rows <= 16*C4_RPT).
constexpr int C4_RL = 16, C4_RPT = 16;

__global__ __launch_bounds__(NT) void softmax_col4_kernel(const float* __restrict__ x, float* __restrict__ y, int rows,
                                                          int cols, int causal) {
  __shared__ f32x4 red[C4_RL][16];
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  const int c0 = blockIdx.x * 64 + tx * 4;
  const size_t base = (size_t)blockIdx.y * rows * cols;
  const bool cv = c0 < cols;
  f32x4 v[C4_RPT];
  f32x4 mx = {-FLT_MAX, -FLT_MAX, -FLT_MAX, -FLT_MAX};
#pragma unroll
  for (int i = 0; i < C4_RPT; ++i) {
    const int r = ty + i * C4_RL;
    v[i] = (cv && r < rows) ? ldv(x, base + (size_t)r * cols + c0) : f32x4{-FLT_MAX, -FLT_MAX, -FLT_MAX, -FLT_MAX};
#pragma unroll
    for (int j = 0; j < 4; ++j) mx[j] = fmaxf(mx[j], v[i][j]);
  }
  red[ty][tx] = mx;
  __syncthreads();
  mx = red[0][tx];
#pragma unroll
  for (int k = 1; k < C4_RL; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) mx[j] = fmaxf(mx[j], red[k][tx][j]);
  __syncthreads();
  f32x4 sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < C4_RPT; ++i) {
    const int r = ty + i * C4_RL;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool keep = cv && r < rows && !(causal && c0 + j > r);
      v[i][j] = keep ? expf(v[i][j] - mx[j]) : 0.f;
      sum[j] += v[i][j];
    }
  }
  red[ty][tx] = sum;
  __syncthreads();
  sum = red[0][tx];
#pragma unroll
  for (int k = 1; k < C4_RL; ++k) sum += red[k][tx];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (sum[j] < 1e-45f) sum[j] = 1.0f;
  if (!cv) return;
#pragma unroll
  for (int i = 0; i < C4_RPT; ++i) {
    const int r = ty + i * C4_RL;
    if (r < rows) {
      f32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = v[i][j] / sum[j];
      stv(y, base + (size_t)r * cols + c0, o);
    }
  }
}

__global__ __launch_bounds__(NT) void softmax_col4_bwd_kernel(const float* __restrict__ y, const float* __restrict__ dy,
                                                              float* __restrict__ dx, int rows, int cols, int acc) {
  __shared__ f32x4 red[C4_RL][16];
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  const int c0 = blockIdx.x * 64 + tx * 4;
  const size_t base = (size_t)blockIdx.y * rows * cols;
  const bool cv = c0 < cols;
  f32x4 yv[C4_RPT], gv[C4_RPT];
  f32x4 dot = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < C4_RPT; ++i) {
    const int r = ty + i * C4_RL;
    const bool ok = cv && r < rows;
    yv[i] = ok ? ldv(y, base + (size_t)r * cols + c0) : f32x4{0.f, 0.f, 0.f, 0.f};
    gv[i] = ok ? ldv(dy, base + (size_t)r * cols + c0) : f32x4{0.f, 0.f, 0.f, 0.f};
    dot += gv[i] * yv[i];
  }
  red[ty][tx] = dot;
  __syncthreads();
  dot = red[0][tx];
#pragma unroll
  for (int k = 1; k < C4_RL; ++k) dot += red[k][tx];
  if (!cv) return;
#pragma unroll
  for (int i = 0; i < C4_RPT; ++i) {
    const int r = ty + i * C4_RL;
    if (r < rows) {
      const size_t o = base + (size_t)r * cols + c0;
      const f32x4 v = yv[i] * (gv[i] - dot);
      stv(dx, o, acc ? ldv(dx, o) + v : v);
    }
  }
}

// ---------------------------------------------------------------------------
// Deterministic sums into a scalar: per-block double partials, then one block
// adds them in a fixed order.
// With dx set, the same pass also writes the last loss node's gradient,
// dx = 2 (x - t) / n (assigned), as mse_bwd_kernel computes it.
__global__ __launch_bounds__(NT) void mse_partial_kernel(const float* __restrict__ x, const float* __restrict__ t,
                                                         size_t n, double* __restrict__ part,
                                                         float* __restrict__ dx = nullptr) {
  __shared__ double red[NT / 64];
  double acc = 0.0;
  const size_t stride = (size_t)gridDim.x * NT;
  const float fn = (float)n;
  for (size_t i = (size_t)blockIdx.x * NT + threadIdx.x; i < n; i += stride) {
    const float xi = x[i], ti = t[i];
    const double d = (double)ti - (double)xi;
    acc += d * d;
    if (dx) dx[i] = 2.0f * (xi - ti) / fn;
  }
  acc = block_sum<NT>(acc, red);
  if (threadIdx.x == 0) part[blockIdx.x] = acc;
}

// The same sum with 16-byte loads (n % 4 == 0, every operand aligned): a
// thread adds its float4 groups in grid-stride order, each group's four
// squares in element order, in double.
__global__ __launch_bounds__(NT) void mse_partial4_kernel(const float* __restrict__ x, const float* __restrict__ t,
                                                          size_t n4, double* __restrict__ part,
                                                          float* __restrict__ dx = nullptr) {
  __shared__ double red[NT / 64];
  double acc = 0.0;
  const size_t stride = (size_t)gridDim.x * NT;
  const float fn = (float)(n4 * 4);
  for (size_t i = (size_t)blockIdx.x * NT + threadIdx.x; i < n4; i += stride) {
    const f32x4 xv = ldv(x, i * 4), tv = ldv(t, i * 4);
    f32x4 g;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const double d = (double)tv[j] - (double)xv[j];
      acc += d * d;
      g[j] = 2.0f * (xv[j] - tv[j]) / fn;
    }
    if (dx) stv(dx, i * 4, g);
  }
  acc = block_sum<NT>(acc, red);
  if (threadIdx.x == 0) part[blockIdx.x] = acc;
}

// The last MSE node's forward when its prediction is an activation's output
// x = act(z): the partial sums of mse_partial_kernel / mse_partial4_kernel
// (the same grid, order and terms; x recomputed from z with the activation's
// own function, the bits the activation stored), x's gradient g = 2 (x - t) /
// n and z's gradient act'(z) g with the product rounded (the activation
// backward's formula), both assigned, in one pass over z and t.
template <int K>
__device__ __forceinline__ float mse_act_dz(float z, float g) {
#pragma clang fp contract(off)
  return act_df<K>(z) * g;
}

// Contraction off in this kernel's own arithmetic, so that x - t is not fused
// with the activation's last product: x is rounded first, as when it is
// stored and read back.  With ADD, z is not read but formed as a + b (an Add
// node's forward, the same float additions) and stored to zout unless zout
// is null: the Add, the activation after it and the loss in one pass over a,
// b and t.
template <int K, bool VEC, bool ADD>
__global__ __launch_bounds__(NT) void mse_act_partial_kernel(const float* __restrict__ z, const float* __restrict__ t,
                                                             size_t n, double* __restrict__ part,
                                                             float* __restrict__ dx, float* __restrict__ dz,
                                                             const float* __restrict__ a, const float* __restrict__ b,
                                                             float* __restrict__ zout) {
#pragma clang fp contract(off)
  __shared__ double red[NT / 64];
  double acc = 0.0;
  const size_t stride = (size_t)gridDim.x * NT;
  const float fn = (float)n;
  if (VEC) {
    for (size_t i = (size_t)blockIdx.x * NT + threadIdx.x; i < n / 4; i += stride) {
      f32x4 zv;
      if (ADD) {
        zv = ldv(a, i * 4) + ldv(b, i * 4);
        if (zout) stv(zout, i * 4, zv);
      } else {
        zv = ldv(z, i * 4);
      }
      const f32x4 tv = ldv(t, i * 4);
      f32x4 g, d;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float xj = act_f<K>(zv[j]);
        const double e = (double)tv[j] - (double)xj;
        acc += e * e;
        g[j] = 2.0f * (xj - tv[j]) / fn;
        d[j] = mse_act_dz<K>(zv[j], g[j]);
      }
      stv(dx, i * 4, g);
      stv(dz, i * 4, d);
    }
  } else {
    for (size_t i = (size_t)blockIdx.x * NT + threadIdx.x; i < n; i += stride) {
      float zi;
      if (ADD) {
        zi = a[i] + b[i];
        if (zout) zout[i] = zi;
      } else {
        zi = z[i];
      }
      const float ti = t[i];
      const float xi = act_f<K>(zi);
      const double e = (double)ti - (double)xi;
      acc += e * e;
      const float g = 2.0f * (xi - ti) / fn;
      dx[i] = g;
      dz[i] = mse_act_dz<K>(zi, g);
    }
  }
  acc = block_sum<NT>(acc, red);
  if (threadIdx.x == 0) part[blockIdx.x] = acc;
}

// One 1024-thread workgroup; four loads in flight per thread, fixed order.
constexpr int FIN_NT = 1024;
// With a slot, the value is also published for the host (mle_read_scalar),
// so a loss read-back needs no kernel of its own.
__global__ __launch_bounds__(FIN_NT) void finish_scalar_kernel(const double* __restrict__ part, size_t nparts,
                                                               double denom, float* __restrict__ out,
                                                               mle::ScalarSlot* slot = nullptr, unsigned seq = 0) {
  __shared__ double red[FIN_NT / 64];
  double a[4] = {0.0, 0.0, 0.0, 0.0};
  size_t i = threadIdx.x;
  for (; i + 3 * FIN_NT < nparts; i += 4 * FIN_NT) {
#pragma unroll
    for (int u = 0; u < 4; ++u) a[u] += part[i + u * FIN_NT];
  }
  for (; i < nparts; i += FIN_NT) a[0] += part[i];
  double acc = (a[0] + a[1]) + (a[2] + a[3]);
  acc = block_sum<FIN_NT>(acc, red);
  if (threadIdx.x == 0) {
    const float v = (float)(acc / denom);
    out[0] = v;
    if (slot) mle::publish_scalar(slot, __builtin_bit_cast(unsigned, v), seq);
  }
}

__global__ __launch_bounds__(NT) void mse_bwd_kernel(const float* __restrict__ x, const float* __restrict__ t,
                                                     const float* __restrict__ up, float* __restrict__ dx, size_t n,
                                                     int acc) {
  const size_t stride = (size_t)gridDim.x * NT;
  const float fn = (float)n;
  for (size_t i = (size_t)blockIdx.x * NT + threadIdx.x; i < n; i += stride) {
    const float d = x[i] - t[i];
    const float g = up ? (2.0f * d * up[0]) / fn : 2.0f * d / fn;
    dx[i] = (acc ? dx[i] : 0.f) + g;
  }
}

// Vector form, used when n % 4 == 0 and every operand is 16-byte aligned.
__global__ __launch_bounds__(NT) void mse_bwd4_kernel(const float* __restrict__ x, const float* __restrict__ t,
                                                      const float* __restrict__ up, float* __restrict__ dx, size_t n4,
                                                      float fn, int acc) {
  const size_t stride = (size_t)gridDim.x * NT;
  const float u = up ? up[0] : 1.0f;
  for (size_t i = (size_t)blockIdx.x * NT + threadIdx.x; i < n4; i += stride) {
    const f32x4 xv = ldv(x, i * 4), tv = ldv(t, i * 4);
    f32x4 g;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float d = xv[j] - tv[j];
      g[j] = up ? (2.0f * d * u) / fn : 2.0f * d / fn;
    }
    stv(dx, i * 4, acc ? ldv(dx, i * 4) + g : g);
  }
}

__global__ __launch_bounds__(NT) void xent_bwd_kernel(const float* __restrict__ p, const float* __restrict__ t,
                                                      const float* __restrict__ up, float* __restrict__ dl, size_t n,
                                                      float batch) {
  const size_t stride = (size_t)gridDim.x * NT;
  for (size_t i = (size_t)blockIdx.x * NT + threadIdx.x; i < n; i += stride) {
    float g = p[i] + (-1.0f) * t[i];
    if (up) g *= up[0];
    dl[i] = g / batch;
  }
}

__global__ __launch_bounds__(NT) void xent_bwd4_kernel(const float* __restrict__ p, const float* __restrict__ t,
                                                       const float* __restrict__ up, float* __restrict__ dl, size_t n4,
                                                       float batch) {
  const size_t stride = (size_t)gridDim.x * NT;
  for (size_t i = (size_t)blockIdx.x * NT + threadIdx.x; i < n4; i += stride) {
    f32x4 g = ldv(p, i * 4) + (-1.0f) * ldv(t, i * 4);
    if (up) g *= up[0];
    stv(dl, i * 4, g / batch);
  }
}

// dlogits = (p - t) * (upstream ? upstream[0] : 1) / batch with t from key
// targets and p = exp(x - max) / sum recomputed from the forward's row stats,
// in the operations the probability path uses (same values, bit for bit).
// Grid: x over float4 column groups, y over rows (looping past 65535).
// A thread owns 4 columns and walks rows blockIdx.y, + gridDim.y, ... four
// at a time with the four rows' loads issued together (a workgroup per row
// left each thread one 16-byte load in flight: 65536 workgroups of one load
// and one store each ran at 63 % of HBM bandwidth).
// POW2: batch is a power of two, so g / batch is the product with its exact
// reciprocal (the same correctly rounded value, subnormals included) and the
// division sequence drops out of the per-element work.
template <bool POW2>
__global__ __launch_bounds__(NT) void xent_keys_bwd4_kernel(const float* __restrict__ x, const float* __restrict__ stats,
                                                            KeyTargets kt, const float* __restrict__ up,
                                                            float* __restrict__ dl, int rows, int cols, float batch) {
  const int c = (blockIdx.x * NT + threadIdx.x) * 4;
  if (c >= cols) return;
  const float u = up ? up[0] : 1.0f;
  const float inv_batch = 1.0f / batch;
  constexpr int R = 4;
  const int step = gridDim.y;
  for (int line0 = blockIdx.y; line0 < rows; line0 += R * step) {
    f32x4 xv[R];
    float mx[R], sum[R];
    int key[R];
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int line = line0 + k * step;
      if (line < rows) {
        xv[k] = ldv(x, (size_t)line * cols + c);
        mx[k] = stats[2 * line];
        sum[k] = stats[2 * line + 1];
        key[k] = kt.key(line, cols);
      }
    }
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int line = line0 + k * step;
      if (line < rows) {
        f32x4 g;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float p = expf(xv[k][j] - mx[k]) / sum[k];
          g[j] = p + (-1.0f) * (c + j == key[k] ? 1.0f : 0.0f);
        }
        if (up) g *= u;
        stv(dl, (size_t)line * cols + c, POW2 ? g * inv_batch : g / batch);
      }
    }
  }
}

__global__ __launch_bounds__(NT) void xent_keys_bwd_kernel(const float* __restrict__ x, const float* __restrict__ stats,
                                                           KeyTargets kt, const float* __restrict__ up,
                                                           float* __restrict__ dl, int rows, int cols, float batch) {
  const int c = blockIdx.x * NT + threadIdx.x;
  if (c >= cols) return;
  for (int line = blockIdx.y; line < rows; line += gridDim.y) {
    const float mx = stats[2 * line], sum = stats[2 * line + 1];
    const float p = expf(x[(size_t)line * cols + c] - mx) / sum;
    float g = p + (-1.0f) * (c == kt.key(line, cols) ? 1.0f : 0.0f);
    if (up) g *= up[0];
    dl[(size_t)line * cols + c] = g / batch;
  }
}

constexpr unsigned kMsePartCap = 2048;

// Cross-entropy against key targets for small logits (rows <= FIN_NT,
// cols <= 64) in one workgroup: the row's max and sum of exp as the GEMM-side
// rowstats_kernel forms them over one 64-column block, the loss term
// -log(p_key + 1e-27) of xent_keys_partials_kernel, and the loss as the
// workgroup's sum of the row terms over rows * cols in finish_scalar_kernel's
// order, published for the host when a slot is given.  With dl set, the
// gradient (p - t) / batch of xent_keys_bwd_kernel too, from the row's own
// exponentials.  Each row is taken by 16 lanes holding columns 4 l + v: the
// maximum by shuffles (its value does not depend on the order), then the
// 64-lane butterfly of rowstats_kernel over the exponentials (level `off`
// pairs columns j and j ^ off: lanes l ^ 8, 4, 2, 1 for off = 32 .. 4, then
// registers v ^ 2, v ^ 1), so each pair is added as there and the bits are
// the same.  x is global memory, or the LDS copy the Linear + cross-entropy
// kernel keeps.
__device__ __forceinline__ void xent_small_body(const float* x, KeyTargets kt, int rows, int cols, float batch,
                                                float* __restrict__ loss, float* __restrict__ dl,
                                                mle::ScalarSlot* slot, unsigned seq) {
  __shared__ double red[FIN_NT / 64];
  __shared__ double slp[FIN_NT];  // each row's loss term, summed in row order below
  const int grp = threadIdx.x >> 4, gl = threadIdx.x & 15;
  for (int rb = 0; rb < rows; rb += FIN_NT / 16) {
    const int row = rb + grp;
    const bool live = row < rows;
    float e[4] = {-FLT_MAX, -FLT_MAX, -FLT_MAX, -FLT_MAX};
    int key = -1;
    float xk = 0.f;
    if (live) {
      const float* xr = x + (size_t)row * cols;
      key = kt.key((size_t)row, cols);
      if (key >= 0) xk = xr[key];
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (4 * gl + v < cols) e[v] = xr[4 * gl + v];
    }
    float m = fmaxf(fmaxf(e[0], e[1]), fmaxf(e[2], e[3]));
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 16));
#pragma unroll
    for (int v = 0; v < 4; ++v) e[v] = (live && 4 * gl + v < cols) ? expf(e[v] - m) : 0.f;
    const float p[4] = {e[0], e[1], e[2], e[3]};  // exp(x - m) of this lane's columns
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1)
#pragma unroll
      for (int v = 0; v < 4; ++v) e[v] = e[v] + __shfl_xor(e[v], o, 16);
    e[0] = e[0] + e[2];
    e[1] = e[1] + e[3];
    e[0] = e[0] + e[1];
    const float sum = e[0] < 1e-45f ? 1.0f : e[0];
    if (live && gl == 0) {
      slp[row] = key >= 0 ? -log((double)(expf(xk - m) / sum) + 1e-27) : 0.0;
      kt.stats[2 * row] = m;
      kt.stats[2 * row + 1] = sum;
    }
    if (dl && live)  // the gradient (p - t) / batch from the same exponentials
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int c = 4 * gl + v;
        if (c < cols) dl[(size_t)row * cols + c] = (p[v] / sum + (-1.0f) * (c == key ? 1.0f : 0.0f)) / batch;
      }
  }
  __syncthreads();
  const double lp = (int)threadIdx.x < rows ? slp[threadIdx.x] : 0.0;
  double acc = (lp + 0.0) + (0.0 + 0.0);  // finish_scalar_kernel's four accumulators, three of them empty
  acc = block_sum<FIN_NT>(acc, red);
  if (threadIdx.x == 0) {
    const float vv = (float)(acc / ((double)rows * (double)cols));
    loss[0] = vv;
    if (slot) mle::publish_scalar(slot, __builtin_bit_cast(unsigned, vv), seq);
  }
}

__global__ __launch_bounds__(FIN_NT) void xent_keys_small_kernel(const float* __restrict__ x, KeyTargets kt, int rows,
                                                                 int cols, float batch, float* __restrict__ loss,
                                                                 float* __restrict__ dl, mle::ScalarSlot* slot,
                                                                 unsigned seq) {
  xent_small_body(x, kt, rows, cols, batch, loss, dl, slot, seq);
}

// A classifier head, Linear then cross-entropy against key targets, in one
// workgroup: logits = X W + bias (X [rows, in], W [in, cols]) on fp32 MFMA,
// the 16 x 16 tiles of the logits (at most LXS_T of them) each taken by
// 16 / tiles waves that split `in` in whole 16-deep slabs and add their
// partial tiles in wave order through LDS; the logits are written out (the
// Linear's output) and kept in LDS, and xent_keys_small_kernel's body runs on
// them: the loss, its read-back, the row statistics and the early gradient.
// Lane group q = l / 16 of a wave feeds k = 4q + e of a slab to MFMA step e,
// so a row of X is read with one 16-byte load per lane and slab.
constexpr int LXS_T = 16, LXS_MAXN = 4096;

__global__ __launch_bounds__(FIN_NT) void linear_xent_small_kernel(const float* __restrict__ X,
                                                                   const float* __restrict__ W,
                                                                   const float* __restrict__ bias,
                                                                   float* __restrict__ logits, int rows, int in,
                                                                   int cols, KeyTargets kt, float batch,
                                                                   float* __restrict__ loss, float* __restrict__ dl,
                                                                   mle::ScalarSlot* slot, unsigned seq) {
  __shared__ __attribute__((aligned(16))) float part[FIN_NT / 64][256];
  __shared__ float lg[LXS_MAXN];
  const int lane = threadIdx.x & 63, li = lane & 15, lq = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int tn = (cols + 15) / 16, tiles = ((rows + 15) / 16) * tn;
  const int wpt = (FIN_NT / 64) / tiles;  // waves per tile
  if (w < tiles * wpt) {
    const int tile = w / wpt, q = w - tile * wpt;
    const int r = (tile / tn) * 16 + li, c = (tile % tn) * 16 + li;  // this lane's X row and W column
    const bool rok = r < rows, cok = c < cols;
    const int kc = ((in + wpt - 1) / wpt + 15) / 16 * 16;
    const int k0 = q * kc, k1 = min(in, k0 + kc);
    const bool vec = in % 4 == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int kb = k0; kb < k1; kb += 64) {  // four slabs: every load issued before the products
      f32x4 a[4], b[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        a[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        b[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int kq = kb + 16 * t + 4 * lq;
        if (kb + 16 * t < k1) {
          if (rok) {
            const float* p = X + (size_t)r * in + kq;
            if (vec && kq + 3 < k1) {
              a[t] = *reinterpret_cast<const f32x4*>(p);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (kq + e < k1) a[t][e] = p[e];
            }
          }
          if (cok)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (kq + e < k1) b[t][e] = W[(size_t)(kq + e) * cols + c];
        }
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (kb + 16 * t >= k1) break;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][e], b[t][e], acc, 0, 0, 0);
      }
    }
    // result lane l holds rows 4 (l / 16) + i of column l % 16
#pragma unroll
    for (int i = 0; i < 4; ++i) part[w][(4 * lq + i) * 16 + li] = acc[i];
  }
  __syncthreads();
  const int n = rows * cols;
  for (int o = threadIdx.x; o < n; o += FIN_NT) {
    const int r = o / cols, c = o - r * cols;
    const int tile = (r / 16) * tn + c / 16, at = (r % 16) * 16 + c % 16;
    float v = part[tile * wpt][at];
    for (int q = 1; q < wpt; ++q) v += part[tile * wpt + q][at];
    if (bias) v += bias[c];
    lg[o] = v;
    logits[o] = v;
  }
  __syncthreads();
  xent_small_body(lg, kt, rows, cols, batch, loss, dl, slot, seq);
}

}  // namespace

extern "C" {

int mle_softmax_fwd(mle_stream stream, const float* x, float* y, int bc, int rows, int cols, int axis, int causal) {
  MLE_CHECK_ARG(x && y && bc >= 0 && rows >= 0 && cols >= 0 && (axis == 0 || axis == 1), "mle_softmax_fwd: bad argument");
  if ((size_t)bc * rows * cols == 0) return MLE_OK;
  hipStream_t s = as_stream(stream);
  const bool vec = cols % 4 == 0 && aligned16(x) && aligned16(y);
  if (axis == 0) {
    const size_t lines = (size_t)bc * rows;
    MLE_CHECK_ARG(lines <= 2147483647u, "mle_softmax_fwd: too many rows");
    if (vec && cols <= 4 * NT * RV4)
      softmax_row4_kernel<<<(unsigned)lines, NT, 0, s>>>(x, y, rows, cols, causal, nullptr, nullptr, KeyTargets{});
    else if (cols <= NT * ROW_CPT)
      softmax_row_kernel<true><<<(unsigned)lines, NT, 0, s>>>(x, y, rows, cols, causal, nullptr, nullptr, KeyTargets{});
    else
      softmax_row_kernel<false><<<(unsigned)lines, NT, 0, s>>>(x, y, rows, cols, causal, nullptr, nullptr, KeyTargets{});
  } else {
    MLE_CHECK_ARG(bc <= 65535, "mle_softmax_fwd: bc %d > 65535", bc);
    dim3 grid((cols + COL_W - 1) / COL_W, bc);
    if (vec && rows <= C4_RL * C4_RPT) softmax_col4_kernel<<<grid, NT, 0, s>>>(x, y, rows, cols, causal);
    else if (rows <= COL_RL * COL_RPT) softmax_col_kernel<true><<<grid, NT, 0, s>>>(x, y, rows, cols, causal);
    else softmax_col_kernel<false><<<grid, NT, 0, s>>>(x, y, rows, cols, causal);
  }
  return check_launch("mle_softmax_fwd");
}

int mle_softmax_bwd(mle_stream stream, const float* y, const float* dy, float* dx, int bc, int rows, int cols,
                    int axis, int accumulate) {
  MLE_CHECK_ARG(y && dy && dx && (axis == 0 || axis == 1), "mle_softmax_bwd: bad argument");
  if ((size_t)bc * rows * cols == 0) return MLE_OK;
  hipStream_t s = as_stream(stream);
  if (axis == 0) {
    const size_t lines = (size_t)bc * rows;
    MLE_CHECK_ARG(lines <= 2147483647u, "mle_softmax_bwd: too many rows");
    if (cols <= NT * ROW_CPT) softmax_row_bwd_kernel<true><<<(unsigned)lines, NT, 0, s>>>(y, dy, dx, cols, accumulate);
    else softmax_row_bwd_kernel<false><<<(unsigned)lines, NT, 0, s>>>(y, dy, dx, cols, accumulate);
  } else {
    MLE_CHECK_ARG(bc <= 65535, "mle_softmax_bwd: bc %d > 65535", bc);
    dim3 grid((cols + COL_W - 1) / COL_W, bc);
    const bool vec = cols % 4 == 0 && aligned16(y) && aligned16(dy) && aligned16(dx);
    if (vec && rows <= C4_RL * C4_RPT)
      softmax_col4_bwd_kernel<<<grid, NT, 0, s>>>(y, dy, dx, rows, cols, accumulate);
    else if (rows <= COL_RL * COL_RPT)
      softmax_col_bwd_kernel<true><<<grid, NT, 0, s>>>(y, dy, dx, rows, cols, accumulate);
    else
      softmax_col_bwd_kernel<false><<<grid, NT, 0, s>>>(y, dy, dx, rows, cols, accumulate);
  }
  return check_launch("mle_softmax_bwd");
}

size_t mle_loss_ws_bytes(size_t n) {
  // MSE: one double per partial block; cross-entropy: one double per row (<= n).
  size_t parts = n < kMsePartCap ? n : kMsePartCap;
  size_t rows = n;
  size_t b = (parts > rows ? parts : rows) * sizeof(double);
  return b < 256 ? 256 : b;
}

static int mse_fwd_impl(mle_stream stream, const float* x, const float* t, size_t n, float* loss, void* ws,
                        size_t ws_bytes, float* loss_host, const char* who, float* dx = nullptr) {
  MLE_CHECK_ARG(x && t && loss && ws && n > 0, "%s: bad argument", who);
  const unsigned g = stream_grid(n, NT, kMsePartCap);
  if (ws_bytes < g * sizeof(double)) return set_error(MLE_ERR_WORKSPACE, "%s: workspace too small", who);
  hipStream_t s = as_stream(stream);
  double* part = static_cast<double*>(ws);
  mle::ScalarRead r;
  if (loss_host) {
    const int rc = mle::scalar_read_begin(r, who);
    if (rc) return rc;
  }
  unsigned np = g;
  if (n % 4 == 0 && aligned16(x) && aligned16(t) && (!dx || aligned16(dx))) {
    np = stream_grid(n / 4, NT, kMsePartCap);
    mse_partial4_kernel<<<np, NT, 0, s>>>(x, t, n / 4, part, dx);
  } else {
    mse_partial_kernel<<<g, NT, 0, s>>>(x, t, n, part, dx);
  }
  finish_scalar_kernel<<<1, FIN_NT, 0, s>>>(part, np, (double)n, loss, r.slot, r.seq);
  const int rc = check_launch(who);
  if (rc || !loss_host) return rc;
  return mle::scalar_read_finish(s, r, loss_host, who);
}

int mle_mse_fwd(mle_stream stream, const float* x, const float* t, size_t n, float* loss, void* ws, size_t ws_bytes) {
  return mse_fwd_impl(stream, x, t, n, loss, ws, ws_bytes, nullptr, "mle_mse_fwd");
}

int mle_mse_fwd_read(mle_stream stream, const float* x, const float* t, size_t n, float* loss, void* ws,
                     size_t ws_bytes, float* loss_host) {
  MLE_CHECK_ARG(loss_host != nullptr, "mle_mse_fwd_read: null loss_host");
  return mse_fwd_impl(stream, x, t, n, loss, ws, ws_bytes, loss_host, "mle_mse_fwd_read");
}

int mle_mse_fwd_bwd_read(mle_stream stream, const float* x, const float* t, size_t n, float* loss, float* dx,
                         void* ws, size_t ws_bytes, float* loss_host) {
  MLE_CHECK_ARG(loss_host != nullptr && dx != nullptr, "mle_mse_fwd_bwd_read: null pointer");
  return mse_fwd_impl(stream, x, t, n, loss, ws, ws_bytes, loss_host, "mle_mse_fwd_bwd_read", dx);
}

static int mse_act_impl(mle_stream stream, const float* z, float* zout, const float* a, const float* b, const float* t, size_t n,
                        int act_kind, float* loss, float* dx, float* dz, void* ws, size_t ws_bytes, float* loss_host,
                        const char* who) {
  const bool add = a != nullptr;
  MLE_CHECK_ARG((add ? b != nullptr : z != nullptr) && t && loss && dx && dz && ws && loss_host && n > 0 &&
                    act_kind >= MLE_RELU && act_kind <= MLE_LEAKY_RELU,
                "%s: bad argument", who);
  MLE_CHECK_ARG(dx != dz && dx != t && dz != t && (!z || dx != z), "%s: dx and dz must differ from each other and t",
                who);
  if (add)
    MLE_CHECK_ARG(!z || (z != a && z != b && z != t && z != dz), "%s: z must not alias a, b, t or dz", who);
  if (add)
    MLE_CHECK_ARG(dx != a && dx != b && dz != a && dz != b,
                  "%s: z, dx and dz must not alias a, b or t", who);
  const unsigned g = stream_grid(n, NT, kMsePartCap);
  if (ws_bytes < g * sizeof(double)) return set_error(MLE_ERR_WORKSPACE, "%s: workspace too small", who);
  hipStream_t s = as_stream(stream);
  double* part = static_cast<double*>(ws);
  mle::ScalarRead r;
  int rc = mle::scalar_read_begin(r, who);
  if (rc) return rc;
  const bool vec = n % 4 == 0 && (!z || aligned16(z)) && aligned16(t) && aligned16(dx) && aligned16(dz) &&
                   (!add || (aligned16(a) && aligned16(b)));
  const unsigned np = vec ? stream_grid(n / 4, NT, kMsePartCap) : g;  // mse_fwd_impl's grids
#define MLE_MSE_ACT_A(K, A)                                                                                    \
  (vec ? mse_act_partial_kernel<K, true, A><<<np, NT, 0, s>>>(z, t, n, part, dx, dz, a, b, zout)               \
       : mse_act_partial_kernel<K, false, A><<<np, NT, 0, s>>>(z, t, n, part, dx, dz, a, b, zout))
#define MLE_MSE_ACT(K) (add ? MLE_MSE_ACT_A(K, true) : MLE_MSE_ACT_A(K, false))
  switch (act_kind) {
    case MLE_RELU: MLE_MSE_ACT(MLE_RELU); break;
    case MLE_GELU: MLE_MSE_ACT(MLE_GELU); break;
    case MLE_SILU: MLE_MSE_ACT(MLE_SILU); break;
    case MLE_TANH: MLE_MSE_ACT(MLE_TANH); break;
    case MLE_SIGMOID: MLE_MSE_ACT(MLE_SIGMOID); break;
    default: MLE_MSE_ACT(MLE_LEAKY_RELU); break;
  }
#undef MLE_MSE_ACT
#undef MLE_MSE_ACT_A
  finish_scalar_kernel<<<1, FIN_NT, 0, s>>>(part, np, (double)n, loss, r.slot, r.seq);
  rc = check_launch(who);
  if (rc) return rc;
  return mle::scalar_read_finish(s, r, loss_host, who);
}

int mle_mse_act_fwd_bwd_read(mle_stream stream, const float* z, const float* t, size_t n, int act_kind, float* loss,
                             float* dx, float* dz, void* ws, size_t ws_bytes, float* loss_host) {
  return mse_act_impl(stream, z, nullptr, nullptr, nullptr, t, n, act_kind, loss, dx, dz, ws, ws_bytes, loss_host,
                      "mle_mse_act_fwd_bwd_read");
}

int mle_add_mse_act_fwd_bwd_read(mle_stream stream, const float* a, const float* b, float* z, const float* t,
                                 size_t n, int act_kind, float* loss, float* dx, float* dz, void* ws, size_t ws_bytes,
                                 float* loss_host) {
  MLE_CHECK_ARG(a && b, "mle_add_mse_act_fwd_bwd_read: null pointer");
  return mse_act_impl(stream, z, z, a, b, t, n, act_kind, loss, dx, dz, ws, ws_bytes, loss_host,
                      "mle_add_mse_act_fwd_bwd_read");
}

int mle_mse_bwd(mle_stream stream, const float* x, const float* t, const float* upstream, float* dx, size_t n,
                int accumulate) {
  MLE_CHECK_ARG(x && t && dx, "mle_mse_bwd: bad argument");
  if (n == 0) return MLE_OK;
  if (n % 4 == 0 && aligned16(x) && aligned16(t) && aligned16(dx))
    mse_bwd4_kernel<<<stream_grid(n / 4, NT, 8192), NT, 0, as_stream(stream)>>>(x, t, upstream, dx, n / 4, (float)n,
                                                                               accumulate);
  else
    mse_bwd_kernel<<<stream_grid(n, NT, 8192), NT, 0, as_stream(stream)>>>(x, t, upstream, dx, n, accumulate);
  return check_launch("mle_mse_bwd");
}

int mle_softmax_xent_fwd(mle_stream stream, const float* logits, const float* target, float* probs, int rows, int cols,
                         float* loss, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(logits && target && probs && loss && ws && rows > 0 && cols > 0, "mle_softmax_xent_fwd: bad argument");
  if (ws_bytes < (size_t)rows * sizeof(double))
    return set_error(MLE_ERR_WORKSPACE, "mle_softmax_xent_fwd: workspace too small");
  hipStream_t s = as_stream(stream);
  double* part = static_cast<double*>(ws);
  if (cols % 4 == 0 && cols <= 4 * NT * RV4 && aligned16(logits) && aligned16(probs) && aligned16(target))
    softmax_row4_kernel<<<rows, NT, 0, s>>>(logits, probs, rows, cols, 0, target, part, KeyTargets{});
  else if (cols <= NT * ROW_CPT)
    softmax_row_kernel<true><<<rows, NT, 0, s>>>(logits, probs, rows, cols, 0, target, part, KeyTargets{});
  else
    softmax_row_kernel<false><<<rows, NT, 0, s>>>(logits, probs, rows, cols, 0, target, part, KeyTargets{});
  finish_scalar_kernel<<<1, FIN_NT, 0, s>>>(part, (size_t)rows, (double)rows * (double)cols, loss);
  return check_launch("mle_softmax_xent_fwd");
}

int mle_softmax_xent_bwd(mle_stream stream, const float* probs, const float* target, const float* upstream,
                         float* dlogits, size_t n, int batch) {
  MLE_CHECK_ARG(probs && target && dlogits && batch > 0, "mle_softmax_xent_bwd: bad argument");
  if (n == 0) return MLE_OK;
  if (n % 4 == 0 && aligned16(probs) && aligned16(target) && aligned16(dlogits))
    xent_bwd4_kernel<<<stream_grid(n / 4, NT, 8192), NT, 0, as_stream(stream)>>>(probs, target, upstream, dlogits,
                                                                                n / 4, (float)batch);
  else
    xent_bwd_kernel<<<stream_grid(n, NT, 8192), NT, 0, as_stream(stream)>>>(probs, target, upstream, dlogits, n,
                                                                           (float)batch);
  return check_launch("mle_softmax_xent_bwd");
}

int mle_softmax_xent_keys_fwd(mle_stream stream, const float* logits, const int32_t* keys, int clen, int max_clen,
                              float* stats, int rows, int cols, float* loss, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(logits && keys && stats && loss && ws && rows > 0 && cols > 0 && clen > 0 && max_clen >= clen &&
                    rows % clen == 0,
                "mle_softmax_xent_keys_fwd: bad argument");
  if (ws_bytes < (size_t)rows * sizeof(double))
    return set_error(MLE_ERR_WORKSPACE, "mle_softmax_xent_keys_fwd: workspace too small");
  hipStream_t s = as_stream(stream);
  double* part = static_cast<double*>(ws);
  const KeyTargets kt{keys, clen, max_clen, stats};
  // The kernel choice matches mle_softmax_xent_fwd's, so sums and loss agree bit for bit.
  if (cols % 4 == 0 && cols <= 4 * NT * RV4 && aligned16(logits))
    softmax_row4_kernel<<<rows, NT, 0, s>>>(logits, nullptr, rows, cols, 0, nullptr, part, kt);
  else if (cols <= NT * ROW_CPT)
    softmax_row_kernel<true><<<rows, NT, 0, s>>>(logits, nullptr, rows, cols, 0, nullptr, part, kt);
  else
    softmax_row_kernel<false><<<rows, NT, 0, s>>>(logits, nullptr, rows, cols, 0, nullptr, part, kt);
  finish_scalar_kernel<<<1, FIN_NT, 0, s>>>(part, (size_t)rows, (double)rows * (double)cols, loss);
  return check_launch("mle_softmax_xent_keys_fwd");
}

static int xent_rowstats_impl(mle_stream stream, const float* logits, const float* rowpart, int64_t ldp, const int32_t* keys,
                       int clen, int max_clen, float* stats, int rows, int cols, float* loss, void* ws, size_t ws_bytes,
                       float* loss_host, const char* who) {
  const int nblk = (cols + 63) / 64;
  MLE_CHECK_ARG(logits && rowpart && keys && stats && loss && ws && rows > 0 && cols > 0 && clen > 0 &&
                    max_clen >= clen && rows % clen == 0 && ldp >= 2 * (int64_t)nblk,
                "%s: bad argument", who);
  if (ws_bytes < (size_t)rows * sizeof(double)) return set_error(MLE_ERR_WORKSPACE, "%s: workspace too small", who);
  hipStream_t s = as_stream(stream);
  double* part = static_cast<double*>(ws);
  const KeyTargets kt{keys, clen, max_clen, stats};
  const unsigned grid = (unsigned)((rows + 3) / 4);
  const double denom = (double)rows * (double)cols;
  mle::ScalarRead r;
  if (loss_host) {
    const int rc = mle::scalar_read_begin(r, who);
    if (rc) return rc;
  }
  xent_keys_partials_kernel<<<grid, 256, 0, s>>>(logits, rowpart, ldp, nblk, rows, cols, kt, part);
  finish_scalar_kernel<<<1, FIN_NT, 0, s>>>(part, (size_t)rows, denom, loss, r.slot, r.seq);
  const int rc = check_launch(who);
  if (rc || !loss_host) return rc;
  return mle::scalar_read_finish(s, r, loss_host, who);
}

int mle_softmax_xent_keys_fwd_rowstats(mle_stream stream, const float* logits, const float* rowpart, int64_t ldp,
                                       const int32_t* keys, int clen, int max_clen, float* stats, int rows, int cols,
                                       float* loss, void* ws, size_t ws_bytes) {
  return xent_rowstats_impl(stream, logits, rowpart, ldp, keys, clen, max_clen, stats, rows, cols, loss, ws, ws_bytes,
                            nullptr, "mle_softmax_xent_keys_fwd_rowstats");
}

int mle_softmax_xent_keys_fwd_rowstats_read(mle_stream stream, const float* logits, const float* rowpart,
                                            int64_t ldp, const int32_t* keys, int clen, int max_clen, float* stats,
                                            int rows, int cols, float* loss, void* ws, size_t ws_bytes,
                                            float* loss_host) {
  MLE_CHECK_ARG(loss_host != nullptr, "mle_softmax_xent_keys_fwd_rowstats_read: null loss_host");
  return xent_rowstats_impl(stream, logits, rowpart, ldp, keys, clen, max_clen, stats, rows, cols, loss, ws, ws_bytes,
                            loss_host, "mle_softmax_xent_keys_fwd_rowstats_read");
}

int mle_softmax_xent_keys_small_read(mle_stream stream, const float* logits, const int32_t* keys, int clen,
                                     int max_clen, float* stats, int rows, int cols, int batch, float* loss,
                                     float* dlogits, float* loss_host) {
  MLE_CHECK_ARG(logits && keys && stats && loss && rows > 0 && cols > 0 && clen > 0 && max_clen >= clen &&
                    rows % clen == 0 && batch > 0,
                "mle_softmax_xent_keys_small_read: bad argument");
  MLE_CHECK_ARG(rows <= FIN_NT && cols <= 64, "mle_softmax_xent_keys_small_read: %d x %d logits exceed %d x 64", rows,
                cols, FIN_NT);
  hipStream_t s = as_stream(stream);
  const KeyTargets kt{keys, clen, max_clen, stats};
  mle::ScalarRead r;
  if (loss_host) {
    const int rc = mle::scalar_read_begin(r, "mle_softmax_xent_keys_small_read");
    if (rc) return rc;
  }
  xent_keys_small_kernel<<<1, FIN_NT, 0, s>>>(logits, kt, rows, cols, (float)batch, loss, dlogits, r.slot, r.seq);
  const int rc = check_launch("mle_softmax_xent_keys_small_read");
  if (rc || !loss_host) return rc;
  return mle::scalar_read_finish(s, r, loss_host, "mle_softmax_xent_keys_small_read");
}

int mle_linear_xent_keys_small_read(mle_stream stream, int rows, int in, int cols, const float* X, const float* W,
                                    const float* bias, float* logits, const int32_t* keys, int clen, int max_clen,
                                    float* stats, int batch, float* loss, float* dlogits, float* loss_host) {
  MLE_CHECK_ARG(X && W && logits && keys && stats && loss && rows > 0 && in >= 0 && cols > 0 && clen > 0 &&
                    max_clen >= clen && rows % clen == 0 && batch > 0,
                "mle_linear_xent_keys_small_read: bad argument");
  MLE_CHECK_ARG(rows <= FIN_NT && cols <= 64, "mle_linear_xent_keys_small_read: %d x %d logits exceed %d x 64", rows,
                cols, FIN_NT);
  MLE_CHECK_ARG(dlogits != logits && logits != X && logits != W,
                "mle_linear_xent_keys_small_read: logits must differ from X, W and dlogits");
  const int tiles = ((rows + 15) / 16) * ((cols + 15) / 16);
  if (tiles > LXS_T || rows * cols > LXS_MAXN) {  // the two launches
    const int rc = mle_gemm_ex(stream, 0, 0, rows, cols, in, 1.0f, X, in, 0, W, cols, 0, 0.0f, logits, cols, 0, 1,
                               nullptr, bias, nullptr, 0);
    if (rc) return rc;
    return mle_softmax_xent_keys_small_read(stream, logits, keys, clen, max_clen, stats, rows, cols, batch, loss,
                                            dlogits, loss_host);
  }
  hipStream_t s = as_stream(stream);
  const KeyTargets kt{keys, clen, max_clen, stats};
  mle::ScalarRead r;
  if (loss_host) {
    const int rc = mle::scalar_read_begin(r, "mle_linear_xent_keys_small_read");
    if (rc) return rc;
  }
  linear_xent_small_kernel<<<1, FIN_NT, 0, s>>>(X, W, bias, logits, rows, in, cols, kt, (float)batch, loss, dlogits,
                                                r.slot, r.seq);
  const int rc = check_launch("mle_linear_xent_keys_small_read");
  if (rc || !loss_host) return rc;
  return mle::scalar_read_finish(s, r, loss_host, "mle_linear_xent_keys_small_read");
}

int mle_softmax_xent_keys_bwd(mle_stream stream, const float* logits, const float* stats, const int32_t* keys, int clen,
                              int max_clen, const float* upstream, float* dlogits, int rows, int cols, int batch) {
  MLE_CHECK_ARG(logits && stats && keys && dlogits && batch > 0 && rows > 0 && cols > 0 && clen > 0 &&
                    max_clen >= clen && rows % clen == 0,
                "mle_softmax_xent_keys_bwd: bad argument");
  hipStream_t s = as_stream(stream);
  const KeyTargets kt{keys, clen, max_clen, nullptr};
  const unsigned gy = (unsigned)std::min(rows, 65535);
  if (cols % 4 == 0 && aligned16(logits) && aligned16(dlogits)) {
    const dim3 grid((cols / 4 + NT - 1) / NT, std::min(gy, 1024u));
    if ((batch & (batch - 1)) == 0 && batch <= (1 << 24))
      xent_keys_bwd4_kernel<true><<<grid, NT, 0, s>>>(logits, stats, kt, upstream, dlogits, rows, cols, (float)batch);
    else
      xent_keys_bwd4_kernel<false><<<grid, NT, 0, s>>>(logits, stats, kt, upstream, dlogits, rows, cols, (float)batch);
  } else
    xent_keys_bwd_kernel<<<dim3((cols + NT - 1) / NT, gy), NT, 0, s>>>(logits, stats, kt, upstream, dlogits, rows,
                                                                       cols, (float)batch);
  return check_launch("mle_softmax_xent_keys_bwd");
}

}  // extern "C"
