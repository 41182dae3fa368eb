// ORACLE -- test infrastructure only.
//
// A CPU (OpenMP C++) restatement of the ML_Engine arithmetic on the backward /
// optimizer hot path.  Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg load it, as the checker and the CPU baseline; the product
// (ml_engine_amd) never calls it.  Each function names the reference code it
// restates (paths relative to the reference repository root).
//
// Accumulation rule: where the reference's summation order is not reproducible
// (fp32 atomicAdd epilogues of bcmm*, per-thread serial sums inside blocks whose
// partials are combined by atomics) the oracle accumulates in double and rounds
// once, giving an order-independent value to compare against.  Element-wise
// formulas keep the reference's float/double promotions exactly.
//
// How each function is pinned (tests/test_oracle_pins.py): torch CPU autograd /
// matmul / conv2d cross-checks, central finite differences, closed forms and
// brute-force identities -- see the test file for the list per function.
#include <math.h>
#include <float.h>
#include <limits.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#include <vector>
#include <algorithm>
#include <omp.h>

#define OEXPORT extern "C" __attribute__((visibility("default")))

namespace {
constexpr float kPI = 3.14159265359f;  // Includes/kernels.h:10

// batch_chan_offset (Engine/kernels.cu:371-385)
inline long long bco(int flag, int b, int c, int C, long long inner) {
  const int hb = flag & 1, hc = (flag >> 1) & 1;
  const long long cs = hc ? C : 1;
  return (hb ? (long long)b * cs : 0) * inner + (hc ? (long long)c : 0) * inner;
}
}  // namespace

OEXPORT int orc_num_threads(void) { return omp_get_max_threads(); }
OEXPORT void orc_set_threads(int n) { if (n > 0) omp_set_num_threads(n); }

// ---------------------------------------------------------------------------
// GEMM family: bcmm / bcmmABT / bcmmATB / bcmmT (Engine/kernels.cu:387-539).
// kind 0: C[m x p] (+)= s * A[m x n] B[n x p]
// kind 1: C[m x p] (+)= s * A[m x n] B[p x n]^T
// kind 2: C[m x p] (+)= s * A[n x m]^T B[n x p]
// kind 3: C[m x p] (+)= s * A[n x m]^T B[p x n]^T
// backward == 0 assigns, 1 accumulates (the reference's atomicAdd); flags are
// the batch/channel broadcast codes A, B, C of batch_chan_offset.
namespace {
// Register tile of the packed GEMM: MR rows x NR columns of C per work step.
constexpr int kMR = 4, kNR = 32, kRowTiles = 8;

// op(A) element (r, k) and op(B) element (k, c) of the four bcmm kinds.
inline float a_at(const float* a, int kind, int m, int n, long long r, long long k) {
  return (kind & 2) ? a[k * m + r] : a[r * n + k];
}
inline float b_at(const float* b, int kind, int n, int p, long long k, long long c) {
  return (kind & 1) ? b[c * n + k] : b[k * p + c];
}

// C tile = sum_k op(A)[r, k] op(B)[k, c] with one double accumulator per
// element, the k terms added one at a time in increasing k -- the same
// operations in the same order as a scalar triple loop, so the result is
// bit-identical to it (the build disables FMA contraction).  The column loop
// vectorises; only the accumulators' layout differs from the scalar loop.
inline void gemm_tile(const float* ap, const float* bp, long long n, double acc[kMR][kNR]) {
  for (int i = 0; i < kMR; ++i)
    for (int j = 0; j < kNR; ++j) acc[i][j] = 0.0;
  for (long long k = 0; k < n; ++k) {
    double bv[kNR];
    for (int j = 0; j < kNR; ++j) bv[j] = (double)bp[k * kNR + j];
    for (int i = 0; i < kMR; ++i) {
      const double av = (double)ap[k * kMR + i];
      for (int j = 0; j < kNR; ++j) acc[i][j] += av * bv[j];
    }
  }
}

// C[r, c] = sum_k A(r, k) B(k, c) for r < m, c < p, k < n, with the operands
// given by element functions: each is read once into a packed copy (op(A) as
// [row tile][k][kMR], op(B) as [column tile][k][kNR], zero past the matrix
// edge -- those products only reach discarded tile elements), then every tile
// is summed by gemm_tile and handed to store(r, c, sum).
template <class AF, class BF, class SF>
void packed_gemm(long long m, long long n, long long p, const AF& a_el, const BF& b_el, const SF& store) {
  const long long rt = (m + kMR - 1) / kMR, ct = (p + kNR - 1) / kNR;
  std::vector<float> ap((size_t)(rt * kMR * n)), bp((size_t)(ct * kNR * n));
#pragma omp parallel for schedule(static)
  for (long long t = 0; t < rt; ++t)
    for (int i = 0; i < kMR; ++i) {
      const long long r = t * kMR + i;
      float* dst = ap.data() + t * kMR * n + i;
      for (long long k = 0; k < n; ++k) dst[k * kMR] = r < m ? a_el(r, k) : 0.0f;
    }
#pragma omp parallel for schedule(static)
  for (long long t = 0; t < ct; ++t)
    for (long long k = 0; k < n; ++k)
      for (int j = 0; j < kNR; ++j) {
        const long long col = t * kNR + j;
        bp[(size_t)((t * n + k) * kNR + j)] = col < p ? b_el(k, col) : 0.0f;
      }
  const long long rblocks = (rt + kRowTiles - 1) / kRowTiles;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (long long cb = 0; cb < ct; ++cb)
    for (long long rb = 0; rb < rblocks; ++rb)
      for (long long t = rb * kRowTiles; t < std::min(rt, (rb + 1) * kRowTiles); ++t) {
        double acc[kMR][kNR];
        gemm_tile(ap.data() + t * kMR * n, bp.data() + cb * kNR * n, n, acc);
        for (int i = 0; i < kMR && t * kMR + i < m; ++i)
          for (int j = 0; j < kNR && cb * kNR + j < p; ++j) store(t * kMR + i, cb * kNR + j, acc[i][j]);
      }
}
}  // namespace

OEXPORT void orc_bcmm(int kind, const float* a, const float* b, float* c, int batch, int channels, int m, int n, int p,
                      int backward, int fa, int fb, int fc, float scale) {
  for (int z = 0; z < batch * channels; ++z) {
    const int bi = z / channels, ci = z % channels;
    const float* A = a + bco(fa, bi, ci, channels, (long long)m * n);
    const float* B = b + bco(fb, bi, ci, channels, (long long)n * p);
    float* Cz = c + bco(fc, bi, ci, channels, (long long)m * p);
    packed_gemm(
        m, n, p, [&](long long r, long long k) { return a_at(A, kind, m, n, r, k); },
        [&](long long k, long long col) { return b_at(B, kind, n, p, k, col); },
        [&](long long r, long long col, double acc) {
          const float sum = (float)acc;
          float* dst = Cz + r * p + col;
          if (backward == 0) *dst = scale * sum;
          else *dst += scale * sum;
        });
  }
}

// The scalar triple loop orc_bcmm restates in packed form; kept to check that
// the two agree bit for bit (tests/test_oracle_pins.py).
OEXPORT void orc_bcmm_naive(int kind, const float* a, const float* b, float* c, int batch, int channels, int m, int n,
                            int p, int backward, int fa, int fb, int fc, float scale) {
  for (int z = 0; z < batch * channels; ++z) {
    const int bi = z / channels, ci = z % channels;
    const float* A = a + bco(fa, bi, ci, channels, (long long)m * n);
    const float* B = b + bco(fb, bi, ci, channels, (long long)n * p);
    float* Cz = c + bco(fc, bi, ci, channels, (long long)m * p);
#pragma omp parallel for schedule(static)
    for (int row = 0; row < m; ++row)
      for (int col = 0; col < p; ++col) {
        double acc = 0.0;
        for (int k = 0; k < n; ++k) acc += (double)a_at(A, kind, m, n, row, k) * (double)b_at(B, kind, n, p, k, col);
        const float sum = (float)acc;
        float* dst = Cz + (long long)row * p + col;
        if (backward == 0) *dst = scale * sum;
        else *dst += scale * sum;
      }
  }
}

// BCompress (Engine/kernels.cu:1562-1584): Y[col] += scale * sum over all rows.
OEXPORT void orc_bcompress(const float* x, float* y, long long rows, int cols, float scale) {
#pragma omp parallel for schedule(static)
  for (int c = 0; c < cols; ++c) {
    double acc = 0.0;
    for (long long r = 0; r < rows; ++r) acc += x[r * cols + c];
    y[c] += (float)acc * scale;
  }
}

// BCumAdd (Engine/kernels.cu:1586-1592): X[row, :] += Y[:].
OEXPORT void orc_bcumadd(float* x, const float* y, long long rows, int cols) {
#pragma omp parallel for schedule(static)
  for (long long r = 0; r < rows; ++r)
    for (int c = 0; c < cols; ++c) x[r * cols + c] += y[c];
}

// Channel_Squeeze1D (Engine/kernels.cu:1734-1761) launched with `nblocks`
// blocks: average[c] += sum_{b,s} X[b, c, s] for c < nblocks.
OEXPORT void orc_channel_squeeze(const float* x, float* avg, int batch, int depth, long long spatial, int nblocks) {
  const int nb = std::min(nblocks, depth);
#pragma omp parallel for schedule(static)
  for (int c = 0; c < nb; ++c) {
    double acc = 0.0;
    for (int b = 0; b < batch; ++b)
      for (long long s = 0; s < spatial; ++s) acc += x[((long long)b * depth + c) * spatial + s];
    avg[c] += (float)acc;
  }
}

// broadcast_add (Engine/kernels.cu:1661-1668).
OEXPORT void orc_broadcast_add(const float* x, const float* bias, float* out, int batch, int kernels, long long hw) {
  const long long total = (long long)batch * kernels * hw;
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < total; ++i) out[i] = x[i] + bias[(i / hw) % kernels];
}

// ---------------------------------------------------------------------------
// Element-wise ops.
// ScaleAdd (Engine/kernels.cu:1718-1724)
OEXPORT void orc_scale_add(const float* x, const float* y, float* z, float scale, long long n) {
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) z[i] = x[i] + scale * y[i];
}
// Accumulate (Engine/kernels.cu:1693-1699): Y += scale*X in double, stored float.
OEXPORT void orc_accumulate(const float* x, float* y, double scale, long long n) {
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) y[i] = (float)((double)y[i] + scale * (double)x[i]);
}
// Scale_Write (Engine/kernels.cu:1677-1682)
OEXPORT void orc_scale_write(const float* x, float* y, float scale, long long n) {
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) y[i] = scale * x[i];
}

// Activations and derivatives (Engine/kernels.cu:1214-1328).  kind: 0 ReLU,
// 1 GELU (tanh form), 2 SiLU, 3 tanh, 4 sigmoid, 5 leaky ReLU.
static inline float act_f(int kind, float x) {
  switch (kind) {
    case 0: return (x < 0) ? 0.0f : x;
    case 1: {
      const float val = sqrtf(2.0f / kPI) * (x + 0.044715f * x * x * x);
      return 0.5f * x * (1.0f + tanhf(val));
    }
    case 2: return x * (1.0f / (1.0f + expf(-x)));
    case 3: return tanhf(x);
    case 4: return 1.0f / (1.0f + expf(-1.0f * x));
    default: return (x < 0) ? 0.01f * x : x;
  }
}
static inline float act_df(int kind, float x) {
  switch (kind) {
    case 0: return (x > 0.0f) ? 1.0f : 0.0f;
    case 1: {
      const float root = sqrtf(2.0f / kPI);
      const float u = root * (x + 0.044715f * x * x * x);
      const float du = root * (1.0f + 0.134145f * x * x);
      const float t = tanhf(u);
      return 0.5f + 0.5f * t + 0.5f * x * (1.0f - t * t) * du;
    }
    case 2: {
      const float e = expf(x), ne = 1.0f / e, sg = 1.0f / (1.0f + ne);
      return sg + (x / (e + ne + 2.0f));
    }
    case 3: {
      const float e2 = expf(2.0f * x), ne2 = 1.0f / e2;
      return 4.0f / (e2 + ne2 + 2.0f);
    }
    case 4: {
      const float e = expf(x), ne = 1.0f / e;
      return 1.0f / (e + ne + 2.0f);
    }
    default: return (x < 0.0f) ? 0.01f : 1.0f;
  }
}
OEXPORT void orc_act_fwd(int kind, const float* x, float* y, long long n) {
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) y[i] = act_f(kind, x[i]);
}
// deriv_*: grad_out += f'(x) * grad_in
OEXPORT void orc_act_bwd(int kind, const float* x, const float* dy, float* dx, long long n) {
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) dx[i] += act_df(kind, x[i]) * dy[i];
}

// HeadifyColChannel (Engine/kernels.cu:1371-1406), flags 0..3.
OEXPORT void orc_headify(const float* in, float* out, int batch, int heads, int seq, int hd, int flag) {
  const long long total = (long long)batch * heads * seq * hd;
  const long long embed = (long long)heads * hd;
#pragma omp parallel for schedule(static)
  for (long long idx = 0; idx < total; ++idx) {
    const long long d = idx % hd, s = (idx / hd) % seq, h = (idx / ((long long)hd * seq)) % heads;
    const long long b = idx / ((long long)hd * seq * heads);
    const long long hidx = b * (heads * (long long)seq * hd) + h * ((long long)seq * hd) + s * hd + d;
    const long long fidx = b * ((long long)seq * embed) + s * embed + h * hd + d;
    if (flag == 0) out[hidx] = in[fidx];
    else if (flag == 1) out[fidx] += in[hidx];
    else if (flag == 2) out[fidx] = in[hidx];
    else out[hidx] += in[fidx];
  }
}

// MatPEncoding (Engine/kernels.cu:166-185)
OEXPORT void orc_matpe(const float* x, float* out, int batch, int row, int col, int start_idx) {
  const long long total = (long long)batch * row * col;
#pragma omp parallel for schedule(static)
  for (long long g = 0; g < total; ++g) {
    const int pos = (int)((g % ((long long)row * col)) / col) + start_idx;
    const int dim = (int)(g % col);
    const int i = dim / 2;
    const double expo = (2.0 * i) / col;
    const double freq = 1.0 / pow(10000.0, expo);
    const double ang = (double)pos * freq;
    out[g] = x[g] + ((dim % 2 == 0) ? (float)sin(ang) : (float)cos(ang));
  }
}

// PEncoding (Engine/kernels.cu:147-164)
OEXPORT void orc_pe(float* x, int t, int dim) {
  const int half = dim / 2;
  for (int g = 0; g < dim; ++g) {
    const int fi = (g < half) ? g : g - half;
    const double expo = -(double)fi * log(10000.0) / (half - 1);
    const double ang = (double)t * exp(expo);
    x[g] = (g < half) ? (float)cos(ang) : (float)sin(ang);
  }
}

// ---------------------------------------------------------------------------
// Softmax: SoftMax / SoftMask (Engine/kernels.cu:2183-2235) = FindMax,
// exponentiate(M), SumCols/SumRows (sum < 1e-45 -> 1), Scale_arr(divide).
// type 0 normalises each row, type 1 each column; masked: c > r -> 0.
OEXPORT void orc_softmax(const float* x, float* y, int bc, int rows, int cols, int type, int masked) {
  if (type == 0) {
#pragma omp parallel for schedule(static)
    for (long long line = 0; line < (long long)bc * rows; ++line) {
      const int r = (int)(line % rows);
      const float* xr = x + line * cols;
      float* yr = y + line * cols;
      float m = -FLT_MAX;
      for (int c = 0; c < cols; ++c) m = fmaxf(m, xr[c]);
      for (int c = 0; c < cols; ++c) yr[c] = (masked && c > r) ? 0.0f : expf(xr[c] - m);
      double acc = 0.0;
      for (int c = 0; c < cols; ++c) acc += yr[c];
      float sum = (float)acc;
      if (sum < 1e-45f) sum = 1.0f;
      for (int c = 0; c < cols; ++c) yr[c] /= sum;
    }
  } else {
#pragma omp parallel for schedule(static)
    for (long long line = 0; line < (long long)bc * cols; ++line) {
      const long long bcI = line / cols;
      const int c = (int)(line % cols);
      const float* xb = x + bcI * rows * cols;
      float* yb = y + bcI * rows * cols;
      float m = -FLT_MAX;
      for (int r = 0; r < rows; ++r) m = fmaxf(m, xb[(long long)r * cols + c]);
      double acc = 0.0;
      for (int r = 0; r < rows; ++r) {
        const float e = (masked && c > r) ? 0.0f : expf(xb[(long long)r * cols + c] - m);
        yb[(long long)r * cols + c] = e;
        acc += e;
      }
      float sum = (float)acc;
      if (sum < 1e-45f) sum = 1.0f;
      for (int r = 0; r < rows; ++r) yb[(long long)r * cols + c] /= sum;
    }
  }
}

// deriv_softmax (Engine/kernels.cu:2149-2181): dx += y (dy - <dy, y>).
OEXPORT void orc_softmax_bwd(const float* y, const float* dy, float* dx, int bc, int rows, int cols, int type) {
  if (type == 0) {
#pragma omp parallel for schedule(static)
    for (long long line = 0; line < (long long)bc * rows; ++line) {
      const long long o = line * cols;
      double dot = 0.0;
      for (int c = 0; c < cols; ++c) dot += (double)dy[o + c] * (double)y[o + c];
      const float d = (float)dot;
      for (int c = 0; c < cols; ++c) dx[o + c] += y[o + c] * (dy[o + c] - d);
    }
  } else {
#pragma omp parallel for schedule(static)
    for (long long line = 0; line < (long long)bc * cols; ++line) {
      const long long base = (line / cols) * rows * cols;
      const int c = (int)(line % cols);
      double dot = 0.0;
      for (int r = 0; r < rows; ++r) dot += (double)dy[base + (long long)r * cols + c] * (double)y[base + (long long)r * cols + c];
      const float d = (float)dot;
      for (int r = 0; r < rows; ++r) {
        const long long o = base + (long long)r * cols + c;
        dx[o] += y[o] * (dy[o] - d);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Normalisation.  Group g covers N = (channels/groups)*hw contiguous floats;
// groups == 1 is LayerNorm (LayerMean/LayerStd/LNorm, Engine/kernels.cu:541-572,
// 670-699, 794-804), groups > 1 GroupNorm (GroupMean/GroupStd/GNorm,
// Engine/kernels.cu:607-639, 732-763, 818-834).  stats[2g] = mean,
// stats[2g+1] = sum (x - mean)^2.  gamma = 1, beta = 0, eps as passed.
OEXPORT void orc_norm_fwd(const float* x, float* y, float* stats, int batch, int channels, long long hw, int groups,
                          float eps) {
  const long long N = (long long)(channels / groups) * hw;
#pragma omp parallel for schedule(static)
  for (int g = 0; g < batch * groups; ++g) {
    const float* xg = x + (long long)g * N;
    float* yg = y + (long long)g * N;
    double s = 0.0;
    for (long long i = 0; i < N; ++i) s += xg[i];
    const float mean = (float)(s / (double)N);
    double ss = 0.0;
    for (long long i = 0; i < N; ++i) {
      const float d = xg[i] - mean;
      ss += (double)d * (double)d;
    }
    const float ssd = (float)ss;
    const float r = 1.0f / sqrtf((1.0f / (float)N) * ssd + eps);
    for (long long i = 0; i < N; ++i) yg[i] = (xg[i] - mean) * r;
    stats[2 * g] = mean;
    stats[2 * g + 1] = ssd;
  }
}

// LayerBackward / GroupBackward (Engine/kernels.cu:849-896) after ggamma =
// dy (gamma = 1), ggammanode = dy*y and their per-group sums
// (Engine/engine.cu:3116-3130, 3262-3276).  reference_layout reproduces
// LayerBackward's `idx >= batch*row*col` guard for channels > 1.
OEXPORT void orc_norm_bwd(const float* y, const float* dy, float* dx, const float* stats, int batch, int channels,
                          long long hw, int groups, float eps, int reference_layout) {
  const long long N = (long long)(channels / groups) * hw;
  const int G = batch * groups;
  std::vector<float> sg(G), sgy(G);
#pragma omp parallel for schedule(static)
  for (int g = 0; g < G; ++g) {
    double a = 0.0, b = 0.0;
    for (long long i = 0; i < N; ++i) {
      const long long o = (long long)g * N + i;
      a += dy[o];
      b += (double)(dy[o] * y[o]);
    }
    sg[g] = (float)a;
    sgy[g] = (float)b;
  }
  const bool quirk = reference_layout && groups == 1 && channels > 1;
  const long long total = quirk ? (long long)batch * hw : (long long)G * N;
  const float fN = (float)N;
#pragma omp parallel for schedule(static)
  for (long long idx = 0; idx < total; ++idx) {
    const int g = quirk ? (int)(idx / hw) : (int)(idx / N);
    const float r = 1.0f / sqrtf(stats[2 * g + 1] / fN + eps);
    dx[idx] += r * (dy[idx] - (sg[g] / fN) - y[idx] * (sgy[g] / fN));
  }
}

// ---------------------------------------------------------------------------
// Convolution (NCHW, OIHW).
// Convolute2D as GEMMs over gathered operands (implicit im2col).  Each sum
// runs over the same index order as the direct 7-loop form below it (the
// *_naive functions, kept to pin this one bit for bit): an out-of-image tap
// enters as a 0 product, which leaves a nonzero double sum unchanged and keeps
// a zero sum +0.
// CV2D (Engine/kernels.cu:985-1019): y[n, co, p] = sum_{ci, kh, kw} x w + b[co].
OEXPORT void orc_conv_fwd(const float* x, const float* w, const float* bias, float* y, int N, int Cin, int H, int W,
                          int Cout, int KH, int KW, int pad, int stride) {
  const int OH = (2 * pad + H - KH) / stride + 1, OW = (2 * pad + W - KW) / stride + 1;
  const long long P = (long long)OH * OW, K = (long long)Cin * KH * KW;
  packed_gemm(
      Cout, K, (long long)N * P, [&](long long co, long long k) { return w[co * K + k]; },
      [&](long long k, long long c) {
        const long long n = c / P, pix = c % P;
        const int ci = (int)(k / (KH * KW)), kh = (int)(k / KW % KH), kw = (int)(k % KW);
        const int iy = (int)(pix / OW) * stride - pad + kh, ix = (int)(pix % OW) * stride - pad + kw;
        if (iy < 0 || iy >= H || ix < 0 || ix >= W) return 0.0f;
        return x[((n * Cin + ci) * H + iy) * W + ix];
      },
      [&](long long co, long long c, double acc) {
        const long long n = c / P, pix = c % P;
        const float sv = (float)acc;
        y[(n * Cout + co) * P + pix] = bias ? sv + bias[co] : sv;
      });
}

// CV2D_GradInput (Engine/kernels.cu:1053-1089): dx[n, ci, q] += sum_{co, kh, kw} dy w.
OEXPORT void orc_conv_dgrad(const float* dy, const float* w, float* dx, int N, int Cin, int H, int W, int Cout, int KH,
                            int KW, int pad, int stride) {
  const int OH = (2 * pad + H - KH) / stride + 1, OW = (2 * pad + W - KW) / stride + 1;
  const long long HW = (long long)H * W, KK = (long long)KH * KW;
  packed_gemm(
      Cin, (long long)Cout * KK, (long long)N * HW,
      [&](long long ci, long long k) { return w[((k / KK) * Cin + ci) * KK + k % KK]; },
      [&](long long k, long long c) {
        const long long n = c / HW, q = c % HW;
        const int oc = (int)(k / KK), kh = (int)(k / KW % KH), kw = (int)(k % KW);
        const int nr = (int)(q / W) + pad - kh, nc = (int)(q % W) + pad - kw;
        if (nr < 0 || nr % stride != 0 || nc < 0 || nc % stride != 0) return 0.0f;
        const int oy = nr / stride, ox = nc / stride;
        if (oy >= OH || ox >= OW) return 0.0f;
        return dy[((n * Cout + oc) * OH + oy) * OW + ox];
      },
      [&](long long ci, long long c, double acc) { dx[(c / HW * Cin + ci) * HW + c % HW] += (float)acc; });
}

// GV2D (Engine/kernels.cu:1021-1051): dw[co, (ci, kh, kw)] = sum_{n, oy, ox} x dy (assign).
OEXPORT void orc_conv_wgrad(const float* x, const float* dy, float* dw, int N, int Cin, int H, int W, int Cout, int KH,
                            int KW, int pad, int stride) {
  const int OH = (2 * pad + H - KH) / stride + 1, OW = (2 * pad + W - KW) / stride + 1;
  const long long P = (long long)OH * OW, KK = (long long)KH * KW;
  packed_gemm(
      Cout, (long long)N * P, (long long)Cin * KK,
      [&](long long co, long long k) { return dy[(k / P * Cout + co) * P + k % P]; },
      [&](long long k, long long c) {
        const long long n = k / P, pix = k % P;
        const int ci = (int)(c / KK), kh = (int)(c / KW % KH), kw = (int)(c % KW);
        const int iy = (int)(pix / OW) * stride - pad + kh, ix = (int)(pix % OW) * stride - pad + kw;
        if (iy < 0 || iy >= H || ix < 0 || ix >= W) return 0.0f;
        return x[((n * Cin + ci) * H + iy) * W + ix];
      },
      [&](long long co, long long c, double acc) { dw[co * Cin * KK + c] = (float)acc; });
}

// CV2D (Engine/kernels.cu:985-1019)
OEXPORT void orc_conv_fwd_naive(const float* x, const float* w, const float* bias, float* y, int N, int Cin, int H, int W,
                          int Cout, int KH, int KW, int pad, int stride) {
  const int OH = (2 * pad + H - KH) / stride + 1, OW = (2 * pad + W - KW) / stride + 1;
#pragma omp parallel for collapse(2) schedule(static)
  for (int n = 0; n < N; ++n)
    for (int co = 0; co < Cout; ++co)
      for (int oy = 0; oy < OH; ++oy)
        for (int ox = 0; ox < OW; ++ox) {
          double acc = 0.0;
          for (int ci = 0; ci < Cin; ++ci)
            for (int kh = 0; kh < KH; ++kh)
              for (int kw = 0; kw < KW; ++kw) {
                const int iy = oy * stride - pad + kh, ix = ox * stride - pad + kw;
                if (iy < 0 || iy >= H || ix < 0 || ix >= W) continue;
                acc += (double)x[(((long long)n * Cin + ci) * H + iy) * W + ix] *
                       (double)w[(((long long)co * Cin + ci) * KH + kh) * KW + kw];
              }
          const float s = (float)acc;
          y[(((long long)n * Cout + co) * OH + oy) * OW + ox] = bias ? s + bias[co] : s;
        }
}

// CV2D_GradInput (Engine/kernels.cu:1053-1089): dX += ...
OEXPORT void orc_conv_dgrad_naive(const float* dy, const float* w, float* dx, int N, int Cin, int H, int W, int Cout, int KH,
                            int KW, int pad, int stride) {
  const int OH = (2 * pad + H - KH) / stride + 1, OW = (2 * pad + W - KW) / stride + 1;
#pragma omp parallel for collapse(2) schedule(static)
  for (int n = 0; n < N; ++n)
    for (int ic = 0; ic < Cin; ++ic)
      for (int ih = 0; ih < H; ++ih)
        for (int iw = 0; iw < W; ++iw) {
          double acc = 0.0;
          for (int oc = 0; oc < Cout; ++oc)
            for (int kh = 0; kh < KH; ++kh) {
              const int nr = ih + pad - kh;
              if (nr < 0 || nr % stride != 0) continue;
              const int oy = nr / stride;
              if (oy >= OH) continue;
              for (int kw = 0; kw < KW; ++kw) {
                const int nc = iw + pad - kw;
                if (nc < 0 || nc % stride != 0) continue;
                const int ox = nc / stride;
                if (ox >= OW) continue;
                acc += (double)dy[(((long long)n * Cout + oc) * OH + oy) * OW + ox] *
                       (double)w[(((long long)oc * Cin + ic) * KH + kh) * KW + kw];
              }
            }
          dx[(((long long)n * Cin + ic) * H + ih) * W + iw] += (float)acc;
        }
}

// GV2D (Engine/kernels.cu:1021-1051): dK = ... (assign)
OEXPORT void orc_conv_wgrad_naive(const float* x, const float* dy, float* dw, int N, int Cin, int H, int W, int Cout, int KH,
                            int KW, int pad, int stride) {
  const int OH = (2 * pad + H - KH) / stride + 1, OW = (2 * pad + W - KW) / stride + 1;
#pragma omp parallel for collapse(2) schedule(static)
  for (int co = 0; co < Cout; ++co)
    for (int ci = 0; ci < Cin; ++ci)
      for (int kh = 0; kh < KH; ++kh)
        for (int kw = 0; kw < KW; ++kw) {
          double acc = 0.0;
          for (int n = 0; n < N; ++n)
            for (int oy = 0; oy < OH; ++oy)
              for (int ox = 0; ox < OW; ++ox) {
                const int iy = oy * stride - pad + kh, ix = ox * stride - pad + kw;
                if (iy < 0 || iy >= H || ix < 0 || ix >= W) continue;
                acc += (double)x[(((long long)n * Cin + ci) * H + iy) * W + ix] *
                       (double)dy[(((long long)n * Cout + co) * OH + oy) * OW + ox];
              }
          dw[(((long long)co * Cin + ci) * KH + kh) * KW + kw] = (float)acc;
        }
}

// ---------------------------------------------------------------------------
// Losses.
// scalar_mse_kernel (Engine/kernels.cu:1808-1816): sum (t - x)^2 / n.
OEXPORT float orc_mse_loss(const float* x, const float* t, long long n) {
  double acc = 0.0;
#pragma omp parallel for reduction(+ : acc) schedule(static)
  for (long long i = 0; i < n; ++i) {
    const double d = (double)t[i] - (double)x[i];
    acc += d * d;
  }
  return (float)(acc / (double)n);
}
// deriv_mse_kernel (Engine/kernels.cu:1838-1848), full == false.
OEXPORT void orc_mse_bwd(const float* x, const float* t, const float* up, float* dx, long long n) {
  const float fn = (float)n;
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) {
    if (up) dx[i] += (2.0f * (x[i] - t[i]) * up[0]) / fn;
    else dx[i] += 2.0f * (x[i] - t[i]) / fn;
  }
}
// SoftMaxCrossEntropy forward (Engine/engine.cu:2088-2100): row softmax, then
// scalar_ce_kernel (Engine/kernels.cu:1818-1826).
OEXPORT float orc_softmax_xent_fwd(const float* logits, const float* target, float* probs, int rows, int cols) {
  orc_softmax(logits, probs, 1, rows, cols, 0, 0);
  const long long n = (long long)rows * cols;
  double acc = 0.0;
#pragma omp parallel for reduction(+ : acc) schedule(static)
  for (long long i = 0; i < n; ++i) acc += -(double)target[i] * log((double)probs[i] + 1e-27);
  return (float)(acc / (double)n);
}
// SoftMaxCrossEntropy backward (Engine/engine.cu:2104-2110): ScaleAdd(-1),
// optional ScalePtr(upstream), ScaleValue(/batch).  Assigns.
OEXPORT void orc_softmax_xent_bwd(const float* probs, const float* target, const float* up, float* dl, long long n,
                                  int batch) {
  const float fb = (float)batch;
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) {
    float g = probs[i] + (-1.0f) * target[i];
    if (up) g *= up[0];
    dl[i] = g / fb;
  }
}

// ---------------------------------------------------------------------------
// Optimizer.
// SumSquared (Engine/kernels.cu:1486-1506): *scale += sum (double)g^2.
OEXPORT void orc_sumsq(const float* g, long long n, double* accum) {
  long double acc = 0.0L;  // order-independent at double precision
  for (long long i = 0; i < n; ++i) acc += (long double)((double)g[i] * (double)g[i]);
  *accum += (double)acc;
}
// Sqrt_Scale type 0 (Engine/kernels.cu:1763-1773).
OEXPORT void orc_sqrt_scale(double* x, double scale) {
  if (x[0] == x[0]) {
    const double cur = sqrt(x[0]);
    x[0] = (cur > 1.0) ? cur * scale : scale;
  }
}
// SP type 1 via ScalePtr (Includes/kernels.h:293-300): g /= (float)s.
OEXPORT void orc_clip(float* g, long long n, const double* s) {
  const float f = (float)s[0];
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) g[i] /= f;
}
// AdamUpdate / AdamWUpdate (Engine/kernels.cu:1508-1534).
OEXPORT void orc_adam(float* out, const float* grad, long long n, int t, float* m, float* v, float b1, float b2,
                      float eps, float lambda, float lr, int adamw) {
  const double c1 = adamw ? (1.0 - pow((double)b1, (double)t)) : (1.0 - (double)powf(b1, (float)t));
  const double c2 = adamw ? (1.0 - pow((double)b2, (double)t)) : (1.0 - (double)powf(b2, (float)t));
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) {
    const float g = grad[i];
    m[i] = (float)((double)(b1 * m[i]) + (1.0 - (double)b1) * (double)g);
    v[i] = (float)((double)(b2 * v[i]) + ((1.0 - (double)b2) * (double)g) * (double)g);
    const float m_hat = (float)((double)m[i] / c1);
    const float v_hat = (float)((double)v[i] / c2);
    const float vs = sqrtf(v_hat);
    if (adamw) out[i] -= lr * ((m_hat / (vs + eps)) + lambda * out[i]);
    else out[i] -= lr * m_hat / (vs + eps);
  }
}

// ---------------------------------------------------------------------------
// Integer / index paths.
// GatherEmbeddings (Engine/kernels.cu:2279-2296)
OEXPORT void orc_gather(float* out, const float* table, const int32_t* keys, int batch, int c, int max_c, int dim) {
  const long long total = (long long)batch * c * dim;
#pragma omp parallel for schedule(static)
  for (long long g = 0; g < total; ++g) {
    const long long b = g / ((long long)c * dim), kr = g % ((long long)c * dim);
    const long long tok = kr / dim, d = kr % dim;
    const int key = keys[b * max_c + tok];
    out[g] = (key == INT_MIN || key < 0) ? 0.0f : table[(long long)key * dim + d];
  }
}
// KeyUpdate (Engine/kernels.cu:1536-1549) applied serially in token order
// (the reference races on repeated keys): table[key] += scale * grad[token].
// Keys >= vocab are skipped (the reference would write out of bounds).
OEXPORT void orc_scatter_add(float* table, const float* grad, const int32_t* keys, int batch, int c, int max_c,
                             int dim, int vocab, float scale) {
  for (int b = 0; b < batch; ++b)
    for (int s = 0; s < c; ++s) {
      const int key = keys[(long long)b * max_c + s];
      if (key == INT_MIN || key < 0 || key >= vocab) continue;
      const float* gr = grad + ((long long)b * c + s) * dim;
      float* tr = table + (long long)key * dim;
      for (int d = 0; d < dim; ++d) tr[d] += scale * gr[d];
    }
}
// OneHotEmbeddings (Engine/kernels.cu:1551-1560); out must be zeroed.
OEXPORT void orc_onehot(float* out, const int32_t* keys, int batch, int clen, int max_clen, int vocab) {
  for (long long g = 0; g < (long long)batch * clen; ++g) {
    const long long row = g / clen, col = g % clen;
    const int key = keys[row * max_clen + col];
    if (key == INT_MIN || key < 0 || key >= vocab) continue;
    out[g * vocab + key] = 1.0f;
  }
}
// ArgMax (Engine/kernels.cu:2353-2366), per row.
OEXPORT void orc_argmax(const float* x, int rows, int cols, int32_t* out) {
  for (int r = 0; r < rows; ++r) {
    const float* a = x + (long long)r * cols;
    int mi = 0;
    float mv = a[0];
    for (int i = 1; i < cols; ++i)
      if (a[i] > mv) {
        mv = a[i];
        mi = i;
      }
    out[r] = mi;
  }
}

// ---------------------------------------------------------------------------
// RMSNorm (Engine/engine.cu:2613-2648): a copy of x, then SumSquaredSqrtCols
// (type 0, per row over the columns) or SumSquaredSqrtRows (type 1, per column
// over the rows) (Engine/kernels.cu:2246-2277), then Scale_arr divide
// (Engine/kernels.cu:2058-2071).  No 1/N and no epsilon: an L2 normalisation.
// norms[line] = sqrtf(sum x^2).
OEXPORT void orc_rmsnorm_fwd(const float* x, float* y, float* norms, int bc, int rows, int cols, int type) {
  const long long lines = type == 0 ? (long long)bc * rows : (long long)bc * cols;
  const int len = type == 0 ? cols : rows;
#pragma omp parallel for schedule(static)
  for (long long line = 0; line < lines; ++line) {
    long long base, step;
    if (type == 0) {
      base = line * cols;
      step = 1;
    } else {
      base = (line / cols) * (long long)rows * cols + line % cols;
      step = cols;
    }
    double s = 0.0;
    for (int i = 0; i < len; ++i) {
      const float v = x[base + i * step];
      s += (double)v * (double)v;
    }
    const float n = sqrtf((float)s);
    norms[line] = n;
    for (int i = 0; i < len; ++i) y[base + i * step] = x[base + i * step] / n;
  }
}

// Accumulate_rmsnorm_kernel (Engine/kernels.cu:2073-2105):
// dx += (dy - y * <dy, y>) / norm along the same axis.
OEXPORT void orc_rmsnorm_bwd(const float* y, const float* dy, const float* norms, float* dx, int bc, int rows, int cols,
                             int type) {
  const long long lines = type == 0 ? (long long)bc * rows : (long long)bc * cols;
  const int len = type == 0 ? cols : rows;
#pragma omp parallel for schedule(static)
  for (long long line = 0; line < lines; ++line) {
    long long base, step;
    if (type == 0) {
      base = line * cols;
      step = 1;
    } else {
      base = (line / cols) * (long long)rows * cols + line % cols;
      step = cols;
    }
    double dot = 0.0;
    for (int i = 0; i < len; ++i) dot += (double)dy[base + i * step] * (double)y[base + i * step];
    const float d = (float)dot, inv = 1.0f / norms[line];
    for (int i = 0; i < len; ++i) {
      const long long o = base + i * step;
      dx[o] += (dy[o] - y[o] * d) * inv;
    }
  }
}

// BatchNorm (Engine/engine.cu:3148-3210): per channel over (batch, H, W) --
// BatchMean / BatchStd / BNorm (Engine/kernels.cu:574-604, 701-730, 806-816),
// gamma 1, beta 0.  stats[2c] = mean, stats[2c+1] = sum (x - mean)^2.
OEXPORT void orc_batchnorm_fwd(const float* x, float* y, float* stats, int batch, int channels, long long hw,
                               float eps) {
  const long long N = (long long)batch * hw;
#pragma omp parallel for schedule(static)
  for (int c = 0; c < channels; ++c) {
    double s = 0.0;
    for (int b = 0; b < batch; ++b)
      for (long long i = 0; i < hw; ++i) s += x[((long long)b * channels + c) * hw + i];
    const float mean = (float)(s / (double)N);
    double ss = 0.0;
    for (int b = 0; b < batch; ++b)
      for (long long i = 0; i < hw; ++i) {
        const float d = x[((long long)b * channels + c) * hw + i] - mean;
        ss += (double)d * (double)d;
      }
    const float ssd = (float)ss;
    const float r = 1.0f / sqrtf((1.0f / (float)N) * ssd + eps);
    for (int b = 0; b < batch; ++b)
      for (long long i = 0; i < hw; ++i) {
        const long long o = ((long long)b * channels + c) * hw + i;
        y[o] = (x[o] - mean) * r;
      }
    stats[2 * c] = mean;
    stats[2 * c + 1] = ssd;
  }
}

// BatchBackward (Engine/kernels.cu:864-876) after the per-channel sums of
// ggamma = dy and ggammanode = dy * y (Engine/engine.cu:3185-3194).
OEXPORT void orc_batchnorm_bwd(const float* y, const float* dy, float* dx, const float* stats, int batch, int channels,
                               long long hw, float eps) {
  const long long N = (long long)batch * hw;
  const float fN = (float)N;
#pragma omp parallel for schedule(static)
  for (int c = 0; c < channels; ++c) {
    double a = 0.0, b2 = 0.0;
    for (int b = 0; b < batch; ++b)
      for (long long i = 0; i < hw; ++i) {
        const long long o = ((long long)b * channels + c) * hw + i;
        a += dy[o];
        b2 += (double)(dy[o] * y[o]);
      }
    const float sg = (float)a, sgy = (float)b2;
    const float r = 1.0f / sqrtf(stats[2 * c + 1] / fN + eps);
    for (int b = 0; b < batch; ++b)
      for (long long i = 0; i < hw; ++i) {
        const long long o = ((long long)b * channels + c) * hw + i;
        dx[o] += r * (dy[o] - (sg / fN) - y[o] * (sgy / fN));
      }
  }
}

// CopyCrop (Engine/engine.cu:2855-2920) for the cropping case h1 >= h, w1 >= w:
// CopynCrop centres x1's (h1, w1) window on (h, w) (Engine/kernels.cu:1330-1348),
// then Channel_Concat puts its c1 channels before x2's c2 (Engine/kernels.cu:1408-1419).
OEXPORT void orc_copy_crop_fwd(const float* x1, const float* x2, float* y, int batch, int c1, int h1, int w1, int c2,
                               int h, int w) {
  const int dr = (h1 - h) / 2, dc = (w1 - w) / 2;
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < batch; ++b)
    for (int ch = 0; ch < c1 + c2; ++ch)
      for (int r = 0; r < h; ++r)
        for (int c = 0; c < w; ++c) {
          const long long o = (((long long)b * (c1 + c2) + ch) * h + r) * w + c;
          y[o] = ch < c1 ? x1[(((long long)b * c1 + ch) * h1 + r + dr) * w1 + c + dc]
                         : x2[(((long long)b * c2 + ch - c1) * h + r) * w + c];
        }
}

// CopyCrop backward: Channel_Split (Engine/kernels.cu:1421-1433) into a
// (c1, h, w) temporary and x2's gradient, then PaddingCrop adds the temporary
// back into x1's gradient at the centred window (Engine/kernels.cu:1350-1369).
OEXPORT void orc_copy_crop_bwd(const float* dy, float* dx1, float* dx2, int batch, int c1, int h1, int w1, int c2, int h,
                               int w) {
  const int dr = (h1 - h) / 2, dc = (w1 - w) / 2;
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < batch; ++b)
    for (int ch = 0; ch < c1 + c2; ++ch)
      for (int r = 0; r < h; ++r)
        for (int c = 0; c < w; ++c) {
          const float g = dy[(((long long)b * (c1 + c2) + ch) * h + r) * w + c];
          if (ch < c1) dx1[(((long long)b * c1 + ch) * h1 + r + dr) * w1 + c + dc] += g;
          else dx2[(((long long)b * c2 + ch - c1) * h + r) * w + c] += g;
        }
}

// Transposed convolution, weights [out][inp][kh][kw] (Includes/engine.h:257-280).
// CVT2D (Engine/kernels.cu:1091-1135): out_h = (H - 1) * stride - 2 pad + kh.
OEXPORT void orc_convT_fwd(const float* x, const float* w, const float* bias, float* y, int N, int Cin, int H, int W,
                           int Cout, int KH, int KW, int pad, int stride) {
  const int OH = (H - 1) * stride - 2 * pad + KH, OW = (W - 1) * stride - 2 * pad + KW;
#pragma omp parallel for collapse(2) schedule(static)
  for (int n = 0; n < N; ++n)
    for (int oc = 0; oc < Cout; ++oc)
      for (int row = 0; row < OH; ++row)
        for (int col = 0; col < OW; ++col) {
          double acc = 0.0;
          for (int ic = 0; ic < Cin; ++ic)
            for (int kh = 0; kh < KH; ++kh)
              for (int kw = 0; kw < KW; ++kw) {
                int ir = row + pad - kh, icl = col + pad - kw;
                if (ir % stride != 0 || icl % stride != 0) continue;
                ir /= stride;
                icl /= stride;
                if (ir < 0 || ir >= H || icl < 0 || icl >= W) continue;
                acc += (double)x[(((long long)n * Cin + ic) * H + ir) * W + icl] *
                       (double)w[(((long long)oc * Cin + ic) * KH + kh) * KW + kw];
              }
          const float s = (float)acc;
          y[(((long long)n * Cout + oc) * OH + row) * OW + col] = bias ? s + bias[oc] : s;
        }
}

// CVT2D_GradInput (Engine/kernels.cu:1178-1212): dx = ... (assign).
OEXPORT void orc_convT_dgrad(const float* dy, const float* w, float* dx, int N, int Cin, int H, int W, int Cout, int KH,
                             int KW, int pad, int stride) {
  const int OH = (H - 1) * stride - 2 * pad + KH, OW = (W - 1) * stride - 2 * pad + KW;
#pragma omp parallel for collapse(2) schedule(static)
  for (int n = 0; n < N; ++n)
    for (int ic = 0; ic < Cin; ++ic)
      for (int row = 0; row < H; ++row)
        for (int col = 0; col < W; ++col) {
          double acc = 0.0;
          for (int oc = 0; oc < Cout; ++oc)
            for (int kh = 0; kh < KH; ++kh)
              for (int kw = 0; kw < KW; ++kw) {
                const int orow = row * stride - pad + kh, ocol = col * stride - pad + kw;
                if (orow < 0 || orow >= OH || ocol < 0 || ocol >= OW) continue;
                acc += (double)dy[(((long long)n * Cout + oc) * OH + orow) * OW + ocol] *
                       (double)w[(((long long)oc * Cin + ic) * KH + kh) * KW + kw];
              }
          dx[(((long long)n * Cin + ic) * H + row) * W + col] = (float)acc;
        }
}

// GVT2D (Engine/kernels.cu:1137-1176): dW = ... (assign).
OEXPORT void orc_convT_wgrad(const float* x, const float* dy, float* dw, int N, int Cin, int H, int W, int Cout, int KH,
                             int KW, int pad, int stride) {
  const int OH = (H - 1) * stride - 2 * pad + KH, OW = (W - 1) * stride - 2 * pad + KW;
#pragma omp parallel for collapse(2) schedule(static)
  for (int oc = 0; oc < Cout; ++oc)
    for (int ic = 0; ic < Cin; ++ic)
      for (int kh = 0; kh < KH; ++kh)
        for (int kw = 0; kw < KW; ++kw) {
          double acc = 0.0;
          for (int n = 0; n < N; ++n)
            for (int ir = 0; ir < H; ++ir)
              for (int icl = 0; icl < W; ++icl) {
                const int orow = ir * stride - pad + kh, ocol = icl * stride - pad + kw;
                if (orow < 0 || orow >= OH || ocol < 0 || ocol >= OW) continue;
                acc += (double)x[(((long long)n * Cin + ic) * H + ir) * W + icl] *
                       (double)dy[(((long long)n * Cout + oc) * OH + orow) * OW + ocol];
              }
          dw[(((long long)oc * Cin + ic) * KH + kh) * KW + kw] = (float)acc;
        }
}
