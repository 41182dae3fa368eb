// Layout movers for the U-Net ops: CopyCrop's channel concatenation with a
// centred crop (Engine/engine.cu:2855-2920) and the [out][inp] <-> [inp][out]
// weight swap that lets Convolute2DT (Engine/engine.cu:3819-3900) run on the
// convolution kernels.  All HBM-bound gathers: each output element is written
// once by one thread, so no atomics and no ordering questions.
#include "common.hpp"

using namespace mle;

namespace {

constexpr int NT = 256;

struct CropShape {
  int batch, c1, h1, w1, c2, h, w, dr, dc;
};

// y[b][ch][r][c] = ch < c1 ? x1[b][ch][r + dr][c + dc] : x2[b][ch - c1][r][c]
// (CopynCrop then Channel_Concat, Engine/kernels.cu:1330-1348, 1408-1419).
__global__ __launch_bounds__(NT) void copy_crop_fwd_kernel(const float* __restrict__ x1, const float* __restrict__ x2,
                                                           float* __restrict__ y, CropShape s, size_t total) {
  const size_t hw = (size_t)s.h * s.w;
  for (size_t i = (size_t)blockIdx.x * NT + threadIdx.x; i < total; i += (size_t)gridDim.x * NT) {
    const int c = (int)(i % s.w), r = (int)((i / s.w) % s.h);
    const size_t bc = i / hw;
    const int ch = (int)(bc % (s.c1 + s.c2)), b = (int)(bc / (s.c1 + s.c2));
    y[i] = ch < s.c1 ? x1[(((size_t)b * s.c1 + ch) * s.h1 + r + s.dr) * s.w1 + c + s.dc]
                     : x2[(((size_t)b * s.c2 + ch - s.c1) * s.h + r) * s.w + c];
  }
}

// dx1 (+)= dy[:, :c1] at the centred window (zero outside it when assigning);
// dx2 (+)= dy[:, c1:] (Channel_Split then PaddingCrop, Engine/kernels.cu:
// 1421-1433, 1350-1369).  Threads walk dx1's and dx2's elements, so every
// gradient element has one writer.
__global__ __launch_bounds__(NT) void copy_crop_bwd_kernel(const float* __restrict__ dy, float* __restrict__ dx1,
                                                           float* __restrict__ dx2, CropShape s, size_t n1, size_t n2,
                                                           int acc1, int acc2) {
  for (size_t i = (size_t)blockIdx.x * NT + threadIdx.x; i < n1 + n2; i += (size_t)gridDim.x * NT) {
    if (i < n1) {
      const int c = (int)(i % s.w1), r = (int)((i / s.w1) % s.h1);
      const size_t bc = i / ((size_t)s.h1 * s.w1);
      const int ch = (int)(bc % s.c1), b = (int)(bc / s.c1);
      const int rr = r - s.dr, cc = c - s.dc;
      float v = 0.f;
      if (rr >= 0 && rr < s.h && cc >= 0 && cc < s.w) v = dy[(((size_t)b * (s.c1 + s.c2) + ch) * s.h + rr) * s.w + cc];
      dx1[i] = acc1 ? dx1[i] + v : v;
    } else {
      const size_t j = i - n1;
      const size_t hw = (size_t)s.h * s.w;
      const size_t bc = j / hw;
      const int ch = (int)(bc % s.c2), b = (int)(bc / s.c2);
      const float v = dy[((size_t)b * (s.c1 + s.c2) + s.c1 + ch) * hw + j % hw];
      dx2[j] = acc2 ? dx2[j] + v : v;
    }
  }
}

// dst[i][o][k] (+)= src[o][i][k], k < khw.
__global__ __launch_bounds__(NT) void weight_swap_kernel(const float* __restrict__ src, float* __restrict__ dst, int o_n,
                                                         int i_n, int khw, size_t total, int acc) {
  for (size_t e = (size_t)blockIdx.x * NT + threadIdx.x; e < total; e += (size_t)gridDim.x * NT) {
    const int k = (int)(e % khw);
    const size_t oi = e / khw;
    const int o = (int)(oi % o_n), i = (int)(oi / o_n);  // e indexes dst = [i][o][k]
    const float v = src[((size_t)o * i_n + i) * khw + k];
    dst[e] = acc ? dst[e] + v : v;
  }
}

int crop_shape(int batch, int c1, int h1, int w1, int c2, int h, int w, CropShape& s) {
  if (batch <= 0 || c1 <= 0 || c2 <= 0 || h <= 0 || w <= 0 || h1 <= 0 || w1 <= 0)
    return set_error(MLE_ERR_INVALID, "copy_crop: bad shape");
  // The reference's CopynCrop reads outside x1 when x1 is smaller than x2
  // (negative centring offset), so only the cropping direction is defined.
  if (h1 < h || w1 < w)
    return set_error(MLE_ERR_UNSUPPORTED, "copy_crop: x1 (%d x %d) smaller than x2 (%d x %d) is not supported", h1, w1,
                     h, w);
  s = CropShape{batch, c1, h1, w1, c2, h, w, (h1 - h) / 2, (w1 - w) / 2};
  return MLE_OK;
}

}  // namespace

extern "C" {

int mle_copy_crop_fwd(mle_stream stream, const float* x1, const float* x2, float* y, int batch, int c1, int h1, int w1,
                      int c2, int h, int w) {
  MLE_CHECK_ARG(x1 && x2 && y, "mle_copy_crop_fwd: null pointer");
  CropShape s;
  int rc = crop_shape(batch, c1, h1, w1, c2, h, w, s);
  if (rc) return rc;
  const size_t total = (size_t)batch * (c1 + c2) * h * w;
  copy_crop_fwd_kernel<<<stream_grid(total, NT), NT, 0, as_stream(stream)>>>(x1, x2, y, s, total);
  return check_launch("mle_copy_crop_fwd");
}

int mle_copy_crop_bwd(mle_stream stream, const float* dy, float* dx1, float* dx2, int batch, int c1, int h1, int w1,
                      int c2, int h, int w, int accumulate1, int accumulate2) {
  MLE_CHECK_ARG(dy && dx1 && dx2, "mle_copy_crop_bwd: null pointer");
  CropShape s;
  int rc = crop_shape(batch, c1, h1, w1, c2, h, w, s);
  if (rc) return rc;
  const size_t n1 = (size_t)batch * c1 * h1 * w1, n2 = (size_t)batch * c2 * h * w;
  copy_crop_bwd_kernel<<<stream_grid(n1 + n2, NT), NT, 0, as_stream(stream)>>>(dy, dx1, dx2, s, n1, n2, accumulate1,
                                                                               accumulate2);
  return check_launch("mle_copy_crop_bwd");
}

int mle_weight_swap(mle_stream stream, const float* src, float* dst, int o, int i, int khw, int accumulate) {
  MLE_CHECK_ARG(src && dst && src != dst, "mle_weight_swap: null or aliased pointer");
  MLE_CHECK_ARG(o > 0 && i > 0 && khw > 0, "mle_weight_swap: bad shape");
  const size_t total = (size_t)o * i * khw;
  weight_swap_kernel<<<stream_grid(total, NT), NT, 0, as_stream(stream)>>>(src, dst, o, i, khw, total, accumulate);
  return check_launch("mle_weight_swap");
}

}  // extern "C"
