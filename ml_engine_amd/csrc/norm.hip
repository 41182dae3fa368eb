// LayerNorm (whole-sample statistics), GroupNorm / InstanceNorm and BatchNorm
// forward/backward with gamma = 1, beta = 0 (Engine/engine.cu:3080-3347), and
// the reference's RMSNorm (an L2 normalisation along rows or columns,
// Engine/engine.cu:2613-2648).
//
// A group (one batch item for LayerNorm, one (batch, group) for GroupNorm) is
// a contiguous span of N = (C/G)*HW floats in NCHW.  A BatchNorm group is one
// channel across the batch: `batch` segments of HW floats, C*HW apart.  The reference reduces a
// group with a single 512-thread block (LayerMean/LayerStd, GroupMean/GroupStd,
// Engine/kernels.cu:541-763), i.e. 32 blocks for the transformer LayerNorm.
// Here each group is split into chunks of CH floats so every CU gets work:
//   pass 1: per chunk (mean, M2) from registers -> workspace (double)
//   pass 2: each chunk's workgroup combines its group's chunk partials in a
//           fixed order (Chan et al. pairwise update) and normalises.
// The backward uses the same split for sum(dy) and sum(dy*y).
#include "activation.hpp"
#include "common.hpp"

#include <initializer_list>
#include <type_traits>

using namespace mle;

namespace {

constexpr int NT = 256;
constexpr int VPT = 16;          // floats per thread per chunk
constexpr int CH = NT * VPT;     // 4096 floats per chunk

struct NormShape {
  size_t N;        // elements per group
  int nchunk;      // chunks per group
  int groups_tot;  // groups in the launch
  // Segmented groups (SEG kernels): element e of group g sits at
  // g * group_stride + (e / seg) * seg_stride + e % seg.
  uint32_t seg;
  size_t seg_stride, group_stride;
};

// Offset of element e of group g.  Contiguous groups: g * N + e.
template <bool SEG>
__device__ __forceinline__ size_t at(const NormShape& sh, int g, size_t e) {
  if (!SEG) return (size_t)g * sh.N + e;
  const uint32_t e32 = (uint32_t)e;  // N < 2^32 on this path (checked on the host)
  return (size_t)g * sh.group_stride + (size_t)(e32 / sh.seg) * sh.seg_stride + e32 % sh.seg;
}

// Element e of thread slot i in a chunk starting at c0.  VEC: thread t owns
// the float4s t, t + NT, t + 2 NT, t + 3 NT of the chunk (16-byte loads; the
// host checks that N, the segment length and the base are multiples of 4, so
// a float4 never straddles a group or segment end); otherwise floats
// t + i NT.
template <bool VEC>
__device__ __forceinline__ size_t elem(size_t c0, int i) {
  return VEC ? c0 + 4 * (threadIdx.x + (size_t)(i / 4) * NT) + (i % 4) : c0 + threadIdx.x + (size_t)i * NT;
}

template <bool SEG, bool VEC>
__device__ __forceinline__ void load_chunk(const float* __restrict__ src, const NormShape& sh, int g, size_t c0,
                                           float (&v)[VPT]) {
  if (VEC) {
#pragma unroll
    for (int u = 0; u < VPT / 4; ++u) {
      const size_t e = elem<true>(c0, 4 * u);
      f32x4 t = {0.f, 0.f, 0.f, 0.f};
      if (e < sh.N) t = *reinterpret_cast<const f32x4*>(src + at<SEG>(sh, g, e));
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 * u + k] = t[k];
    }
  } else {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const size_t e = elem<false>(c0, i);
      v[i] = (e < sh.N) ? src[at<SEG>(sh, g, e)] : 0.f;
    }
  }
}

// Inverse of load_chunk: the chunk's in-range elements from registers.
template <bool SEG, bool VEC>
__device__ __forceinline__ void store_chunk(float* __restrict__ dst, const NormShape& sh, int g, size_t c0,
                                            const float (&v)[VPT]) {
  if (VEC) {
#pragma unroll
    for (int u = 0; u < VPT / 4; ++u) {
      const size_t e = elem<true>(c0, 4 * u);
      if (e < sh.N)
        *reinterpret_cast<f32x4*>(dst + at<SEG>(sh, g, e)) = f32x4{v[4 * u], v[4 * u + 1], v[4 * u + 2], v[4 * u + 3]};
    }
  } else {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const size_t e = elem<false>(c0, i);
      if (e < sh.N) dst[at<SEG>(sh, g, e)] = v[i];
    }
  }
}

// Pass 1 of the forward: per chunk (mean, M2) in double.
template <bool SEG, bool VEC>
__global__ __launch_bounds__(NT) void norm_stats_partial(const float* __restrict__ x, NormShape sh,
                                                         double* __restrict__ part) {
  __shared__ double red[NT / 64];
  const int g = blockIdx.y, ck = blockIdx.x;
  const size_t c0 = (size_t)ck * CH;
  float v[VPT];
  load_chunk<SEG, VEC>(x, sh, g, c0, v);
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) s += v[i];
  s = block_sum<NT>(s, red);
  const size_t n_c = (sh.N - c0 < (size_t)CH) ? sh.N - c0 : (size_t)CH;
  const double mean = s / (double)n_c;
  double m2 = 0.0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const double d = (double)v[i] - mean;
    if (elem<VEC>(c0, i) < sh.N) m2 += d * d;
  }
  m2 = block_sum<NT>(m2, red);
  if (threadIdx.x == 0) {
    double* p = part + ((size_t)g * sh.nchunk + ck) * 2;
    p[0] = mean;
    p[1] = m2;
  }
}

// Pass 1 fused into the producer of x: y = a + b (b read at i % b_period, a
// broadcast over the groups when b_period < N), stored, then this chunk's
// (mean, M2) exactly as norm_stats_partial computes them from y (same
// element-to-thread map, same double sums and block reduction), so the
// normalisation that follows is bit-identical.  Contiguous groups only.
template <bool VEC>
__global__ __launch_bounds__(NT) void add_stats_partial(const float* __restrict__ a, const float* __restrict__ b,
                                                        size_t b_period, float* __restrict__ y, NormShape sh,
                                                        double* __restrict__ part) {
  __shared__ double red[NT / 64];
  const int g = blockIdx.y, ck = blockIdx.x;
  const size_t c0 = (size_t)ck * CH;
  float v[VPT];
  if (VEC) {
    // Every load of the thread before its first store; FULL chunks without
    // per-lane branches (see norm_apply).
    auto body = [&](auto full) {
      constexpr bool FULL = decltype(full)::value;
      constexpr int U = VPT / 4;
      f32x4 av[U], bv[U];
      size_t o[U], ob[U];
      bool in[U];
      // b's offsets: the thread's float4s are 4 NT floats apart, so with
      // b_period >= 4 NT each step wraps at most once (one division per
      // thread instead of one per float4).
      const bool step = b_period >= (size_t)(4 * NT);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const size_t e = elem<true>(c0, 4 * u);
        in[u] = FULL || e < sh.N;
        o[u] = at<false>(sh, g, e);
        if (u == 0 || !step) {
          ob[u] = o[u] % b_period;
        } else {
          const size_t nb = ob[u - 1] + 4 * NT;
          ob[u] = nb >= b_period ? nb - b_period : nb;
        }
        av[u] = bv[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (!in[u]) continue;
        av[u] = *reinterpret_cast<const f32x4*>(a + o[u]);
        bv[u] = *reinterpret_cast<const f32x4*>(b + ob[u]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const f32x4 t = av[u] + bv[u];
        if (in[u]) *reinterpret_cast<f32x4*>(y + o[u]) = t;
#pragma unroll
        for (int k = 0; k < 4; ++k) v[4 * u + k] = t[k];
      }
    };
    if (c0 + CH <= sh.N) body(std::true_type{});
    else body(std::false_type{});
  } else {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const size_t e = elem<false>(c0, i);
      v[i] = 0.f;
      if (e < sh.N) {
        const size_t o = at<false>(sh, g, e);
        v[i] = a[o] + b[o % b_period];
        y[o] = v[i];
      }
    }
  }
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) s += v[i];
  s = block_sum<NT>(s, red);
  const size_t n_c = (sh.N - c0 < (size_t)CH) ? sh.N - c0 : (size_t)CH;
  const double mean = s / (double)n_c;
  double m2 = 0.0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const double d = (double)v[i] - mean;
    if (elem<VEC>(c0, i) < sh.N) m2 += d * d;
  }
  m2 = block_sum<NT>(m2, red);
  if (threadIdx.x == 0) {
    double* p = part + ((size_t)g * sh.nchunk + ck) * 2;
    p[0] = mean;
    p[1] = m2;
  }
}

// Chunk c's element count.
__device__ __forceinline__ double chunk_n(const NormShape& sh, int c) {
  const size_t c0 = (size_t)c * CH;
  return (double)((sh.N - c0 < (size_t)CH) ? sh.N - c0 : (size_t)CH);
}

// Chan et al. pairwise update: (n, mean, M2) of a followed by b.
__device__ __forceinline__ void chan_merge(double& n, double& mu, double& M, double nb, double mub, double Mb) {
  const double nn = n + nb;
  if (nb == 0.0) return;
  const double d = mub - mu;
  mu += d * (nb / nn);
  M += Mb + d * d * (n * nb / nn);
  n = nn;
}

// Lane l's first chunk partial (chunk l; lanes past the last chunk load an
// in-range one that the merge below skips), loaded without a branch: a
// caller can issue its own loads after it and still wait for it alone.
struct PartPre {
  double a, b;
};
__device__ __forceinline__ PartPre part_pre(const double* __restrict__ part, const NormShape& sh, int g) {
  const int c = min((int)(threadIdx.x & 63), sh.nchunk - 1);
  const double* p = part + ((size_t)g * sh.nchunk + c) * 2;
  return {p[0], p[1]};
}

// The group's (mean, M2) from its chunk partials, computed by every wave of
// the workgroup with the same fixed order: lane l first merges chunks l,
// l + 64, ... in turn, then lanes merge pairwise in a tree (lower lane first).
// `pre` holds chunk l's partial (part_pre).
__device__ __forceinline__ void group_stats_from(const PartPre& pre, const double* __restrict__ part,
                                                 const NormShape& sh, int g, double& mean, double& m2) {
  const int lane = threadIdx.x & 63;
  const double* p = part + (size_t)g * sh.nchunk * 2;
  double n = 0.0, mu = 0.0, M = 0.0;
  if (lane < sh.nchunk) chan_merge(n, mu, M, chunk_n(sh, lane), pre.a, pre.b);
  for (int c = lane + 64; c < sh.nchunk; c += 64) chan_merge(n, mu, M, chunk_n(sh, c), p[2 * c], p[2 * c + 1]);
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const double nb = __shfl_down(n, off, 64), mub = __shfl_down(mu, off, 64), Mb = __shfl_down(M, off, 64);
    if ((lane & (2 * off - 1)) == 0 && lane + off < 64) chan_merge(n, mu, M, nb, mub, Mb);
  }
  mean = __shfl(mu, 0, 64);
  m2 = __shfl(M, 0, 64);
}

// The group's sum(dy) and sum(dy * y), same fixed order.
__device__ __forceinline__ void group_sums_from(const PartPre& pre, const double* __restrict__ part,
                                                const NormShape& sh, int g, double& a, double& b) {
  const int lane = threadIdx.x & 63;
  const double* p = part + (size_t)g * sh.nchunk * 2;
  a = 0.0;
  b = 0.0;
  if (lane < sh.nchunk) {
    a += pre.a;
    b += pre.b;
  }
  for (int c = lane + 64; c < sh.nchunk; c += 64) {
    a += p[2 * c];
    b += p[2 * c + 1];
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const double ab = __shfl_down(a, off, 64), bb = __shfl_down(b, off, 64);
    if ((lane & (2 * off - 1)) == 0 && lane + off < 64) {
      a += ab;
      b += bb;
    }
  }
  a = __shfl(a, 0, 64);
  b = __shfl(b, 0, 64);
}
__device__ __forceinline__ void group_sums(const double* __restrict__ part, const NormShape& sh, int g, double& a,
                                           double& b) {
  group_sums_from(part_pre(part, sh, g), part, sh, g, a, b);
}

// ACT >= 0 (an mle_act_kind): also act_out = act(y), the activation that
// follows the normalisation (same formula as the activation kernels), plus
// cbias[channel] when cbias is set (a broadcast channel add after the
// activation; the channel of element offset o is (o / cb_hw) % cb_ch).
template <bool SEG, bool VEC, int ACT = -1>
__global__ __launch_bounds__(NT) void norm_apply(const float* __restrict__ x, float* __restrict__ y,
                                                 float* __restrict__ stats, NormShape sh, const double* __restrict__ part,
                                                 float eps, float* __restrict__ act_out = nullptr,
                                                 const float* __restrict__ cbias = nullptr, uint32_t cb_hw = 1,
                                                 uint32_t cb_ch = 1) {
  const int g = blockIdx.y, ck = blockIdx.x;
  // The group's partials first, then (VEC) this thread's x, then the merge:
  // the x loads are in flight while the merge runs.
  const PartPre pre = part_pre(part, sh, g);
  float mean = 0.f, r = 0.f;
  auto finish_stats = [&]() {
    double mean_d, m2_d;
    group_stats_from(pre, part, sh, g, mean_d, m2_d);
    mean = (float)mean_d;
    const float ssd = (float)m2_d;
    r = rsqrtf((1.0f / (float)sh.N) * ssd + eps);  // LNorm/GNorm (Engine/kernels.cu:794-834)
    if (ck == 0 && threadIdx.x == 0) {
      stats[2 * g] = mean;
      stats[2 * g + 1] = ssd;
    }
  };
  const size_t c0 = (size_t)ck * CH;
  if (VEC) {
    // Every load of the thread before its first store: the vector memory
    // counter counts stores too, so a load issued after a store would make
    // its wait cover that store.  A chunk wholly inside the group (FULL, the
    // same for the whole block) loads and stores without per-lane branches,
    // which lets each wait name just the load it needs.
    auto body = [&](auto full) {
      constexpr bool FULL = decltype(full)::value;
      constexpr int U = VPT / 4;
      f32x4 xv[U];
      size_t o[U];
      bool in[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const size_t e = elem<true>(c0, 4 * u);
        in[u] = FULL || e < sh.N;
        o[u] = in[u] ? at<SEG>(sh, g, e) : 0;
        if (in[u]) xv[u] = *reinterpret_cast<const f32x4*>(x + o[u]);
      }
      finish_stats();
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (!in[u]) continue;
        f32x4 yv;
#pragma unroll
        for (int k = 0; k < 4; ++k) yv[k] = (xv[u][k] - mean) * r;
        *reinterpret_cast<f32x4*>(y + o[u]) = yv;
        if (ACT >= 0) {
          f32x4 av;
#pragma unroll
          for (int k = 0; k < 4; ++k) av[k] = act_f<ACT < 0 ? 0 : ACT>(yv[k]);
          if (cbias) {  // a float4 never straddles a channel (the host checks cb_hw % 4 == 0)
            const float cb = cbias[(o[u] / cb_hw) % cb_ch];
#pragma unroll
            for (int k = 0; k < 4; ++k) av[k] = av[k] + cb;
          }
          *reinterpret_cast<f32x4*>(act_out + o[u]) = av;
        }
      }
    };
    if (c0 + CH <= sh.N) body(std::true_type{});
    else body(std::false_type{});
  } else {
    finish_stats();
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const size_t e = elem<false>(c0, i);
      if (e < sh.N) {
        const size_t o = at<SEG>(sh, g, e);
        const float yo = (x[o] - mean) * r;
        y[o] = yo;
        if (ACT >= 0) {
          const float av = act_f<ACT < 0 ? 0 : ACT>(yo);
          act_out[o] = cbias ? av + cbias[(o / cb_hw) % cb_ch] : av;
        }
      }
    }
  }
}

// Backward pass 1: per chunk sum(dy) and sum(dy * y) in double.  ACT >= 0:
// dy is first formed from the gradient `da` of the activation that follows
// the normalisation, dy (+)= act'(y) * da (acc_dy 1 adds to the stored dy),
// exactly as the activation's backward kernel forms it, and stored.
template <bool SEG, bool VEC, int ACT = -1>
__global__ __launch_bounds__(NT) void norm_bwd_partial(const float* __restrict__ y, const float* __restrict__ dy,
                                                       NormShape sh, double* __restrict__ part,
                                                       const float* __restrict__ da = nullptr,
                                                       float* __restrict__ dy_out = nullptr, int acc_dy = 0) {
  __shared__ double red[NT / 64];
  const int g = blockIdx.y, ck = blockIdx.x;
  const size_t c0 = (size_t)ck * CH;
  float yv[VPT], gv[VPT];
  load_chunk<SEG, VEC>(y, sh, g, c0, yv);
  if (ACT >= 0) {
    float av[VPT];
    load_chunk<SEG, VEC>(da, sh, g, c0, av);
    if (acc_dy) load_chunk<SEG, VEC>(dy_out, sh, g, c0, gv);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      // product rounded, then the add (no fma): the activation kernel's steps
#pragma clang fp contract(off)
      const float v = act_df<ACT < 0 ? 0 : ACT>(yv[i]) * av[i];
      gv[i] = acc_dy ? gv[i] + v : v;
    }
    store_chunk<SEG, VEC>(dy_out, sh, g, c0, gv);
  } else {
    load_chunk<SEG, VEC>(dy, sh, g, c0, gv);
  }
  double sg = 0.0, sgy = 0.0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    sg += gv[i];
    sgy += (double)(gv[i] * yv[i]);
  }
  sg = block_sum<NT>(sg, red);
  sgy = block_sum<NT>(sgy, red);
  if (threadIdx.x == 0) {
    double* p = part + ((size_t)g * sh.nchunk + ck) * 2;
    p[0] = sg;
    p[1] = sgy;
  }
}

// Per group, once (the LayerNorm layout quirk reads other groups' sums per
// element): fin[2g] = sum(dy), fin[2g+1] = sum(dy * y), same order as group_sums.
__global__ __launch_bounds__(64) void norm_bwd_final(const double* __restrict__ part, NormShape sh,
                                                     double* __restrict__ fin) {
  double a, b;
  group_sums(part, sh, blockIdx.x, a, b);
  if (threadIdx.x == 0) {
    fin[2 * blockIdx.x] = a;
    fin[2 * blockIdx.x + 1] = b;
  }
}

// dx (+)= r (dy - sum(dy)/N - y sum(dy*y)/N)  (LayerBackward/GroupBackward,
// Engine/kernels.cu:849-896); acc = 0 assigns.  dx2 and dx3, when set, then
// receive dx's new value (acc2, acc3 each: add or assign): the gradients of
// the two inputs of the Add that produced the normalised tensor, whose
// backward (Engine/engine.cu:1650-1672) adds its whole output gradient -- dx
// -- into both.  `quirk_hw` != 0 reproduces
// LayerBackward for channels > 1: only elements e < batch*hw receive a
// gradient, with group e / hw (the others are left alone, or set to 0 when
// assigning, which is what adding nothing to a cleared gradient gives).
// With acc the gradient is added to dx_in's values (dx_in may be dx).
template <bool SEG, bool VEC, bool EXTRA = false>  // EXTRA: dx2 set (dx3 may be)
__global__ __launch_bounds__(NT) void norm_bwd_apply(const float* __restrict__ y, const float* __restrict__ dy,
                                                     float* dx, const float* __restrict__ stats,
                                                     NormShape sh, const double* __restrict__ part,
                                                     const double* __restrict__ fin, float eps, size_t quirk_hw,
                                                     int acc, const float* dx_in, float* __restrict__ dx2, int acc2,
                                                     float* __restrict__ dx3, int acc3) {
  const int g = blockIdx.y, ck = blockIdx.x;
  const size_t c0 = (size_t)ck * CH;
  const float fN = (float)(int)sh.N;
  // fin: precomputed per-group sums (quirk path); otherwise this group's own.
  auto terms = [&](int gs, float& sg, float& sgy, float& r) {
    sg = (float)fin[2 * gs];
    sgy = (float)fin[2 * gs + 1];
    r = rsqrtf(stats[2 * gs + 1] / fN + eps);
  };
  float sg = 0.f, sgy = 0.f, r = 0.f;
  if (quirk_hw) terms(g, sg, sgy, r);
  // Non-quirk: the group's partials and ssd first, then (VEC) this thread's
  // loads, then the sums, so the loads are in flight while the sums run.
  const PartPre pre = part_pre(part, sh, g);
  const float ssd_g = stats[2 * g + 1];
  auto finish_sums = [&]() {
    double a, b;
    group_sums_from(pre, part, sh, g, a, b);
    sg = (float)a;
    sgy = (float)b;
    r = rsqrtf(ssd_g / fN + eps);
  };
  if (VEC && !quirk_hw) {
    // Every load of the thread before its first store; FULL chunks without
    // per-lane branches (see norm_apply).
    auto body = [&](auto full) {
      constexpr bool FULL = decltype(full)::value;
      constexpr int U = VPT / 4;
      const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
      f32x4 yv[U], gv[U], d[U], d2[U], d3[U];
      size_t o[U];
      bool in[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const size_t e = elem<true>(c0, 4 * u);
        in[u] = FULL || e < sh.N;
        o[u] = in[u] ? at<SEG>(sh, g, e) : 0;
        d[u] = d2[u] = d3[u] = z4;
        if (!in[u]) continue;
        yv[u] = *reinterpret_cast<const f32x4*>(y + o[u]);
        gv[u] = *reinterpret_cast<const f32x4*>(dy + o[u]);
        if (acc) d[u] = *reinterpret_cast<const f32x4*>(dx_in + o[u]);
        if (EXTRA && acc2) d2[u] = *reinterpret_cast<const f32x4*>(dx2 + o[u]);
        if (EXTRA && dx3 && acc3) d3[u] = *reinterpret_cast<const f32x4*>(dx3 + o[u]);
      }
      finish_sums();
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (!in[u]) continue;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float v = r * (gv[u][k] - (sg / fN) - yv[u][k] * (sgy / fN));
          d[u][k] = acc ? d[u][k] + v : v;
          d2[u][k] = acc2 ? d2[u][k] + d[u][k] : d[u][k];
          d3[u][k] = acc3 ? d3[u][k] + d[u][k] : d[u][k];
        }
        *reinterpret_cast<f32x4*>(dx + o[u]) = d[u];
        if (EXTRA) *reinterpret_cast<f32x4*>(dx2 + o[u]) = d2[u];
        if (EXTRA && dx3) *reinterpret_cast<f32x4*>(dx3 + o[u]) = d3[u];
      }
    };
    if (c0 + CH <= sh.N) body(std::true_type{});
    else body(std::false_type{});
    return;
  }
  if (!quirk_hw) finish_sums();
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const size_t e = elem<false>(c0, i);
    if (e >= sh.N) continue;
    const size_t idx = at<SEG>(sh, g, e);
    if (!SEG && quirk_hw) {
      if (idx >= (size_t)sh.groups_tot * quirk_hw) {
        const float nv = acc ? dx_in[idx] : 0.f;
        dx[idx] = nv;
        if (EXTRA) dx2[idx] = acc2 ? dx2[idx] + nv : nv;
        if (EXTRA && dx3) dx3[idx] = acc3 ? dx3[idx] + nv : nv;
        continue;
      }
      terms((int)(idx / quirk_hw), sg, sgy, r);
    }
    const float v = r * (dy[idx] - (sg / fN) - y[idx] * (sgy / fN));
    const float nv = acc ? dx_in[idx] + v : v;
    dx[idx] = nv;
    if (EXTRA) dx2[idx] = acc2 ? dx2[idx] + nv : nv;
    if (EXTRA && dx3) dx3[idx] = acc3 ? dx3[idx] + nv : nv;
  }
}

// The 16-byte path: every group (segment) length and base a multiple of 4 floats.
bool vec_ok(const NormShape& sh, std::initializer_list<const void*> ptrs) {
  if (sh.N % 4 != 0) return false;
  if (sh.seg && (sh.seg % 4 != 0 || sh.seg_stride % 4 != 0 || sh.group_stride % 4 != 0)) return false;
  for (const void* p : ptrs)
    if (!aligned16(p)) return false;
  return true;
}

// Workspace: per-chunk partials, then the per-group finals.
size_t ws_need(const NormShape& sh) { return ((size_t)sh.groups_tot * sh.nchunk * 2 + (size_t)sh.groups_tot * 2) * sizeof(double); }

// f(std::integral_constant<int, K>) for the activation kind K (-1: none).
template <class F>
void with_act(int kind, F f) {
  switch (kind) {
    case MLE_RELU: f(std::integral_constant<int, MLE_RELU>{}); break;
    case MLE_GELU: f(std::integral_constant<int, MLE_GELU>{}); break;
    case MLE_SILU: f(std::integral_constant<int, MLE_SILU>{}); break;
    case MLE_TANH: f(std::integral_constant<int, MLE_TANH>{}); break;
    case MLE_SIGMOID: f(std::integral_constant<int, MLE_SIGMOID>{}); break;
    case MLE_LEAKY_RELU: f(std::integral_constant<int, MLE_LEAKY_RELU>{}); break;
    default: f(std::integral_constant<int, -1>{}); break;
  }
}

// act >= 0: the normalisation also writes act_out = act(y) (+ cbias[channel]).
void launch_fwd(hipStream_t s, const NormShape& sh, const float* x, float* y, float* stats, void* ws, float eps,
                bool stats_ready = false, int act = -1, float* act_out = nullptr, const float* cbias = nullptr,
                uint32_t cb_hw = 1, uint32_t cb_ch = 1) {
  dim3 grid(sh.nchunk, sh.groups_tot);
  double* part = static_cast<double*>(ws);
  const bool v = vec_ok(sh, {x, y}) && (act < 0 || aligned16(act_out));
  if (!stats_ready || sh.seg) {  // otherwise pass 1 ran in the producer of x
    if (sh.seg) {
      if (v) norm_stats_partial<true, true><<<grid, NT, 0, s>>>(x, sh, part);
      else norm_stats_partial<true, false><<<grid, NT, 0, s>>>(x, sh, part);
    } else {
      if (v) norm_stats_partial<false, true><<<grid, NT, 0, s>>>(x, sh, part);
      else norm_stats_partial<false, false><<<grid, NT, 0, s>>>(x, sh, part);
    }
  }
  with_act(act, [&](auto K) {
    constexpr int A = decltype(K)::value;
    if (sh.seg) {
      if (v) norm_apply<true, true, A><<<grid, NT, 0, s>>>(x, y, stats, sh, part, eps, act_out, cbias, cb_hw, cb_ch);
      else norm_apply<true, false, A><<<grid, NT, 0, s>>>(x, y, stats, sh, part, eps, act_out, cbias, cb_hw, cb_ch);
    } else {
      if (v) norm_apply<false, true, A><<<grid, NT, 0, s>>>(x, y, stats, sh, part, eps, act_out, cbias, cb_hw, cb_ch);
      else norm_apply<false, false, A><<<grid, NT, 0, s>>>(x, y, stats, sh, part, eps, act_out, cbias, cb_hw, cb_ch);
    }
  });
}

// The backward's first pass: per-chunk sums of dy and dy*y (act >= 0: dy (+)=
// act'(y) * da first (acc_dy), stored, and the sums taken of that).
void launch_bwd_partials(hipStream_t s, const NormShape& sh, const float* y, const float* dy, void* ws, size_t quirk,
                         int act = -1, const float* da = nullptr, int acc_dy = 0) {
  dim3 grid(sh.nchunk, sh.groups_tot);
  double* part = static_cast<double*>(ws);
  double* fin = part + (size_t)sh.groups_tot * sh.nchunk * 2;
  const bool v = vec_ok(sh, {y, dy}) && (act < 0 || aligned16(da));
  float* dyw = const_cast<float*>(dy);  // written only with act >= 0
  with_act(act, [&](auto K) {
    constexpr int A = decltype(K)::value;
    if (sh.seg) {
      if (v) norm_bwd_partial<true, true, A><<<grid, NT, 0, s>>>(y, dy, sh, part, da, dyw, acc_dy);
      else norm_bwd_partial<true, false, A><<<grid, NT, 0, s>>>(y, dy, sh, part, da, dyw, acc_dy);
    } else {
      if (v) norm_bwd_partial<false, true, A><<<grid, NT, 0, s>>>(y, dy, sh, part, da, dyw, acc_dy);
      else norm_bwd_partial<false, false, A><<<grid, NT, 0, s>>>(y, dy, sh, part, da, dyw, acc_dy);
    }
  });
  if (!sh.seg && quirk) norm_bwd_final<<<sh.groups_tot, 64, 0, s>>>(part, sh, fin);
}

// The second pass, from the first pass's sums in ws: dx (and dx2, dx3 when set).
void launch_bwd_apply(hipStream_t s, const NormShape& sh, const float* y, const float* dy, float* dx, int accumulate,
                      const float* stats, void* ws, float eps, size_t quirk, float* dx2 = nullptr, int acc2 = 0,
                      float* dx3 = nullptr, int acc3 = 0, const float* dx_in = nullptr) {
  dim3 grid(sh.nchunk, sh.groups_tot);
  double* part = static_cast<double*>(ws);
  double* fin = part + (size_t)sh.groups_tot * sh.nchunk * 2;
  if (!dx_in) dx_in = dx;
  const bool v = vec_ok(sh, {y, dy, dx, dx_in}) && (!dx2 || aligned16(dx2)) && (!dx3 || aligned16(dx3));
  auto go = [&](auto kern, size_t qk) {
    hipLaunchKernelGGL(kern, grid, dim3(NT), 0, s, y, dy, dx, stats, sh, part, fin, eps, qk, accumulate, dx_in, dx2,
                       acc2, dx3, acc3);
  };
  if (dx2) {
    if (sh.seg) go(v ? norm_bwd_apply<true, true, true> : norm_bwd_apply<true, false, true>, 0);
    else go(v ? norm_bwd_apply<false, true, true> : norm_bwd_apply<false, false, true>, quirk);
  } else {
    if (sh.seg) go(v ? norm_bwd_apply<true, true> : norm_bwd_apply<true, false>, 0);
    else go(v ? norm_bwd_apply<false, true> : norm_bwd_apply<false, false>, quirk);
  }
}

void launch_bwd(hipStream_t s, const NormShape& sh, const float* y, const float* dy, float* dx, const float* stats,
                void* ws, float eps, size_t quirk, int accumulate, int act = -1, const float* da = nullptr,
                int acc_dy = 0) {
  launch_bwd_partials(s, sh, y, dy, ws, quirk, act, da, acc_dy);
  launch_bwd_apply(s, sh, y, dy, dx, accumulate, stats, ws, eps, quirk);
}

int shape_of(int batch, int channels, size_t hw, int groups, NormShape& sh) {
  if (batch <= 0 || channels <= 0 || hw == 0 || groups <= 0 || channels % groups != 0)
    return set_error(MLE_ERR_INVALID, "norm: bad shape batch %d channels %d hw %zu groups %d", batch, channels, hw,
                     groups);
  sh.N = (size_t)(channels / groups) * hw;
  sh.nchunk = (int)((sh.N + CH - 1) / CH);
  sh.groups_tot = batch * groups;
  sh.seg = 0;
  sh.seg_stride = sh.group_stride = 0;
  if (sh.groups_tot > 65535) return set_error(MLE_ERR_UNSUPPORTED, "norm: %d groups > 65535", sh.groups_tot);
  return MLE_OK;
}

// BatchNorm: one group per channel, `batch` segments of hw floats.
int bn_shape_of(int batch, int channels, size_t hw, NormShape& sh) {
  if (batch <= 0 || channels <= 0 || hw == 0)
    return set_error(MLE_ERR_INVALID, "batchnorm: bad shape batch %d channels %d hw %zu", batch, channels, hw);
  sh.N = (size_t)batch * hw;
  if (sh.N > 0xffffffffull || hw > 0xffffffffull)
    return set_error(MLE_ERR_UNSUPPORTED, "batchnorm: %zu elements per channel >= 2^32", sh.N);
  sh.nchunk = (int)((sh.N + CH - 1) / CH);
  sh.groups_tot = channels;
  sh.seg = (uint32_t)hw;
  sh.seg_stride = (size_t)channels * hw;
  sh.group_stride = hw;
  if (channels > 65535) return set_error(MLE_ERR_UNSUPPORTED, "batchnorm: %d channels > 65535", channels);
  return MLE_OK;
}

// RMSNorm.  A line is a row (type 0: `len` = cols contiguous floats) or a
// column (type 1: `len` = rows floats, cols apart).  norms[line] =
// sqrtf(sum x^2) (SumSquaredSqrtCols / SumSquaredSqrtRows, Engine/kernels.cu:
// 2246-2277), y = x / norm (Scale_arr, Engine/kernels.cu:2058-2071).
// Rows: one workgroup per line, sums in double with a fixed-order block
// reduction.  Columns: one thread per column, walking the rows, so a wave
// reads 64 consecutive floats of each row.
__global__ __launch_bounds__(NT) void rms_row_fwd(const float* __restrict__ x, float* __restrict__ y,
                                                  float* __restrict__ norms, int cols) {
  __shared__ double red[NT / 64];
  const size_t base = (size_t)blockIdx.x * cols;
  double s = 0.0;
  for (int i = threadIdx.x; i < cols; i += NT) {
    const float v = x[base + i];
    s += (double)v * (double)v;
  }
  s = block_sum<NT>(s, red);
  const float n = sqrtf((float)s);
  if (threadIdx.x == 0) norms[blockIdx.x] = n;
  for (int i = threadIdx.x; i < cols; i += NT) y[base + i] = x[base + i] / n;
}

__global__ __launch_bounds__(NT) void rms_col_fwd(const float* __restrict__ x, float* __restrict__ y,
                                                  float* __restrict__ norms, int rows, int cols) {
  const int c = blockIdx.x * NT + threadIdx.x;
  if (c >= cols) return;
  const size_t base = (size_t)blockIdx.y * rows * cols + c;
  double s = 0.0;
  for (int r = 0; r < rows; ++r) {
    const float v = x[base + (size_t)r * cols];
    s += (double)v * (double)v;
  }
  const float n = sqrtf((float)s);
  norms[(size_t)blockIdx.y * cols + c] = n;
  for (int r = 0; r < rows; ++r) y[base + (size_t)r * cols] = x[base + (size_t)r * cols] / n;
}

// dx (+)= (dy - y <dy, y>) / norm along the line (Accumulate_rmsnorm_kernel,
// Engine/kernels.cu:2073-2105); acc = 0 assigns.
__global__ __launch_bounds__(NT) void rms_row_bwd(const float* __restrict__ y, const float* __restrict__ dy,
                                                  const float* __restrict__ norms, float* __restrict__ dx, int cols,
                                                  int acc) {
  __shared__ double red[NT / 64];
  const size_t base = (size_t)blockIdx.x * cols;
  double s = 0.0;
  for (int i = threadIdx.x; i < cols; i += NT) s += (double)dy[base + i] * (double)y[base + i];
  s = block_sum<NT>(s, red);
  const float d = (float)s, inv = 1.0f / norms[blockIdx.x];
  for (int i = threadIdx.x; i < cols; i += NT) {
    const float v = (dy[base + i] - y[base + i] * d) * inv;
    dx[base + i] = acc ? dx[base + i] + v : v;
  }
}

__global__ __launch_bounds__(NT) void rms_col_bwd(const float* __restrict__ y, const float* __restrict__ dy,
                                                  const float* __restrict__ norms, float* __restrict__ dx, int rows,
                                                  int cols, int acc) {
  const int c = blockIdx.x * NT + threadIdx.x;
  if (c >= cols) return;
  const size_t base = (size_t)blockIdx.y * rows * cols + c;
  double s = 0.0;
  for (int r = 0; r < rows; ++r) s += (double)dy[base + (size_t)r * cols] * (double)y[base + (size_t)r * cols];
  const float d = (float)s, inv = 1.0f / norms[(size_t)blockIdx.y * cols + c];
  for (int r = 0; r < rows; ++r) {
    const size_t o = base + (size_t)r * cols;
    const float v = (dy[o] - y[o] * d) * inv;
    dx[o] = acc ? dx[o] + v : v;
  }
}

int rms_check(int bc, int rows, int cols, int type) {
  if (bc <= 0 || rows <= 0 || cols <= 0 || (type != 0 && type != 1))
    return set_error(MLE_ERR_INVALID, "rmsnorm: bad shape bc %d rows %d cols %d type %d", bc, rows, cols, type);
  if (type == 0 && (long long)bc * rows > 0x7fffffffLL)
    return set_error(MLE_ERR_UNSUPPORTED, "rmsnorm: too many rows");
  if (type == 1 && bc > 65535) return set_error(MLE_ERR_UNSUPPORTED, "rmsnorm: bc %d > 65535", bc);
  return MLE_OK;
}

}  // namespace

extern "C" {

size_t mle_norm_ws_bytes(int batch, int channels, size_t hw, int groups) {
  NormShape sh;
  if (shape_of(batch, channels, hw, groups, sh) != MLE_OK) return 0;
  return ws_need(sh);
}

int mle_norm_fwd(mle_stream stream, const float* x, float* y, float* stats, int batch, int channels, size_t hw,
                 int groups, float eps, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(x && y && stats && ws, "mle_norm_fwd: null pointer");
  NormShape sh;
  int rc = shape_of(batch, channels, hw, groups, sh);
  if (rc) return rc;
  if (ws_bytes < ws_need(sh)) return set_error(MLE_ERR_WORKSPACE, "mle_norm_fwd: workspace too small");
  launch_fwd(as_stream(stream), sh, x, y, stats, ws, eps);
  return check_launch("mle_norm_fwd");
}

int mle_norm_fwd_ex(mle_stream stream, const float* x, float* y, float* stats, int batch, int channels, size_t hw,
                    int groups, float eps, void* ws, size_t ws_bytes, int stats_ready) {
  MLE_CHECK_ARG(x && y && stats && ws, "mle_norm_fwd: null pointer");
  NormShape sh;
  int rc = shape_of(batch, channels, hw, groups, sh);
  if (rc) return rc;
  if (ws_bytes < ws_need(sh)) return set_error(MLE_ERR_WORKSPACE, "mle_norm_fwd: workspace too small");
  launch_fwd(as_stream(stream), sh, x, y, stats, ws, eps, stats_ready != 0);
  return check_launch("mle_norm_fwd");
}

int mle_norm_fwd_act(mle_stream stream, const float* x, float* y, float* act_out, int kind, float* stats, int batch,
                     int channels, size_t hw, int groups, float eps, void* ws, size_t ws_bytes, int stats_ready) {
  MLE_CHECK_ARG(x && y && act_out && stats && ws && kind >= MLE_RELU && kind <= MLE_LEAKY_RELU,
                "mle_norm_fwd_act: bad argument");
  NormShape sh;
  int rc = shape_of(batch, channels, hw, groups, sh);
  if (rc) return rc;
  if (ws_bytes < ws_need(sh)) return set_error(MLE_ERR_WORKSPACE, "mle_norm_fwd_act: workspace too small");
  launch_fwd(as_stream(stream), sh, x, y, stats, ws, eps, stats_ready != 0, kind, act_out);
  return check_launch("mle_norm_fwd_act");
}

int mle_norm_fwd_act_bias(mle_stream stream, const float* x, float* y, float* out, int kind, const float* cbias,
                          float* stats, int batch, int channels, size_t hw, int groups, float eps, void* ws,
                          size_t ws_bytes, int stats_ready) {
  MLE_CHECK_ARG(x && y && out && cbias && stats && ws && kind >= MLE_RELU && kind <= MLE_LEAKY_RELU,
                "mle_norm_fwd_act_bias: bad argument");
  MLE_CHECK_ARG(hw % 4 == 0 && hw < ((size_t)1 << 32) && channels > 0, "mle_norm_fwd_act_bias: bad plane size");
  NormShape sh;
  int rc = shape_of(batch, channels, hw, groups, sh);
  if (rc) return rc;
  MLE_CHECK_ARG(!sh.seg, "mle_norm_fwd_act_bias: contiguous groups only");
  if (ws_bytes < ws_need(sh)) return set_error(MLE_ERR_WORKSPACE, "mle_norm_fwd_act_bias: workspace too small");
  launch_fwd(as_stream(stream), sh, x, y, stats, ws, eps, stats_ready != 0, kind, out, cbias, (uint32_t)hw,
             (uint32_t)channels);
  return check_launch("mle_norm_fwd_act_bias");
}

int mle_norm_bwd_act(mle_stream stream, const float* y, const float* da, int kind, float* dy, int accumulate_dy,
                     float* dx, const float* stats, int batch, int channels, size_t hw, int groups, float eps,
                     int reference_layout, void* ws, size_t ws_bytes, int accumulate) {
  MLE_CHECK_ARG(y && da && dy && dx && stats && ws && kind >= MLE_RELU && kind <= MLE_LEAKY_RELU,
                "mle_norm_bwd_act: bad argument");
  NormShape sh;
  int rc = shape_of(batch, channels, hw, groups, sh);
  if (rc) return rc;
  if (ws_bytes < ws_need(sh)) return set_error(MLE_ERR_WORKSPACE, "mle_norm_bwd_act: workspace too small");
  const size_t quirk = (reference_layout && groups == 1 && channels > 1) ? hw : 0;
  launch_bwd(as_stream(stream), sh, y, dy, dx, stats, ws, eps, quirk, accumulate, kind, da, accumulate_dy);
  return check_launch("mle_norm_bwd_act");
}

int mle_add_norm_partials(mle_stream stream, const float* a, const float* b, size_t b_period, float* y, int batch,
                          int channels, size_t hw, int groups, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(a && b && y && ws && b_period > 0, "mle_add_norm_partials: bad argument");
  NormShape sh;
  int rc = shape_of(batch, channels, hw, groups, sh);
  if (rc) return rc;
  const size_t total = (size_t)batch * channels * hw;
  MLE_CHECK_ARG(total % b_period == 0, "mle_add_norm_partials: b period %zu does not divide %zu", b_period, total);
  if (ws_bytes < ws_need(sh)) return set_error(MLE_ERR_WORKSPACE, "mle_add_norm_partials: workspace too small");
  dim3 grid(sh.nchunk, sh.groups_tot);
  double* part = static_cast<double*>(ws);
  const bool v = vec_ok(sh, {a, b, y}) && b_period % 4 == 0;
  hipStream_t s = as_stream(stream);
  if (v) add_stats_partial<true><<<grid, NT, 0, s>>>(a, b, b_period, y, sh, part);
  else add_stats_partial<false><<<grid, NT, 0, s>>>(a, b, b_period, y, sh, part);
  return check_launch("mle_add_norm_partials");
}

int mle_norm_bwd_partials(mle_stream stream, const float* y, float* dy, const float* da, int kind, int accumulate_dy,
                          int batch, int channels, size_t hw, int groups, int reference_layout, void* ws,
                          size_t ws_bytes) {
  MLE_CHECK_ARG(y && dy && ws && (kind < 0 || (da && kind >= MLE_RELU && kind <= MLE_LEAKY_RELU)),
                "mle_norm_bwd_partials: bad argument");
  NormShape sh;
  int rc = shape_of(batch, channels, hw, groups, sh);
  if (rc) return rc;
  if (ws_bytes < ws_need(sh)) return set_error(MLE_ERR_WORKSPACE, "mle_norm_bwd_partials: workspace too small");
  const size_t quirk = (reference_layout && groups == 1 && channels > 1) ? hw : 0;
  launch_bwd_partials(as_stream(stream), sh, y, dy, ws, quirk, kind < 0 ? -1 : kind, kind < 0 ? nullptr : da,
                      accumulate_dy);
  return check_launch("mle_norm_bwd_partials");
}

int mle_norm_bwd_apply_add(mle_stream stream, const float* y, const float* dy, float* dx, int accumulate,
                           const float* dx_in, float* dxa, int accumulate_a, float* dxb, int accumulate_b,
                           const float* stats, int batch, int channels, size_t hw, int groups, float eps,
                           int reference_layout, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(y && dy && dx && stats && ws && (dxa || !dxb), "mle_norm_bwd_apply_add: bad argument");
  MLE_CHECK_ARG(dxa != dx && (!dxb || (dxb != dx && dxb != dxa)), "mle_norm_bwd_apply_add: outputs must differ");
  MLE_CHECK_ARG(!dx_in || (dx_in != dxa && dx_in != dxb), "mle_norm_bwd_apply_add: dx_in must not be an output");
  NormShape sh;
  int rc = shape_of(batch, channels, hw, groups, sh);
  if (rc) return rc;
  if (ws_bytes < ws_need(sh)) return set_error(MLE_ERR_WORKSPACE, "mle_norm_bwd_apply_add: workspace too small");
  const size_t quirk = (reference_layout && groups == 1 && channels > 1) ? hw : 0;
  launch_bwd_apply(as_stream(stream), sh, y, dy, dx, accumulate, stats, ws, eps, quirk, dxa, accumulate_a, dxb,
                   accumulate_b, dx_in);
  return check_launch("mle_norm_bwd_apply_add");
}

int mle_norm_bwd(mle_stream stream, const float* y, const float* dy, float* dx, const float* stats, int batch,
                 int channels, size_t hw, int groups, float eps, int reference_layout, void* ws, size_t ws_bytes,
                 int accumulate) {
  MLE_CHECK_ARG(y && dy && dx && stats && ws, "mle_norm_bwd: null pointer");
  NormShape sh;
  int rc = shape_of(batch, channels, hw, groups, sh);
  if (rc) return rc;
  if (ws_bytes < ws_need(sh)) return set_error(MLE_ERR_WORKSPACE, "mle_norm_bwd: workspace too small");
  const size_t quirk = (reference_layout && groups == 1 && channels > 1) ? hw : 0;
  launch_bwd(as_stream(stream), sh, y, dy, dx, stats, ws, eps, quirk, accumulate);
  return check_launch("mle_norm_bwd");
}

size_t mle_batchnorm_ws_bytes(int batch, int channels, size_t hw) {
  NormShape sh;
  if (bn_shape_of(batch, channels, hw, sh) != MLE_OK) return 0;
  return ws_need(sh);
}

int mle_batchnorm_fwd(mle_stream stream, const float* x, float* y, float* stats, int batch, int channels, size_t hw,
                      float eps, void* ws, size_t ws_bytes) {
  MLE_CHECK_ARG(x && y && stats && ws, "mle_batchnorm_fwd: null pointer");
  NormShape sh;
  int rc = bn_shape_of(batch, channels, hw, sh);
  if (rc) return rc;
  if (ws_bytes < ws_need(sh)) return set_error(MLE_ERR_WORKSPACE, "mle_batchnorm_fwd: workspace too small");
  launch_fwd(as_stream(stream), sh, x, y, stats, ws, eps);
  return check_launch("mle_batchnorm_fwd");
}

int mle_batchnorm_bwd(mle_stream stream, const float* y, const float* dy, float* dx, const float* stats, int batch,
                      int channels, size_t hw, float eps, void* ws, size_t ws_bytes, int accumulate) {
  MLE_CHECK_ARG(y && dy && dx && stats && ws, "mle_batchnorm_bwd: null pointer");
  NormShape sh;
  int rc = bn_shape_of(batch, channels, hw, sh);
  if (rc) return rc;
  if (ws_bytes < ws_need(sh)) return set_error(MLE_ERR_WORKSPACE, "mle_batchnorm_bwd: workspace too small");
  launch_bwd(as_stream(stream), sh, y, dy, dx, stats, ws, eps, 0, accumulate);
  return check_launch("mle_batchnorm_bwd");
}

int mle_rmsnorm_fwd(mle_stream stream, const float* x, float* y, float* norms, int bc, int rows, int cols, int type) {
  MLE_CHECK_ARG(x && y && norms, "mle_rmsnorm_fwd: null pointer");
  int rc = rms_check(bc, rows, cols, type);
  if (rc) return rc;
  hipStream_t s = as_stream(stream);
  if (type == 0) rms_row_fwd<<<(unsigned)((long long)bc * rows), NT, 0, s>>>(x, y, norms, cols);
  else rms_col_fwd<<<dim3((cols + NT - 1) / NT, bc), NT, 0, s>>>(x, y, norms, rows, cols);
  return check_launch("mle_rmsnorm_fwd");
}

int mle_rmsnorm_bwd(mle_stream stream, const float* y, const float* dy, const float* norms, float* dx, int bc, int rows,
                    int cols, int type, int accumulate) {
  MLE_CHECK_ARG(y && dy && norms && dx, "mle_rmsnorm_bwd: null pointer");
  int rc = rms_check(bc, rows, cols, type);
  if (rc) return rc;
  hipStream_t s = as_stream(stream);
  if (type == 0) rms_row_bwd<<<(unsigned)((long long)bc * rows), NT, 0, s>>>(y, dy, norms, dx, cols, accumulate);
  else rms_col_bwd<<<dim3((cols + NT - 1) / NT, bc), NT, 0, s>>>(y, dy, norms, dx, rows, cols, accumulate);
  return check_launch("mle_rmsnorm_bwd");
}

}  // extern "C"
