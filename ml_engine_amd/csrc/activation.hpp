// Activation functions and their derivatives (the reference's formulas), shared
// by the elementwise kernels and the GEMM epilogues so both compute the same
// values: forward (Engine/kernels.cu:1214, 1248, 1286) and derivative
// (Engine/kernels.cu:1223, 1256, 1297) kernels of ReLU, SiLU, GELU, plus
// tanh, sigmoid and leaky ReLU.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include "../../include/mle_hip.h"

namespace mle {

constexpr float kPI = 3.14159265359f;  // Includes/kernels.h:10

template <int K>
__device__ __forceinline__ float act_f(float x) {
  if (K == MLE_RELU) return (x < 0) ? 0.0f : x;
  if (K == MLE_GELU) {
    const float val = sqrtf(2.0f / kPI) * (x + 0.044715f * x * x * x);
    return 0.5f * x * (1.0f + tanhf(val));
  }
  if (K == MLE_SILU) return x * (1.0f / (1.0f + expf(-x)));
  if (K == MLE_TANH) return tanhf(x);
  if (K == MLE_SIGMOID) return 1.0f / (1.0f + expf(-1.0f * x));
  return (x < 0) ? 0.01f * x : x;  // leaky
}

template <int K>
__device__ __forceinline__ float act_df(float x) {
  if (K == MLE_RELU) return (x > 0.0f) ? 1.0f : 0.0f;
  if (K == MLE_GELU) {
    const float root = sqrtf(2.0f / kPI);
    const float u = root * (x + 0.044715f * x * x * x);
    const float du = root * (1.0f + 0.134145f * x * x);
    const float t = tanhf(u);
    return 0.5f + 0.5f * t + 0.5f * x * (1.0f - t * t) * du;
  }
  if (K == MLE_SILU) {
    const float e = expf(x);
    const float ne = 1.0f / e;
    const float sg = 1.0f / (1.0f + ne);
    return sg + (x / (e + ne + 2.0f));
  }
  if (K == MLE_TANH) {
    const float e2 = expf(2.0f * x);
    const float ne2 = 1.0f / e2;
    return 4.0f / (e2 + ne2 + 2.0f);
  }
  if (K == MLE_SIGMOID) {
    const float e = expf(x);
    const float ne = 1.0f / e;
    return 1.0f / (e + ne + 2.0f);
  }
  return (x < 0.0f) ? 0.01f : 1.0f;
}

// act_f for a kind known only at run time.
__device__ __forceinline__ float act_rt(int kind, float x) {
  switch (kind) {
    case MLE_RELU: return act_f<MLE_RELU>(x);
    case MLE_GELU: return act_f<MLE_GELU>(x);
    case MLE_SILU: return act_f<MLE_SILU>(x);
    case MLE_TANH: return act_f<MLE_TANH>(x);
    case MLE_SIGMOID: return act_f<MLE_SIGMOID>(x);
    default: return act_f<MLE_LEAKY_RELU>(x);
  }
}

// act_df for a kind known only at run time.
__device__ __forceinline__ float act_drt(int kind, float x) {
  switch (kind) {
    case MLE_RELU: return act_df<MLE_RELU>(x);
    case MLE_GELU: return act_df<MLE_GELU>(x);
    case MLE_SILU: return act_df<MLE_SILU>(x);
    case MLE_TANH: return act_df<MLE_TANH>(x);
    case MLE_SIGMOID: return act_df<MLE_SIGMOID>(x);
    default: return act_df<MLE_LEAKY_RELU>(x);
  }
}

// dx (+)= f'(x) * dy as the elementwise activation backward forms it: the
// product is rounded before the add (acc = false assigns and `old` is unused).
template <int K>
__device__ __forceinline__ float act_bwd_k(float x, float dy, float old, bool acc) {
#pragma clang fp contract(off)
  const float v = act_df<K>(x) * dy;
  return acc ? old + v : v;
}

// dx (+)= f'(x) * dy for a run-time kind, as the elementwise activation
// backward forms it: the product is rounded before the add (acc = false
// assigns and `old` is unused).
__device__ __forceinline__ float act_bwd_rt(int kind, float x, float dy, float old, bool acc) {
#pragma clang fp contract(off)
  const float v = act_drt(kind, x) * dy;
  return acc ? old + v : v;
}

}  // namespace mle
