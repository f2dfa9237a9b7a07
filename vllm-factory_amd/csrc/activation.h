// Activation functions shared by the elementwise kernels and the fused
// projection epilogues (fp32 arithmetic on gfx950).
#pragma once

#include <math.h>

#include "vfk_common.h"

namespace vfk {

// a * sigmoid(t) = a / (1 + e^-t) with the hardware exp2 and reciprocal
// (relative error a few ulp; e^-t = inf gives 0, the limit).
__device__ inline float mul_sigmoid(float a, float t) {
  return a * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-t * 1.4426950408889634f));
}

// erf(u) by Abramowitz & Stegun, Handbook of Mathematical Functions, 7.1.26
// (absolute error <= 1.5e-7): 1 - (a1 t + ... + a5 t^5) e^(-u^2), t = 1 / (1 + p|u|).
__device__ inline float erf_as(float u) {
  const float x = fabsf(u);
  const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * x);
  float poly = 1.061405429f;
  poly = poly * t - 1.453152027f;
  poly = poly * t + 1.421413741f;
  poly = poly * t - 0.284496736f;
  poly = poly * t + 0.254829592f;
  const float y = 1.0f - poly * t * __builtin_amdgcn_exp2f(-x * x * 1.4426950408889634f);
  return copysignf(y, u);
}

template <int ACT>
__device__ inline float act_f(float a) {
  if (ACT == VFK_ACT_GELU_ERF) return 0.5f * a * (1.0f + erf_as(a * 0.70710678118654752f));
  if (ACT == VFK_ACT_GELU_TANH) {
    // 0.5 a (1 + tanh(z)) = a sigmoid(2 z): the same identity as the
    // reference's kernels/ff_fused.py:47-53, without the cancellation of
    // 1 + tanh(z) for large negative z
    const float z = 0.7978845608028654f * (a + 0.044715f * a * a * a);
    return mul_sigmoid(a, 2.0f * z);
  }
  if (ACT == VFK_ACT_SILU) return mul_sigmoid(a, a);
  return fmaxf(a, 0.f);  // VFK_ACT_RELU
}

}  // namespace vfk
