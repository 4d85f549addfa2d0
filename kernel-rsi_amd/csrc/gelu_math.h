// GELU of the GEGLU kernels (geglu.hip and the fused projection in geglu_linear.hip), so
// both compute bitwise the same gelu(a) and gelu'(a).
//   tanh form (the reference's _gelu_parts, library/geglu.py:20-24):
//     z = sqrt(2/pi) (a + 0.044715 a^3);  t = 1 - 2 / (exp(2z) + 1);  gelu = 0.5 a (1 + t)
//   erf form (torch.nn.functional.gelu(approximate="none")):
//     gelu = 0.5 a (1 + erf(a / sqrt 2)),  gelu' = 0.5 (1 + erf(a / sqrt 2)) + a exp(-a^2 / 2) / sqrt(2 pi)
#pragma once

#include <hip/hip_runtime.h>

namespace krsi {
namespace gelu_detail {

constexpr float kSqrt2OverPi = 0.7978845608028654f;
constexpr float kKappa = 0.044715f;
constexpr float kKappa3 = 0.134145f;  // 3 * 0.044715
constexpr float kInvSqrt2 = 0.70710678118654752f;
constexpr float kInvSqrt2Pi = 0.3989422804014327f;
constexpr float kLog2eG = 1.4426950408889634f;

// tanh(z) = 1 - 2 / (e^{2z} + 1), the identity the reference uses; e^{2z}
// overflows to +inf for large z and the quotient then gives exactly 1.
__device__ __forceinline__ float tanh_via_exp(float z) {
  const float e = __builtin_amdgcn_exp2f(2.0f * z * kLog2eG);
  return 1.0f - 2.0f / (e + 1.0f);
}

// erf by Abramowitz & Stegun, Handbook of Mathematical Functions, 7.1.26:
// erf(x) = 1 - t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) e^{-x^2}, t = 1 / (1 + p x), x >= 0,
// absolute error <= 1.5e-7 (<= 6e-7 evaluated in fp32), far below a bf16 ulp of the output.
// Returns erf(a / sqrt 2); ex must be e^{-a^2 / 2}, which gelu' needs as well.
__device__ __forceinline__ float erf_as(float a, float ex) {
  const float x = fabsf(a) * kInvSqrt2;
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f, x, 1.0f));
  float q = __builtin_fmaf(1.061405429f, t, -1.453152027f);
  q = __builtin_fmaf(q, t, 1.421413741f);
  q = __builtin_fmaf(q, t, -0.284496736f);
  q = __builtin_fmaf(q, t, 0.254829592f);
  return copysignf(1.0f - q * t * ex, a);
}
__device__ __forceinline__ float exp_half_sq(float a) {
  return __builtin_amdgcn_exp2f(-0.5f * kLog2eG * a * a);
}

template <bool TANH>
__device__ __forceinline__ float gelu_fwd(float a) {
  if (TANH) {
    const float z = kSqrt2OverPi * (a + kKappa * a * a * a);
    return 0.5f * a * (1.0f + tanh_via_exp(z));
  }
  return 0.5f * a * (1.0f + erf_as(a, exp_half_sq(a)));
}

// Returns gelu(a) and writes gelu'(a) to d.
template <bool TANH>
__device__ __forceinline__ float gelu_fwd_bwd(float a, float& d) {
  if (TANH) {
    const float z = kSqrt2OverPi * (a + kKappa * a * a * a);
    const float t = tanh_via_exp(z);
    const float dz = kSqrt2OverPi * (1.0f + kKappa3 * a * a);
    d = 0.5f * (1.0f + t) + 0.5f * a * (1.0f - t * t) * dz;
    return 0.5f * a * (1.0f + t);
  }
  const float ex = exp_half_sq(a);
  const float e = erf_as(a, ex);
  const float pdf = ex * kInvSqrt2Pi;
  d = 0.5f * (1.0f + e) + a * pdf;
  return 0.5f * a * (1.0f + e);  // the forward's expression, so bf16(gelu) matches it
}

}  // namespace gelu_detail

using gelu_detail::gelu_fwd;
using gelu_detail::gelu_fwd_bwd;

}  // namespace krsi
