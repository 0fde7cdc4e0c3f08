// Elementwise math of the layer around the recurrence (the short
// convolution's input rounding, SiLU, softplus, sigmoid), shared by the
// layer kernels and the fused decode step.
#pragma once

#include "common.hpp"

namespace pbgdn {

// The value a float takes after a round trip through `dtype` (the reference
// casts the carried tail to the input's dtype before the convolution).
__device__ __forceinline__ float through(float x, int dtype) {
  if (dtype == PBGDN_BF16) return bf16_bits_to_float(float_to_bf16_bits(x));
  if (dtype == PBGDN_F16) return static_cast<float>(static_cast<half_t>(x));
  return x;
}

__device__ __forceinline__ float sigmoidf(float x) { return 1.f / (1.f + expf(-x)); }
// x sigmoid(x) on v_exp_f32 and v_rcp_f32 (about 1e-7 relative error; the
// IEEE-exact forms cost ~25 VALU operations per element and made both
// kernels VALU-bound)
__device__ __forceinline__ float siluf(float x) {
  return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}
// torch.nn.functional.softplus with beta 1, threshold 20
__device__ __forceinline__ float softplusf(float x) { return x > 20.f ? x : log1pf(expf(x)); }

// The same three on v_exp_f32, v_log_f32 and v_rcp_f32 (a few ulp relative
// error, ~1e-6 for exp of |x| ~ 20 through the rounding of x log2(e)): the
// IEEE-exact forms cost ~100 VALU operations per gate and sat on the
// prologue's critical tiles.
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float sigmoid_fast(float x) { return __builtin_amdgcn_rcpf(1.f + exp_fast(-x)); }
// log1p(e) as log(u) e / (u - 1), u = 1 + e rounded: the factor cancels the
// rounding of u (Goldberg's form), so small e keep their relative precision
__device__ __forceinline__ float softplus_fast(float x) {
  if (x > 20.f) return x;
  const float e = exp_fast(x);
  const float u = 1.f + e;
  const float d = u - 1.f;
  return d == 0.f ? e : __builtin_amdgcn_logf(u) * 0.6931471805599453f * e * __builtin_amdgcn_rcpf(d);
}

}  // namespace pbgdn
