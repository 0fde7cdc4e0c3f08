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

}  // namespace pbgdn
