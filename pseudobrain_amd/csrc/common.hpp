// Device helpers shared by the Gated DeltaNet kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pbgdn.h"

namespace pbgdn {

typedef _Float16 half_t;
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint16_t u16;
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t v2u32_t __attribute__((ext_vector_type(2)));
typedef uint32_t v4u32_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Scalar element access. bf16 is handled as raw bits (no compiler bf16
// arithmetic is needed): widening is a shift, narrowing rounds to nearest even.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_float(u16 b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ u16 float_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u) {  // inf / nan: keep, quiet the nan
    return static_cast<u16>((u >> 16) | ((u & 0xffffu) ? 0x40u : 0u));
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<u16>(u >> 16);
}

// Load element i of a tensor of element type `dtype` as float.
__device__ __forceinline__ float load_elem(const void *p, long i, int dtype) {
  if (dtype == PBGDN_F32) return static_cast<const float *>(p)[i];
  if (dtype == PBGDN_BF16) return bf16_bits_to_float(static_cast<const u16 *>(p)[i]);
  return static_cast<float>(static_cast<const half_t *>(p)[i]);
}

__device__ __forceinline__ void store_elem(void *p, long i, int dtype, float x) {
  if (dtype == PBGDN_F32) {
    static_cast<float *>(p)[i] = x;
  } else if (dtype == PBGDN_BF16) {
    static_cast<u16 *>(p)[i] = float_to_bf16_bits(x);
  } else {
    static_cast<half_t *>(p)[i] = static_cast<half_t>(x);
  }
}

// ---------------------------------------------------------------------------
// Buffer resources: a base address and a byte range; a load outside the range
// returns zeros and a store outside it is dropped, so per-lane conditions need
// no branches around the memory operations.
// ---------------------------------------------------------------------------
constexpr int RSRC_WORD3 = 0x00020000;  // raw buffer resource, gfx9 family

// Offset that is past the range of every buffer resource here (ranges stay
// below 2^31): a load from it returns zeros, a store to it is dropped.
constexpr uint32_t OUT_OF_RANGE = 0x7ffffff0u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, long bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                           static_cast<int>(bytes > 0 ? bytes : 0), RSRC_WORD3);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// ---------------------------------------------------------------------------
// Wavefront reductions (64 lanes).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, 64));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// ---------------------------------------------------------------------------
// MFMA wrappers. Lane layouts (l = lane, g = l >> 4, c = l & 15):
//   16x16x32 f16: A[m=c][k-slots 8g..8g+7], B[k-slots 8g..8g+7][n=c]
//   16x16x16 f16: A[m=c][k-slots 4g..4g+3], B[k-slots 4g..4g+3][n=c]
//   D (both):     D[rows 4g..4g+3][n=c]
// A and B use the same slot->k assignment, so any consistent permutation of
// the contraction index between A and B leaves the product unchanged.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float4_t mfma32(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float4_t mfma16(half4_t a, half4_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half8_t cat8(half4_t lo, half4_t hi) {
  return half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ half4_t to_half4(float4_t x) {
  return half4_t{static_cast<half_t>(x[0]), static_cast<half_t>(x[1]),
                 static_cast<half_t>(x[2]), static_cast<half_t>(x[3])};
}

__device__ __forceinline__ float4_t to_float4(half4_t x) {
  return float4_t{static_cast<float>(x[0]), static_cast<float>(x[1]),
                  static_cast<float>(x[2]), static_cast<float>(x[3])};
}

}  // namespace pbgdn
