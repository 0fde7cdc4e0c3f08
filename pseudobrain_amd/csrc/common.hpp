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
// Lane exchanges on the VALU (no LDS round trip). Lane group g = lanes
// 16 g .. 16 g + 15.
// ---------------------------------------------------------------------------
// DPP move of a float inside 16-lane rows (every lane's source in its row).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}

// Sum over aligned groups of `width` lanes (1, 2, 4, 8 or 16) inside a 16-lane
// row; every lane of a group gets the group's sum: a butterfly of DPP moves
// (quad_perm [1,0,3,2] and [2,3,0,1], then row_half_mirror and row_mirror:
// gfx9-family controls 0xb1, 0x4e, 0x141, 0x140).
__device__ __forceinline__ float group_sum(float x, int width) {
  if (width > 1) x += dpp_mov<0xb1>(x);
  if (width > 2) x += dpp_mov<0x4e>(x);
  if (width > 4) x += dpp_mov<0x141>(x);
  if (width > 8) x += dpp_mov<0x140>(x);
  return x;
}

// swap32 exchanges lanes 32-63 of a with lanes 0-31 of b; swap16 lane groups
// 1 and 3 of a with groups 0 and 2 of b (v_permlane32_swap,
// v_permlane16_swap). Written as assembly: this ROCm's clang builtins for them
// (__builtin_amdgcn_permlane{16,32}_swap) return the first result in both
// elements of their pair. The nops give the two wait states between a VALU
// write and the swap's read, and between the swap and the next VALU read.
__device__ __forceinline__ void swap32(float &a, float &b) {
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap16(float &a, float &b) {
  asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
// x + x of lane ^ 32, and of lane ^ 16, in every lane.
__device__ __forceinline__ float add_xor32(float x) {
  float a = x, b = x;
  swap32(a, b);
  return a + b;
}
__device__ __forceinline__ float add_xor16(float x) {
  float a = x, b = x;
  swap16(a, b);
  return a + b;
}
// Sum over the lanes congruent to this one modulo CG (a power of two): every
// lane gets its class's sum. Within a row, DPP rotations by 8, 4, 2, 1 lanes
// (row_ror, controls 0x128, 0x124, 0x122, 0x121); across rows the swaps.
template <int CG>
__device__ __forceinline__ float sum_mod_lanes(float x) {
  static_assert(CG >= 1 && CG <= 64 && (CG & (CG - 1)) == 0, "a power of two up to 64");
  if constexpr (CG <= 8) x += dpp_mov<0x128>(x);
  if constexpr (CG <= 4) x += dpp_mov<0x124>(x);
  if constexpr (CG <= 2) x += dpp_mov<0x122>(x);
  if constexpr (CG <= 1) x += dpp_mov<0x121>(x);
  if constexpr (CG <= 16) x = add_xor16(x);
  if constexpr (CG <= 32) x = add_xor32(x);
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

// Debug build (PBGDN_DEBUG): a kernel fills its LDS with a quiet NaN in every
// 32-bit word before its first use (PBGDN_POISON_LDS on each region, then
// PBGDN_POISON_SYNC), so that a read of LDS the launch has not written first
// gives NaN and shows in the outputs. Nothing in a normal build.
#ifdef PBGDN_DEBUG
__device__ __forceinline__ void debug_poison_lds(void *base, uint32_t bytes) {
  uint32_t *w = static_cast<uint32_t *>(base);
  for (uint32_t i = threadIdx.x; i < bytes / 4; i += blockDim.x) w[i] = 0x7fc00000u;
}
#define PBGDN_POISON_LDS(base, bytes) ::pbgdn::debug_poison_lds((base), static_cast<uint32_t>(bytes))
#define PBGDN_POISON_SYNC() __syncthreads()
#else
#define PBGDN_POISON_LDS(base, bytes) ((void)0)
#define PBGDN_POISON_SYNC() ((void)0)
#endif

}  // namespace pbgdn
