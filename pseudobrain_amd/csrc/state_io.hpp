// Element I/O shared by the kernels that carry the recurrent state: a
// token's inputs picked out of loaded words, and the state moved in pieces of
// four columns through buffer resources in float32, bf16 or fp16.
#pragma once

#include "common.hpp"

namespace pbgdn {

// Element `half` (0 low, 1 high) of a loaded word for 16-bit dtypes, the word
// itself for float32.
__device__ __forceinline__ float widen_word(uint32_t w, int half, int dtype) {
  if (dtype == PBGDN_F32) return __uint_as_float(w);
  const uint32_t bits = half ? w >> 16 : w & 0xffffu;
  if (dtype == PBGDN_BF16) return __uint_as_float(bits << 16);
  return static_cast<float>(__builtin_bit_cast(half_t, static_cast<u16>(bits)));
}

// Four consecutive elements from two loaded 8-byte pieces (w1 only for float32).
__device__ __forceinline__ float4_t widen_words(v2u32_t w0, v2u32_t w1, int dtype) {
  if (dtype == PBGDN_F32) {
    return float4_t{__uint_as_float(w0[0]), __uint_as_float(w0[1]), __uint_as_float(w1[0]), __uint_as_float(w1[1])};
  }
  if (dtype == PBGDN_BF16) {
    return float4_t{__uint_as_float(w0[0] << 16), __uint_as_float(w0[0] & 0xffff0000u),
                    __uint_as_float(w0[1] << 16), __uint_as_float(w0[1] & 0xffff0000u)};
  }
  return to_float4(__builtin_bit_cast(half4_t, w0));
}

// Cache policy of the state's loads and stores (the aux bits of a buffer
// instruction on gfx950: sc0 = 1, nt = 2, sc1 = 16). Measured on the decode
// step at the Qwen3-Next head shape, B = 64 (read + write bytes per second
// against 8 TB/s): with the 128 MiB float32 state resident in the 256 MB
// last-level cache (the same pool stepped again and again), sc0|sc1 83%, nt
// 71%; with it outside (pools rotated between steps, as the layers of a model
// do), nt 69%, sc0|sc1 61%; a bf16 state outside, sc1|nt 70.5%, nt 68.5%. A
// 1 GiB streaming copy (pbgdn_stream_probe, nt) sustains 75%.
constexpr int STATE_CACHED = 17;  // sc0 | sc1
template <typename TS>
constexpr int state_streamed() { return sizeof(TS) == 4 ? 2 : 18; }  // nt; sc1 | nt for 16-bit states
constexpr long STATE_CACHE_BYTES = 192L << 20;  // a call moving more state than this streams it

// State element I/O: Raw is what a thread loads for 4 consecutive columns;
// AUX is the cache policy above.
//
// Stores take their whole offset in the VGPR and a constant zero soffset.
// A buffer store of more than 64 bits reads its data VGPRs after it issues,
// and the compiler puts a wait state before a VALU write of those VGPRs only
// when soffset is a constant: with the row step in an SGPR soffset, a VALU
// write of the first data VGPR right after the store corrupted the stored
// value on gfx950 (only the first element of the piece, only where the write
// came next), so the store form here is the one the compiler protects.
template <typename TS>
struct StateIO;
template <>
struct StateIO<float> {
  using Raw = float4_t;
  template <int AUX = 0>
  __device__ static Raw load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, AUX));
  }
  __device__ static float4_t widen(Raw x) { return x; }
  template <int AUX = 0>
  __device__ static void store(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, float4_t x) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u32_t, x), r, voff + soff, 0, AUX);
  }
};
template <>
struct StateIO<u16> {
  using Raw = v2u32_t;
  template <int AUX = 0>
  __device__ static Raw load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, AUX);
  }
  __device__ static float4_t widen(Raw w) {
    return float4_t{__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u),
                    __uint_as_float(w[1] << 16), __uint_as_float(w[1] & 0xffff0000u)};
  }
  // Round to nearest even (v_cvt_pk_bf16_f32).
  template <int AUX = 0>
  __device__ static void store(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, float4_t x) {
    const bf16x4_t b = {static_cast<__bf16>(x[0]), static_cast<__bf16>(x[1]), static_cast<__bf16>(x[2]),
                        static_cast<__bf16>(x[3])};
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u32_t, b), r, voff + soff, 0, AUX);
  }
};
template <>
struct StateIO<half_t> {
  using Raw = v2u32_t;
  template <int AUX = 0>
  __device__ static Raw load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, AUX);
  }
  __device__ static float4_t widen(Raw w) { return to_float4(__builtin_bit_cast(half4_t, w)); }
  template <int AUX = 0>
  __device__ static void store(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, float4_t x) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u32_t, to_half4(x)), r, voff + soff, 0, AUX);
  }
};

}  // namespace pbgdn
