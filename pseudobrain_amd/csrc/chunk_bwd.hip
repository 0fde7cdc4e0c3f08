// Backward of the chunked Gated DeltaNet operator: the gradients that
// pseudobrain::gated_delta_chunk_backward returns (pseudobrain/
// gated_deltanet.py:230-277), from the chunk form of the forward
//
//   X = V - Gamma K S,   U = Tb X,   O = scale Gamma Q S + M U,
//   S' = gamma_C S + K^T E U,
//   Tb = (I + A)^-1 diag(beta),  A_ts = beta_t (k_t.k_s) e^{c_t - c_s} (t > s),
//   M_ts = scale (q_t.k_s) e^{c_t - c_s} (t >= s),  Gamma = diag(e^{c_t}),
//   E = diag(e^{c_last - c_t}),  gamma_C = e^{c_last},
//
// with c the in-chunk inclusive cumulative sum of g. Reverse mode through it:
// the state adjoint runs backward over the chunks,
//   dU = M^T dO + E K dS',  dX = Tb^T dU,
//   dS = gamma_C dS' + scale (Gamma Q)^T dO - (Gamma K)^T dX,
// and each chunk's gradients follow from its start state S, its end adjoint
// dS' and its own inputs. Four launches on the caller's stream:
//
//   bwd_local_kernel     per (chunk, value head): T = (I + A)^-1 by block
//                        substitution, dU0 = M^T dO, J = scale (Gamma Q)^T dO
//   bwd_scans_kernel     per (value head, 16 value columns), serial over the
//                        chunks, two independent roles in one launch: the
//                        state at every chunk start (forward), and the
//                        adjoint at every chunk end and dh0 (reverse)
//   bwd_grad_kernel      per (chunk, value head): dq, dk, dv, dbeta, dg
//   bwd_gqa_reduce_kernel  dq, dk summed over the value heads of a key head
//
// Accumulation is float32. With bf16 inputs the products of inputs and states
// run on bf16 MFMA, a float32 operand entering as a high/low pair of bf16
// parts (A B_hi + A B_lo, or three products when both are paired: about
// 2^-16 relative); the rest, and every product for fp16 / fp32 inputs, on the
// 16x16x4 fp32 MFMA with four consecutive k per lane group.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "device.hpp"
#include "schedule.hpp"

namespace pbgdn {
namespace {

constexpr int BC = 64;    // chunk length
constexpr int BNT = 256;  // threads per workgroup (4 waves)
constexpr int LC = BC + 4;
constexpr int LT = 16 + 4;  // row stride of 16-column tiles

struct BwdParams {
  const void *q, *k, *v;
  const float *g;
  const void *beta;
  const float *h0;
  const void *dout;
  const float *dht;
  void *dq, *dk, *dv;
  float *dg;
  void *dbeta;
  float *dh0;
  float *ws_T, *ws_c, *ws_beta, *ws_dU0, *ws_J, *ws_S, *ws_dS, *ws_dq, *ws_dk;
  int in_dtype, beta_dtype;
  int B, T, Hk, Hv, K, V, n;
  float scale;
  int xcds;  // the device's XCDs (device.hpp)
};

// fp32 MFMA: acc (16x16) += A (16x4) B (4x16). Lane l, c = l & 15, g = l >> 4:
// A[m=c][k=g], B[k=g][n=c]; acc[r] is D[row 4g + r][col c].
__device__ __forceinline__ float4_t mfma_f32(float a, float b, float4_t acc) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
}

// acc += sum_{k < KD} a(i, k) b(k, j) over a 16x16 tile; a(i, k) is row i of
// the tile's A rows, b(k, j) column j of its B columns; U k-steps unrolled.
template <int KD, int U = 8, typename FA, typename FB>
__device__ __forceinline__ float4_t tile_mm(float4_t acc, FA a, FB b) {
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, g = lane >> 4;
#pragma unroll U
  for (int k = 0; k < KD; k += 4) acc = mfma_f32(a(c, k + g), b(k + g, c), acc);
  return acc;
}

// The same sum with k grouped per lane: in each block of 16 k, lane group g
// supplies k = 4g .. 4g+3 over four products (the products sum over all k,
// so which k a step carries is free). a4(i, k) and b4(k, j) return the four
// values a(i, k..k+3) and b(k..k+3, j): one 128-bit LDS read where they are
// contiguous (ld4), else four reads 16 lanes x 4 groups wide that fall in
// distinct banks for the padded strides used here (ld4s). U blocks unrolled.
template <int KD, int U = 4, typename FA, typename FB>
__device__ __forceinline__ float4_t tile_mm4(float4_t acc, FA a4, FB b4) {
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, g = lane >> 4;
#pragma unroll U
  for (int kb = 0; kb < KD; kb += 16) {
    const float4_t a = a4(c, kb + 4 * g), b = b4(kb + 4 * g, c);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = mfma_f32(a[j], b[j], acc);
  }
  return acc;
}

__device__ __forceinline__ float4_t ld4(const float *p) { return *reinterpret_cast<const float4_t *>(p); }
__device__ __forceinline__ float4_t ld4s(const float *p, int stride) {
  return float4_t{p[0], p[stride], p[2 * stride], p[3 * stride]};
}

__device__ __forceinline__ float4_t zero4() { return float4_t{0.f, 0.f, 0.f, 0.f}; }

template <typename T>
constexpr int dtype_of_bwd() {
  return sizeof(T) == 4 ? PBGDN_F32 : (std::is_same<T, u16>::value ? PBGDN_BF16 : PBGDN_F16);
}

// Sum over the 16 lanes that share lane >> 4 (the columns of one tile row).
__device__ __forceinline__ float row16_sum(float x) {
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// Eight (four for float32) consecutive elements of TIn in a 16-byte piece, as float.
template <typename TIn>
__device__ __forceinline__ void decode16(const uint4 &u, float *x) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
  if constexpr (sizeof(TIn) == 4) {
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = __uint_as_float(w[e]);
  } else if constexpr (dtype_of_bwd<TIn>() == PBGDN_BF16) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = __uint_as_float(w[e] << 16);
      x[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = static_cast<float>(__builtin_bit_cast(half_t, static_cast<u16>(w[e] & 0xffffu)));
      x[2 * e + 1] = static_cast<float>(__builtin_bit_cast(half_t, static_cast<u16>(w[e] >> 16)));
    }
  }
}

// Element idx of an LDS array of TIn, as float.
template <typename TIn>
__device__ __forceinline__ float ld_el(const TIn *m, int idx) {
  if constexpr (sizeof(TIn) == 4) {
    return m[idx];
  } else if constexpr (dtype_of_bwd<TIn>() == PBGDN_BF16) {
    return __uint_as_float(static_cast<uint32_t>(m[idx]) << 16);
  } else {
    return static_cast<float>(m[idx]);
  }
}

// Four consecutive elements of TIn (idx a multiple of 4; one 8- or 16-byte
// LDS read), and four elements `stride` apart, as float.
template <typename TIn>
__device__ __forceinline__ float4_t ld4e(const TIn *m, int idx) {
  if constexpr (sizeof(TIn) == 4) {
    return ld4(reinterpret_cast<const float *>(m) + idx);
  } else {
    const uint2 w = *reinterpret_cast<const uint2 *>(m + idx);
    if constexpr (dtype_of_bwd<TIn>() == PBGDN_BF16) {
      return float4_t{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u), __uint_as_float(w.y << 16),
                      __uint_as_float(w.y & 0xffff0000u)};
    } else {
      return float4_t{static_cast<float>(__builtin_bit_cast(half_t, static_cast<u16>(w.x & 0xffffu))),
                      static_cast<float>(__builtin_bit_cast(half_t, static_cast<u16>(w.x >> 16))),
                      static_cast<float>(__builtin_bit_cast(half_t, static_cast<u16>(w.y & 0xffffu))),
                      static_cast<float>(__builtin_bit_cast(half_t, static_cast<u16>(w.y >> 16)))};
    }
  }
}

template <typename TIn>
__device__ __forceinline__ float4_t ld4es(const TIn *m, int idx, int stride) {
  return float4_t{ld_el(m, idx), ld_el(m, idx + stride), ld_el(m, idx + 2 * stride), ld_el(m, idx + 3 * stride)};
}

typedef __bf16 bh8_t __attribute__((ext_vector_type(8)));

// x = hi + lo, each rounded to bf16 in turn (16 significant bits together),
// as packed bf16 pairs: element j in bits 16 (j & 1) of word j >> 1. (The
// words are taken apart with integer shifts: reading the elements of a
// __bf16 vector one by one compiled to element 0 four times.)
__device__ __forceinline__ void split_bf16(float4_t x, v2u32_t &hi, v2u32_t &lo) {
  hi = __builtin_bit_cast(v2u32_t, __builtin_convertvector(x, bf16x4_t));
  const float4_t back = {__uint_as_float(hi[0] << 16), __uint_as_float(hi[0] & 0xffff0000u),
                         __uint_as_float(hi[1] << 16), __uint_as_float(hi[1] & 0xffff0000u)};
  lo = __builtin_bit_cast(v2u32_t, __builtin_convertvector(x - back, bf16x4_t));
}

// bf16 MFMA: acc (16x16) += A (16x32) B (32x16). Lane l, c = l & 15, g = l >> 4:
// A[m=c][k=8g..8g+7], B[k=8g..8g+7][n=c]; acc[r] is D[row 4g + r][col c].
__device__ __forceinline__ float4_t mfma_bf16(bh8_t a, bh8_t b, float4_t acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}

// Rows row0 .. row0+15 of a [64][ldr] bf16 array (exact inputs) times a
// state tile given as its transpose in two bf16 parts, hiT + loT ([16][lds],
// x = hi + lo to 16 bits): sum over k < KD, on bf16 MFMA with fp32
// accumulation. Both operands are read k-contiguous, 16 bytes a lane.
template <int KD>
__device__ __forceinline__ float4_t rows_times_state(const u16 *rows, int ldr, int row0, const u16 *hiT,
                                                     const u16 *loT, int ldt) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
  for (int kb = 0; kb < KD; kb += 32) {
    const bh8_t a = *reinterpret_cast<const bh8_t *>(rows + (row0 + c) * ldr + kb + 8 * g);
    acc = mfma_bf16(a, *reinterpret_cast<const bh8_t *>(hiT + c * ldt + kb + 8 * g), acc);
    acc = mfma_bf16(a, *reinterpret_cast<const bh8_t *>(loT + c * ldt + kb + 8 * g), acc);
  }
  return acc;
}

// Rows a0 .. a0+15 of one [64][ld] bf16 array times the transpose of rows
// b0 .. b0+15 of another (exact inputs, sum over k < KD) on bf16 MFMA.
template <int KD>
__device__ __forceinline__ float4_t rows_times_rows(const u16 *a, const u16 *b, int ld, int a0, int b0) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
  for (int kb = 0; kb < KD; kb += 32) {
    acc = mfma_bf16(*reinterpret_cast<const bh8_t *>(a + (a0 + c) * ld + kb + 8 * g),
                    *reinterpret_cast<const bh8_t *>(b + (b0 + c) * ld + kb + 8 * g), acc);
  }
  return acc;
}

typedef short bw_i16x4_t __attribute__((ext_vector_type(4)));

// x (rows k0 .. k0+3 of column c) into a transposed pair of bf16 tiles
// (high at hiT, low 16 rows of ld after it): 8 bytes each.
__device__ __forceinline__ void put_t_pair(u16 *hiT, int ld, int k0, int c, float4_t x) {
  v2u32_t hi, lo;
  split_bf16(x, hi, lo);
  *reinterpret_cast<v2u32_t *>(hiT + c * ld + k0) = hi;
  *reinterpret_cast<v2u32_t *>(hiT + 16 * ld + c * ld + k0) = lo;
}

// Rows row0 .. row0+15 of an A pair (high ah, low al; rows of lda) times a B
// pair given transposed (bh, bl: [16][ldb]), over k < KD: A_hi B_hi + A_hi
// B_lo + A_lo B_hi on bf16 MFMA (fp32 accurate to about 2^-16).
template <int KD>
__device__ __forceinline__ float4_t pair_times_pair(const u16 *ah, const u16 *al, int lda, int row0, const u16 *bh,
                                                    const u16 *bl, int ldb) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < KD; kb += 32) {
    const bh8_t a_h = *reinterpret_cast<const bh8_t *>(ah + (row0 + c) * lda + kb + 8 * g);
    const bh8_t a_l = *reinterpret_cast<const bh8_t *>(al + (row0 + c) * lda + kb + 8 * g);
    const bh8_t b_h = *reinterpret_cast<const bh8_t *>(bh + c * ldb + kb + 8 * g);
    const bh8_t b_l = *reinterpret_cast<const bh8_t *>(bl + c * ldb + kb + 8 * g);
    acc = mfma_bf16(a_h, b_h, acc);
    acc = mfma_bf16(a_h, b_l, acc);
    acc = mfma_bf16(a_l, b_h, acc);
  }
  return acc;
}

// The A fragment of columns col0 .. col0+15 of a row-major bf16 array (rows
// of ld) taken as rows, contraction rows k0 + 8g .. k0 + 8g + 7: two
// transposing reads (lanes 4k .. 4k+3 of group g address row k0 + 8g + k
// (+ 4), 8 bytes at column col0 + 4 (c & 3); lane c receives column col0 + c).
__device__ __forceinline__ bh8_t tr_frag(const u16 *m, int ld, int k0, int col0) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  const u16 *a = m + (k0 + 8 * g + (c >> 2)) * ld + col0 + 4 * (c & 3);
  const bw_i16x4_t lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) bw_i16x4_t *)(a));
  const bw_i16x4_t hi4 =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) bw_i16x4_t *)(a + 4 * ld));
  return __builtin_bit_cast(bh8_t, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
}

// bf16 MFMA with four k per lane: acc (16x16) += A (16x16) B (16x16); lane l,
// c = l & 15, g = l >> 4: A[m=c][k=4g..4g+3], B[k=4g..4g+3][n=c].
__device__ __forceinline__ float4_t mfma_bf16_k16(bw_i16x4_t a, bw_i16x4_t b, float4_t acc) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc, 0, 0, 0);
}

// Rows 4g .. 4g+3 of column col0 + c of a row-major 16-bit array (rows of
// ld) in lane (c, g): one transposing read (lanes 4k .. 4k+3 of group g
// address row 4g + k, 8 bytes at column col0 + 4 (c & 3)). Taken from a
// transposed tile M^T it is the A or B operand of M's rows col0 .. col0+15
// with k the 16 rows of M^T.
__device__ __forceinline__ bw_i16x4_t tr4(const u16 *m, int ld, int col0) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) bw_i16x4_t *)(m + (4 * g + (c >> 2)) * ld + col0 + 4 * (c & 3)));
}

// (columns k0 .. k0+15 of the K rows)^T times a B pair given transposed,
// over the 64 tokens: K is exact in bf16, so two products per step.
__device__ __forceinline__ float4_t kt_times_pair(const u16 *sk, int ldk, int k0, const u16 *bh, const u16 *bl,
                                                  int ldb) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ts = 0; ts < BC; ts += 32) {
    const bh8_t a = tr_frag(sk, ldk, ts, k0);
    acc = mfma_bf16(a, *reinterpret_cast<const bh8_t *>(bh + c * ldb + ts + 8 * g), acc);
    acc = mfma_bf16(a, *reinterpret_cast<const bh8_t *>(bl + c * ldb + ts + 8 * g), acc);
  }
  return acc;
}

// (columns col0 .. col0+15 of T)^T, T a high/low pair of rows of ldt, times
// a B pair given transposed, over the 64 rows of T.
__device__ __forceinline__ float4_t tt_times_pair(const u16 *th, const u16 *tl, int ldt, int col0, const u16 *bh,
                                                  const u16 *bl, int ldb) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ts = 0; ts < BC; ts += 32) {
    const bh8_t a_h = tr_frag(th, ldt, ts, col0), a_l = tr_frag(tl, ldt, ts, col0);
    const bh8_t b_h = *reinterpret_cast<const bh8_t *>(bh + c * ldb + ts + 8 * g);
    const bh8_t b_l = *reinterpret_cast<const bh8_t *>(bl + c * ldb + ts + 8 * g);
    acc = mfma_bf16(a_h, b_h, acc);
    acc = mfma_bf16(a_h, b_l, acc);
    acc = mfma_bf16(a_l, b_h, acc);
  }
  return acc;
}

// Round to the nearest bf16 (ties to even) of a finite float, as its bits.
__device__ __forceinline__ u16 bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<u16>(u >> 16);
}

// Element i of an output of the kernel's input type from float, with the
// rounding store_elem applies for that dtype, chosen at compile time (no
// branch on the runtime dtype around each store).
template <typename TIn>
__device__ __forceinline__ void store_el(void *p, long i, float x) {
  if constexpr (sizeof(TIn) == 4) {
    static_cast<float *>(p)[i] = x;
  } else if constexpr (std::is_same<TIn, u16>::value) {
    static_cast<u16 *>(p)[i] = float_to_bf16_bits(x);
  } else {
    static_cast<half_t *>(p)[i] = static_cast<half_t>(x);
  }
}

// The value of a bf16 high/low pair.
__device__ __forceinline__ float pair_val(const u16 *m, int lo_off, int e) {
  return __uint_as_float(static_cast<uint32_t>(m[e]) << 16) + __uint_as_float(static_cast<uint32_t>(m[lo_off + e]) << 16);
}

// x as a bf16 high/low pair: element e of the high array, e + lo_off of the low.
__device__ __forceinline__ void put_pair1(u16 *m, int lo_off, int e, float x) {
  const u16 hi = bf16_bits(x);
  m[e] = hi;
  m[lo_off + e] = bf16_bits(x - __uint_as_float(static_cast<uint32_t>(hi) << 16));
}

// Workspace records of (batch b, value head h, chunk i).
__device__ __forceinline__ long rec(const BwdParams &p, int b, int h, int i) {
  return (static_cast<long>(b) * p.Hv + h) * p.n + i;
}

// A 64 x 64 float32 record (T) into LDS rows of LC floats.
__device__ __forceinline__ void load_t(float *st, const float *src) {
  const float4_t *w = reinterpret_cast<const float4_t *>(src);
  float4_t raw[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) raw[m] = w[threadIdx.x + BNT * m];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int e = threadIdx.x + BNT * m;
    *reinterpret_cast<float4_t *>(&st[(e >> 4) * LC + 4 * (e & 15)]) = raw[m];
  }
}

// A 64 x 64 float32 record (T) into LDS as a bf16 high/low pair of rows ld.
__device__ __forceinline__ void load_t_pair(u16 *tp, int ld, const float *src) {
  const float4_t *w = reinterpret_cast<const float4_t *>(src);
  float4_t raw[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) raw[m] = w[threadIdx.x + BNT * m];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int e = threadIdx.x + BNT * m;
    v2u32_t hi, lo;
    split_bf16(raw[m], hi, lo);
    *reinterpret_cast<v2u32_t *>(tp + (e >> 4) * ld + 4 * (e & 15)) = hi;
    *reinterpret_cast<v2u32_t *>(tp + BC * ld + (e >> 4) * ld + 4 * (e & 15)) = lo;
  }
}

// c (in-chunk cumulative log decay), e^c, e^(c_last - c) and beta of one chunk,
// from the workspace record (c, and beta as float: 0 past T). Every lane
// loads; the first wave stores.
__device__ __forceinline__ void load_decays(const BwdParams &p, int b, int h, int i, float *sc, float *sgam, float *se,
                                            float *sbeta) {
  const int tid = threadIdx.x;
  const long r = rec(p, b, h, i) * BC;
  const float c = p.ws_c[r + (tid & (BC - 1))], last = p.ws_c[r + BC - 1], bt = p.ws_beta[r + (tid & (BC - 1))];
  if (tid < BC) {
    sc[tid] = c;
    sgam[tid] = expf(c);
    se[tid] = expf(last - c);
    sbeta[tid] = bt;
  }
}

// ---------------------------------------------------------------------------
// Per (chunk, value head): T, dU0 = M^T dO, J = scale (Gamma Q)^T dO, c and
// beta as float.
// ---------------------------------------------------------------------------
// Rows t0 .. t0+63 of a [B,T,H,W] tensor of TIn (head hd, columns 0 ..
// COLS-1) as 16-byte pieces in registers, then into LDS as they are (rows of
// ld elements, ld a multiple of 16 bytes), zero past T. Every lane issues the
// same loads (rows clamped into the sequence, zeroed after), so a kernel can
// issue several tensors' rows before its first wait, and that wait is one
// round trip rather than one per tensor.
template <typename TIn, int COLS>
struct RawRows {
  static constexpr int EPP = 16 / sizeof(TIn), PPR = COLS / EPP, TOTAL = BC * PPR, PER = TOTAL / BNT;
  static_assert(TOTAL % BNT == 0, "whole pieces per thread");
  uint4 raw[PER];

  __device__ __forceinline__ void load(const void *src, const BwdParams &p, int b, int t0, int heads, int hd,
                                       int width) {
    const unsigned char *base = static_cast<const unsigned char *>(src);
#pragma unroll
    for (int m = 0; m < PER; ++m) {
      const int e = threadIdx.x + BNT * m, row = e / PPR, part = e % PPR, t = t0 + row, tc = t < p.T ? t : p.T - 1;
      const long off = ((static_cast<long>(b) * p.T + tc) * heads + hd) * width * static_cast<long>(sizeof(TIn));
      const uint4 x = *reinterpret_cast<const uint4 *>(base + off + part * 16);
      raw[m] = t < p.T ? x : uint4{0u, 0u, 0u, 0u};
    }
  }
  __device__ __forceinline__ void put(TIn *dst, int ld) const {
#pragma unroll
    for (int m = 0; m < PER; ++m) {
      const int e = threadIdx.x + BNT * m, row = e / PPR, part = e % PPR;
      *reinterpret_cast<uint4 *>(&dst[row * ld + part * EPP]) = raw[m];
    }
  }
};

// q, k and dO stay in LDS in the input dtype (converted on read), and M is
// formed in A's place once T has been written out: 72 KiB for 16-bit inputs at
// K = V = 128, so two workgroups share a CU.
template <int K, int V, typename TIn>
constexpr size_t local_lds() {
  return sizeof(TIn) * BC * (2 * (K + 16 / sizeof(TIn)) + V + 16 / sizeof(TIn)) +
         sizeof(float) * (BC * LC + 3 * BC + 3 * 256);
}

template <int K, int V, typename TIn>
__global__ __launch_bounds__(BNT) void bwd_local_kernel(BwdParams p) {
  constexpr int PADE = 16 / sizeof(TIn), LK = K + PADE, LV = V + PADE;
  extern __shared__ __align__(16) float lds[];
  PBGDN_POISON_LDS(lds, (local_lds<K, V, TIn>()));
  PBGDN_POISON_SYNC();
  TIn *sq = reinterpret_cast<TIn *>(lds), *sk = sq + BC * LK, *sdo = sk + BC * LK;
  float *sa = reinterpret_cast<float *>(sdo + BC * LV);
  float *sc = sa + BC * LC, *sgam = sc + BC, *sbeta = sgam + BC, *sr = sbeta + BC;
  // bf16 inputs: M as a bf16 high/low pair (rows of LM) in sa's bytes, and
  // dU0, J on bf16 MFMA
  constexpr bool BF = std::is_same<TIn, u16>::value;
  constexpr int LM = LC;
  u16 *mh = reinterpret_cast<u16 *>(sa);
  const int i = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = lane & 15, g4 = lane >> 4;
  const int hk = h / (p.Hv / p.Hk);
  const int t0 = i * BC;
  {
    RawRows<TIn, K> rq, rk;
    RawRows<TIn, V> rd;
    rq.load(p.q, p, b, t0, p.Hk, hk, K);
    rk.load(p.k, p, b, t0, p.Hk, hk, K);
    rd.load(p.dout, p, b, t0, p.Hv, h, V);
    rq.put(sq, LK);
    rk.put(sk, LK);
    rd.put(sdo, LV);
  }
  if (wave == 0) {  // inclusive cumulative sum of g over the chunk (zero past T)
    const int t = t0 + lane;
    float x = t < p.T ? p.g[(static_cast<long>(b) * p.T + t) * p.Hv + h] : 0.f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(x, off, 64);
      if (lane >= off) x += y;
    }
    sc[lane] = x;
    sgam[lane] = expf(x);
    const float bt = t < p.T ? load_elem(p.beta, (static_cast<long>(b) * p.T + t) * p.Hv + h, p.beta_dtype) : 0.f;
    sbeta[lane] = bt;
    p.ws_c[rec(p, b, h, i) * BC + lane] = x;
    p.ws_beta[rec(p, b, h, i) * BC + lane] = bt;
  }
  __syncthreads();
  auto krow = [&](int kk, int j, int tc) { return ld4e(sk, (16 * tc + j) * LK + kk); };
  // A = strict_lower(beta_t (K K^T) o D), rows 16w .. of this wave
  for (int tc = 0; tc < 4; ++tc) {
    float4_t kk_acc;
    if constexpr (std::is_same<TIn, u16>::value) {
      kk_acc = rows_times_rows<K>(sk, sk, LK, 16 * wave, 16 * tc);
    } else {
      kk_acc = tile_mm4<K>(zero4(), [&](int r, int kk) { return ld4e(sk, (16 * wave + r) * LK + kk); },
                           [&](int kk, int j) { return krow(kk, j, tc); });
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * wave + 4 * g4 + r, s2 = 16 * tc + c;
      sa[t * LC + s2] = t > s2 ? sbeta[t] * kk_acc[r] * expf(sc[t] - sc[s2]) : 0.f;
    }
  }
  __syncthreads();
  // T = (I + A)^-1 (unit lower triangular) in place over A, by 16 x 16
  // blocks. Wave w inverts diagonal block w by forward substitution: lane
  // (column j, part) sums the terms s = part mod 4 of
  // T[t][j] = -sum_{s<t} A[t][s] T[s][j] (T is zero above the diagonal, A
  // too), and two shuffles add the parts; every lane reads row t before it is
  // written (one wave, one instruction stream).
  {
    const int j = lane & 15, part = lane >> 4, base = 16 * wave;
    for (int t = 0; t < 16; ++t) {
      float acc = 0.f;
      for (int s2 = part; s2 < t; s2 += 4) acc += sa[(base + t) * LC + base + s2] * sa[(base + s2) * LC + base + j];
      acc += __shfl_xor(acc, 16, 64);
      acc += __shfl_xor(acc, 32, 64);
      if (part == 0) sa[(base + t) * LC + base + j] = t == j ? 1.f : (t < j ? 0.f : -acc);
    }
  }
  __syncthreads();
  // Off-diagonal blocks, one block row at a time:
  // T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj, wave j forming block (i, j).
  for (int bi = 1; bi < 4; ++bi) {
    if (wave < bi) {
      float4_t racc = zero4();
      for (int bk = wave; bk < bi; ++bk) {
        racc = tile_mm<16>(racc, [&](int r, int kk) { return sa[(16 * bi + r) * LC + 16 * bk + kk]; },
                           [&](int kk, int col) { return sa[(16 * bk + kk) * LC + 16 * wave + col]; });
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) sr[wave * 256 + (4 * g4 + r) * 16 + c] = racc[r];
    }
    __syncthreads();  // block row bi of A is read by every wave before any T of it is written
    if (wave < bi) {
      const float4_t tacc = tile_mm<16>(zero4(), [&](int r, int kk) { return sa[(16 * bi + r) * LC + 16 * bi + kk]; },
                                        [&](int kk, int col) { return sr[wave * 256 + kk * 16 + col]; });
#pragma unroll
      for (int r = 0; r < 4; ++r) sa[(16 * bi + 4 * g4 + r) * LC + 16 * wave + c] = -tacc[r];
    }
    __syncthreads();
  }
  float *wt = p.ws_T + rec(p, b, h, i) * BC * BC;
  for (int e = tid; e < BC * BC; e += BNT) wt[e] = sa[(e / BC) * LC + e % BC];
  __syncthreads();  // T is out: M = scale (Q K^T) o D takes its place
  for (int tc = 0; tc < 4; ++tc) {
    float4_t qk_acc;
    if constexpr (std::is_same<TIn, u16>::value) {
      qk_acc = rows_times_rows<K>(sq, sk, LK, 16 * wave, 16 * tc);
    } else {
      qk_acc = tile_mm4<K>(zero4(), [&](int r, int kk) { return ld4e(sq, (16 * wave + r) * LK + kk); },
                           [&](int kk, int j) { return krow(kk, j, tc); });
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * wave + 4 * g4 + r, s2 = 16 * tc + c;
      const float mv = t >= s2 ? p.scale * qk_acc[r] * expf(sc[t] - sc[s2]) : 0.f;
      if constexpr (BF) {  // M as a bf16 high/low pair, rows of LM, in sa's bytes
        const u16 hi = bf16_bits(mv);
        mh[t * LM + s2] = hi;
        mh[BC * LM + t * LM + s2] = bf16_bits(mv - __uint_as_float(static_cast<uint32_t>(hi) << 16));
      } else {
        sa[t * LC + s2] = mv;
      }
    }
  }
  __syncthreads();
  // dU0 = M^T dO: tiles (row tile, 16-column tile)
  float *wu = p.ws_dU0 + rec(p, b, h, i) * BC * V;
  if constexpr (BF) {  // M^T fragments and dO's columns by transposing reads
    for (int tile = wave; tile < 4 * (V / 16); tile += 4) {
      const int tr = tile & 3, tv = tile >> 2;
      float4_t acc = zero4();
#pragma unroll
      for (int ts = 0; ts < BC; ts += 32) {
        const bh8_t d = tr_frag(sdo, LV, ts, 16 * tv);
        acc = mfma_bf16(tr_frag(mh, LM, ts, 16 * tr), d, acc);
        acc = mfma_bf16(tr_frag(mh + BC * LM, LM, ts, 16 * tr), d, acc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) wu[(16 * tr + 4 * g4 + r) * V + 16 * tv + c] = acc[r];
    }
  }
  for (int tile = wave; tile < (BF ? 0 : 4 * (V / 16)); tile += 4) {
    const int tr = tile & 3, tv = tile >> 2;
    const float4_t acc = tile_mm4<BC>(zero4(), [&](int r, int s2) { return ld4s(&sa[s2 * LC + 16 * tr + r], LC); },
                                      [&](int s2, int col) {
                                        const int e = s2 * LV + 16 * tv + col;
                                        return float4_t{ld_el(sdo, e), ld_el(sdo, e + LV), ld_el(sdo, e + 2 * LV),
                                                        ld_el(sdo, e + 3 * LV)};
                                      });
#pragma unroll
    for (int r = 0; r < 4; ++r) wu[(16 * tr + 4 * g4 + r) * V + 16 * tv + c] = acc[r];
  }
  // J = scale (Gamma Q)^T dO: K x V
  float *wj = p.ws_J + rec(p, b, h, i) * static_cast<long>(K) * V;
  if constexpr (BF) {
    // per column tile of this wave: (Gamma dO)'s columns as bf16 pairs once,
    // then every key tile's Q^T fragments (transposing reads of the q rows)
    for (int tv = wave; tv < V / 16; tv += 4) {
      bh8_t bh[2], bl[2];
#pragma unroll
      for (int s8 = 0; s8 < 2; ++s8) {
        const v4u32_t w = __builtin_bit_cast(v4u32_t, tr_frag(sdo, LV, 32 * s8, 16 * tv));
        const float4_t g0 = ld4(&sgam[32 * s8 + 8 * g4]), g1 = ld4(&sgam[32 * s8 + 8 * g4 + 4]);
        const float4_t x0 = float4_t{__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u),
                                     __uint_as_float(w[1] << 16), __uint_as_float(w[1] & 0xffff0000u)} * g0;
        const float4_t x1 = float4_t{__uint_as_float(w[2] << 16), __uint_as_float(w[2] & 0xffff0000u),
                                     __uint_as_float(w[3] << 16), __uint_as_float(w[3] & 0xffff0000u)} * g1;
        v2u32_t h0, l0, h1, l1;
        split_bf16(x0, h0, l0);
        split_bf16(x1, h1, l1);
        bh[s8] = __builtin_bit_cast(bh8_t, v4u32_t{h0[0], h0[1], h1[0], h1[1]});
        bl[s8] = __builtin_bit_cast(bh8_t, v4u32_t{l0[0], l0[1], l1[0], l1[1]});
      }
      for (int tk = 0; tk < K / 16; ++tk) {
        float4_t acc = zero4();
#pragma unroll
        for (int s8 = 0; s8 < 2; ++s8) {
          const bh8_t a = tr_frag(sq, LK, 32 * s8, 16 * tk);
          acc = mfma_bf16(a, bh[s8], acc);
          acc = mfma_bf16(a, bl[s8], acc);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) wj[(16 * tk + 4 * g4 + r) * V + 16 * tv + c] = p.scale * acc[r];
      }
    }
  }
  for (int tile = wave; tile < (BF ? 0 : (K / 16) * (V / 16)); tile += 4) {
    const int tk = tile % (K / 16), tv = tile / (K / 16);
    const float4_t acc = tile_mm4<BC>(
        zero4(),
        [&](int r, int t) {
          const int e = t * LK + 16 * tk + r;
          return float4_t{ld_el(sq, e), ld_el(sq, e + LK), ld_el(sq, e + 2 * LK), ld_el(sq, e + 3 * LK)} *
                 ld4(&sgam[t]);
        },
        [&](int t, int col) {
          const int e = t * LV + 16 * tv + col;
          return float4_t{ld_el(sdo, e), ld_el(sdo, e + LV), ld_el(sdo, e + 2 * LV), ld_el(sdo, e + 3 * LV)};
        });
#pragma unroll
    for (int r = 0; r < 4; ++r) wj[(16 * tk + 4 * g4 + r) * V + 16 * tv + c] = p.scale * acc[r];
  }
}

// One chunk's inputs to a scan step, held in registers a step ahead: K rows
// (16-byte pieces of TIn), T, c and beta, and the step's 16-column tile (V for
// the forward pass; dU0 and J, the latter in the accumulator layout, for the
// reverse pass). Loaded while the previous step computes, written to LDS
// between steps.
template <int K, typename TIn, bool ADJ>
struct ScanStage {
  static constexpr int EPP = 16 / sizeof(TIn);  // elements per 16-byte piece
  static constexpr int ROW16 = K / EPP;         // pieces per K row
  static constexpr int KP = BC * ROW16 / BNT;   // K pieces per thread
  static constexpr int TILE16 = 16 / EPP;       // pieces per row of a 16-column tile
  uint4 kr[KP];
  float4_t tr[4];
  float cv, bv;
  uint4 xr;
  float4_t dur;
  float jr[K / 64][4];

  __device__ __forceinline__ void load(const BwdParams &p, int b, int h, int hk, int i, int v0) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = lane & 15, g4 = lane >> 4;
    const int t0 = i * BC;
    const long r = rec(p, b, h, i);
    const unsigned char *kb = static_cast<const unsigned char *>(p.k);
#pragma unroll
    for (int m = 0; m < KP; ++m) {
      // rows clamped into the sequence and zeroed after: every path issues
      // the same loads, so the waits for them can be partial
      const int e = tid + BNT * m, row = e / ROW16, part = e % ROW16, t = t0 + row, tc = t < p.T ? t : p.T - 1;
      const long off = ((static_cast<long>(b) * p.T + tc) * p.Hk + hk) * K * static_cast<long>(sizeof(TIn)) + part * 16;
      const uint4 kx = *reinterpret_cast<const uint4 *>(kb + off);
      kr[m] = t < p.T ? kx : uint4{0u, 0u, 0u, 0u};
    }
    const float4_t *wt = reinterpret_cast<const float4_t *>(p.ws_T + r * BC * BC);
#pragma unroll
    for (int m = 0; m < 4; ++m) tr[m] = wt[tid + BNT * m];
    // every lane loads (wave 0's values are used): c and beta as float from
    // the workspace, no load that only some paths issue
    cv = p.ws_c[r * BC + (tid & (BC - 1))];
    bv = p.ws_beta[r * BC + (tid & (BC - 1))];
    if constexpr (!ADJ) {
      const int row = tid / TILE16, part = tid % TILE16, t = t0 + row;
      const unsigned char *vb = static_cast<const unsigned char *>(p.v);
      const long off = (((static_cast<long>(b) * p.T + t) * p.Hv + h) * p.V + v0) * static_cast<long>(sizeof(TIn)) +
                       part * 16;
      xr = tid < BC * TILE16 && t < p.T ? *reinterpret_cast<const uint4 *>(vb + off) : uint4{0u, 0u, 0u, 0u};
    } else {
      dur = *reinterpret_cast<const float4_t *>(p.ws_dU0 + r * BC * p.V + (tid >> 2) * p.V + v0 + 4 * (tid & 3));
      const float *wj = p.ws_J + r * K * p.V;
#pragma unroll
      for (int m = 0; m < K / 64; ++m) {
#pragma unroll
        for (int q = 0; q < 4; ++q) jr[m][q] = wj[static_cast<long>(16 * (wave + 4 * m) + 4 * g4 + q) * p.V + v0 + c];
      }
    }
  }

  // K rows, T, the decays and the tile into LDS (sk, st, vectors, tile). K
  // rows go in as they are for bf16 inputs (rows of K + 8), else as float
  // (rows of K + 4).
  __device__ __forceinline__ void store(void *sk, void *st, float *sc, float *sgam, float *se, float *sbeta,
                                        float *tile) const {
    const int tid = threadIdx.x;
#pragma unroll
    for (int m = 0; m < KP; ++m) {
      const int e = tid + BNT * m, row = e / ROW16, part = e % ROW16;
      if constexpr (std::is_same<TIn, u16>::value) {
        *reinterpret_cast<uint4 *>(static_cast<u16 *>(sk) + row * (K + 8) + part * EPP) = kr[m];
      } else {
        float x[EPP];
        decode16<TIn>(kr[m], x);
#pragma unroll
        for (int j = 0; j < EPP; j += 4) {
          *reinterpret_cast<float4_t *>(static_cast<float *>(sk) + row * (K + 4) + part * EPP + j) =
              float4_t{x[j], x[j + 1], x[j + 2], x[j + 3]};
        }
      }
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int e = tid + BNT * m;
      if constexpr (std::is_same<TIn, u16>::value) {  // T as bf16 high/low rows of BC + 8
        u16 *th = static_cast<u16 *>(st);
        v2u32_t hi, lo;
        split_bf16(tr[m], hi, lo);
        *reinterpret_cast<v2u32_t *>(th + (e >> 4) * (BC + 8) + 4 * (e & 15)) = hi;
        *reinterpret_cast<v2u32_t *>(th + BC * (BC + 8) + (e >> 4) * (BC + 8) + 4 * (e & 15)) = lo;
      } else {
        *reinterpret_cast<float4_t *>(static_cast<float *>(st) + (e >> 4) * LC + 4 * (e & 15)) = tr[m];
      }
    }
    if (tid < BC) {
      const float last = __shfl(cv, BC - 1, 64);
      sc[tid] = cv;
      sgam[tid] = expf(cv);
      se[tid] = expf(last - cv);
      sbeta[tid] = bv;
    }
    if constexpr (!ADJ) {
      if (tid < BC * TILE16) {
        float x[EPP];
        decode16<TIn>(xr, x);
#pragma unroll
        for (int j = 0; j < EPP; j += 4) {
          *reinterpret_cast<float4_t *>(&tile[(tid / TILE16) * LT + (tid % TILE16) * EPP + j]) =
              float4_t{x[j], x[j + 1], x[j + 2], x[j + 3]};
        }
      }
    } else {
      *reinterpret_cast<float4_t *>(&tile[(tid >> 2) * LT + 4 * (tid & 3)]) = dur;
    }
  }
};

// ---------------------------------------------------------------------------
// Forward over the chunks for 16 value columns: the state at every chunk
// start. Wave w holds key-row tiles w, w+4 (K/64 of them) of the state. The
// next chunk's inputs load during each step.
// ---------------------------------------------------------------------------
// LDS of one scan workgroup. bf16 inputs: K rows as they are and the state
// tile as its transpose in bf16 high/low parts (for K S on bf16 MFMA); other
// inputs: K rows and the state tile in float.
template <int K, typename TIn>
struct ScanLds {
  static constexpr bool BF = std::is_same<TIn, u16>::value;
  static constexpr int LK = BF ? K + 8 : K + 4, LS = K + 8, LB = BC + 8;
  // K rows; T (bf16: high and low parts, rows of LB); the state tile (bf16:
  // its transpose, high and low); the step's V or dU0 tile in float; the
  // tiles the next products read (bf16: two transposed high/low pairs
  // [16][LB], float: one [64][LT] tile); decay vectors.
  static constexpr size_t K_BYTES = BF ? sizeof(u16) * BC * LK : sizeof(float) * BC * LK;
  static constexpr size_t T_BYTES = BF ? sizeof(u16) * 2 * BC * LB : sizeof(float) * BC * LC;
  static constexpr size_t S_BYTES = BF ? sizeof(u16) * 2 * 16 * LS : sizeof(float) * K * LT;
  static constexpr size_t A_BYTES = BF ? sizeof(u16) * 2 * 2 * 16 * LB : sizeof(float) * BC * LT;
  static constexpr size_t OFF_T = K_BYTES, OFF_S = OFF_T + T_BYTES, OFF_TILE = OFF_S + S_BYTES,
                          OFF_A = OFF_TILE + sizeof(float) * BC * LT, OFF_VEC = OFF_A + A_BYTES;
  static constexpr size_t BYTES = OFF_VEC + sizeof(float) * 4 * BC;
};

// K rows (row0 + r) times the state tile kept in LDS: bf16 MFMA on the high
// and low parts of its transpose, or the fp32 MFMA on the float tile.
template <int K, typename TIn>
__device__ __forceinline__ float4_t k_times_state(const void *sk, int row0, const void *sstate) {
  using L = ScanLds<K, TIn>;
  if constexpr (L::BF) {
    const u16 *hiT = static_cast<const u16 *>(sstate);
    return rows_times_state<K>(static_cast<const u16 *>(sk), L::LK, row0, hiT, hiT + 16 * L::LS, L::LS);
  } else {
    const float *kf = static_cast<const float *>(sk), *sf = static_cast<const float *>(sstate);
    return tile_mm4<K>(zero4(), [&](int r, int kk) { return ld4(&kf[(row0 + r) * L::LK + kk]); },
                       [&](int kk, int col) { return ld4s(&sf[kk * LT + col], LT); });
  }
}

// Rows kk0 .. kk0+3 (4 g4 + 16 m ..) of the state tile, column c, into LDS: the
// float tile, or the high/low parts of its transpose (8 bytes each).
template <int K, typename TIn>
__device__ __forceinline__ void put_state_rows(void *sstate, int kk0, int c, float4_t x) {
  using L = ScanLds<K, TIn>;
  if constexpr (L::BF) {
    u16 *hiT = static_cast<u16 *>(sstate);
    v2u32_t hi, lo;
    split_bf16(x, hi, lo);
    *reinterpret_cast<v2u32_t *>(hiT + c * L::LS + kk0) = hi;
    *reinterpret_cast<v2u32_t *>(hiT + 16 * L::LS + c * L::LS + kk0) = lo;
  } else {
    float *sf = static_cast<float *>(sstate);
#pragma unroll
    for (int r = 0; r < 4; ++r) sf[(kk0 + r) * LT + c] = x[r];
  }
}

// (diag(w) K)^T rows k0 + r, four tokens t .. t+3 of the K rows in LDS.
template <int K, typename TIn>
__device__ __forceinline__ float4_t k_cols(const void *sk, int t, int col) {
  using L = ScanLds<K, TIn>;
  if constexpr (L::BF) {
    return ld4es(static_cast<const u16 *>(sk), t * L::LK + col, L::LK);
  } else {
    return ld4s(static_cast<const float *>(sk) + t * L::LK + col, L::LK);
  }
}

template <int K, typename TIn>
__device__ __forceinline__ void state_pass(const BwdParams &p, float *lds, int b, int h, int v0) {
  using L = ScanLds<K, TIn>;
  constexpr int PER = K / 64, LB = L::LB;
  unsigned char *base = reinterpret_cast<unsigned char *>(lds);
  void *sk = base, *st = base + L::OFF_T, *ss = base + L::OFF_S;
  float *sx = reinterpret_cast<float *>(base + L::OFF_TILE), *su = reinterpret_cast<float *>(base + L::OFF_A);
  float *sc = reinterpret_cast<float *>(base + L::OFF_VEC), *sgam = sc + BC, *se = sgam + BC, *sbeta = se + BC;
  // bf16 inputs: (beta X)^T and (E U)^T as high/low pairs
  u16 *xT = reinterpret_cast<u16 *>(base + L::OFF_A), *uT = xT + 2 * 16 * LB;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = lane & 15, g4 = lane >> 4;
  const int hk = h / (p.Hv / p.Hk);
  const long kv = (static_cast<long>(b) * p.Hv + h) * K * p.V;
  float4_t s[PER];
#pragma unroll
  for (int m = 0; m < PER; ++m) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int kk = 16 * (wave + 4 * m) + 4 * g4 + r;
      s[m][r] = p.h0 ? p.h0[kv + static_cast<long>(kk) * p.V + v0 + c] : 0.f;
    }
  }
  ScanStage<K, TIn, false> stage;
  if (p.n > 0) stage.load(p, b, h, hk, 0, v0);
  for (int i = 0; i < p.n; ++i) {
    float *ws = p.ws_S + rec(p, b, h, i) * K * p.V;
#pragma unroll
    for (int m = 0; m < PER; ++m) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kk = 16 * (wave + 4 * m) + 4 * g4 + r;
        ws[static_cast<long>(kk) * p.V + v0 + c] = s[m][r];
      }
      put_state_rows<K, TIn>(ss, 16 * (wave + 4 * m) + 4 * g4, c, s[m]);
    }
    stage.store(sk, st, sc, sgam, se, sbeta, sx);
    if (i + 1 < p.n) stage.load(p, b, h, hk, i + 1, v0);
    __syncthreads();
    // X = V - Gamma K S (rows 16w ..)
    const float4_t ks = k_times_state<K, TIn>(sk, 16 * wave, ss);
    if constexpr (L::BF) {
      float4_t xb;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * wave + 4 * g4 + r;
        xb[r] = (sx[t * LT + c] - sgam[t] * ks[r]) * sbeta[t];
      }
      put_t_pair(xT, LB, 16 * wave + 4 * g4, c, xb);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * wave + 4 * g4 + r;
        sx[t * LT + c] -= sgam[t] * ks[r];
      }
    }
    __syncthreads();
    // U = T diag(beta) X
    if constexpr (L::BF) {
      const u16 *th = static_cast<const u16 *>(st);
      const float4_t u = pair_times_pair<BC>(th, th + BC * LB, LB, 16 * wave, xT, xT + 16 * LB, LB);
      float4_t eu;
#pragma unroll
      for (int r = 0; r < 4; ++r) eu[r] = se[16 * wave + 4 * g4 + r] * u[r];
      put_t_pair(uT, LB, 16 * wave + 4 * g4, c, eu);
    } else {
      const float *stf = static_cast<const float *>(st);
      const float4_t u = tile_mm4<BC>(
          zero4(), [&](int r, int s2) { return ld4(&stf[(16 * wave + r) * LC + s2]) * ld4(&sbeta[s2]); },
          [&](int s2, int col) { return ld4s(&sx[s2 * LT + col], LT); });
#pragma unroll
      for (int r = 0; r < 4; ++r) su[(16 * wave + 4 * g4 + r) * LT + c] = u[r];
    }
    __syncthreads();
    // S = gamma_C S + K^T E U
    const float gam_c = sgam[BC - 1];
#pragma unroll
    for (int m = 0; m < PER; ++m) {
      const int k0 = 16 * (wave + 4 * m);
      float4_t y;
      if constexpr (L::BF) {
        y = kt_times_pair(static_cast<const u16 *>(sk), L::LK, k0, uT, uT + 16 * LB, LB);
      } else {
        y = tile_mm4<BC>(zero4(), [&](int r, int t) { return k_cols<K, TIn>(sk, t, k0 + r) * ld4(&se[t]); },
                         [&](int t, int col) { return ld4s(&su[t * LT + col], LT); });
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) s[m][r] = gam_c * s[m][r] + y[r];
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Backward over the chunks for 16 value columns: the adjoint dS' at every
// chunk end (the input of that chunk's gradients), then dh0.
// ---------------------------------------------------------------------------
template <int K, typename TIn>
__device__ __forceinline__ void adjoint_pass(const BwdParams &p, float *lds, int b, int h, int v0) {
  using L = ScanLds<K, TIn>;
  constexpr int PER = K / 64, LB = L::LB;
  unsigned char *base = reinterpret_cast<unsigned char *>(lds);
  void *sk = base, *st = base + L::OFF_T, *sds = base + L::OFF_S;
  float *sdu = reinterpret_cast<float *>(base + L::OFF_TILE), *sdx = reinterpret_cast<float *>(base + L::OFF_A);
  float *sc = reinterpret_cast<float *>(base + L::OFF_VEC), *sgam = sc + BC, *se = sgam + BC, *sbeta = se + BC;
  // bf16 inputs: dU^T and (Gamma dX)^T as high/low pairs
  u16 *duT = reinterpret_cast<u16 *>(base + L::OFF_A), *gxT = duT + 2 * 16 * LB;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = lane & 15, g4 = lane >> 4;
  const int hk = h / (p.Hv / p.Hk);
  const long kv = (static_cast<long>(b) * p.Hv + h) * K * p.V;
  float4_t ds[PER];
#pragma unroll
  for (int m = 0; m < PER; ++m) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int kk = 16 * (wave + 4 * m) + 4 * g4 + r;
      ds[m][r] = p.dht ? p.dht[kv + static_cast<long>(kk) * p.V + v0 + c] : 0.f;
    }
  }
  ScanStage<K, TIn, true> stage;
  if (p.n > 0) stage.load(p, b, h, hk, p.n - 1, v0);
  for (int i = p.n - 1; i >= 0; --i) {
    float *wds = p.ws_dS + rec(p, b, h, i) * K * p.V;
#pragma unroll
    for (int m = 0; m < PER; ++m) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kk = 16 * (wave + 4 * m) + 4 * g4 + r;
        wds[static_cast<long>(kk) * p.V + v0 + c] = ds[m][r];
      }
      put_state_rows<K, TIn>(sds, 16 * (wave + 4 * m) + 4 * g4, c, ds[m]);
    }
    stage.store(sk, st, sc, sgam, se, sbeta, sdu);
    float jv[PER][4];
#pragma unroll
    for (int m = 0; m < PER; ++m) {
#pragma unroll
      for (int r = 0; r < 4; ++r) jv[m][r] = stage.jr[m][r];
    }
    if (i > 0) stage.load(p, b, h, hk, i - 1, v0);
    __syncthreads();
    // dU = dU0 + E K dS'
    const float4_t kd = k_times_state<K, TIn>(sk, 16 * wave, sds);
    if constexpr (L::BF) {
      float4_t du;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * wave + 4 * g4 + r;
        du[r] = sdu[t * LT + c] + se[t] * kd[r];
      }
      put_t_pair(duT, LB, 16 * wave + 4 * g4, c, du);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * wave + 4 * g4 + r;
        sdu[t * LT + c] += se[t] * kd[r];
      }
    }
    __syncthreads();
    // dX = (T diag(beta))^T dU
    if constexpr (L::BF) {
      const u16 *th = static_cast<const u16 *>(st);
      const float4_t dx = tt_times_pair(th, th + BC * LB, LB, 16 * wave, duT, duT + 16 * LB, LB);
      float4_t gx;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * wave + 4 * g4 + r;
        gx[r] = sgam[t] * (sbeta[t] * dx[r]);
      }
      put_t_pair(gxT, LB, 16 * wave + 4 * g4, c, gx);
    } else {
      const float *stf = static_cast<const float *>(st);
      const float4_t dx = tile_mm4<BC>(
          zero4(), [&](int r, int s2) { return ld4s(&stf[s2 * LC + 16 * wave + r], LC) * sbeta[16 * wave + r]; },
          [&](int s2, int col) { return ld4s(&sdu[s2 * LT + col], LT); });
#pragma unroll
      for (int r = 0; r < 4; ++r) sdx[(16 * wave + 4 * g4 + r) * LT + c] = dx[r];
    }
    __syncthreads();
    // dS = gamma_C dS' + J - (Gamma K)^T dX
    const float gam_c = sgam[BC - 1];
#pragma unroll
    for (int m = 0; m < PER; ++m) {
      const int k0 = 16 * (wave + 4 * m);
      float4_t y;
      if constexpr (L::BF) {
        y = kt_times_pair(static_cast<const u16 *>(sk), L::LK, k0, gxT, gxT + 16 * LB, LB);
      } else {
        y = tile_mm4<BC>(zero4(), [&](int r, int t) { return k_cols<K, TIn>(sk, t, k0 + r) * ld4(&sgam[t]); },
                         [&](int t, int col) { return ld4s(&sdx[t * LT + col], LT); });
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) ds[m][r] = gam_c * ds[m][r] + jv[m][r] - y[r];
    }
    __syncthreads();
  }
  if (p.dh0) {
#pragma unroll
    for (int m = 0; m < PER; ++m) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kk = 16 * (wave + 4 * m) + 4 * g4 + r;
        p.dh0[kv + static_cast<long>(kk) * p.V + v0 + c] = ds[m][r];
      }
    }
  }
}

// The two scans are independent (the reverse one needs the per-chunk records
// and dht, not the states), so one launch runs both: pair z = (role, batch
// row, value head), role 0 the forward pass, 1 the reverse pass. Two
// workgroups fit a CU, so each CU overlaps a forward and a reverse scan.
// Workgroups go to the XCDs round-robin by linear index; the V/16 tiles of
// one pair read the same K rows and T records every step, so when the pairs
// fill the XCDs evenly all tiles of a pair are given indices on one XCD
// (xcd_group) and those reads come from its L2 after the first.
template <int K, typename TIn>
constexpr size_t scan_lds();
template <int K, typename TIn>
constexpr size_t grad_lds();

template <int K, typename TIn>
__global__ __launch_bounds__(BNT) void bwd_scans_kernel(BwdParams p) {
  extern __shared__ __align__(16) float lds[];
  PBGDN_POISON_LDS(lds, (scan_lds<K, TIn>()));
  PBGDN_POISON_SYNC();
  const int tiles = p.V / 16, pairs = 2 * p.B * p.Hv;
  const int l = blockIdx.x;
  int pair, tile;
  xcd_group(l, pairs, tiles, p.xcds, pair, tile);
  const int role_b = pair / p.Hv, h = pair % p.Hv;
  if (role_b < p.B) {
    state_pass<K, TIn>(p, lds, role_b, h, 16 * tile);
  } else {
    adjoint_pass<K, TIn>(p, lds, role_b - p.B, h, 16 * tile);
  }
}

// ---------------------------------------------------------------------------
// Per (chunk, value head): the gradients, from the chunk's start state S and
// end adjoint dS'. Eight waves, two per SIMD: waves w and w+4 share token rows
// 16w .. 16w+15 (w = wave & 3) and split the column tiles of every product
// that has more than one; the chain X -> U -> dU -> dX (one 16-column tile per
// row block) runs on waves 0-3 while waves 4-7 form Q S and its dgamma term.
// ---------------------------------------------------------------------------
constexpr int GNT = 512;

// Floats of the gradient kernel's area: the value-column tiles during the
// loop over them (bf16 inputs: S, dS', V/X, dU in float, five transposed bf16
// pairs and the dO rows; else seven float tiles), then the three C x C
// matrices (bf16 inputs: one in float, two as bf16 pairs of rows BC + 8).
template <int K, bool BF>
constexpr int grad_area() {
  constexpr int tiles = BF ? 2 * K * LT + 2 * BC * LT + (6 * 2 * 16 * (BC + 8) + BC * 24) / 2 : 2 * K * LT + 5 * BC * LT;
  constexpr int tri = BF ? 3 * BC * (BC + 8) : 3 * BC * LC;
  return tri > tiles ? tri : tiles;
}

template <int K, int V, typename TIn>
__global__ __launch_bounds__(GNT) void bwd_grad_kernel(BwdParams p) {
  constexpr int LK = K + 16 / sizeof(TIn), KT = K / 16, KH = KT / 2, LS = K + 8;
  // bf16 inputs: K S, K dS' and Q S on bf16 MFMA (q, k exact; the state
  // tiles as high + low parts); other input types on the fp32 MFMA
  constexpr bool BF = std::is_same<TIn, u16>::value;
  extern __shared__ __align__(16) float lds[];
  PBGDN_POISON_LDS(lds, (grad_lds<K, TIn>()));
  PBGDN_POISON_SYNC();
  constexpr int LB = BC + 8, LO = 16 + 8, PAIR = 2 * 16 * LB;
  // T and M: float rows of LC, or (bf16 inputs) bf16 high/low pairs of rows LB
  constexpr int TSZ = BF ? BC * LB : BC * LC;
  TIn *sq = reinterpret_cast<TIn *>(lds), *sk = sq + BC * LK;  // q, k rows as they are
  float *st = reinterpret_cast<float *>(sk + BC * LK), *sm = st + TSZ;
  u16 *tp = reinterpret_cast<u16 *>(st), *mp = reinterpret_cast<u16 *>(sm);
  float *area = sm + TSZ;  // the value-column tiles, then three C x C matrices
  float *ss = area, *sds = ss + K * LT, *sx = sds + K * LT, *sdo = sx + BC * LT, *su = sdo + BC * LT;
  float *sdu = su + BC * LT, *sdx = sdu + BC * LT;
  // bf16 inputs: the per-tile products take their operands from transposed
  // bf16 high/low pairs [16][LB] (X^T, dU^T, U^T, (E U)^T, (-Gamma dX)^T,
  // (beta X)^T) and dO rows as they are [64][LO]; sdu follows sx and these
  // replace sdo, su, sdx
  if constexpr (BF) sdu = sx + BC * LT;
  u16 *xT = reinterpret_cast<u16 *>(sdu + BC * LT), *duT = xT + PAIR, *uT = duT + PAIR, *euT = uT + PAIR,
      *gxT = euT + PAIR, *bxT = gxT + PAIR, *sdo16 = bxT + PAIR;
  float *b1 = area, *b2 = b1 + BC * LC, *b3 = b2 + BC * LC;
  // bf16 inputs: dT (then W), dM o Mt and H + H^T as bf16 high/low pairs, rows of LB
  u16 *b2p = reinterpret_cast<u16 *>(area), *b1p = b2p + 2 * BC * LB, *b3p = b1p + 2 * BC * LB;
  float *vec = area + grad_area<K, BF>();
  float *sc = vec, *sgam = sc + BC, *se = sgam + BC, *sbeta = se + BC;
  float *sdgam = sbeta + BC, *sde = sdgam + BC;
  // per-wave sums of the dc and dbeta terms: over this wave's token rows
  // [wave][16] and over its two column tiles [wave][32]
  float *prc = sde + BC, *prb = prc + 16 * (GNT / 64), *pcc = prb + 16 * (GNT / 64), *pcb = pcc + 32 * (GNT / 64);
  float *sred = pcb + 32 * (GNT / 64);
  // bf16 inputs: the tile's S^T and dS'^T as high and low bf16 parts, [16][LS]
  u16 *shT = reinterpret_cast<u16 *>(sred + GNT / 64 + 8), *slT = shT + 16 * LS, *dhT = slT + 16 * LS,
      *dlT = dhT + 16 * LS;
  const int i = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = lane & 15, g4 = lane >> 4;
  const int half = wave >> 2, tw = 16 * (wave & 3);  // column half; this wave's token rows
  const bool chain = half == 0;
  const int hk = h / (p.Hv / p.Hk);
  const int t0 = i * BC;
  if (tid < BNT) {  // the loads run on the first four waves
    RawRows<TIn, K> rq, rk;
    rq.load(p.q, p, b, t0, p.Hk, hk, K);
    rk.load(p.k, p, b, t0, p.Hk, hk, K);
    rq.put(sq, LK);
    rk.put(sk, LK);
    if constexpr (BF) {
      load_t_pair(tp, LB, p.ws_T + rec(p, b, h, i) * BC * BC);
    } else {
      load_t(st, p.ws_T + rec(p, b, h, i) * BC * BC);
    }
    load_decays(p, b, h, i, sc, sgam, se, sbeta);
    if (tid < BC) {
      sdgam[tid] = 0.f;
      sde[tid] = 0.f;
    }
  }
  __syncthreads();
  // M = scale (Q K^T) o D, this wave's rows and column tiles 2 half, 2 half + 1
  for (int tc = 2 * half; tc < 2 * half + 2; ++tc) {
    float4_t qk;
    if constexpr (BF) {
      qk = rows_times_rows<K>(sq, sk, LK, tw, 16 * tc);
    } else {
      qk = tile_mm4<K>(zero4(), [&](int r, int kk) { return ld4e(sq, (tw + r) * LK + kk); },
                       [&](int kk, int j) { return ld4e(sk, (16 * tc + j) * LK + kk); });
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = tw + 4 * g4 + r, s2 = 16 * tc + c;
      const float mv = t >= s2 ? p.scale * qk[r] * expf(sc[t] - sc[s2]) : 0.f;
      if constexpr (BF) {
        put_pair1(mp, BC * LB, t * LB + s2, mv);
      } else {
        sm[t * LC + s2] = mv;
      }
    }
  }

  float4_t dq[KH], dk[KH], dtb[2], dm[2];
#pragma unroll
  for (int m = 0; m < KH; ++m) dq[m] = dk[m] = zero4();
#pragma unroll
  for (int m = 0; m < 2; ++m) dtb[m] = dm[m] = zero4();
  float dgam_r[4] = {0.f, 0.f, 0.f, 0.f}, de_r[4] = {0.f, 0.f, 0.f, 0.f}, dgc = 0.f;
  const long kv = rec(p, b, h, i) * K * V;
  // Columns v0 .. v0+15 of the start state and end adjoint (K rows of four
  // float4) and of V and dO (16-byte pieces of TIn), fetched into registers a
  // tile ahead by the first four waves and placed in LDS between tiles.
  constexpr int SP = K * 4 / BNT, EPP = 16 / sizeof(TIn), PPR = 16 / EPP;
  float4_t rs[SP], rd[SP];
  uint4 rv, ro;
  auto fetch = [&](int v0) {
    if (tid >= BNT) return;
#pragma unroll
    for (int m = 0; m < SP; ++m) {
      const int e = tid + BNT * m;
      const long o = kv + static_cast<long>(e >> 2) * V + v0 + 4 * (e & 3);
      rs[m] = *reinterpret_cast<const float4_t *>(p.ws_S + o);
      rd[m] = *reinterpret_cast<const float4_t *>(p.ws_dS + o);
    }
    const int row = tid / PPR, part = tid % PPR, t = t0 + row;
    const long off = (((static_cast<long>(b) * p.T + t) * p.Hv + h) * V + v0) * static_cast<long>(sizeof(TIn)) +
                     part * 16;
    const bool ok = tid < BC * PPR && t < p.T;
    rv = ok ? *reinterpret_cast<const uint4 *>(static_cast<const unsigned char *>(p.v) + off) : uint4{0u, 0u, 0u, 0u};
    ro = ok ? *reinterpret_cast<const uint4 *>(static_cast<const unsigned char *>(p.dout) + off)
            : uint4{0u, 0u, 0u, 0u};
  };
  auto place = [&]() {
    if (tid >= BNT) return;
#pragma unroll
    for (int m = 0; m < SP; ++m) {
      const int e = tid + BNT * m;
      *reinterpret_cast<float4_t *>(&ss[(e >> 2) * LT + 4 * (e & 3)]) = rs[m];
      *reinterpret_cast<float4_t *>(&sds[(e >> 2) * LT + 4 * (e & 3)]) = rd[m];
      if constexpr (BF) {  // column c0 + j of the tile -> row c0 + j of the transposes
        const int kk = e >> 2, c0 = 4 * (e & 3);
        v2u32_t hi, lo;
        split_bf16(rs[m], hi, lo);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          shT[(c0 + j) * LS + kk] = static_cast<u16>(hi[j >> 1] >> (16 * (j & 1)));
          slT[(c0 + j) * LS + kk] = static_cast<u16>(lo[j >> 1] >> (16 * (j & 1)));
        }
        split_bf16(rd[m], hi, lo);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dhT[(c0 + j) * LS + kk] = static_cast<u16>(hi[j >> 1] >> (16 * (j & 1)));
          dlT[(c0 + j) * LS + kk] = static_cast<u16>(lo[j >> 1] >> (16 * (j & 1)));
        }
      }
    }
    if (tid < BC * PPR) {
      float x[EPP], y[EPP];
      decode16<TIn>(rv, x);
      decode16<TIn>(ro, y);
      const int row = tid / PPR, part = tid % PPR;
      if constexpr (BF) *reinterpret_cast<uint4 *>(sdo16 + row * LO + part * EPP) = ro;
#pragma unroll
      for (int j = 0; j < EPP; j += 4) {
        *reinterpret_cast<float4_t *>(&sx[row * LT + part * EPP + j]) = float4_t{x[j], x[j + 1], x[j + 2], x[j + 3]};
        if constexpr (!BF) {
          *reinterpret_cast<float4_t *>(&sdo[row * LT + part * EPP + j]) = float4_t{y[j], y[j + 1], y[j + 2], y[j + 3]};
        }
      }
    }
  };
  auto rows_of = [&](const float *m2, int ld) { return [=](int r, int kk) { return ld4(&m2[(tw + r) * ld + kk]); }; };
  auto in_rows = [&](const TIn *m2) { return [=](int r, int kk) { return ld4e(m2, (tw + r) * LK + kk); }; };
  auto state_cols = [&](const float *m2) { return [=](int kk, int col) { return ld4s(&m2[kk * LT + col], LT); }; };
  fetch(0);
  for (int v0 = 0; v0 < V; v0 += 16) {
    __syncthreads();  // the previous tile's readers are done (and sm is complete)
    place();
    if (v0 + 16 < V) fetch(v0 + 16);
    __syncthreads();
    float4_t ks = zero4(), kd = zero4();
    if (chain) {
      if constexpr (BF) {
        ks = rows_times_state<K>(sk, LK, tw, shT, slT, LS);
        kd = rows_times_state<K>(sk, LK, tw, dhT, dlT, LS);
      } else {
        ks = tile_mm4<K>(zero4(), in_rows(sk), state_cols(ss));
        kd = tile_mm4<K>(zero4(), in_rows(sk), state_cols(sds));
      }
      float4_t xv;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = tw + 4 * g4 + r;
        xv[r] = sx[t * LT + c] - sgam[t] * ks[r];  // X = V - Gamma K S
        sx[t * LT + c] = xv[r];
      }
      if constexpr (BF) {
        put_t_pair(xT, LB, tw + 4 * g4, c, xv);
        put_t_pair(bxT, LB, tw + 4 * g4, c, xv * ld4(&sbeta[tw + 4 * g4]));
      }
    } else {
      float4_t qs;
      if constexpr (BF) {
        qs = rows_times_state<K>(sq, LK, tw, shT, slT, LS);
      } else {
        qs = tile_mm4<K>(zero4(), in_rows(sq), state_cols(ss));
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = tw + 4 * g4 + r;
        dgam_r[r] += p.scale * qs[r] * (BF ? ld_el(sdo16, t * LO + c) : sdo[t * LT + c]);
      }
    }
    __syncthreads();
    if (chain) {
      float4_t u, du;
      if constexpr (BF) {  // U = T (beta X), dU0 part M^T dO (M^T, dO columns by transposing reads)
        u = pair_times_pair<BC>(tp, tp + BC * LB, LB, tw, bxT, bxT + 16 * LB, LB);
        du = zero4();
#pragma unroll
        for (int ts = 0; ts < BC; ts += 32) {
          const bh8_t dof = tr_frag(sdo16, LO, ts, 0);
          du = mfma_bf16(tr_frag(mp, LB, ts, tw), dof, du);
          du = mfma_bf16(tr_frag(mp + BC * LB, LB, ts, tw), dof, du);
        }
      } else {
        u = tile_mm4<BC>(zero4(), [&](int r, int s2) { return ld4(&st[(tw + r) * LC + s2]) * ld4(&sbeta[s2]); },
                         [&](int s2, int col) { return ld4s(&sx[s2 * LT + col], LT); });
        du = tile_mm4<BC>(zero4(), [&](int r, int s2) { return ld4s(&sm[s2 * LC + tw + r], LC); },
                          [&](int s2, int col) { return ld4s(&sdo[s2 * LT + col], LT); });
      }
      float4_t eu;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = tw + 4 * g4 + r;
        if constexpr (!BF) su[t * LT + c] = u[r];
        eu[r] = se[t] * u[r];
        de_r[r] += kd[r] * u[r];
        du[r] += se[t] * kd[r];
        sdu[t * LT + c] = du[r];
      }
      if constexpr (BF) {
        put_t_pair(uT, LB, tw + 4 * g4, c, u);
        put_t_pair(euT, LB, tw + 4 * g4, c, eu);
        put_t_pair(duT, LB, tw + 4 * g4, c, du);
      }
    }
    __syncthreads();
    if (chain) {
      float4_t dx;
      if constexpr (BF) {  // dX = diag(beta) T^T dU
        dx = tt_times_pair(tp, tp + BC * LB, LB, tw, duT, duT + 16 * LB, LB);
#pragma unroll
        for (int r = 0; r < 4; ++r) dx[r] *= sbeta[tw + 4 * g4 + r];
      } else {
        dx = tile_mm4<BC>(zero4(), [&](int r, int s2) { return ld4s(&st[s2 * LC + tw + r], LC) * sbeta[tw + r]; },
                          [&](int s2, int col) { return ld4s(&sdu[s2 * LT + col], LT); });
      }
      float4_t gx;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = tw + 4 * g4 + r;
        if constexpr (!BF) sdx[t * LT + c] = dx[r];
        gx[r] = -sgam[t] * dx[r];
        if (t0 + t < p.T) {
          store_el<TIn>(p.dv, ((static_cast<long>(b) * p.T + t0 + t) * p.Hv + h) * V + v0 + c, dx[r]);
        }
        dgam_r[r] -= ks[r] * dx[r];
      }
      if constexpr (BF) put_t_pair(gxT, LB, tw + 4 * g4, c, gx);
    }
    for (int e = tid; e < K * 16; e += GNT) dgc += ss[(e >> 4) * LT + (e & 15)] * sds[(e >> 4) * LT + (e & 15)];
    __syncthreads();
    // C x C products over these 16 columns (this wave's two column tiles):
    // dTb += dU X^T, dM += dO U^T; then dQ += scale Gamma dO S^T (bf16
    // inputs: the row scale after the loop), dK += E U dS'^T - Gamma dX S^T
    // (this wave's half of the key tiles)
    if constexpr (BF) {
      // A operands of this wave's rows: dU, E U, -Gamma dX pairs, dO as it is
      const bw_i16x4_t du_h = tr4(duT, LB, tw), du_l = tr4(duT + 16 * LB, LB, tw);
      const bw_i16x4_t eu_h = tr4(euT, LB, tw), eu_l = tr4(euT + 16 * LB, LB, tw);
      const bw_i16x4_t gx_h = tr4(gxT, LB, tw), gx_l = tr4(gxT + 16 * LB, LB, tw);
      const bw_i16x4_t dof = *reinterpret_cast<const bw_i16x4_t *>(sdo16 + (tw + c) * LO + 4 * g4);
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int tc = 2 * half + m;
        const bw_i16x4_t x_h = tr4(xT, LB, 16 * tc), x_l = tr4(xT + 16 * LB, LB, 16 * tc);
        const bw_i16x4_t u_h = tr4(uT, LB, 16 * tc), u_l = tr4(uT + 16 * LB, LB, 16 * tc);
        dtb[m] = mfma_bf16_k16(du_h, x_h, dtb[m]);
        dtb[m] = mfma_bf16_k16(du_h, x_l, dtb[m]);
        dtb[m] = mfma_bf16_k16(du_l, x_h, dtb[m]);
        dm[m] = mfma_bf16_k16(dof, u_h, dm[m]);
        dm[m] = mfma_bf16_k16(dof, u_l, dm[m]);
      }
#pragma unroll
      for (int m = 0; m < KH; ++m) {
        const int kt = half * KH + m;
        const bw_i16x4_t s_h = tr4(shT, LS, 16 * kt), s_l = tr4(slT, LS, 16 * kt);
        const bw_i16x4_t d_h = tr4(dhT, LS, 16 * kt), d_l = tr4(dlT, LS, 16 * kt);
        dq[m] = mfma_bf16_k16(dof, s_h, dq[m]);
        dq[m] = mfma_bf16_k16(dof, s_l, dq[m]);
        dk[m] = mfma_bf16_k16(eu_h, d_h, dk[m]);
        dk[m] = mfma_bf16_k16(eu_h, d_l, dk[m]);
        dk[m] = mfma_bf16_k16(eu_l, d_h, dk[m]);
        dk[m] = mfma_bf16_k16(gx_h, s_h, dk[m]);
        dk[m] = mfma_bf16_k16(gx_h, s_l, dk[m]);
        dk[m] = mfma_bf16_k16(gx_l, s_h, dk[m]);
      }
    } else {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int tc = 2 * half + m;
        dtb[m] = tile_mm4<16>(dtb[m], rows_of(sdu, LT), [&](int j, int col) { return ld4(&sx[(16 * tc + col) * LT + j]); });
        dm[m] = tile_mm4<16>(dm[m], rows_of(sdo, LT), [&](int j, int col) { return ld4(&su[(16 * tc + col) * LT + j]); });
      }
#pragma unroll
      for (int m = 0; m < KH; ++m) {
        const int kt = half * KH + m;
        auto s_t = [&](int j, int col) { return ld4(&ss[(16 * kt + col) * LT + j]); };
        dq[m] = tile_mm4<16>(dq[m], [&](int r, int j) { return ld4(&sdo[(tw + r) * LT + j]) * sgam[tw + r] * p.scale; },
                             s_t);
        dk[m] = tile_mm4<16>(dk[m], [&](int r, int j) { return ld4(&su[(tw + r) * LT + j]) * se[tw + r]; },
                             [&](int j, int col) { return ld4(&sds[(16 * kt + col) * LT + j]); });
        dk[m] = tile_mm4<16>(dk[m], [&](int r, int j) { return ld4(&sdx[(tw + r) * LT + j]) * -sgam[tw + r]; }, s_t);
      }
    }
  }
  if constexpr (BF) {  // dQ's row scale, scale Gamma
#pragma unroll
    for (int m = 0; m < KH; ++m) {
#pragma unroll
      for (int r = 0; r < 4; ++r) dq[m][r] *= sgam[tw + 4 * g4 + r] * p.scale;
    }
  }
  // per-token sums over the value columns (both halves add into sdgam)
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float a = row16_sum(dgam_r[r]), e2 = row16_sum(de_r[r]);
    if (c == 0) {
      atomicAdd(&sdgam[tw + 4 * g4 + r], a);
      if (chain) sde[tw + 4 * g4 + r] = e2;
    }
  }
  dgc = wave_sum(dgc);
  if (lane == 0) sred[wave] = dgc;
  __syncthreads();  // the value tiles are dead: the area now holds b1, b2, b3
  // dM o Mt into b1 (and its dc terms); dT = dTb diag(beta) into b2 (and
  // dbeta). The dc and dbeta terms of token t are summed in registers: rc, rb
  // for this lane's rows t = tw + 4 g4 + r, cc, cb for its columns 16 tc + c.
  float rc[4] = {0.f, 0.f, 0.f, 0.f}, rb[4] = {0.f, 0.f, 0.f, 0.f}, cc[2] = {0.f, 0.f}, cb[2] = {0.f, 0.f};
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int tc = 2 * half + m;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = tw + 4 * g4 + r, s2 = 16 * tc + c;
      const float d = t >= s2 ? p.scale * expf(sc[t] - sc[s2]) : 0.f;
      const float dmv = t >= s2 ? dm[m][r] : 0.f;
      if constexpr (BF) {
        put_pair1(b1p, BC * LB, t * LB + s2, dmv * d);
      } else {
        b1[t * LC + s2] = dmv * d;
      }
      const float dcv = dmv * (BF ? pair_val(mp, BC * LB, t * LB + s2) : sm[t * LC + s2]);
      rc[r] += dcv;
      cc[m] -= dcv;
      if constexpr (BF) {
        put_pair1(b2p, BC * LB, t * LB + s2, dtb[m][r] * sbeta[s2]);
      } else {
        b2[t * LC + s2] = dtb[m][r] * sbeta[s2];
      }
      cb[m] += dtb[m][r] * (BF ? pair_val(tp, BC * LB, t * LB + s2) : st[t * LC + s2]);
    }
  }
  __syncthreads();
  // W = T^T dT (this wave's tiles), then into b2 once every wave has read dT
  float4_t w4[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int tc = 2 * half + m;
    if constexpr (BF) {  // T^T and dT's columns by transposing reads of the pairs
      w4[m] = zero4();
#pragma unroll
      for (int ts = 0; ts < BC; ts += 32) {
        const bh8_t th = tr_frag(tp, LB, ts, tw), tl = tr_frag(tp + BC * LB, LB, ts, tw);
        const bh8_t dh = tr_frag(b2p, LB, ts, 16 * tc), dl = tr_frag(b2p + BC * LB, LB, ts, 16 * tc);
        w4[m] = mfma_bf16(th, dh, w4[m]);
        w4[m] = mfma_bf16(th, dl, w4[m]);
        w4[m] = mfma_bf16(tl, dh, w4[m]);
      }
    } else {
      w4[m] = tile_mm4<BC>(zero4(), [&](int r, int u2) { return ld4s(&st[u2 * LC + tw + r], LC); },
                           [&](int u2, int col) { return ld4s(&b2[u2 * LC + 16 * tc + col], LC); });
    }
  }
  __syncthreads();
#pragma unroll
  for (int m = 0; m < 2; ++m) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int e = (tw + 4 * g4 + r) * (BF ? LB : LC) + 16 * (2 * half + m) + c;
      if constexpr (BF) {
        put_pair1(b2p, BC * LB, e, w4[m][r]);
      } else {
        b2[e] = w4[m][r];
      }
    }
  }
  __syncthreads();
  // dA = -W T^T (strict lower): H = dA beta_t D, stored as H + H^T in b3
  // (symmetric, so one product gives H K + H^T K); dbeta_t, dc terms
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int tc = 2 * half + m;
    float4_t da;
    if constexpr (BF) {  // W rows times T rows (both pairs)
      da = pair_times_pair<BC>(b2p, b2p + BC * LB, LB, tw, tp + 16 * tc * LB, tp + BC * LB + 16 * tc * LB, LB);
    } else {
      da = tile_mm4<BC>(zero4(), [&](int r, int u2) { return ld4(&b2[(tw + r) * LC + u2]); },
                        [&](int u2, int col) { return ld4(&st[(16 * tc + col) * LC + u2]); });
    }
    float4_t gk;
    if constexpr (BF) {
      gk = rows_times_rows<K>(sk, sk, LK, tw, 16 * tc);
    } else {
      gk = tile_mm4<K>(zero4(), [&](int r, int kk) { return ld4e(sk, (tw + r) * LK + kk); },
                       [&](int kk, int col) { return ld4e(sk, (16 * tc + col) * LK + kk); });
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = tw + 4 * g4 + r, s2 = 16 * tc + c;
      if (t > s2) {
        const float d = expf(sc[t] - sc[s2]);
        const float dav = -da[r];
        const float av = sbeta[t] * gk[r] * d;
        const float hv = dav * sbeta[t] * d;
        rb[r] += dav * gk[r] * d;
        rc[r] += dav * av;
        cc[m] -= dav * av;
        if constexpr (BF) {
          put_pair1(b3p, BC * LB, t * LB + s2, hv);
          put_pair1(b3p, BC * LB, s2 * LB + t, hv);
        } else {
          b3[t * LC + s2] = hv;
          b3[s2 * LC + t] = hv;
        }
      } else if (t == s2) {
        if constexpr (BF) {
          put_pair1(b3p, BC * LB, t * LB + s2, 0.f);
        } else {
          b3[t * LC + s2] = 0.f;
        }
      }
    }
  }
  // the sums over this wave's lanes: a row's over its 16 column lanes, a
  // column's over its 4 row groups
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float x = group_sum(rc[r], 16), y = group_sum(rb[r], 16);
    if (c == 0) {
      prc[16 * wave + 4 * g4 + r] = x;
      prb[16 * wave + 4 * g4 + r] = y;
    }
  }
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const float x = add_xor32(add_xor16(cc[m])), y = add_xor32(add_xor16(cb[m]));
    if (g4 == 0) {
      pcc[32 * wave + 16 * m + c] = x;
      pcb[32 * wave + 16 * m + c] = y;
    }
  }
  __syncthreads();
  // dQ += (dM o Mt) K;  dK += (dM o Mt)^T Q + (H + H^T) K
  if constexpr (BF) {  // K and Q columns by transposing reads (exact), the C x C pairs by rows or transposing reads
#pragma unroll
    for (int ts = 0; ts < BC; ts += 32) {
      const int o = (tw + c) * LB + ts + 8 * g4;
      const bh8_t a1h = *reinterpret_cast<const bh8_t *>(b1p + o), a1l = *reinterpret_cast<const bh8_t *>(b1p + BC * LB + o);
      const bh8_t a3h = *reinterpret_cast<const bh8_t *>(b3p + o), a3l = *reinterpret_cast<const bh8_t *>(b3p + BC * LB + o);
      const bh8_t t1h = tr_frag(b1p, LB, ts, tw), t1l = tr_frag(b1p + BC * LB, LB, ts, tw);
#pragma unroll
      for (int m = 0; m < KH; ++m) {
        const int kt = half * KH + m;
        const bh8_t kf = tr_frag(sk, LK, ts, 16 * kt), qf = tr_frag(sq, LK, ts, 16 * kt);
        dq[m] = mfma_bf16(a1h, kf, dq[m]);
        dq[m] = mfma_bf16(a1l, kf, dq[m]);
        dk[m] = mfma_bf16(t1h, qf, dk[m]);
        dk[m] = mfma_bf16(t1l, qf, dk[m]);
        dk[m] = mfma_bf16(a3h, kf, dk[m]);
        dk[m] = mfma_bf16(a3l, kf, dk[m]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < (BF ? 0 : KH); ++m) {
    const int kt = half * KH + m;
    auto kcol = [&](int s2, int col) { return ld4es(sk, s2 * LK + 16 * kt + col, LK); };
    dq[m] = tile_mm4<BC>(dq[m], [&](int r, int s2) { return ld4(&b1[(tw + r) * LC + s2]); }, kcol);
    dk[m] = tile_mm4<BC>(dk[m], [&](int r, int s2) { return ld4s(&b1[s2 * LC + tw + r], LC); },
                         [&](int s2, int col) { return ld4es(sq, s2 * LK + 16 * kt + col, LK); });
    dk[m] = tile_mm4<BC>(dk[m], [&](int r, int s2) { return ld4(&b3[(tw + r) * LC + s2]); }, kcol);
  }
  // dq, dk: straight to the output without GQA, else per value head in float32
  const bool direct = p.Hk == p.Hv;
#pragma unroll
  for (int m = 0; m < KH; ++m) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + tw + 4 * g4 + r, kk = 16 * (half * KH + m) + c;
      if (t >= p.T) continue;
      if (direct) {
        const long o = ((static_cast<long>(b) * p.T + t) * p.Hk + hk) * K + kk;
        store_el<TIn>(p.dq, o, dq[m][r]);
        store_el<TIn>(p.dk, o, dk[m][r]);
      } else {
        const long o = ((static_cast<long>(b) * p.T + t) * p.Hv + h) * K + kk;
        p.ws_dq[o] = dq[m][r];
        p.ws_dk[o] = dk[m][r];
      }
    }
  }
  __syncthreads();
  if (wave == 0) {  // dc -> dg = reverse cumulative sum within the chunk
    const int t = lane;
    // token t's terms: rows t of waves t/16 and t/16 + 4, columns t of the
    // four waves of column half t/32
    float dct = prc[16 * (t >> 4) + (t & 15)] + prc[16 * ((t >> 4) + 4) + (t & 15)];
    float dbt = prb[16 * (t >> 4) + (t & 15)] + prb[16 * ((t >> 4) + 4) + (t & 15)];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      dct += pcc[32 * (4 * (t >> 5) + w) + (t & 31)];
      dbt += pcb[32 * (4 * (t >> 5) + w) + (t & 31)];
    }
    float dcv = dct + sdgam[t] * sgam[t] - sde[t] * se[t];
    const float tail = wave_sum(sde[t] * se[t]);
    float gc = 0.f;
#pragma unroll
    for (int w = 0; w < GNT / 64; ++w) gc += sred[w];
    if (t == BC - 1) dcv += tail + gc * sgam[BC - 1];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_down(dcv, off, 64);
      if (lane + off < 64) dcv += y;
    }
    if (t0 + t < p.T) {
      const long o = (static_cast<long>(b) * p.T + t0 + t) * p.Hv + h;
      p.dg[o] = dcv;
      store_elem(p.dbeta, o, p.beta_dtype, dbt);
    }
  }
}

// dq, dk [B,T,Hk,K] = sum over the Hv/Hk value heads of each key head.
__global__ __launch_bounds__(BNT) void bwd_gqa_reduce_kernel(BwdParams p) {
  const long total = static_cast<long>(p.B) * p.T * p.Hk * p.K;
  const int group = p.Hv / p.Hk;
  for (long e = static_cast<long>(blockIdx.x) * BNT + threadIdx.x; e < total; e += static_cast<long>(gridDim.x) * BNT) {
    const long kk = e % p.K, rest = e / p.K;
    const long hk = rest % p.Hk, bt = rest / p.Hk;
    const long base = (bt * p.Hv + hk * group) * p.K + kk;
    float sq = 0.f, sk = 0.f;
    for (int m = 0; m < group; ++m) {
      sq += p.ws_dq[base + static_cast<long>(m) * p.K];
      sk += p.ws_dk[base + static_cast<long>(m) * p.K];
    }
    store_elem(p.dq, e, p.in_dtype, sq);
    store_elem(p.dk, e, p.in_dtype, sk);
  }
}

// LDS bytes of each kernel.
template <int K, typename TIn>
constexpr size_t scan_lds() { return ScanLds<K, TIn>::BYTES; }
template <int K, typename TIn>
constexpr size_t grad_lds() {
  return sizeof(TIn) * 2 * BC * (K + 16 / sizeof(TIn)) +
         sizeof(float) * (2 * (std::is_same<TIn, u16>::value ? BC * (BC + 8) : BC * LC) +
                          grad_area<K, std::is_same<TIn, u16>::value>() + 6 * BC + 96 * (GNT / 64) + GNT / 64 + 8) +
         (std::is_same<TIn, u16>::value ? sizeof(u16) * 4 * 16 * (K + 8) : 0);
}

template <typename Kern>
int launch(Kern kernel, dim3 grid, size_t lds, hipStream_t st, const BwdParams &p, int threads = BNT) {
  if (hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(lds)) != hipSuccess) {
    return PBGDN_ERR_LAUNCH;
  }
  hipLaunchKernelGGL(kernel, grid, dim3(threads), lds, st, p);
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}

template <int K, int V>
int run_backward(const BwdParams &p, hipStream_t st) {
  static_assert(grad_lds<K, float>() <= 160 * 1024 && grad_lds<K, u16>() <= 160 * 1024 && local_lds<K, V, float>() <= 160 * 1024, "LDS budget");
  const dim3 per_chunk(p.n, p.Hv, p.B), per_tile2((V / 16) * p.Hv * 2 * p.B);
  int rc = PBGDN_OK;
  if (p.n > 0) {
    switch (p.in_dtype) {
      case PBGDN_F32: rc = launch(bwd_local_kernel<K, V, float>, per_chunk, local_lds<K, V, float>(), st, p); break;
      case PBGDN_BF16: rc = launch(bwd_local_kernel<K, V, u16>, per_chunk, local_lds<K, V, u16>(), st, p); break;
      default: rc = launch(bwd_local_kernel<K, V, half_t>, per_chunk, local_lds<K, V, half_t>(), st, p); break;
    }
  }
  if (rc == PBGDN_OK) {  // both scans in one launch (with T = 0 only the reverse one writes: dh0 = dht)
    switch (p.in_dtype) {
      case PBGDN_F32: rc = launch(bwd_scans_kernel<K, float>, per_tile2, scan_lds<K, float>(), st, p); break;
      case PBGDN_BF16: rc = launch(bwd_scans_kernel<K, u16>, per_tile2, scan_lds<K, u16>(), st, p); break;
      default: rc = launch(bwd_scans_kernel<K, half_t>, per_tile2, scan_lds<K, half_t>(), st, p); break;
    }
  }
  if (rc == PBGDN_OK && p.n > 0) {
    switch (p.in_dtype) {
      case PBGDN_F32: rc = launch(bwd_grad_kernel<K, V, float>, per_chunk, grad_lds<K, float>(), st, p, GNT); break;
      case PBGDN_BF16: rc = launch(bwd_grad_kernel<K, V, u16>, per_chunk, grad_lds<K, u16>(), st, p, GNT); break;
      default: rc = launch(bwd_grad_kernel<K, V, half_t>, per_chunk, grad_lds<K, half_t>(), st, p, GNT); break;
    }
  }
  if (rc == PBGDN_OK && p.n > 0 && p.Hk != p.Hv) {
    const long total = static_cast<long>(p.B) * p.T * p.Hk * K;
    const unsigned blocks = static_cast<unsigned>(std::min<long>((total + BNT - 1) / BNT, 65535L));
    hipLaunchKernelGGL(bwd_gqa_reduce_kernel, dim3(blocks), dim3(BNT), 0, st, p);
    rc = hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
  }
  return rc;
}

// Workspace floats per (batch, value head, chunk), and the GQA scratch.
long ws_record_floats(int K, int V) {
  return static_cast<long>(BC) * BC + 2 * BC + static_cast<long>(BC) * V + 3L * K * V;
}

}  // namespace
}  // namespace pbgdn

extern "C" size_t pbgdn_chunk_bwd_workspace_size(int B, int T, int Hk, int Hv, int K, int V) {
  using namespace pbgdn;
  if (B < 0 || T < 0 || Hk <= 0 || Hv <= 0 || K <= 0 || V <= 0) return 0;
  const long n = (static_cast<long>(T) + BC - 1) / BC;
  long floats = static_cast<long>(B) * Hv * n * ws_record_floats(K, V);
  if (Hk != Hv) floats += 2L * B * T * Hv * K;
  return static_cast<size_t>(floats) * sizeof(float) + 256;
}

extern "C" int pbgdn_chunk_bwd(const void *q, const void *k, const void *v, int in_dtype, const float *g,
                               const void *beta, int beta_dtype, const float *h0, const void *dout, int do_dtype,
                               const float *dht, void *dq, void *dk, void *dv, float *dg, void *dbeta, float *dh0,
                               void *workspace, size_t workspace_bytes, int B, int T, int Hk, int Hv, int K, int V,
                               float scale, void *stream) {
  using namespace pbgdn;
  if (B < 0 || T < 0 || Hk <= 0 || Hv <= 0 || K <= 0 || V <= 0 || Hv % Hk != 0) return PBGDN_ERR_INVALID_ARGUMENT;
  auto dtype_ok = [](int d) { return d == PBGDN_F32 || d == PBGDN_BF16 || d == PBGDN_F16; };
  if (!dtype_ok(in_dtype) || !dtype_ok(beta_dtype) || !dtype_ok(do_dtype)) return PBGDN_ERR_INVALID_ARGUMENT;
  if (!((K == 64 || K == 128) && (V == 64 || V == 128)) || do_dtype != in_dtype) return PBGDN_ERR_UNSUPPORTED;
  if (static_cast<long>(B) * T == 0) {
    if (B > 0 && dh0 == nullptr) return PBGDN_OK;
  }
  const long n = (static_cast<long>(T) + BC - 1) / BC;
  if (n > 0 && (!q || !k || !v || !g || !beta || !dout || !dq || !dk || !dv || !dg || !dbeta)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (B == 0) return PBGDN_OK;
  if (n > 65535 || Hv > 65535 || B > 32767) return PBGDN_ERR_UNSUPPORTED;
  if (static_cast<long>(V / 16) * Hv * 2 * B > 0x7fffffffL) return PBGDN_ERR_UNSUPPORTED;  // the scans' 1-D grid
  if (!workspace || workspace_bytes < pbgdn_chunk_bwd_workspace_size(B, T, Hk, Hv, K, V) ||
      reinterpret_cast<uintptr_t>(workspace) % 16 != 0) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  float *ws = static_cast<float *>(workspace);
  const long recs = static_cast<long>(B) * Hv * n;
  {  // debug builds: the gradients and the workspace start as NaN
    hipStream_t s = static_cast<hipStream_t>(stream);
    const long isz = in_dtype == PBGDN_F32 ? 4 : 2, bsz = beta_dtype == PBGDN_F32 ? 4 : 2;
    const long bt = static_cast<long>(B) * T;
    debug_poison(dq, static_cast<size_t>(bt * Hk * K * isz), s);
    debug_poison(dk, static_cast<size_t>(bt * Hk * K * isz), s);
    debug_poison(dv, static_cast<size_t>(bt * Hv * V * isz), s);
    debug_poison(dg, static_cast<size_t>(bt * Hv * 4), s);
    debug_poison(dbeta, static_cast<size_t>(bt * Hv * bsz), s);
    debug_poison(dh0, static_cast<size_t>(static_cast<long>(B) * Hv * K * V * 4), s);
    debug_poison(workspace, workspace_bytes, s);
  }
  BwdParams p{};
  DeviceShape shape;
  if (!device_shape(shape)) return PBGDN_ERR_LAUNCH;
  p.xcds = shape.xcds;
  p.q = q;
  p.k = k;
  p.v = v;
  p.g = g;
  p.beta = beta;
  p.h0 = h0;
  p.dout = dout;
  p.dht = dht;
  p.dq = dq;
  p.dk = dk;
  p.dv = dv;
  p.dg = dg;
  p.dbeta = dbeta;
  p.dh0 = dh0;
  p.ws_T = ws;
  p.ws_c = p.ws_T + recs * BC * BC;
  p.ws_beta = p.ws_c + recs * BC;
  p.ws_dU0 = p.ws_beta + recs * BC;
  p.ws_J = p.ws_dU0 + recs * BC * V;
  p.ws_S = p.ws_J + recs * K * V;
  p.ws_dS = p.ws_S + recs * K * V;
  p.ws_dq = p.ws_dS + recs * K * V;
  p.ws_dk = Hk != Hv ? p.ws_dq + static_cast<long>(B) * T * Hv * K : nullptr;
  if (Hk == Hv) p.ws_dq = nullptr;
  p.in_dtype = in_dtype;
  p.beta_dtype = beta_dtype;
  p.B = B;
  p.T = T;
  p.Hk = Hk;
  p.Hv = Hv;
  p.K = K;
  p.V = V;
  p.n = static_cast<int>(n);
  p.scale = scale;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (K == 64) return V == 64 ? run_backward<64, 64>(p, st) : run_backward<64, 128>(p, st);
  return V == 64 ? run_backward<128, 64>(p, st) : run_backward<128, 128>(p, st);
}
