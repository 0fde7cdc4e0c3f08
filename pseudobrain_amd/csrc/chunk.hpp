// Shared pieces of the chunkwise Gated DeltaNet prefill for gfx950 (CDNA4):
// parameters, the workspace record format, MFMA and buffer helpers, and the
// staging of one chunk's inputs from HBM into LDS.
//
// Reference algorithm: delta_rule_chunked, pseudobrain/gated_deltanet.py:110-165.
// Within a chunk of C = 64 tokens with inclusive cumulative log decay c_t,
// gamma_t = exp(c_t), D_ts = exp(c_t - c_s) (s <= t), every exponent <= 0:
//   A   = strict_lower(b_t (k_t . k_s) D_ts)                        (:143-146)
//   T   = (I + A)^-1,  Tb = T diag(b)                                (:147-149)
//   X   = V - diag(gamma) K S                                        (U = U' - W S with
//   U   = Tb X                                                        W = Tb diag(gamma) K,
//                                                                     U' = Tb V, :150-159)
//   O   = diag(gamma scale) Q S + (scale Q K^T o D) U                (:160-161)
//   S  <- gamma_C S + K^T diag(exp(c_C - c)) U                       (:162-163)
//
// Two kernels carry it:
//   * prep (chunk_prep.hip): every (chunk, value head) independently: A, the
//     inverse T, Tb and QKD = scale (Q K^T o D) and the decay vectors, written
//     to a workspace record in the operand layout the scan kernel consumes;
//   * scan (chunk_scan.hip): per (sequence, value head, 16-column tile of V),
//     the chunks in order: only the products that involve the state.
//
// Fragment layouts (lane l, g = l >> 4, c = l & 15). 16x16x32: A holds
// A[m = c][k = 8g + j], B holds B[k = 8g + j][n = c], j = 0..7; 16x16x16:
// k = 4g + j, j = 0..3; the accumulator holds D[4g + i][c], i = 0..3. Any
// consistent assignment of contraction slots works, as long as A and B agree.
// Written tile(X) for the accumulator layout of a 16x16 X: tile(X) is the B
// operand of X and the A operand of X^T, so MFMA(tile(P^T), tile(Q)) = tile(PQ)
// and MFMA(tile(Q), tile(P^T)) = tile((PQ)^T).
//
// LDS rows are an odd multiple of 32 bytes long and the 16-byte chunk index
// within a row is XORed with bit 2 of the row index ("swz"): conflict-free for
// 16-byte fragment reads and 8-byte accumulator-tile writes alike, and the
// swizzle folds into each lane's base address.
#pragma once

#include "common.hpp"
#include "device.hpp"
#include "schedule.hpp"

namespace pbgdn {

typedef __bf16 bf16_t;
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));

constexpr int CH = 64;                  // chunk length (CHUNK, gated_deltanet.py:49)
constexpr int VT = 16;                  // value columns per scan workgroup

// Workspace record of one (chunk, value head), REC_BYTES bytes:
//   REC_SC   fp32 [64] gamma_t, [64] scale gamma_t, [64] exp(c_63 - c_t),
//            then 256 bytes not written
//   REC_TB   6 fragments of Tb as 16x16x32 fp16 A operands (64 lanes x 16 B):
//            row tile r, contraction step kk <= r / 2 (the others are zero),
//            at fragment frag_index(r, kk); lane (g, c) holds
//            Tb[16 r + c][32 kk + 8 g .. + 7]
//   REC_QKD  the same for QKD = scale (Q K^T o D)
//   REC_TBL  float32 inputs only: the low fp16 part of Tb (Tb - fp16(Tb)) in
//            the layout of REC_TB, so that U = Tb X is formed to ~22 bits
//            (REC_BYTES_F32 bytes a record)
// Records are indexed (chunk record, value head); the chunk record of chunk j
// of sequence s is rec_base(s) + j with rec_base(s) = floor(bos_s / 64) + s,
// which is increasing in s, leaves room for every sequence's chunks, and is
// below floor(total_tokens / 64) + num_seqs + 1 (see chunk_records()).
constexpr int FRAG_BYTES = 64 * 16;
constexpr int NFRAG = 6;
constexpr int REC_SC = 0;
constexpr int SC_GAM = 0, SC_GSC = 256, SC_DEC = 512;
constexpr int REC_TB = 1024;
constexpr int REC_QKD = REC_TB + NFRAG * FRAG_BYTES;
constexpr int REC_BYTES = REC_QKD + NFRAG * FRAG_BYTES;
constexpr int REC_TBL = REC_BYTES;
constexpr int REC_BYTES_F32 = REC_TBL + NFRAG * FRAG_BYTES;
// Bytes of a record for inputs of type TIn / of dtype code `in_dtype`.
template <typename TIn>
__host__ __device__ constexpr int rec_bytes() { return sizeof(TIn) == 4 ? REC_BYTES_F32 : REC_BYTES; }
__host__ __device__ constexpr int rec_bytes_of(int in_dtype) { return in_dtype == PBGDN_F32 ? REC_BYTES_F32 : REC_BYTES; }

__host__ __device__ constexpr int frag_index(int r, int kk) { return r < 2 ? r : 2 * r - 2 + kk; }
// The record's 16-byte units that hold nothing a scan reads: the lanes
// (g, c) of a fragment (r, kk) whose 8 columns 32 kk + 8 g .. all lie past
// their row 16 r + c, where the lower-triangular Tb, QKD (and Tb's low part)
// vanish (32 of the 64 lanes of fragments (0, 0) and (2, 1), 8 of the others
// but (2, 0) and (3, 0): 3 KiB of a 13 KiB record), and the vector of c after
// the three decay vectors (no scan uses it). The prep kernel does not store
// them and the scans do not fetch them: their loads go out of range, and the
// zeros such a load returns are what they stage.
__host__ __device__ constexpr bool rec_unused_unit(int byte) {
  if (byte >= REC_SC + 768 && byte < REC_TB) return true;  // c
  if (byte < REC_TB) return false;
  const int f = ((byte - REC_TB) / FRAG_BYTES) % NFRAG;
  const int lane = ((byte - REC_TB) % FRAG_BYTES) / 16;
  const int r = f < 2 ? f : 2 + (f - 2) / 2, kk = f < 2 ? 0 : (f - 2) % 2;  // frag_index(r, kk) == f
  return 32 * kk + 8 * (lane >> 4) > 16 * r + (lane & 15);
}
static_assert(frag_index(2, 1) == 3 && frag_index(3, 0) == 4 && frag_index(3, 1) == 5, "fragment order");
static_assert(!rec_unused_unit(REC_TB + 7 * 16) && rec_unused_unit(REC_TB + 16 * 16) &&
                  !rec_unused_unit(REC_TB + 24 * 16) && rec_unused_unit(REC_TB + 32 * 16) &&
                  rec_unused_unit(REC_QKD + 3 * FRAG_BYTES + 63 * 16) &&
                  !rec_unused_unit(REC_QKD + 2 * FRAG_BYTES + 63 * 16) &&
                  rec_unused_unit(REC_QKD + FRAG_BYTES + 48 * 16) && !rec_unused_unit(REC_QKD + FRAG_BYTES + 56 * 16) &&
                  !rec_unused_unit(REC_SC + 512) && rec_unused_unit(REC_SC + 768),
              "units of the record no scan reads");

__host__ __device__ inline long rec_base(long bos, int s) { return bos / CH + s; }

// Upper bound of the chunk records of a call (the workspace holds
// chunk_records() x Hv records).
__host__ __device__ inline long chunk_records(long total_tokens, int num_seqs) {
  return total_tokens / CH + num_seqs + 1;
}

struct ChunkParams {
  const void *q, *k, *v;
  const float *g;
  const void *beta;
  int beta_dtype;
  const void *h0;  // initial states, or NULL for zeros
  void *ht;        // final states, or NULL
  int state_dtype;
  const int32_t *state_idx;          // [N] state slot of each sequence, or NULL for slot n
  const uint8_t *has_initial_state;  // [N] 0: start from zeros, or NULL (all read h0)
  int num_states;                    // slots in h0/ht when state_idx is set
  const int32_t *cu_seqlens;
  void *o;
  unsigned char *ws;  // workspace records
  int T, Hk, Hv, V, num_seqs;
  int seq_groups;  // the scan's sequence groups (a workgroup runs one group's sequences back to back)
  float scale;
  int cus, xcds;   // the device's compute units and XCDs (device.hpp)
  // The layer's epilogue, when the scan applies it (the wide scan at V = 128):
  // o is then hs = RMSNorm(o) o_norm SiLU(gate) per (token, value head).
  const void *gate;   // [T, gate_stride] in the inputs' dtype, head h at columns h V ..
  long gate_stride;   // elements per token row
  const float *o_norm;
  float eps;
  // float32 inputs: the power of two that brings v and the initial states
  // into the kernels' range (a device scalar written before the scan), or NULL
  const float *in_scale;
  // float32 inputs: the RANGE_BLOCKS partial maxima the scale is made from
  // (the prep kernel's first wave reduces them into *in_scale), or NULL
  const float *range_part;
};

// float32 inputs' range scale: v and the initial states are brought within
// RANGE_LIMIT by a power of two, from RANGE_BLOCKS partial maxima of their
// magnitudes.
constexpr float RANGE_LIMIT = 1024.f;
constexpr int RANGE_BLOCKS = 512;

// One wave: the scale 2^-e, e = max(0, ceil(log2(max / RANGE_LIMIT))), from
// the partial maxima; 1 for a maximum that is not finite.
__device__ __forceinline__ void range_scale_wave(const float *part, float *scale) {
  const int lane = threadIdx.x & 63;
  float m = 0.f;
  for (int i = lane; i < RANGE_BLOCKS; i += 64) m = fmaxf(m, part[i]);
  m = wave_max(m);
  if (lane == 0) {
    float down = 1.f;
    if (__builtin_isfinite(m) && m > RANGE_LIMIT) {
      int e = 0;
      const float mant = frexpf(m / RANGE_LIMIT, &e);  // m / RANGE_LIMIT = mant 2^e, mant in [0.5, 1)
      down = ldexpf(1.f, mant == 0.5f ? 1 - e : -e);   // 2^-ceil(log2(m / RANGE_LIMIT))
    }
    *scale = down;
  }
}

// Sequence s (wave-uniform): first token and end. cu_seqlens is read through
// the constant address space (it is not written during a call), so these are
// scalar loads. Whatever cu_seqlens holds, the bounds are clamped to
// 0 <= bos <= eos <= T (B == 1 with cu_seqlens), so every token, record and
// output row a sequence touches lies inside the call's buffers; a decreasing
// cu_seqlens gives meaningless results, never an access out of bounds.
typedef const __attribute__((address_space(4))) int32_t const_i32;
__device__ __forceinline__ void seq_bounds(const ChunkParams &p, int s, long &bos, long &eos) {
  if (p.cu_seqlens) {
    const_i32 *cu = (const_i32 *)p.cu_seqlens;  // C-style: an address-space cast
    const long total = p.T;
    const long b = cu[s], e = cu[s + 1];
    bos = b < 0 ? 0 : (b > total ? total : b);
    eos = e < bos ? bos : (e > total ? total : e);
  } else {
    bos = static_cast<long>(s) * p.T;
    eos = bos + p.T;
  }
}

// Operand type of the q/k products: bf16 for bf16 inputs, fp16 otherwise.
template <typename TIn>
struct OpOf {
  using T4 = half4_t;
  using T8 = half8_t;
  __device__ static T4 from(float4_t x) { return __builtin_convertvector(x, half4_t); }
  __device__ static float4_t to(T4 x) { return __builtin_convertvector(x, float4_t); }
  __device__ static float4_t bits_to_float(i16x4_t x) { return to(__builtin_bit_cast(half4_t, x)); }
  // x = hi + lo, each rounded to the operand type in turn (packed conversions)
  __device__ static void split(float4_t x, T4 &hi, T4 &lo) {
    hi = from(x);
    lo = from(x - to(hi));
  }
};
template <>
struct OpOf<u16> {
  using T4 = bf16x4_t;
  using T8 = bf16x8_t;
  // round to nearest even, two values per conversion
  __device__ static T4 from(float4_t x) { return __builtin_convertvector(x, bf16x4_t); }
  // widening is exact: the bf16 bits are the high half of the float
  __device__ static float4_t to(T4 x) {
    const v2u32_t w = __builtin_bit_cast(v2u32_t, x);
    return float4_t{__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u), __uint_as_float(w[1] << 16),
                    __uint_as_float(w[1] & 0xffff0000u)};
  }
  __device__ static float4_t bits_to_float(i16x4_t x) { return to(__builtin_bit_cast(bf16x4_t, x)); }
  // x = hi + lo, each rounded to bf16 in turn (packed conversions)
  __device__ static void split(float4_t x, T4 &hi, T4 &lo) {
    hi = from(x);
    lo = from(x - to(hi));
  }
};

// Range of the fp16 operands X (and through Tb X, U). A tile of X whose largest
// magnitude m exceeds X_LIMIT is scaled by 2^-e, e = the least power that
// brings it to at most X_LIMIT (exact: a power of two), so that U' = Tb X'
// (at most 64 |Tb| X_LIMIT) stays inside fp16; U = U' 2^e is restored in fp32.
constexpr float X_LIMIT = 256.f;
// 2^-e for a tile maximum m > X_LIMIT (m finite): scales m to at most X_LIMIT.
__device__ __forceinline__ float range_scale(float m) {
  int e;
  frexpf(m / X_LIMIT, &e);  // m / X_LIMIT = f 2^e, f in [0.5, 1)
  return ldexpf(1.f, -e);
}
__device__ __forceinline__ float tile_max(const float4_t (&x)[4]) {
  float m = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) m = fmaxf(m, fmaxf(fmaxf(fabsf(x[r][0]), fabsf(x[r][1])), fmaxf(fabsf(x[r][2]), fabsf(x[r][3]))));
  return m;
}

__device__ __forceinline__ float4_t mma(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float4_t mma(bf16x8_t a, bf16x8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Workgroup barrier for LDS traffic: waits for this wave's LDS operations, not
// for its outstanding global loads (prefetched chunks) or stores.
__device__ __forceinline__ void block_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}


// Output element stores through a buffer resource (stores past its range are dropped).
template <typename T>
__device__ __forceinline__ void put_out(__amdgpu_buffer_rsrc_t r, uint32_t off, float x);
template <>
__device__ __forceinline__ void put_out<u16>(__amdgpu_buffer_rsrc_t r, uint32_t off, float x) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(u16, static_cast<bf16_t>(x)), r, off, 0, 0);
}
template <>
__device__ __forceinline__ void put_out<half_t>(__amdgpu_buffer_rsrc_t r, uint32_t off, float x) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(u16, static_cast<half_t>(x)), r, off, 0, 0);
}
template <>
__device__ __forceinline__ void put_out<float>(__amdgpu_buffer_rsrc_t r, uint32_t off, float x) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, x), r, off, 0, 0);
}

// DPP move of a float: lanes of disabled rows (row_mask) and, with
// bound_ctrl, lanes whose source is outside the row, get 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp0(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK, 0xf, true));
}

// Inclusive prefix sum over the 64 lanes of a wave: row_shr 1, 2, 4, 8 scan
// each row of 16 lanes; row_bcast 15 adds the last lane of rows 0, 2 to rows
// 1, 3 and row_bcast 31 adds lane 31 to rows 2, 3 (gfx9-family DPP controls
// 0x111..0x118, 0x142, 0x143).
__device__ __forceinline__ float wave_prefix_sum(float x) {
  x += dpp0<0x111, 0xf>(x);
  x += dpp0<0x112, 0xf>(x);
  x += dpp0<0x114, 0xf>(x);
  x += dpp0<0x118, 0xf>(x);
  x += dpp0<0x142, 0xa>(x);
  x += dpp0<0x143, 0xc>(x);
  return x;
}

__device__ __forceinline__ float lane_value(float x, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}

__device__ __forceinline__ float pick(float4_t v, int i) {
  return (i == 0) ? v[0] : (i == 1) ? v[1] : (i == 2) ? v[2] : v[3];
}


// One chunk of raw inputs held in registers between its buffer load and its
// store into LDS. LY gives the LDS placement (KQ, KQ_MAT, KPB; V16, V16_BUF
// when WITH_V; SC when WITH_SCAN). Per-lane byte offsets are fixed; a chunk
// only sets the scalar base and range of each buffer resource, and tokens at
// or past the end of the sequence load as zeros (k = v = g = beta = 0: the
// identity steps of the reference's padding, gated_deltanet.py:127).
//
// Every thread issues the same loads whatever its role (threads without a V
// unit load from OUT_OF_RANGE, every lane loads g and beta): the compiler
// counts outstanding memory operations per wave statically, and a load issued
// on only some paths would make it wait for all of them at the next use.
template <int K, typename TIn, int NT, typename LY, bool WITH_V, bool WITH_SCAN>
struct ChunkInputs {
  static constexpr int EPU = 16 / sizeof(TIn);       // elements per 16-byte unit
  static constexpr int ROW_UNITS = K / EPU;
  static constexpr int MAT_UNITS = CH * ROW_UNITS;   // units of one of K, Q
  static constexpr int UPT = 2 * MAT_UNITS / NT;     // K then Q units per thread
  static constexpr int V_UNITS = CH * VT / EPU;
  static_assert(UPT >= 1 && (2 * MAT_UNITS) % NT == 0 && MAT_UNITS % 64 == 0, "K/Q units must tile the workgroup");
  static_assert(!WITH_V || V_UNITS <= NT, "V units exceed the workgroup");

  uint32_t qk_off[UPT];  // global byte offset of this thread's units within a chunk
  uint32_t qk_lds[UPT];  // LDS byte offset of the same units within a K or Q matrix
  uint32_t v_off, v_lds, g_off, b_off;
  uint4 x[UPT], vx;
  float g;
  uint32_t b32;  // beta as loaded: fp32 bits, or
  u16 b16;       // its 16-bit form (beta_dtype bf16 / fp16)
  int bdt;       // beta_dtype

  // Unit i of this thread belongs to Q (1) or K (0); uniform across a wave.
  __device__ static int mat_of(int tid, int i) { return (tid + NT * i) / MAT_UNITS; }

  __device__ void init(const ChunkParams &p, int tid, int lane) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = (tid + NT * i) % MAT_UNITS;
      const int t = u / ROW_UNITS;
      const int byte = (u % ROW_UNITS) * EPU * 2;  // staged as 16-bit elements
      qk_off[i] = (t * p.Hk * K + (u % ROW_UNITS) * EPU) * sizeof(TIn);
      qk_lds[i] = t * LY::KPB + (byte ^ (((t >> 2) & 1) << 4));
    }
    const int tv = tid / (VT / EPU);
    const int c0 = (tid % (VT / EPU)) * EPU;
    v_off = tid < V_UNITS ? (tv * p.Hv * p.V + c0) * sizeof(TIn) : OUT_OF_RANGE;
    v_lds = tv * 32 + c0 * 2;
    g_off = lane * p.Hv * 4;
    b_off = lane * p.Hv * 2;
    bdt = p.beta_dtype;
  }

  // Issue the loads of the chunk starting at token t0 with `len` (may be <= 0
  // or > CH) tokens left in the sequence; value columns v0.. of head h.
  __device__ void load(const ChunkParams &p, long t0, long len, int hk, int h, int v0) {
    const long rows = len < CH ? len : CH;
    const long qk_bytes = rows > 0 ? ((rows - 1) * p.Hk * K + K) * static_cast<long>(sizeof(TIn)) : 0;
    const long qk_base = (t0 * p.Hk + hk) * static_cast<long>(K);
    const __amdgpu_buffer_rsrc_t rk = rsrc(static_cast<const TIn *>(p.k) + qk_base, qk_bytes);
    const __amdgpu_buffer_rsrc_t rq = rsrc(static_cast<const TIn *>(p.q) + qk_base, qk_bytes);
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      // wave-uniform (MAT_UNITS is a multiple of 64): keep the resource in SGPRs
      const int m = __builtin_amdgcn_readfirstlane(mat_of(threadIdx.x, i));
      x[i] = buf_load16(m ? rq : rk, qk_off[i]);
    }
    if constexpr (WITH_V) {
      const long v_bytes = rows > 0 ? ((rows - 1) * p.Hv * p.V + VT) * static_cast<long>(sizeof(TIn)) : 0;
      const __amdgpu_buffer_rsrc_t rv =
          rsrc(static_cast<const TIn *>(p.v) + (t0 * p.Hv + h) * static_cast<long>(p.V) + v0, v_bytes);
      vx = buf_load16(rv, v_off);
    }
    if constexpr (WITH_SCAN) {
      const long gi = t0 * p.Hv + h;
      const long n = rows > 0 ? (rows - 1) * p.Hv + 1 : 0;
      g = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc(p.g + gi, n * 4), g_off, 0, 0));
      // both forms are loaded (one from a zero-size resource); converted when stored
      const bool f32 = bdt == PBGDN_F32;
      b32 = __builtin_amdgcn_raw_buffer_load_b32(rsrc(static_cast<const float *>(p.beta) + gi, f32 ? n * 4 : 0),
                                                 2 * b_off, 0, 0);
      b16 = __builtin_amdgcn_raw_buffer_load_b16(rsrc(static_cast<const u16 *>(p.beta) + gi, f32 ? 0 : n * 2),
                                                 b_off, 0, 0);
    }
  }

  // A 16-byte unit as staged: 16-bit elements unchanged, fp32 rounded to fp16.
  __device__ static void put_unit(unsigned char *dst, const uint4 &x) {
    if constexpr (EPU == 8) {
      *reinterpret_cast<uint4 *>(dst) = x;
    } else {
      *reinterpret_cast<half4_t *>(dst) = to_half4(float4_t{__uint_as_float(x.x), __uint_as_float(x.y),
                                                            __uint_as_float(x.z), __uint_as_float(x.w)});
    }
  }

  // Registers -> LDS buffer `buf`: K and Q [t][key], V [t][col], and (scan
  // wave) the decay and beta tables of the chunk (below).
  __device__ void store(unsigned char *lds, int buf, int tid, int lane, bool scan, float scale, int sc_off = 0) const {
#pragma unroll
    for (int i = 0; i < UPT; ++i) put_unit(lds + LY::KQ + (2 * buf + mat_of(tid, i)) * LY::KQ_MAT + qk_lds[i], x[i]);
    if constexpr (WITH_V) {
      if (tid < V_UNITS) put_unit(lds + LY::V16 + buf * LY::V16_BUF + v_lds, vx);
    }
    if constexpr (WITH_SCAN) {
      if (scan) scan_tables(reinterpret_cast<float *>(lds + LY::SC + sc_off), lane, scale);
    }
  }

  // Inclusive cumulative sum c of g over the chunk, then fp32 [64] tables:
  // CUM c, GAM exp(c), DEC exp(c_63 - c), BET beta; [16][4] tables (entry
  // (i, r) is token 16 r + i): CUM4 c, BET4 beta, BU4 beta u, SU4 scale u with
  // u_t = exp(c_t - c_16(t/16)); and W_R[s] = exp(c_16R - c_s) for s < 16 R
  // (R = 1, 2, 3; else 0) at W1 + (R - 1) * 256.
  __device__ void scan_tables(float *sc, int lane, float scale) const {
    const float b = bdt == PBGDN_F32    ? __uint_as_float(b32)
                    : bdt == PBGDN_BF16 ? __uint_as_float(static_cast<uint32_t>(b16) << 16)
                                        : static_cast<float>(__builtin_bit_cast(half_t, b16));
    const float x = wave_prefix_sum(g);
    const float c16 = lane_value(x, 16), c32 = lane_value(x, 32), c48 = lane_value(x, 48);
    const float last = lane_value(x, 63);
    const int t4 = (lane & 15) * 4 + (lane >> 4);
    const float row0 = lane < 16 ? lane_value(x, 0) : lane < 32 ? c16 : lane < 48 ? c32 : c48;
    const float u = __expf(x - row0);
    sc[LY::CUM / 4 + lane] = x;
    sc[LY::GAM / 4 + lane] = __expf(x);
    sc[LY::DEC / 4 + lane] = __expf(last - x);
    sc[LY::BET / 4 + lane] = b;
    sc[LY::CUM4 / 4 + t4] = x;
    sc[LY::BET4 / 4 + t4] = b;
    sc[LY::BU4 / 4 + t4] = b * u;
    sc[LY::SU4 / 4 + t4] = scale * u;
    sc[LY::W1 / 4 + lane] = (lane < 16) ? __expf(c16 - x) : 0.f;
    sc[LY::W1 / 4 + CH + lane] = (lane < 32) ? __expf(c32 - x) : 0.f;
    sc[LY::W1 / 4 + 2 * CH + lane] = (lane < 48) ? __expf(c48 - x) : 0.f;
  }
};

// Launchers (explicitly instantiated in chunk_prep.hip, chunk_scan.hip,
// chunk_wide.hip and chunk_k256.hip).
template <int K, typename TIn>
int launch_prep(const ChunkParams &p, long records, hipStream_t stream);
template <int K, typename TIn, typename TOut>
int launch_scan(const ChunkParams &p, hipStream_t stream);
template <int K, typename TIn, typename TOut, bool EPI>
int launch_wide(const ChunkParams &p, hipStream_t stream);
// The scan for 256-wide keys (chunk_k256.hip): `wt` tiles (4 or 2) of 16
// columns per workgroup, each held by `kh` waves (1, or 2 with wt = 2: each
// wave a half of the keys); k256_waves picks wt for a call.
template <typename TIn, typename TOut>
int launch_k256(const ChunkParams &p, int wt, int kh, hipStream_t stream);
int k256_waves(int V, long pairs_of_seq_and_head, int cus);

}  // namespace pbgdn
