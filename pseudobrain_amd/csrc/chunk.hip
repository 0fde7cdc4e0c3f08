// Chunkwise Gated DeltaNet prefill for gfx950 (CDNA4).
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
// Decomposition. The recurrence is separable along the value columns, so a
// workgroup owns one (sequence, value head, 16-column tile of V): grid =
// V/16 x Hv x N, 512 threads (8 waves), one workgroup per CU (~150 KB LDS).
// The fp32 state tile S [K, 16] lives in MFMA accumulators for the whole
// sequence (wave w owns key rows 16w..16w+15) and is written out once.
//
// Pipeline. Each loop iteration ("tick" n) has three barrier-separated phases
// and overlaps three chunks:
//   phase 1: chain   K S, X = V - gamma K S              (chunk n, waves 0-3)
//            output  Q S                                 (chunk n, waves 4-7)
//            inverse off-diagonal 16x16 blocks of T, Tb  (chunk n, waves 6-7)
//            inputs  chunk n+1 registers -> LDS, cumsum of g;
//                    buffer loads of chunk n+2 issued into registers
//   phase 2: chain   U = Tb X                            (chunk n, waves 0-3)
//            prep    K K^T -> A, Q K^T -> QKD            (chunk n+1, all waves)
//   phase 3: chain   S <- gamma_C S + K^T (dec U)        (chunk n, waves owning S)
//            output  O = gamma scale Q S + QKD U, store  (chunk n, waves 4-7)
//            inverse diagonal 16x16 blocks of T          (chunk n+1, waves 0-3)
// so the S-dependent chain of one chunk runs beside the S-independent work of
// the next. Barriers wait for LDS traffic only, so the prefetch of chunk n+2
// stays in flight for a whole tick.
//
// Costs that shape the code (measured on MI355X): a wave64 VALU instruction
// occupies its SIMD for 4 cycles and a 16x16x32 MFMA for ~14-16, and the LDS
// delivers ~200 B/clk per CU for conflict-free 16-byte reads. Hence:
//   * global traffic uses buffer instructions: per-lane byte offsets are fixed
//     for the whole sequence and each chunk only moves a scalar base, whose
//     range check also zero-fills tokens past the end (no address arithmetic
//     or masking in the vector unit);
//   * every LDS row pitch is its length + 32 bytes, the conflict-free stride
//     for 16-byte fragment reads;
//   * the A and QKD tiles are computed transposed so each lane stores 4
//     consecutive elements of a row with one write;
//   * K^T fragments for the state update come from ds_read_b64_tr_b16, which
//     transposes 16-bit elements across each group of 16 lanes;
//   * role parameters (tile indices, buffers) are wave-uniform runtime values,
//     so the loop body stays small for the instruction cache.
//
// Arithmetic (fp32 accumulation throughout):
//   * q/k products use the input's own 16-bit type on v_mfma_f32_16x16x32:
//     bf16 inputs are fed to the bf16 MFMA unconverted; fp16 inputs as fp16;
//     fp32 inputs are rounded to fp16 once when staged.
//   * S enters K S as a high + low pair of that type (two MFMAs), so X sees
//     the fp32 state to ~16 bits; Q S, which only reaches the output, uses the
//     high part. The state update K^T (dec U) uses dec U as a pair.
//   * Tb, X, U and QKD are fp16 (11-bit significand) on the fp16 MFMA.
//   * The diagonal 16x16 blocks of T come from the nilpotent product
//     (I + M)(I + M^2)(I + M^4)(I + M^8) on fp16 high/low MFMAs (~22-bit
//     products); the off-diagonal blocks from 16x16x16 fp16 MFMAs.
//
// Fragment layouts (lane l, g = l >> 4, c = l & 15). 16x16x32: A holds
// A[m = c][k = 8g + j], B holds B[k = 8g + j][n = c], j = 0..7; 16x16x16:
// k = 4g + j, j = 0..3; the accumulator holds D[4g + i][c], i = 0..3. Any
// consistent assignment of contraction slots works, as long as A and B agree.
// B operands are kept in LDS transposed ([n][k]) so both fragments are one
// 16-byte read, and an accumulator tile is written there as one 8-byte store.
#include "common.hpp"

namespace pbgdn {

typedef __bf16 bf16_t;
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));

constexpr int CH = 64;        // chunk length (CHUNK, gated_deltanet.py:49)
constexpr int VT = 16;        // value columns per workgroup
constexpr int NT = 512;       // threads per workgroup
constexpr int NW = NT / 64;   // waves per workgroup
constexpr int SCAN_WAVE = 5;  // wave that loads g, beta and scans them
constexpr int RSRC_WORD3 = 0x00020000;  // raw buffer resource, gfx9 family

struct ChunkParams {
  const void *q, *k, *v;
  const float *g;
  const void *beta;
  int beta_dtype;
  const float *h0;
  float *ht;
  const int32_t *cu_seqlens;
  void *o;
  int T, Hk, Hv, V, num_seqs;
  float scale;
};

// Operand type of the q/k products: bf16 for bf16 inputs, fp16 otherwise.
template <typename TIn>
struct OpOf {
  using T4 = half4_t;
  using T8 = half8_t;
  __device__ static T4 from(float4_t x) { return to_half4(x); }
  __device__ static float4_t to(T4 x) { return to_float4(x); }
};
template <>
struct OpOf<u16> {
  using T4 = bf16x4_t;
  using T8 = bf16x8_t;
  __device__ static T4 from(float4_t x) {
    return T4{static_cast<bf16_t>(x[0]), static_cast<bf16_t>(x[1]), static_cast<bf16_t>(x[2]),
              static_cast<bf16_t>(x[3])};
  }
  __device__ static float4_t to(T4 x) {
    return float4_t{static_cast<float>(x[0]), static_cast<float>(x[1]), static_cast<float>(x[2]),
                    static_cast<float>(x[3])};
  }
};

__device__ __forceinline__ float4_t mma(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float4_t mma(bf16x8_t a, bf16x8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <typename V8>
__device__ __forceinline__ V8 ld8(const void *p) { return *reinterpret_cast<const V8 *>(p); }
template <typename V4>
__device__ __forceinline__ void st4(void *p, V4 x) { *reinterpret_cast<V4 *>(p) = x; }
__device__ __forceinline__ half8_t lds8(const half_t *p) { return *reinterpret_cast<const half8_t *>(p); }
__device__ __forceinline__ float4_t ldf4(const float *p) { return *reinterpret_cast<const float4_t *>(p); }

// Transposing LDS read of four 16-bit elements (ds_read_b64_tr_b16). Within
// each group of 16 lanes, lane o receives element (o & 3) of the 8 bytes read
// by lanes 4k + (o >> 2), k = 0..3: if lanes 4k..4k+3 of a group point at row
// r_k, columns 0-3, 4-7, 8-11, 12-15 of a 16-column block, lane o gets column
// o of rows r_0..r_3.
__device__ __forceinline__ i16x4_t ld_tr(const u16 *p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4_t *)(reinterpret_cast<uintptr_t>(p)));
}

// Workgroup barrier for LDS traffic: waits for this wave's LDS operations, not
// for its outstanding global loads (the prefetched chunk) or stores.
__device__ __forceinline__ void block_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, long bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                           static_cast<int>(bytes > 0 ? bytes : 0), RSRC_WORD3);
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

template <int K>
struct ChunkSmem {
  static constexpr int KP = K + 16;   // pitch (16-bit elements) of [t][key] and [col][key] rows
  static constexpr int SP = CH + 16;  // pitch (16-bit elements) of [.][t] rows
  static constexpr int FP = CH + 8;   // pitch (floats) of fp32 rows of 64
  alignas(16) u16 kq[2][2][CH][KP];   // [buffer][K, Q][t][key], operand type
  alignas(16) float vt[2][VT][FP];    // V column tile, transposed [col][t]
  alignas(16) float cum[2][CH];       // inclusive cumsum of g
  alignas(16) float gam[2][CH];       // exp(cum)
  alignas(16) float dec[2][CH];       // exp(cum[C-1] - cum)
  alignas(16) float bet[2][CH];       // beta
  alignas(16) float at[CH][FP];       // A, then T's diagonal blocks in place (fp32)
  alignas(16) half_t tb[CH][SP];      // Tb = T diag(beta), [t][s]
  alignas(16) half_t qkd[2][CH][SP];  // scale (Q K^T o D), inclusive lower, [t][s]
  alignas(16) half_t xt[VT][SP];      // X^T [col][t]
  alignas(16) half_t ut[VT][SP];      // U^T [col][t]
  alignas(16) u16 uh[VT][SP];         // (dec U)^T high part, operand type
  alignas(16) u16 ul[VT][SP];         // (dec U)^T low part
  alignas(16) u16 sh[VT][KP];         // S^T [col][key] high part, operand type
  alignas(16) u16 sl[VT][KP];         // S^T low part
};

// One chunk of raw inputs held in registers between its buffer load (issued a
// tick ahead) and its store into LDS. Per-lane byte offsets are fixed for the
// whole sequence; a chunk only sets the scalar base and range of each buffer
// resource, and tokens at or past the end of the sequence load as zeros
// (k = v = g = beta = 0: the identity steps of the reference's padding,
// gated_deltanet.py:127).
template <int K, typename TIn>
struct ChunkInputs {
  static constexpr int EPU = 16 / sizeof(TIn);              // elements per 16-byte unit
  static constexpr int ROW_UNITS = K / EPU;
  static constexpr int MAT_UNITS = CH * ROW_UNITS;          // units of one of K, Q
  static constexpr int PER_MAT = MAT_UNITS / NT;            // units per thread per matrix
  static constexpr int V_UNITS = CH * VT / EPU;
  static_assert(MAT_UNITS % NT == 0, "K/Q units must tile the workgroup");
  static_assert(V_UNITS <= NT, "V units exceed the workgroup");

  uint32_t qk_off[PER_MAT];  // byte offset of this thread's units within a chunk
  uint32_t v_off, g_off, b_off;
  uint4 kx[PER_MAT], qx[PER_MAT], vx;
  float g, b;

  __device__ void init(const ChunkParams &p, int tid, int lane) {
#pragma unroll
    for (int i = 0; i < PER_MAT; ++i) {
      const int u = tid + NT * i;
      qk_off[i] = ((u / ROW_UNITS) * p.Hk * K + (u % ROW_UNITS) * EPU) * sizeof(TIn);
    }
    const int tv = tid / (VT / EPU);
    v_off = (tv * p.Hv * p.V + (tid % (VT / EPU)) * EPU) * sizeof(TIn);
    g_off = lane * p.Hv * 4;
    b_off = lane * p.Hv * (p.beta_dtype == PBGDN_F32 ? 4 : 2);
  }

  // Issue the loads of the chunk starting at token t0 with `len` (may be <= 0
  // or > CH) tokens left in the sequence.
  __device__ void load(const ChunkParams &p, long t0, long len, int hk, int h, int v0, int tid, bool scan) {
    const long rows = len < CH ? len : CH;
    const long qk_bytes = rows > 0 ? ((rows - 1) * p.Hk * K + K) * static_cast<long>(sizeof(TIn)) : 0;
    const long qk_base = (t0 * p.Hk + hk) * static_cast<long>(K);
    const __amdgpu_buffer_rsrc_t rk = rsrc(static_cast<const TIn *>(p.k) + qk_base, qk_bytes);
    const __amdgpu_buffer_rsrc_t rq = rsrc(static_cast<const TIn *>(p.q) + qk_base, qk_bytes);
#pragma unroll
    for (int i = 0; i < PER_MAT; ++i) {
      kx[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, qk_off[i], 0, 0));
      qx[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, qk_off[i], 0, 0));
    }
    if (tid < V_UNITS) {
      const long v_bytes = rows > 0 ? ((rows - 1) * p.Hv * p.V + VT) * static_cast<long>(sizeof(TIn)) : 0;
      const __amdgpu_buffer_rsrc_t rv =
          rsrc(static_cast<const TIn *>(p.v) + (t0 * p.Hv + h) * static_cast<long>(p.V) + v0, v_bytes);
      vx = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, v_off, 0, 0));
    }
    if (scan) {
      const long gi = t0 * p.Hv + h;
      const long n = rows > 0 ? (rows - 1) * p.Hv + 1 : 0;
      g = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc(p.g + gi, n * 4), g_off, 0, 0));
      if (p.beta_dtype == PBGDN_F32) {
        b = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                          rsrc(static_cast<const float *>(p.beta) + gi, n * 4), b_off, 0, 0));
      } else {
        const u16 raw =
            __builtin_amdgcn_raw_buffer_load_b16(rsrc(static_cast<const u16 *>(p.beta) + gi, n * 2), b_off, 0, 0);
        b = (p.beta_dtype == PBGDN_BF16) ? __uint_as_float(static_cast<uint32_t>(raw) << 16)
                                         : static_cast<float>(__builtin_bit_cast(half_t, raw));
      }
    }
  }

  __device__ static float elem(const uint4 &raw, int i) {
    const uint32_t w = (EPU == 4) ? ((i == 0) ? raw.x : (i == 1) ? raw.y : (i == 2) ? raw.z : raw.w)
                                  : ((i < 2) ? raw.x : (i < 4) ? raw.y : (i < 6) ? raw.z : raw.w);
    if constexpr (EPU == 4) {
      return __uint_as_float(w);
    } else if constexpr (__is_same(TIn, u16)) {  // bf16
      return (i & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
    } else {
      const u16 bits = (i & 1) ? static_cast<u16>(w >> 16) : static_cast<u16>(w & 0xffffu);
      return static_cast<float>(__builtin_bit_cast(half_t, bits));
    }
  }

  __device__ static void put_unit(u16 *dst, const uint4 &x) {
    if constexpr (EPU == 8) {
      *reinterpret_cast<uint4 *>(dst) = x;
    } else {
      st4(dst, to_half4(float4_t{__uint_as_float(x.x), __uint_as_float(x.y), __uint_as_float(x.z),
                                 __uint_as_float(x.w)}));
    }
  }

  // Registers -> LDS buffer `buf`: K and Q in the operand type [t][key], V^T in
  // fp32, and (scan wave) the cumulative decays and beta of the chunk.
  __device__ void store(ChunkSmem<K> &sm, int buf, int tid, int lane, bool scan) const {
#pragma unroll
    for (int i = 0; i < PER_MAT; ++i) {
      const int u = tid + NT * i;
      put_unit(&sm.kq[buf][0][u / ROW_UNITS][(u % ROW_UNITS) * EPU], kx[i]);
      put_unit(&sm.kq[buf][1][u / ROW_UNITS][(u % ROW_UNITS) * EPU], qx[i]);
    }
    if (tid < V_UNITS) {
      const int t = tid / (VT / EPU);
      const int c0 = (tid % (VT / EPU)) * EPU;
#pragma unroll
      for (int j = 0; j < EPU; ++j) sm.vt[buf][c0 + j][t] = elem(vx, j);
    }
    if (scan) {
      float x = g;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
      }
      const float last = __shfl(x, 63, 64);
      sm.cum[buf][lane] = x;
      sm.gam[buf][lane] = __expf(x);
      sm.dec[buf][lane] = __expf(last - x);
      sm.bet[buf][lane] = b;
    }
  }
};

// Block index -> (sequence, value head, column tile). All column tiles of the
// value heads that share one query/key head of one sequence form a group; a
// group is kept on one XCD (workgroups are dispatched round-robin over the 8
// XCDs) so that its q/k chunks are fetched into that XCD's L2 once.
__device__ __forceinline__ void decode_block(int L, int total, int nv, int group_heads, int Hk, int &seq, int &h,
                                             int &vtile) {
  const int gsize = nv * group_heads;
  const int ngroups = total / gsize;
  int grp, in;
  if (ngroups % 8 == 0) {
    const int xcd = L & 7;
    const int slot = L >> 3;
    grp = (slot / gsize) * 8 + xcd;
    in = slot % gsize;
  } else {
    grp = L / gsize;
    in = L % gsize;
  }
  const int hk = grp % Hk;
  seq = grp / Hk;
  h = hk * group_heads + in / nv;
  vtile = in % nv;
}

template <int K, typename TIn, typename TOut>
struct ChunkBlock {
  using Smem = ChunkSmem<K>;
  using Op = OpOf<TIn>;
  using O4 = typename Op::T4;
  using O8 = typename Op::T8;
  static constexpr int NKT = K / 16;  // key tiles of S, one per wave
  static constexpr int KS = K / 32;   // contraction steps over keys
  static_assert(K == 64 || K == 128, "K must be 64 or 128");
  static_assert(NKT <= NW, "one S key tile per wave");

  Smem &sm;
  const ChunkParams &p;
  int tid, lane, c16, g4, wave, seq, h, hk, v0;
  long bos, eos, nchunks;
  uint32_t o_off;  // byte offset of this lane's first output element in a chunk
  float4_t sacc, qs;
  ChunkInputs<K, TIn> in;

  __device__ ChunkBlock(Smem &s, const ChunkParams &prm) : sm(s), p(prm) {
    tid = threadIdx.x;
    lane = tid & 63;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    c16 = lane & 15;
    g4 = lane >> 4;
    const int group_heads = p.Hv / p.Hk;
    int vtile;
    decode_block(blockIdx.x, gridDim.x, p.V / VT, group_heads, p.Hk, seq, h, vtile);
    hk = h / group_heads;
    v0 = vtile * VT;
    if (p.cu_seqlens) {
      bos = p.cu_seqlens[seq];
      eos = p.cu_seqlens[seq + 1];
    } else {
      bos = static_cast<long>(seq) * p.T;
      eos = bos + p.T;
    }
    nchunks = (eos - bos + CH - 1) / CH;
    sacc = float4_t{0.f, 0.f, 0.f, 0.f};
    qs = sacc;
    in.init(p, tid, lane);
    o_off = ((16 * (wave & 3) + 4 * g4) * p.Hv * p.V + c16) * sizeof(TOut);
  }

  __device__ void load_chunk(long n) {
    const long t0 = bos + n * CH;
    in.load(p, t0, eos - t0, hk, h, v0, tid, wave == SCAN_WAVE);
  }

  // ---------------------------------------------------------------- phase 1
  // Waves 0-3: chain X = V - gamma K S for token rows 16w.. (S as a high/low
  // pair); waves 4-7: Q S (high part) for token rows 16(w-4)..; waves 6, 7
  // also the off-diagonal blocks of T.
  __device__ void phase1(long n, int b) {
    const int r = wave & 3;
    const bool chain = wave < 4;
    O8 a[KS], shi[KS], slo[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      a[kk] = ld8<O8>(&sm.kq[b][chain ? 0 : 1][16 * r + c16][32 * kk + 8 * g4]);
      shi[kk] = ld8<O8>(&sm.sh[c16][32 * kk + 8 * g4]);
    }
    const int tr = 16 * r + 4 * g4;
    float4_t vv, gg;
    if (chain) {
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) slo[kk] = ld8<O8>(&sm.sl[c16][32 * kk + 8 * g4]);
      vv = ldf4(&sm.vt[b][c16][tr]);
      gg = ldf4(&sm.gam[b][tr]);
    }
    in.store(sm, b ^ 1, tid, lane, wave == SCAN_WAVE);
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) acc = mma(a[kk], shi[kk], acc);
    if (chain) {
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) acc = mma(a[kk], slo[kk], acc);
      st4(&sm.xt[c16][tr], to_half4(vv - gg * acc));
    } else {
      qs = acc;
      if (wave >= 6) offdiag(b, wave == 6);
    }
    load_chunk(n + 2);
  }

  // Off-diagonal blocks of T for the chunk in buffer b:
  //   T_rs = -D_r sum_{s<=j<r} A_rj T_js,  D_r = T_rr (fp32 in `at`),
  // written as Tb blocks T_rs diag(beta). First: T10, T20, T30; else T21, T31, T32.
  __device__ void offdiag(int b, bool first) {
    const float4_t z = {0.f, 0.f, 0.f, 0.f};
    auto aop = [&](int R, int C) {  // A[m = c][k = 4g + j] = at[R + m][C + k]
      return to_half4(ldf4(&sm.at[R + c16][C + 4 * g4]));
    };
    auto dop = [&](int S) {  // B[k = 4g + j][n = c] = D_S[k][n]
      half4_t x;
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = static_cast<half_t>(sm.at[16 * S + 4 * g4 + j][16 * S + c16]);
      return x;
    };
    auto put = [&](int r, int s, float4_t mv, float bs) {  // mv = -T_rs
#pragma unroll
      for (int i = 0; i < 4; ++i) sm.tb[16 * r + 4 * g4 + i][16 * s + c16] = static_cast<half_t>(-mv[i] * bs);
    };
    if (first) {
      const half4_t a10 = aop(16, 0), a20 = aop(32, 0), a21 = aop(32, 16);
      const half4_t a30 = aop(48, 0), a31 = aop(48, 16), a32 = aop(48, 32);
      const half4_t d1 = aop(16, 16), d2 = aop(32, 32), d3 = aop(48, 48), d0 = dop(0);
      const float bs = sm.bet[b][c16];
      const float4_t m10 = mfma16(d1, to_half4(mfma16(a10, d0, z)), z);
      const half4_t t10 = to_half4(-m10);
      const float4_t m20 = mfma16(d2, to_half4(mfma16(a21, t10, mfma16(a20, d0, z))), z);
      const half4_t t20 = to_half4(-m20);
      const float4_t m30 = mfma16(d3, to_half4(mfma16(a32, t20, mfma16(a31, t10, mfma16(a30, d0, z)))), z);
      put(1, 0, m10, bs);
      put(2, 0, m20, bs);
      put(3, 0, m30, bs);
    } else {
      const half4_t a21 = aop(32, 16), a31 = aop(48, 16), a32 = aop(48, 32);
      const half4_t d2 = aop(32, 32), d3 = aop(48, 48), d1b = dop(1), d2b = dop(2);
      const float bs1 = sm.bet[b][16 + c16], bs2 = sm.bet[b][32 + c16];
      const float4_t m21 = mfma16(d2, to_half4(mfma16(a21, d1b, z)), z);
      const half4_t t21 = to_half4(-m21);
      const float4_t m31 = mfma16(d3, to_half4(mfma16(a32, t21, mfma16(a31, d1b, z))), z);
      const float4_t m32 = mfma16(d3, to_half4(mfma16(a32, d2b, z)), z);
      put(2, 1, m21, bs1);
      put(3, 1, m31, bs1);
      put(3, 2, m32, bs2);
    }
  }

  // ---------------------------------------------------------------- phase 2
  // Waves 0-3: chain U = Tb X for token rows 16w.. (the zero upper blocks of
  // Tb make two contraction steps exact for every row tile); then every wave
  // computes its tiles of A and QKD for chunk n+1.
  __device__ void phase2(int b) {
    const int nb = b ^ 1;
    if (wave < 4) {
      half8_t ta[2], xb[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        ta[ks] = lds8(&sm.tb[16 * wave + c16][32 * ks + 8 * g4]);
        xb[ks] = lds8(&sm.xt[c16][32 * ks + 8 * g4]);
      }
      const int tr = 16 * wave + 4 * g4;
      const float4_t dd = ldf4(&sm.dec[b][tr]);
      float4_t u = mfma32(ta[0], xb[0], float4_t{0.f, 0.f, 0.f, 0.f});
      u = mfma32(ta[1], xb[1], u);
      st4(&sm.ut[c16][tr], to_half4(u));
      const float4_t du = u * dd;
      const O4 hi = Op::from(du);
      st4(&sm.uh[c16][tr], hi);
      st4(&sm.ul[c16][tr], Op::from(du - Op::to(hi)));
    }
    products(nb);
  }

  // The 10 lower 16x16 tile pairs (R, S) of A and QKD: (3,0), (3,1), (2,0),
  // (2,1) on waves 0-3 (which also run U = Tb X), two pairs on waves 4 and 5,
  // one on waves 6 and 7.
  __device__ void products(int nb) {
    if (wave < 4) {
      tile_pair(nb, 3 - (wave >> 1), wave & 1);
    } else if (wave == 4) {
      tile_pair(nb, 3, 2);
      tile_pair(nb, 3, 3);
    } else if (wave == 5) {
      tile_pair(nb, 2, 2);
      tile_pair(nb, 1, 1);
    } else {
      tile_pair(nb, wave == 6 ? 1 : 0, 0);
    }
  }

  // Tile (R, S), S <= R, of A = strict_lower(b_t K K^T o D) and of
  // QKD = scale (Q K^T o D) (inclusive) for the chunk in buffer nb. The
  // products are formed transposed (rows s from K_S, columns t from K_R and
  // Q_R), so lane (g, c) holds row t = 16R + c, columns s = 16S + 4g..4g+3 and
  // stores them with one write each; the decays exp(c_t - c_s) are shared.
  __device__ void tile_pair(int nb, int R, int S) {
    O8 ks[KS], kr[KS], qr[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      ks[kk] = ld8<O8>(&sm.kq[nb][0][16 * S + c16][32 * kk + 8 * g4]);
      kr[kk] = ld8<O8>(&sm.kq[nb][0][16 * R + c16][32 * kk + 8 * g4]);
      qr[kk] = ld8<O8>(&sm.kq[nb][1][16 * R + c16][32 * kk + 8 * g4]);
    }
    const int t = 16 * R + c16;
    const int s0 = 16 * S + 4 * g4;
    const float ct = sm.cum[nb][t];
    const float bt = sm.bet[nb][t];
    const float4_t cs = ldf4(&sm.cum[nb][s0]);
    float4_t acck = {0.f, 0.f, 0.f, 0.f}, accq = acck;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      acck = mma(ks[kk], kr[kk], acck);
      accq = mma(ks[kk], qr[kk], accq);
    }
    float4_t av, qv;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float d = __expf(ct - cs[i]);
      av[i] = (s0 + i < t) ? bt * acck[i] * d : 0.f;
      qv[i] = (s0 + i <= t) ? p.scale * accq[i] * d : 0.f;
    }
    *reinterpret_cast<float4_t *>(&sm.at[t][s0]) = av;
    st4(&sm.qkd[nb][t][s0], to_half4(qv));
  }

  // ---------------------------------------------------------------- phase 3
  // Waves owning S: S <- gamma_C S + K^T (dec U); waves 4-7: O = gamma scale
  // Q S + QKD U for token rows 16(w-4).., stored; waves 0-3: diagonal blocks
  // of T for chunk n+1.
  __device__ void phase3(long n, int b) {
    if (wave < NKT) {
      // K^T fragment of key tile w, token step ts: contraction slot j of lane
      // group g is token 32 ts + 8 g + j, the slot order of uh / ul.
      O8 ka[2], hb[2], lb[2];
      const int trow = 8 * g4 + (c16 >> 2);
      const int tcol = 16 * wave + 4 * (c16 & 3);
#pragma unroll
      for (int ts = 0; ts < 2; ++ts) {
        const i16x4_t lo4 = ld_tr(&sm.kq[b][0][32 * ts + trow][tcol]);
        const i16x4_t hi4 = ld_tr(&sm.kq[b][0][32 * ts + trow + 4][tcol]);
        ka[ts] = __builtin_bit_cast(O8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
        hb[ts] = ld8<O8>(&sm.uh[c16][32 * ts + 8 * g4]);
        lb[ts] = ld8<O8>(&sm.ul[c16][32 * ts + 8 * g4]);
      }
      sacc *= sm.gam[b][CH - 1];
#pragma unroll
      for (int ts = 0; ts < 2; ++ts) {
        sacc = mma(ka[ts], hb[ts], sacc);
        sacc = mma(ka[ts], lb[ts], sacc);
      }
      const O4 hi = Op::from(sacc);
      st4(&sm.sh[c16][16 * wave + 4 * g4], hi);
      st4(&sm.sl[c16][16 * wave + 4 * g4], Op::from(sacc - Op::to(hi)));
    }
    if (wave >= 4) {
      const int r = wave - 4;
      half8_t qa[2], ub[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        qa[ks] = lds8(&sm.qkd[b][16 * r + c16][32 * ks + 8 * g4]);
        ub[ks] = lds8(&sm.ut[c16][32 * ks + 8 * g4]);
      }
      const int tr = 16 * r + 4 * g4;
      float4_t o = qs * ldf4(&sm.gam[b][tr]) * p.scale;
      o = mfma32(qa[0], ub[0], o);
      o = mfma32(qa[1], ub[1], o);
      const long t0 = bos + n * CH;
      const long len = eos - t0;
      const long rows = len < CH ? len : CH;
      const long bytes = ((rows - 1) * p.Hv * p.V + VT) * static_cast<long>(sizeof(TOut));
      const __amdgpu_buffer_rsrc_t ro =
          rsrc(static_cast<TOut *>(p.o) + (t0 * p.Hv + h) * static_cast<long>(p.V) + v0, bytes);
      const uint32_t row = p.Hv * p.V * sizeof(TOut);
#pragma unroll
      for (int i = 0; i < 4; ++i) put_out<TOut>(ro, o_off + i * row, o[i]);
    } else {
      diag(b ^ 1);
    }
  }

  // fp16 high/low pair of an fp32 tile, and c + a b from pairs (3 MFMAs, the
  // low*low term dropped): a product accurate to ~22 bits.
  struct Pair16 {
    half4_t h, l;
  };
  __device__ static Pair16 split16(float4_t x) {
    Pair16 r;
    r.h = to_half4(x);
    r.l = to_half4(x - to_float4(r.h));
    return r;
  }
  __device__ static float4_t mul3(const Pair16 &a, const Pair16 &b, float4_t c) {
    c = mfma16(a.h, b.h, c);
    c = mfma16(a.h, b.l, c);
    return mfma16(a.l, b.h, c);
  }

  // Diagonal block D_w = (I + A_ww)^-1 (w = this wave) of the chunk in buffer
  // nb. A_ww is strictly lower triangular (nilpotent), so with M = -A_ww
  //   D = (I + M)(I + M^2)(I + M^4)(I + M^8).
  // A 16x16 matrix X held as an accumulator tile (lane (g, c): X[4g + i][c]) is
  // the B operand of a 16x16x16 MFMA as is, and the A operand of X^T; keeping
  // P_k = M^k and its transpose as tiles gives every operand without LDS, and
  // Y = D is built transposed: Y^T <- Y^T + P_k^T Y^T. D replaces A_ww in `at`
  // (fp32), and D diag(beta) is the diagonal block of Tb.
  __device__ void diag(int nb) {
    const int base = 16 * wave;
    const float4_t z = {0.f, 0.f, 0.f, 0.f};
    float4_t p1;  // M as a tile
#pragma unroll
    for (int i = 0; i < 4; ++i) p1[i] = -sm.at[base + 4 * g4 + i][base + c16];
    const float4_t p1t = -ldf4(&sm.at[base + c16][base + 4 * g4]);  // M^T as a tile
    const float4_t bw = ldf4(&sm.bet[nb][base + 4 * g4]);
    float4_t yt = p1t;  // (I + M)^T
#pragma unroll
    for (int i = 0; i < 4; ++i) yt[i] += (4 * g4 + i == c16) ? 1.f : 0.f;
    const Pair16 s1 = split16(p1), s1t = split16(p1t);
    const Pair16 s2 = split16(mul3(s1t, s1, z)), s2t = split16(mul3(s1, s1t, z));  // M^2, (M^2)^T
    yt = mul3(s2, split16(yt), yt);
    const Pair16 s4 = split16(mul3(s2t, s2, z)), s4t = split16(mul3(s2, s2t, z));  // M^4, (M^4)^T
    yt = mul3(s4, split16(yt), yt);
    const Pair16 s8 = split16(mul3(s4t, s4, z));                                    // M^8
    yt = mul3(s8, split16(yt), yt);
    // yt holds D^T: lane (g, c) has D[c][4g + i].
    *reinterpret_cast<float4_t *>(&sm.at[base + c16][base + 4 * g4]) = yt;
    st4(&sm.tb[base + c16][base + 4 * g4], to_half4(yt * bw));
  }

  __device__ void tick(long n) {
    // Re-define the lane indices opaquely each tick: the per-lane LDS addresses
    // derived from them are then formed where they are used instead of being
    // hoisted out of the loop, where they would hold ~100 registers.
    asm volatile("" : "+v"(c16), "+v"(g4), "+v"(lane), "+v"(tid));
    const int b = static_cast<int>(n & 1);
    phase1(n, b);
    block_sync();
    phase2(b);
    block_sync();
    phase3(n, b);
    block_sync();
  }

  __device__ void run() {
    // Blocks of Tb and QKD above the diagonal are read as zeros and never written.
    for (int i = tid; i < CH * Smem::SP; i += NT) {
      (&sm.tb[0][0])[i] = static_cast<half_t>(0.f);
      (&sm.qkd[0][0][0])[i] = static_cast<half_t>(0.f);
      (&sm.qkd[1][0][0])[i] = static_cast<half_t>(0.f);
    }
    // Initial state: wave w owns key rows 16w..16w+15.
    const long state_base = (static_cast<long>(seq) * p.Hv + h) * K * p.V + v0 + c16;
    if (wave < NKT) {
      if (p.h0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sacc[i] = p.h0[state_base + static_cast<long>(16 * wave + 4 * g4 + i) * p.V];
      }
      const O4 hi = Op::from(sacc);
      st4(&sm.sh[c16][16 * wave + 4 * g4], hi);
      st4(&sm.sl[c16][16 * wave + 4 * g4], Op::from(sacc - Op::to(hi)));
    }
    load_chunk(0);
    block_sync();
    // Prologue: chunk 0 into buffer 0 and through the S-independent prep.
    in.store(sm, 0, tid, lane, wave == SCAN_WAVE);
    load_chunk(1);
    block_sync();
    products(0);
    block_sync();
    if (wave < 4) diag(0);
    block_sync();
    for (long n = 0; n < nchunks; ++n) tick(n);
    if (p.ht && wave < NKT) {
#pragma unroll
      for (int i = 0; i < 4; ++i) p.ht[state_base + static_cast<long>(16 * wave + 4 * g4 + i) * p.V] = sacc[i];
    }
  }
};

template <int K, typename TIn, typename TOut>
__global__ __launch_bounds__(NT) void chunk_kernel(ChunkParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  ChunkBlock<K, TIn, TOut> blk(*reinterpret_cast<ChunkSmem<K> *>(smem_raw), p);
  blk.run();
}

template <int K, typename TIn, typename TOut>
static int launch_chunk(const ChunkParams &p, hipStream_t stream) {
  static bool configured = false;  // benign race: the attribute call is idempotent
  const size_t smem = sizeof(ChunkSmem<K>);
  auto kernel = chunk_kernel<K, TIn, TOut>;
  if (!configured) {
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(smem)) != hipSuccess) {
      return PBGDN_ERR_LAUNCH;
    }
    configured = true;
  }
  const int total = (p.V / VT) * p.Hv * p.num_seqs;
  hipLaunchKernelGGL(kernel, dim3(total), dim3(NT), smem, stream, p);
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}

template <int K, typename TIn>
static int dispatch_out(const ChunkParams &p, int out_dtype, int in_dtype, hipStream_t stream) {
  if (out_dtype == PBGDN_F32) return launch_chunk<K, TIn, float>(p, stream);
  if (out_dtype == in_dtype) return launch_chunk<K, TIn, TIn>(p, stream);
  return PBGDN_ERR_UNSUPPORTED;
}

template <int K>
static int dispatch_in(const ChunkParams &p, int in_dtype, int out_dtype, hipStream_t stream) {
  switch (in_dtype) {
    case PBGDN_BF16: return dispatch_out<K, u16>(p, out_dtype, in_dtype, stream);
    case PBGDN_F16: return dispatch_out<K, half_t>(p, out_dtype, in_dtype, stream);
    case PBGDN_F32: return launch_chunk<K, float, float>(p, stream);
    default: return PBGDN_ERR_INVALID_ARGUMENT;
  }
}

}  // namespace pbgdn

static bool valid_dtype(int d) { return d == PBGDN_F32 || d == PBGDN_BF16 || d == PBGDN_F16; }

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

extern "C" int pbgdn_chunk_fwd(const void *q, const void *k, const void *v, int in_dtype, const float *g,
                               const void *beta, int beta_dtype, const float *h0, float *ht,
                               const int32_t *cu_seqlens, int num_seqs, void *o, int out_dtype, int B, int T,
                               int Hk, int Hv, int K, int V, float scale, int chunk, void *stream) {
  if (B < 0 || T < 0 || Hk <= 0 || Hv <= 0 || K <= 0 || V <= 0 || Hv % Hk != 0 || num_seqs < 0) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype) || !(beta_dtype == PBGDN_F32 || beta_dtype == in_dtype)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (cu_seqlens ? B != 1 : num_seqs != B) return PBGDN_ERR_INVALID_ARGUMENT;
  if (chunk != pbgdn::CH) return PBGDN_ERR_UNSUPPORTED;
  if (!(K == 64 || K == 128) || V % pbgdn::VT != 0) return PBGDN_ERR_UNSUPPORTED;
  if (!(out_dtype == PBGDN_F32 || out_dtype == in_dtype)) return PBGDN_ERR_UNSUPPORTED;
  // Per-chunk buffer ranges and per-lane offsets are 32-bit byte counts.
  if (static_cast<long>(pbgdn::CH) * Hv * V * 4 > 0x7fffffffL ||
      static_cast<long>(pbgdn::CH) * Hk * K * 4 > 0x7fffffffL) {
    return PBGDN_ERR_UNSUPPORTED;
  }
  if (num_seqs == 0) return PBGDN_OK;
  if (T > 0 && (!q || !k || !v || !g || !beta || !o)) return PBGDN_ERR_INVALID_ARGUMENT;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v)) return PBGDN_ERR_INVALID_ARGUMENT;
  const long total = static_cast<long>(V / pbgdn::VT) * Hv * num_seqs;
  if (total > 0x7fffffffL) return PBGDN_ERR_UNSUPPORTED;
  pbgdn::ChunkParams p{q, k, v, g, beta, beta_dtype, h0, ht, cu_seqlens, o, T, Hk, Hv, V, num_seqs, scale};
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (K) {
    case 64: return pbgdn::dispatch_in<64>(p, in_dtype, out_dtype, s);
    case 128: return pbgdn::dispatch_in<128>(p, in_dtype, out_dtype, s);
    default: return PBGDN_ERR_UNSUPPORTED;
  }
}
