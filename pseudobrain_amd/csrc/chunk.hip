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
// V/16 x Hv x N, 1024 threads (16 waves, 4 per SIMD), one workgroup per CU
// (~156 KB LDS).
// The fp32 state tile S [K, 16] lives in MFMA accumulators for the whole
// sequence (wave 8 + j owns key rows 16j..16j+15) and is written out once.
//
// Pipeline. Each loop iteration ("tick" n) has three barrier-separated phases
// and overlaps three chunks:
//   phase 1: chain   K S, X = V - gamma K S              (chunk n, waves 0-3)
//            output  Q S                                 (chunk n, waves 4-7)
//            inverse off-diagonal 16x16 blocks of T, Tb  (chunk n, waves 8-10)
//            inputs  chunk n+1 registers -> LDS, cumsum of g;
//                    buffer loads of chunk n+2 issued into registers
//   phase 2: chain   U = Tb X                            (chunk n, waves 0-3)
//            prep    K K^T -> A, Q K^T -> QKD            (chunk n+1, waves 4-13)
//   phase 3: chain   S <- gamma_C S + K^T (dec U)        (chunk n, waves 8-15)
//            output  O = gamma scale Q S + QKD U, store  (chunk n, waves 4-7)
//            inverse diagonal 16x16 blocks of T          (chunk n+1, waves 0-3)
// so the S-dependent chain of one chunk runs beside the S-independent work of
// the next. Barriers wait for LDS traffic only, so the prefetch of chunk n+2
// stays in flight for a whole tick.
//
// Costs that shape the code (measured on MI355X, CU cycles per wave64
// instruction): VALU 4 per SIMD; 16x16x32 MFMA ~14 per SIMD; LDS 16-byte
// fragment reads 4 and transposing reads 4 (conflict-free layouts), 8-byte
// tile writes 6.7, but 4-byte reads ~17. Hence:
//   * global traffic uses buffer instructions: per-lane byte offsets are fixed
//     for the whole sequence and each chunk only moves a scalar base, whose
//     range check also zero-fills tokens past the end;
//   * LDS rows are an odd multiple of 32 bytes long and the 16-byte chunk
//     index within a row is XORed with bit 2 of the row index: conflict-free
//     for 16-byte fragment reads and 8-byte accumulator-tile writes alike, and
//     the swizzle folds into each lane's base address (no per-access VALU);
//   * no 4-byte LDS accesses in the loop: per-row scalars (cumulative decay,
//     beta) are also kept in a [16][4] layout read as one float4 per lane, V
//     is staged row-major and read column-wise with ds_read_b64_tr_b16, and
//     so are the K^T and D_s operands;
//   * A, QKD and the off-diagonal Tb blocks are computed transposed so that
//     each lane writes 4 consecutive elements of a row at once;
//   * role parameters (tile indices, buffers) are wave-uniform runtime values,
//     so the loop body stays small for the instruction cache.
//
// Arithmetic (fp32 accumulation throughout):
//   * q/k products use the input's own 16-bit type on v_mfma_f32_16x16x32:
//     bf16 inputs are fed to the bf16 MFMA unconverted; fp16 inputs as fp16;
//     fp32 inputs are rounded to fp16 once when staged (V likewise).
//   * S enters K S as a high + low pair of that type (two MFMAs), so X sees
//     the fp32 state to ~16 bits; Q S, which only reaches the output, uses the
//     high part. The state update K^T (dec U) uses dec U as a pair.
//   * Tb, X, U, QKD and the off-diagonal A blocks are fp16 (11-bit
//     significand) on the fp16 MFMA.
//   * The diagonal 16x16 blocks of T come from the nilpotent product
//     (I + M)(I + M^2)(I + M^4)(I + M^8) on fp16 high/low MFMAs (~22-bit
//     products) from fp32 A; the off-diagonal blocks from 16x16x16 fp16 MFMAs.
//
// Fragment layouts (lane l, g = l >> 4, c = l & 15). 16x16x32: A holds
// A[m = c][k = 8g + j], B holds B[k = 8g + j][n = c], j = 0..7; 16x16x16:
// k = 4g + j, j = 0..3; the accumulator holds D[4g + i][c], i = 0..3. Any
// consistent assignment of contraction slots works, as long as A and B agree.
// Written tile(X) for the accumulator layout of a 16x16 X: tile(X) is the B
// operand of X and the A operand of X^T, so MFMA(tile(P^T), tile(Q)) = tile(PQ)
// and MFMA(tile(Q), tile(P^T)) = tile((PQ)^T).
#include "common.hpp"

namespace pbgdn {

typedef __bf16 bf16_t;
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));

constexpr int CH = 64;        // chunk length (CHUNK, gated_deltanet.py:49)
constexpr int VT = 16;        // value columns per workgroup
constexpr int NT = 1024;      // threads per workgroup
constexpr int NW = NT / 64;   // waves per workgroup
constexpr int SCAN_WAVE = 11; // wave that loads g, beta and scans them
constexpr int S_WAVE0 = 8;    // waves S_WAVE0 + j own key tile j of the state
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
  __device__ static float4_t bits_to_float(i16x4_t x) { return to_float4(__builtin_bit_cast(half4_t, x)); }
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
  __device__ static float4_t bits_to_float(i16x4_t x) { return to(__builtin_bit_cast(bf16x4_t, x)); }
};

__device__ __forceinline__ float4_t mma(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float4_t mma(bf16x8_t a, bf16x8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
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

// LDS layout (byte offsets). Rows of [.][K] 16-bit are KPB bytes, rows of
// [.][64] 16-bit SPB bytes and rows of [.][64] fp32 FPB bytes; arrays marked
// (swz) store the 16-byte chunk j of row r at chunk j ^ ((r >> 2) & 1).
template <int K>
struct Layout {
  static constexpr int KPB = 2 * K + 32;
  static constexpr int SPB = 2 * CH + 32;
  static constexpr int FPB = 4 * CH + 32;
  static constexpr int KQ_MAT = CH * KPB;
  static constexpr int KQ = 0;                        // [2 buf][K, Q][64 t][K] operand type (swz)
  static constexpr int V16 = KQ + 4 * KQ_MAT;         // [2 buf][64 t][16] 16-bit, 32-byte rows
  static constexpr int V16_BUF = CH * 32;
  static constexpr int SC = V16 + 2 * V16_BUF;        // [2 buf][11][64] fp32 per-token scalars (below)
  static constexpr int SC_BUF = 11 * CH * 4;
  static constexpr int AT = SC + 2 * SC_BUF;          // [64 t][64 s] fp32 A (diagonal tiles used)
  static constexpr int TB = AT + CH * FPB;            // [64 t][64 s] fp16 Tb (swz)
  static constexpr int QKD = TB + CH * SPB;           // [2 buf][64 t][64 s] fp16 (swz)
  static constexpr int A16 = QKD + 2 * CH * SPB;      // [64 t][64 s] fp16: off-diagonal A, diagonal D (swz)
  static constexpr int XT = A16 + CH * SPB;           // [16 col][64 t] fp16 X^T (swz)
  static constexpr int UT = XT + VT * SPB;            // U^T fp16 (swz)
  static constexpr int UH = UT + VT * SPB;            // (dec U)^T high, operand type (swz)
  static constexpr int UL = UH + VT * SPB;            // (dec U)^T low (swz)
  static constexpr int SH = UL + VT * SPB;            // [16 col][K] S^T high, operand type (swz)
  static constexpr int SL = SH + VT * KPB;            // S^T low (swz)
  static constexpr int BYTES = SL + VT * KPB;
  // scalar arrays within a buffer's SC block
  // Per-token scalars of a chunk (fp32 [64] each): c (inclusive cumsum of g),
  // gamma = exp(c), dec = exp(c_63 - c), beta; [16][4] tables (entry (i, r) is
  // token 16 r + i): c, beta, beta u, scale u with u_t = exp(c_t - c_16(t/16));
  // and W_R[s] = exp(c_16R - c_s) for s < 16 R (R = 1, 2, 3), else 0.
  static constexpr int CUM = 0, GAM = 256, DEC = 512, BET = 768, CUM4 = 1024, BET4 = 1280, BU4 = 1536,
                       SU4 = 1792, W1 = 2048;
};

// One chunk of raw inputs held in registers between its buffer load (issued a
// tick ahead) and its store into LDS. Per-lane byte offsets are fixed for the
// whole sequence; a chunk only sets the scalar base and range of each buffer
// resource, and tokens at or past the end of the sequence load as zeros
// (k = v = g = beta = 0: the identity steps of the reference's padding,
// gated_deltanet.py:127).
template <int K, typename TIn>
struct ChunkInputs {
  using L = Layout<K>;
  static constexpr int EPU = 16 / sizeof(TIn);       // elements per 16-byte unit
  static constexpr int ROW_UNITS = K / EPU;
  static constexpr int MAT_UNITS = CH * ROW_UNITS;   // units of one of K, Q
  static constexpr int UPT = 2 * MAT_UNITS / NT;     // K then Q units per thread
  static constexpr int V_UNITS = CH * VT / EPU;
  static_assert(UPT >= 1 && (2 * MAT_UNITS) % NT == 0 && MAT_UNITS % 64 == 0, "K/Q units must tile the workgroup");
  static_assert(V_UNITS <= NT, "V units exceed the workgroup");

  uint32_t qk_off[UPT];  // global byte offset of this thread's units within a chunk
  uint32_t qk_lds[UPT];  // LDS byte offset of the same units within a K or Q matrix
  uint32_t v_off, v_lds, g_off, b_off;
  uint4 x[UPT], vx;
  float g, b;

  // Unit i of this thread belongs to Q (1) or K (0); uniform across a wave.
  __device__ static int mat_of(int tid, int i) { return (tid + NT * i) / MAT_UNITS; }

  __device__ void init(const ChunkParams &p, int tid, int lane) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = (tid + NT * i) % MAT_UNITS;
      const int t = u / ROW_UNITS;
      const int byte = (u % ROW_UNITS) * EPU * 2;  // staged as 16-bit elements
      qk_off[i] = (t * p.Hk * K + (u % ROW_UNITS) * EPU) * sizeof(TIn);
      qk_lds[i] = t * L::KPB + (byte ^ (((t >> 2) & 1) << 4));
    }
    const int tv = tid / (VT / EPU);
    const int c0 = (tid % (VT / EPU)) * EPU;
    v_off = (tv * p.Hv * p.V + c0) * sizeof(TIn);
    v_lds = tv * 32 + c0 * 2;
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
    for (int i = 0; i < UPT; ++i) {
      x[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(mat_of(tid, i) ? rq : rk, qk_off[i], 0, 0));
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
  // wave) the cumulative decays and beta of the chunk, also as [16][4] tables
  // (entry (c, r) = value of row 16 r + c).
  __device__ void store(unsigned char *lds, int buf, int tid, int lane, bool scan, float scale) const {
#pragma unroll
    for (int i = 0; i < UPT; ++i) put_unit(lds + L::KQ + (2 * buf + mat_of(tid, i)) * L::KQ_MAT + qk_lds[i], x[i]);
    if (tid < V_UNITS) put_unit(lds + L::V16 + buf * L::V16_BUF + v_lds, vx);
    if (scan) {
      float x = g;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
      }
      const float last = __shfl(x, 63, 64);
      float *sc = reinterpret_cast<float *>(lds + L::SC + buf * L::SC_BUF);
      const int t4 = (lane & 15) * 4 + (lane >> 4);
      const float u = __expf(x - __shfl(x, lane & ~15, 64));
      sc[L::CUM / 4 + lane] = x;
      sc[L::GAM / 4 + lane] = __expf(x);
      sc[L::DEC / 4 + lane] = __expf(last - x);
      sc[L::BET / 4 + lane] = b;
      sc[L::CUM4 / 4 + t4] = x;
      sc[L::BET4 / 4 + t4] = b;
      sc[L::BU4 / 4 + t4] = b * u;
      sc[L::SU4 / 4 + t4] = scale * u;
#pragma unroll
      for (int r = 1; r < 4; ++r) {
        const float cr = __shfl(x, 16 * r, 64);
        sc[L::W1 / 4 + (r - 1) * CH + lane] = (lane < 16 * r) ? __expf(cr - x) : 0.f;
      }
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

__device__ __forceinline__ float pick(float4_t v, int i) {
  return (i == 0) ? v[0] : (i == 1) ? v[1] : (i == 2) ? v[2] : v[3];
}

template <int K, typename TIn, typename TOut>
struct ChunkBlock {
  using L = Layout<K>;
  using Op = OpOf<TIn>;
  using O4 = typename Op::T4;
  using O8 = typename Op::T8;
  static constexpr int NKT = K / 16;  // key tiles of S, one per wave
  static constexpr int KS = K / 32;   // contraction steps over keys
  static_assert(K == 64 || K == 128, "K must be 64 or 128");
  static_assert(NKT <= NW, "one S key tile per wave");

  unsigned char *lds;
  const ChunkParams &p;
  int tid, lane, c16, g4, wave, seq, h, hk, v0;
  long bos, eos, nchunks;
  uint32_t o_off;  // byte offset of this lane's first output element in a chunk
  float4_t sacc, qs;
  ChunkInputs<K, TIn> in;
  // Per-lane LDS byte offsets (see tick()).
  uint32_t kp_frag, sp_frag, kp_tile, sp_tile, at_lane, tr_v, tr_a, tr_k0, tr_k1;

  __device__ ChunkBlock(unsigned char *l, const ChunkParams &prm) : lds(l), p(prm) {
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
    lane_offsets();
  }

  // Per-lane parts of LDS addresses; everything else is a wave-uniform or
  // immediate offset. s4 is the swizzle of rows 16 m + c (bit 2 of the row).
  __device__ void lane_offsets() {
    const uint32_t s4 = ((c16 >> 2) & 1) << 4;
    kp_frag = c16 * L::KPB + ((16 * g4) ^ s4);                         // row c, 16 bytes at 16 g
    sp_frag = c16 * L::SPB + ((16 * g4) ^ s4);
    kp_tile = c16 * L::KPB + ((16 * (g4 >> 1)) ^ s4) + 8 * (g4 & 1);  // row c, 8 bytes at 8 g
    sp_tile = c16 * L::SPB + ((16 * (g4 >> 1)) ^ s4) + 8 * (g4 & 1);
    at_lane = c16 * L::FPB + 16 * g4;
    // transposing reads: lanes 4k..4k+3 of group g point at row 4g + k (V, A16)
    // or 8g + k (K), 8 bytes at 8 (c & 3)
    tr_v = (4 * g4 + (c16 >> 2)) * 32 + 8 * (c16 & 3);
    tr_a = (4 * g4 + (c16 >> 2)) * L::SPB + ((8 * (c16 & 3)) ^ ((g4 & 1) << 4));
    tr_k0 = (8 * g4 + (c16 >> 2)) * L::KPB + 8 * (c16 & 3);
    tr_k1 = (8 * g4 + 4 + (c16 >> 2)) * L::KPB + ((8 * (c16 & 3)) ^ 16);
  }

  template <typename T>
  __device__ T ld(uint32_t off) const { return *reinterpret_cast<const T *>(lds + off); }
  template <typename T>
  __device__ void st(uint32_t off, T x) const { *reinterpret_cast<T *>(lds + off) = x; }
  __device__ i16x4_t ld_tr(uint32_t off) const {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t *)(lds + off));
  }
  __device__ uint32_t sc(int buf, int arr) const { return L::SC + buf * L::SC_BUF + arr; }

  __device__ void load_chunk(long n) {
    const long t0 = bos + n * CH;
    in.load(p, t0, eos - t0, hk, h, v0, tid, wave == SCAN_WAVE);
  }

  // ---------------------------------------------------------------- phase 1
  // Waves 0-3: chain X = V - gamma K S for token rows 16w.. (S as a high/low
  // pair); waves 4-7: Q S (high part) for token rows 16(w-4)..; waves 8-10:
  // the off-diagonal blocks of T.
  __device__ void phase1(long n, int b) {
    if (wave >= 8) {
      in.store(lds, b ^ 1, tid, lane, wave == SCAN_WAVE, p.scale);
      load_chunk(n + 2);
      if (wave <= 10) offdiag(b, wave - 8);
      return;
    }
    const int r = wave & 3;
    const bool chain = wave < 4;
    const uint32_t mat = L::KQ + (2 * b + (chain ? 0 : 1)) * L::KQ_MAT + 16 * r * L::KPB + kp_frag;
    O8 a[KS], shi[KS], slo[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      a[kk] = ld<O8>(mat + 64 * kk);
      shi[kk] = ld<O8>(L::SH + kp_frag + 64 * kk);
    }
    float4_t vv, gg;
    if (chain) {
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) slo[kk] = ld<O8>(L::SL + kp_frag + 64 * kk);
      vv = Op::bits_to_float(ld_tr(L::V16 + b * L::V16_BUF + 16 * r * 32 + tr_v));
      gg = ld<float4_t>(sc(b, L::GAM) + (16 * r + 4 * g4) * 4);
    }
    in.store(lds, b ^ 1, tid, lane, wave == SCAN_WAVE, p.scale);
    load_chunk(n + 2);
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) acc = mma(a[kk], shi[kk], acc);
    if (chain) {
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) acc = mma(a[kk], slo[kk], acc);
      st(L::XT + sp_tile + 32 * r, to_half4(vv - gg * acc));
    } else {
      qs = acc;
    }
  }

  // Off-diagonal blocks of T for the chunk in buffer b:
  //   T_rs = -D_r Y_rs,  Y_rs = sum_{s<=j<r} A_rj T_js,  T_ss = D_s,
  // with A_rj and D_r from A16 (fp16). Blocks needed by later products are
  // formed as tiles (tile(D_r Y) = MFMA(A op D_r, tile(Y))); every block is
  // also formed transposed (MFMA(tile(Y), A op D_r) = tile((D_r Y)^T)) and
  // written as Tb rows T_rs diag(beta). The three independent dependency
  // chains run on three waves: T10 -> T20 -> T30; T21 -> T31; T32.
  __device__ void offdiag(int b, int chain) {
    const float4_t z = {0.f, 0.f, 0.f, 0.f};
    auto aop = [&](int r, int s) { return ld<half4_t>(L::A16 + 16 * r * L::SPB + 32 * s + sp_tile); };
    auto dop = [&](int s) {  // tile(D_s) via a transposing read
      return __builtin_bit_cast(half4_t, ld_tr(L::A16 + 16 * s * L::SPB + 32 * s + tr_a));
    };
    auto put = [&](int r, int s, float4_t mt) {  // mt = tile((D_r Y_rs)^T) = -tile(T_rs^T)
      const float4_t bs = ld<float4_t>(sc(b, L::BET) + (16 * s + 4 * g4) * 4);
      st(L::TB + 16 * r * L::SPB + 32 * s + sp_tile, to_half4(-mt * bs));
    };
    if (chain == 0) {
      const half4_t a10 = aop(1, 0), a20 = aop(2, 0), a21 = aop(2, 1);
      const half4_t a30 = aop(3, 0), a31 = aop(3, 1), a32 = aop(3, 2);
      const half4_t d1 = aop(1, 1), d2 = aop(2, 2), d3 = aop(3, 3), d0 = dop(0);
      const half4_t y10 = to_half4(mfma16(a10, d0, z));
      const half4_t t10 = to_half4(-mfma16(d1, y10, z));
      put(1, 0, mfma16(y10, d1, z));
      const half4_t y20 = to_half4(mfma16(a21, t10, mfma16(a20, d0, z)));
      const half4_t t20 = to_half4(-mfma16(d2, y20, z));
      put(2, 0, mfma16(y20, d2, z));
      const half4_t y30 = to_half4(mfma16(a32, t20, mfma16(a31, t10, mfma16(a30, d0, z))));
      put(3, 0, mfma16(y30, d3, z));
    } else if (chain == 1) {
      const half4_t a21 = aop(2, 1), a31 = aop(3, 1), a32 = aop(3, 2);
      const half4_t d2 = aop(2, 2), d3 = aop(3, 3), d1 = dop(1);
      const half4_t y21 = to_half4(mfma16(a21, d1, z));
      const half4_t t21 = to_half4(-mfma16(d2, y21, z));
      put(2, 1, mfma16(y21, d2, z));
      const half4_t y31 = to_half4(mfma16(a32, t21, mfma16(a31, d1, z)));
      put(3, 1, mfma16(y31, d3, z));
    } else {
      const half4_t a32 = aop(3, 2), d3 = aop(3, 3), d2 = dop(2);
      put(3, 2, mfma16(to_half4(mfma16(a32, d2, z)), d3, z));
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
        ta[ks] = ld<half8_t>(L::TB + 16 * wave * L::SPB + sp_frag + 64 * ks);
        xb[ks] = ld<half8_t>(L::XT + sp_frag + 64 * ks);
      }
      const float4_t dd = ld<float4_t>(sc(b, L::DEC) + (16 * wave + 4 * g4) * 4);
      float4_t u = mfma32(ta[0], xb[0], float4_t{0.f, 0.f, 0.f, 0.f});
      u = mfma32(ta[1], xb[1], u);
      const uint32_t o = sp_tile + 32 * wave;
      st(L::UT + o, to_half4(u));
      const float4_t du = u * dd;
      const O4 hi = Op::from(du);
      st(L::UH + o, hi);
      st(L::UL + o, Op::from(du - Op::to(hi)));
    }
    products(nb);
  }

  // The 10 lower 16x16 tile pairs (R, S) of A and QKD for the chunk in buffer
  // nb, one per wave 4..13: (3,0) (3,1) (3,2) (3,3) (2,0) (2,1) (2,2) (1,0)
  // (1,1) (0,0).
  __device__ void products(int nb) {
    const int i = wave - 4;
    if (i >= 0 && i < 10) {
      const int R = (i < 4) ? 3 : (i < 7) ? 2 : (i < 9) ? 1 : 0;
      const int S = i - ((i < 4) ? 0 : (i < 7) ? 4 : (i < 9) ? 7 : 9);
      tile_pair(nb, R, S);
    }
  }

  // Tile (R, S), S <= R, of A = strict_lower(b_t K K^T o D) and of
  // QKD = scale (Q K^T o D) (inclusive) for the chunk in buffer nb. The
  // products are formed transposed (rows s from K_S, columns t from K_R and
  // Q_R), so lane (g, c) holds row t = 16R + c, columns s = 16S + 4g..4g+3 and
  // writes them at once. Off the diagonal, s < 16R <= t and the decay factors
  // as exp(c_t - c_s) = u_t W_R[s] with u_t = exp(c_t - c_16R) and
  // W_R[s] = exp(c_16R - c_s), both <= 1 (no overflow; an underflow only
  // drops a product that is itself below the fp32 range), taken from the
  // chunk's tables: two multiplies per element. Diagonal tiles use
  // exp(c_t - c_s) directly with the triangular masks and go to AT (fp32, for
  // the inverse); off-diagonal A tiles go to A16.
  __device__ void tile_pair(int nb, int R, int S) {
    const uint32_t kmat = L::KQ + 2 * nb * L::KQ_MAT + kp_frag;
    const uint32_t qmat = kmat + L::KQ_MAT;
    const bool diag_tile = R == S;
    O8 kr[KS], qr[KS], ks[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      kr[kk] = ld<O8>(kmat + 16 * R * L::KPB + 64 * kk);
      qr[kk] = ld<O8>(qmat + 16 * R * L::KPB + 64 * kk);
    }
    if (diag_tile) {
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) ks[kk] = kr[kk];
    } else {
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) ks[kk] = ld<O8>(kmat + 16 * S * L::KPB + 64 * kk);
    }
    const int s0 = 16 * S + 4 * g4;
    float4_t acck = {0.f, 0.f, 0.f, 0.f}, accq = acck;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      acck = mma(ks[kk], kr[kk], acck);
      accq = mma(ks[kk], qr[kk], accq);
    }
    const uint32_t qkd_out = L::QKD + nb * CH * L::SPB + 16 * R * L::SPB + 32 * S + sp_tile;
    if (diag_tile) {
      const int t = 16 * R + c16;
      const float ct = pick(ld<float4_t>(sc(nb, L::CUM4) + c16 * 16), R);
      const float bt = pick(ld<float4_t>(sc(nb, L::BET4) + c16 * 16), R);
      const float4_t cs = ld<float4_t>(sc(nb, L::CUM) + s0 * 4);
      float4_t av, qv;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float d = __expf(ct - cs[i]);
        av[i] = (s0 + i < t) ? bt * acck[i] * d : 0.f;
        qv[i] = (s0 + i <= t) ? p.scale * accq[i] * d : 0.f;
      }
      st(L::AT + 16 * R * (L::FPB + 4) + at_lane, av);
      st(qkd_out, to_half4(qv));
    } else {
      const float bu = pick(ld<float4_t>(sc(nb, L::BU4) + c16 * 16), R);
      const float su = pick(ld<float4_t>(sc(nb, L::SU4) + c16 * 16), R);
      const float4_t w = ld<float4_t>(sc(nb, L::W1) + ((R - 1) * CH + s0) * 4);
      st(L::A16 + 16 * R * L::SPB + 32 * S + sp_tile, to_half4(acck * bu * w));
      st(qkd_out, to_half4(accq * su * w));
    }
  }

  // ---------------------------------------------------------------- phase 3
  // Waves owning S: S <- gamma_C S + K^T (dec U); waves 4-7: O = gamma scale
  // Q S + QKD U for token rows 16(w-4).., stored; waves 0-3: diagonal blocks
  // of T for chunk n+1.
  __device__ void phase3(long n, int b) {
    if (wave >= S_WAVE0 && wave < S_WAVE0 + NKT) {
      const int kt = wave - S_WAVE0;
      // K^T fragment of key tile w, token step ts: contraction slot j of lane
      // group g is token 32 ts + 8 g + j, the slot order of uh / ul.
      const uint32_t kmat = L::KQ + 2 * b * L::KQ_MAT + 32 * kt;
      O8 ka[2], hb[2], lb[2];
#pragma unroll
      for (int ts = 0; ts < 2; ++ts) {
        const i16x4_t lo4 = ld_tr(kmat + 32 * ts * L::KPB + tr_k0);
        const i16x4_t hi4 = ld_tr(kmat + 32 * ts * L::KPB + tr_k1);
        ka[ts] = __builtin_bit_cast(O8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
        hb[ts] = ld<O8>(L::UH + sp_frag + 64 * ts);
        lb[ts] = ld<O8>(L::UL + sp_frag + 64 * ts);
      }
      sacc *= ld<float4_t>(sc(b, L::GAM) + (CH - 4) * 4)[3];
#pragma unroll
      for (int ts = 0; ts < 2; ++ts) {
        sacc = mma(ka[ts], hb[ts], sacc);
        sacc = mma(ka[ts], lb[ts], sacc);
      }
      const O4 hi = Op::from(sacc);
      st(L::SH + kp_tile + 32 * kt, hi);
      st(L::SL + kp_tile + 32 * kt, Op::from(sacc - Op::to(hi)));
    }
    if (wave >= 4 && wave < 8) {
      const int r = wave - 4;
      half8_t qa[2], ub[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        qa[ks] = ld<half8_t>(L::QKD + b * CH * L::SPB + 16 * r * L::SPB + sp_frag + 64 * ks);
        ub[ks] = ld<half8_t>(L::UT + sp_frag + 64 * ks);
      }
      float4_t o = qs * ld<float4_t>(sc(b, L::GAM) + (16 * r + 4 * g4) * 4) * p.scale;
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
    } else if (wave < 4) {
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
  // Keeping P_k = M^k both as tile(P_k) and tile(P_k^T) gives every operand
  // in registers; tile(M) comes from tile(M^T) as MFMA(tile(M^T), tile(I)).
  // Y = D is built transposed: Y^T <- Y^T + P_k^T Y^T. D goes to A16 (fp16)
  // for the off-diagonal blocks, D diag(beta) to the diagonal block of Tb.
  __device__ void diag(int nb) {
    const int w = wave;
    const float4_t z = {0.f, 0.f, 0.f, 0.f};
    const float4_t p1t = -ld<float4_t>(L::AT + 16 * w * (L::FPB + 4) + at_lane);  // tile(M^T)
    const float4_t bw = ld<float4_t>(sc(nb, L::BET) + (16 * w + 4 * g4) * 4);
    half4_t eye;
#pragma unroll
    for (int j = 0; j < 4; ++j) eye[j] = static_cast<half_t>((4 * g4 + j == c16) ? 1.f : 0.f);
    float4_t yt = p1t;  // tile((I + M)^T)
#pragma unroll
    for (int i = 0; i < 4; ++i) yt[i] += (4 * g4 + i == c16) ? 1.f : 0.f;
    const Pair16 s1t = split16(p1t);
    Pair16 s1;  // tile(M), exactly, from the pair of tile(M^T)
    s1.h = to_half4(mfma16(s1t.h, eye, z));
    s1.l = to_half4(mfma16(s1t.l, eye, z));
    const Pair16 s2 = split16(mul3(s1t, s1, z)), s2t = split16(mul3(s1, s1t, z));  // M^2, (M^2)^T
    yt = mul3(s2, split16(yt), yt);
    const Pair16 s4 = split16(mul3(s2t, s2, z)), s4t = split16(mul3(s2, s2t, z));  // M^4, (M^4)^T
    yt = mul3(s4, split16(yt), yt);
    const Pair16 s8 = split16(mul3(s4t, s4, z));                                    // M^8
    yt = mul3(s8, split16(yt), yt);
    // yt = tile(D^T): lane (g, c) holds D[c][4g + i], row c of D at columns 4g..
    const uint32_t o = 16 * w * L::SPB + 32 * w + sp_tile;
    st(L::A16 + o, to_half4(yt));
    st(L::TB + o, to_half4(yt * bw));
  }

  __device__ void tick(long n) {
    // Re-define the lane offsets opaquely each tick: addresses derived from
    // them are then formed where they are used instead of being hoisted out
    // of the loop, where they would hold ~100 registers.
    asm volatile("" : "+v"(kp_frag), "+v"(sp_frag), "+v"(kp_tile), "+v"(sp_tile), "+v"(at_lane));
    asm volatile("" : "+v"(tr_v), "+v"(tr_a), "+v"(tr_k0), "+v"(tr_k1), "+v"(c16), "+v"(g4));
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
    for (int i = tid; i < CH * L::SPB / 4; i += NT) {
      reinterpret_cast<uint32_t *>(lds + L::TB)[i] = 0u;
      reinterpret_cast<uint32_t *>(lds + L::QKD)[i] = 0u;
      reinterpret_cast<uint32_t *>(lds + L::QKD + CH * L::SPB)[i] = 0u;
    }
    // Initial state: wave S_WAVE0 + j owns key rows 16j..16j+15.
    const long state_base = (static_cast<long>(seq) * p.Hv + h) * K * p.V + v0 + c16;
    const int kt = wave - S_WAVE0;
    const bool owner = kt >= 0 && kt < NKT;
    if (owner) {
      if (p.h0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sacc[i] = p.h0[state_base + static_cast<long>(16 * kt + 4 * g4 + i) * p.V];
      }
      const O4 hi = Op::from(sacc);
      st(L::SH + kp_tile + 32 * kt, hi);
      st(L::SL + kp_tile + 32 * kt, Op::from(sacc - Op::to(hi)));
    }
    load_chunk(0);
    block_sync();
    // Prologue: chunk 0 into buffer 0 and through the S-independent prep.
    in.store(lds, 0, tid, lane, wave == SCAN_WAVE, p.scale);
    load_chunk(1);
    block_sync();
    products(0);
    block_sync();
    if (wave < 4) diag(0);
    block_sync();
    for (long n = 0; n < nchunks; ++n) tick(n);
    if (p.ht && owner) {
#pragma unroll
      for (int i = 0; i < 4; ++i) p.ht[state_base + static_cast<long>(16 * kt + 4 * g4 + i) * p.V] = sacc[i];
    }
  }
};

template <int K, typename TIn, typename TOut>
__global__ __launch_bounds__(NT) void chunk_kernel(ChunkParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  ChunkBlock<K, TIn, TOut> blk(smem_raw, p);
  blk.run();
}

template <int K, typename TIn, typename TOut>
static int launch_chunk(const ChunkParams &p, hipStream_t stream) {
  static bool configured = false;  // benign race: the attribute call is idempotent
  const size_t smem = Layout<K>::BYTES;
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
