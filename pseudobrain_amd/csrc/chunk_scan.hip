// Scan kernel of the chunkwise prefill: the state-dependent part, chunk by
// chunk (the serial loop of delta_rule_chunked, pseudobrain/gated_deltanet.py:158-165).
//
// The recurrence is separable along the value columns, so a workgroup owns
// one (value head, 16-column tile of V) of a group of sequences: grid = V/16
// x Hv x G. It runs the chunks of the group's sequences back to back as one
// stream (the pipeline below does not drain between sequences, so many short
// sequences cost what one long one of the same total does); at the end of a
// sequence's last chunk the owners write its final state and load the next
// one's initial state. The fp32 state tile S [K, 16] lives in MFMA
// accumulators (compute wave j owns key rows 16j..16j+15) and is read and
// written once per sequence.
// Everything that does not involve S (Tb, QKD, the decay vectors) comes from
// the prep kernel's workspace records.
//
// 12 waves (3 per SIMD): compute waves 0-7 and loader waves 8-11. Per chunk n
// ("tick"), three barrier-separated phases:
//   phase 1: X = V - diag(gamma) K S   (compute 0-3, token rows 16w..)
//            Q S                        (compute 4-7)
//   phase 2: U = Tb X; U^T, (dec U)^T high/low -> LDS   (compute 0-3)
//            O = scale gamma Q S + QKD U of chunk n-1 -> LDS tile (compute 4-7)
//   phase 3: S <- gamma_63 S + K^T (dec U)              (owner of each key tile)
//   loaders: chunk n+1 registers -> LDS and loads of chunk n+3 issued, over
//            the three phases; O of chunk n-1, LDS -> HBM, in phase 3.
// Compute waves read the LDS operands of a phase during the phase before it.
// A chunk's inputs are its K, Q and V tile and its workspace record (Tb and
// QKD fragments, decay vectors), all staged into one LDS buffer of a double
// buffer, loaded two ticks ahead into one of two register sets of the loader
// waves (the loop is unrolled by two so that the sets have fixed registers).
// The compute waves issue no global memory operations in the loop, so the
// state chain never stalls on the memory pipeline. Barriers wait for LDS
// traffic only, so loads stay in flight across them. The two roles run
// separate loops with the same barrier sequence (a workgroup barrier does not
// need its waves at the same instruction), so the registers of one role are
// not held by the other.
//
// Loader threads all issue the same memory operations each tick (units past
// the end use out-of-range offsets or zero-size resources): the compiler
// counts outstanding operations per wave statically, and with identical
// counts on every path the wait before a use lets every newer operation stay
// in flight.
//
// Arithmetic (fp32 accumulation throughout):
//   * K, Q enter MFMA in the input's 16-bit type (bf16 unconverted; fp32
//     inputs staged as fp16); V as staged (fp32 inputs as a bf16 high + low
//     pair, fp32 range).
//   * S enters K S as a high + low pair of that type (two MFMAs), so X sees
//     the fp32 state to ~16 bits; Q S, which only reaches the output, uses the
//     high part. The state update K^T (dec U) uses dec U as a pair.
//   * Tb, X, U and QKD are fp16 (11-bit significand) on the fp16 MFMA. A
//     chunk whose X exceeds X_LIMIT somewhere is scaled by a power of two
//     (chunk.hpp) before it becomes fp16: each X wave publishes its tile's
//     scale, the U waves bring the tiles to the chunk's smallest one through
//     the lanes of their Tb fragments, and U, O are restored in fp32.
//   * float32 inputs form U = Tb X from fp16 high/low pairs of both (three
//     products: high x high, high x low, low x high): the prep kernel's records
//     carry Tb's low part (staged into one buffer, read the tick after), and
//     X's low part goes through the output tile that is idle that tick. This
//     is the product whose fp16 rounding bounded the float32 state error.
//
// LDS costs that shape the code (MI355X, CU cycles per wave64 instruction):
// 16-byte fragment reads and transposing reads 4, 8-byte tile writes 6.7 in
// the swizzled layouts; V is staged row-major and read column-wise with
// ds_read_b64_tr_b16, and so is K^T.
#include "chunk.hpp"

namespace pbgdn {
namespace {

constexpr int NCW = 8;                  // compute waves
constexpr int NLT = 256;                // loader threads (waves 8-11)
constexpr int NT = NCW * 64 + NLT;      // threads per scan workgroup

// LDS layout (byte offsets); (swz) as in chunk.hpp. Two chunk buffers, each
// [K, Q][64 t][K] in the operand type (swz), V [64 t][16] 16-bit in 32-byte
// rows, and the chunk's workspace record as stored; two O tiles [64 t][16].
template <int K, bool LO>
struct ScanLayout {
  static constexpr int KPB = 2 * K + 32;
  static constexpr int SPB = 2 * CH + 32;
  static constexpr int KQ_MAT = CH * KPB;
  static constexpr int V16_OFF = 2 * KQ_MAT;
  static constexpr int V16LO_OFF = V16_OFF + CH * 32;  // fp32 inputs: the low bf16 part of V
  static constexpr int REC_OFF = V16LO_OFF + CH * 32;
  static constexpr int BUF = REC_OFF + REC_BYTES;
  static constexpr int XT = 2 * BUF;                  // [16 col][64 t] fp16 X^T (swz)
  static constexpr int UT = XT + VT * SPB;            // [2] U^T fp16 (swz), by chunk parity
  static constexpr int UH = UT + 2 * VT * SPB;        // (dec U)^T high, operand type (swz)
  static constexpr int UL = UH + VT * SPB;            // (dec U)^T low (swz)
  static constexpr int SH = UL + VT * SPB;            // [16 col][K] S^T high, operand type (swz)
  static constexpr int SL = SH + VT * KPB;            // S^T low (swz)
  static constexpr int OT = SL + VT * KPB;            // [2][64 t][16] output type
  static constexpr int OT_BUF = CH * VT * 4;
  static constexpr int RS = OT + 2 * OT_BUF;          // fp32 range scales: [4] X tiles, [2] chunk by parity
  // LO (float32 inputs): Tb's low fragments of the next chunk, one buffer
  // (staged in the third phase, read in the first of the next tick)
  static constexpr int TBL = RS + 32;
  static constexpr int BYTES = TBL + (LO ? NFRAG * FRAG_BYTES : 0);
  // Chained streams only: the initial state of the sequence whose first
  // chunk is in chunk buffer b ([K rows][16 columns] as stored), staged by the
  // loader waves with that chunk.
  static constexpr int H0_BYTES = K * VT * 4;
  static constexpr int CHAIN_BYTES = BYTES + 2 * H0_BYTES;
  __device__ static constexpr int h0(int b) { return BYTES + b * H0_BYTES; }
  __device__ static constexpr int kq(int b) { return b * BUF; }
  __device__ static constexpr int v16(int b) { return b * BUF + V16_OFF; }
  __device__ static constexpr int v16lo(int b) { return b * BUF + V16LO_OFF; }
  __device__ static constexpr int rec(int b) { return b * BUF + REC_OFF; }
  __device__ static constexpr int ot(int b) { return OT + b * OT_BUF; }
  __device__ static constexpr int ut(int b) { return UT + b * VT * SPB; }
  // LO: X's low part [16 col][64 t] fp16 (swz, as XT) in the O tile of the
  // chunk's own parity, which holds nothing from the tick's first phase until
  // the output waves write the chunk's O a tick later
  __device__ static constexpr int xtl(int b) { return ot(b); }
  static_assert(!LO || VT * SPB <= OT_BUF, "X's low part fits an O tile");
};

// Staging of one chunk by the loader threads: 16-byte units numbered K, Q
// (rows of 64 tokens), V tile, record; loader thread l moves unit
// l + NLT i in slot i. K and Q fill whole slots, so the class of every slot
// but one is a compile-time constant; the slot where V ends and the record
// begins splits at a whole wave. Slot classes are fixed in the code so that
// the loads and stores compile without branches.
template <int K, typename TIn>
struct ScanStage {
  static constexpr bool LO = sizeof(TIn) == 4;
  using L = ScanLayout<K, LO>;
  static constexpr int EPU = 16 / sizeof(TIn);  // elements per unit
  static constexpr int ROW_UNITS = K / EPU;
  static constexpr int MAT_UNITS = CH * ROW_UNITS;
  static constexpr int KQ_UNITS = 2 * MAT_UNITS;
  static constexpr int V_UNITS = CH * VT / EPU;
  static constexpr int R_UNITS = rec_bytes<TIn>() / 16;
  static constexpr int TBL_UNIT = KQ_UNITS + V_UNITS + REC_BYTES / 16;  // LO: units from here on are Tb's low part
  static constexpr int UNITS = KQ_UNITS + V_UNITS + R_UNITS;
  static constexpr int UPT = (UNITS + NLT - 1) / NLT;
  static constexpr int SLOT_K = MAT_UNITS / NLT;   // slots [0, SLOT_K): K; [SLOT_K, SLOT_V): Q
  static constexpr int SLOT_V = KQ_UNITS / NLT;    // slot SLOT_V: V (first V_UNITS threads), then record
  // Slots are staged in three groups, one per phase: [0, SLOT_P2) in phase 1,
  // [SLOT_P2, SLOT_P3) in phase 2 (through the record's decay vectors, which
  // phase 3 reads), [SLOT_P3, UPT) in phase 3 (Tb and QKD fragments, first
  // read in the next tick).
  static constexpr int SLOT_P3 = (KQ_UNITS + V_UNITS + (REC_TB - REC_SC) / 16 - 1) / NLT + 1;
  static constexpr int SLOT_P2 = SLOT_P3 / 2 + 1;
  static_assert(REC_SC == 0 && SLOT_P2 < SLOT_P3 && SLOT_P3 <= UPT, "record vectors lead the record");
  static_assert(MAT_UNITS % NLT == 0, "K and Q must fill whole slots");
  static_assert(V_UNITS % 64 == 0 && V_UNITS <= NLT, "V must end at a wave boundary of its slot");
  static_assert(TBL_UNIT % 64 == 0, "Tb's low part starts at a wave boundary of its slot");

  struct Regs {
    uint4 u[UPT];
  };

  uint32_t src[UPT];  // byte offset of the unit in its source (OUT_OF_RANGE if none)
  uint32_t dst[UPT];  // LDS byte offset of the unit within a chunk buffer (Tb's low part: within LDS)
  uint32_t tbl;       // bit i: this wave's unit of slot i is Tb's low part (one buffer, not per chunk)
  bool v_wave;        // this loader wave's slot SLOT_V unit is V (else record); wave-uniform
  float vscale;       // fp32 inputs: V's range scale (a power of two)

  __device__ __forceinline__ void init(const ChunkParams &p, int l, float in_down) {
    v_wave = __builtin_amdgcn_readfirstlane(l & ~63) < V_UNITS;
    vscale = in_down;
    tbl = 0;
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = l + NLT * i;
      src[i] = OUT_OF_RANGE;
      dst[i] = 0;
      if (u < KQ_UNITS) {
        const int w = u % MAT_UNITS;
        const int t = w / ROW_UNITS;
        const int byte = (w % ROW_UNITS) * EPU * 2;  // staged as 16-bit elements
        src[i] = (t * p.Hk * K + (w % ROW_UNITS) * EPU) * sizeof(TIn);
        dst[i] = (u / MAT_UNITS) * L::KQ_MAT + t * L::KPB + (byte ^ (((t >> 2) & 1) << 4));
      } else if (u < KQ_UNITS + V_UNITS) {
        const int w = u - KQ_UNITS;
        const int tv = w / (VT / EPU);
        const int c0 = (w % (VT / EPU)) * EPU;
        src[i] = (tv * p.Hv * p.V + c0) * sizeof(TIn);
        dst[i] = L::V16_OFF + tv * 32 + c0 * 2;
      } else if (u < UNITS) {
        const int w = u - KQ_UNITS - V_UNITS;
        src[i] = rec_unused_unit(16 * w) ? OUT_OF_RANGE : 16 * w;  // units no scan reads are not fetched
        if (LO && u >= TBL_UNIT) {
          dst[i] = L::TBL + 16 * (u - TBL_UNIT);
          tbl |= 1u << i;
        } else {
          dst[i] = L::REC_OFF + 16 * w;
        }
      }
    }
    tbl = __builtin_amdgcn_readfirstlane(tbl);  // wave-uniform: the boundaries are whole waves
  }

  // Issue the loads of the chunk at tokens t0.. (`len` left, may be <= 0) of
  // value head h, columns v0.., and of its record `rec` (null past the end).
  __device__ __forceinline__ void load(const ChunkParams &p, Regs &r, long t0, long len, int hk, int h, int v0,
                       const unsigned char *rec) const {
    const long rows = len < CH ? len : CH;
    const long qk_bytes = rows > 0 ? ((rows - 1) * p.Hk * K + K) * static_cast<long>(sizeof(TIn)) : 0;
    const long qk_base = (t0 * p.Hk + hk) * static_cast<long>(K);
    const long v_bytes = rows > 0 ? ((rows - 1) * p.Hv * p.V + VT) * static_cast<long>(sizeof(TIn)) : 0;
    const __amdgpu_buffer_rsrc_t rk = rsrc(static_cast<const TIn *>(p.k) + qk_base, qk_bytes);
    const __amdgpu_buffer_rsrc_t rq = rsrc(static_cast<const TIn *>(p.q) + qk_base, qk_bytes);
    const __amdgpu_buffer_rsrc_t rr = rsrc(rec, rec ? rec_bytes<TIn>() : 0);
    const __amdgpu_buffer_rsrc_t rvr =
        v_wave ? rsrc(static_cast<const TIn *>(p.v) + (t0 * p.Hv + h) * static_cast<long>(p.V) + v0, v_bytes) : rr;
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      r.u[i] = buf_load16(i < SLOT_K ? rk : i < SLOT_V ? rq : i == SLOT_V ? rvr : rr, src[i]);
    }
  }

  // Slot by slot: registers -> LDS chunk buffer at byte `base` (as store()),
  // then the slot's register receives the same unit of the chunk at tokens
  // t0.. (as load()), so a load issues as soon as its register is free.
  template <int I0, int I1>
  __device__ __forceinline__ void restage(const ChunkParams &p, unsigned char *lds, int base, Regs &r, int l, long t0, long len,
                          int hk, int h, int v0, const unsigned char *rec) const {
    const long rows = len < CH ? len : CH;
    const long qk_bytes = rows > 0 ? ((rows - 1) * p.Hk * K + K) * static_cast<long>(sizeof(TIn)) : 0;
    const long qk_base = (t0 * p.Hk + hk) * static_cast<long>(K);
    const long v_bytes = rows > 0 ? ((rows - 1) * p.Hv * p.V + VT) * static_cast<long>(sizeof(TIn)) : 0;
    const __amdgpu_buffer_rsrc_t rk = rsrc(static_cast<const TIn *>(p.k) + qk_base, qk_bytes);
    const __amdgpu_buffer_rsrc_t rq = rsrc(static_cast<const TIn *>(p.q) + qk_base, qk_bytes);
    const __amdgpu_buffer_rsrc_t rr = rsrc(rec, rec ? rec_bytes<TIn>() : 0);
    const __amdgpu_buffer_rsrc_t rvr =
        v_wave ? rsrc(static_cast<const TIn *>(p.v) + (t0 * p.Hv + h) * static_cast<long>(p.V) + v0, v_bytes) : rr;
#pragma unroll
    for (int i = I0; i < I1; ++i) {
      store_unit(lds, base, r, l, i);
      r.u[i] = buf_load16(i < SLOT_K ? rk : i < SLOT_V ? rq : i == SLOT_V ? rvr : rr, src[i]);
    }
  }

  __device__ __forceinline__ void store_unit(unsigned char *lds, int base, const Regs &r, int l, int i) const {
    if (l + NLT * i >= UNITS) return;
    unsigned char *d = lds + (LO && ((tbl >> i) & 1) ? 0 : base) + dst[i];
    if (EPU == 4 && i == SLOT_V && v_wave) {  // fp32 V, range-scaled: bf16 high and low parts
      const uint4 x = r.u[i];
      bf16x4_t hi, lo;
      OpOf<u16>::split(float4_t{__uint_as_float(x.x), __uint_as_float(x.y), __uint_as_float(x.z),
                                __uint_as_float(x.w)} * vscale, hi, lo);
      *reinterpret_cast<bf16x4_t *>(d) = hi;
      *reinterpret_cast<bf16x4_t *>(d + (L::V16LO_OFF - L::V16_OFF)) = lo;
    } else if (EPU == 4 && i < SLOT_V) {
      const uint4 x = r.u[i];
      *reinterpret_cast<half4_t *>(d) = to_half4(float4_t{__uint_as_float(x.x), __uint_as_float(x.y),
                                                          __uint_as_float(x.z), __uint_as_float(x.w)});
    } else {
      *reinterpret_cast<uint4 *>(d) = r.u[i];
    }
  }

  // Registers -> LDS chunk buffer at byte `base`: K, Q, V as staged 16-bit
  // elements (fp32 rounded to fp16), the record unchanged. Units without a
  // destination (past the record) write a harmless zero-offset copy of
  // nothing: their slot is skipped by range.
  __device__ __forceinline__ void store(unsigned char *lds, int base, const Regs &r, int l) const {
#pragma unroll
    for (int i = 0; i < UPT; ++i) store_unit(lds, base, r, l, i);
  }
};

// Block index -> (sequence, value head, column tile). All column tiles of the
// value heads that share one query/key head of one sequence form a group; a
// group is kept on one XCD (xcd_group) so that its q/k chunks and Tb/QKD
// records are fetched into that XCD's L2 once.
__device__ __forceinline__ void decode_block(int L, int total, int nv, int group_heads, int Hk, int xcds, int &grp_seq,
                                             int &h, int &vtile, int &member) {
  const int gsize = nv * group_heads;
  int grp, in;
  xcd_group(L, total / gsize, gsize, xcds, grp, in);
  const int hk = grp % Hk;
  grp_seq = grp / Hk;
  h = hk * group_heads + in / nv;
  vtile = in % nv;
  member = in;
}

template <typename T>
__device__ __forceinline__ T out_elem(float x);
template <>
__device__ __forceinline__ u16 out_elem<u16>(float x) { return __builtin_bit_cast(u16, static_cast<bf16_t>(x)); }
template <>
__device__ __forceinline__ half_t out_elem<half_t>(float x) { return static_cast<half_t>(x); }
template <>
__device__ __forceinline__ float out_elem<float>(float x) { return x; }

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// CHAIN: a workgroup runs more than one sequence (the stream crosses sequence
// boundaries); without it the stream is one sequence and the cursors are
// plain counters.
template <int K, typename TIn, typename TOut, bool CHAIN>
struct ScanBlock {
  static constexpr bool LO = sizeof(TIn) == 4;  // U = Tb X from high/low pairs
  using L = ScanLayout<K, LO>;
  using Op = OpOf<TIn>;
  using O4 = typename Op::T4;
  using O8 = typename Op::T8;
  using Stage = ScanStage<K, TIn>;
  static constexpr int NKT = K / 16;  // key tiles of S, one per compute wave
  static constexpr int KS = K / 32;   // contraction steps over keys
  static constexpr int OUT_UNITS = CH * VT * sizeof(TOut) / 16;  // 16-byte units of an O tile
  static_assert(K == 64 || K == 128, "K must be 64 or 128");
  static_assert(NKT <= NCW, "one S key tile per compute wave");
  static_assert(OUT_UNITS <= NLT, "one O unit per loader thread");

  unsigned char *lds;
  const ChunkParams &p;
  int tid, lane, c16, g4, wave, h, hk, v0, lt;  // lt: loader thread index (loader waves)
  int s_begin, s_end;  // the group's sequences
  long nchunks;        // chunks of the group's sequences (the stream's length)
  // Stream positions: compute waves at the current chunk; loader waves at the
  // chunk being loaded (three ahead) and at the chunk whose O goes out (one behind).
  struct Cursor {
    int s;     // sequence (s_end past the stream's end)
    int left;    // chunks of s from this one on
    bool first;  // this chunk is s's first
    long t0, eos, rec;  // this chunk's first token, s's end, this chunk's record
  } cc, lc, oc;
  float4_t sacc;
  // fp32 inputs: v and the initial states enter scaled by in_down (a power of
  // two, so exactly), o and the final states leave scaled back; 1 otherwise
  float in_down, in_up;
  Stage stage;
  typename Stage::Regs regs[2];
  uint4 h0r[2][2];  // chained streams: loader thread's 16-byte units of a chunk's initial state, per register set
  bool h0v[2];      // the set holds a sequence's first chunk (its units go to LDS)
  uint32_t out_src, out_dst;  // loader thread's O unit: LDS offset in a tile, byte offset in a chunk
  // Per-lane LDS byte offsets (see lane_offsets()).
  uint32_t kp_frag, sp_frag, kp_tile, sp_tile, tr_v, tr_k0, tr_k1;

  // Debug builds: the barriers this wave has passed (audited at the end:
  // every wave of the workgroup must pass the same number, whatever its role).
  uint32_t nbar = 0;
  __device__ __forceinline__ void sync() {
    block_sync();
#ifdef PBGDN_DEBUG
    ++nbar;
#endif
  }

  __device__ __forceinline__ ScanBlock(unsigned char *l, const ChunkParams &prm) : lds(l), p(prm) {
    tid = threadIdx.x;
    lane = tid & 63;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    c16 = lane & 15;
    g4 = lane >> 4;
    lt = tid - NCW * 64;
    const int group_heads = p.Hv / p.Hk;
    int vtile, member, grp;
    decode_block(blockIdx.x, gridDim.x, p.V / VT, group_heads, p.Hk, p.xcds, grp, h, vtile, member);
    hk = h / group_heads;
    v0 = vtile * VT;
    s_begin = static_cast<int>(static_cast<long>(grp) * p.num_seqs / p.seq_groups);
    s_end = static_cast<int>(static_cast<long>(grp + 1) * p.num_seqs / p.seq_groups);
    sacc = float4_t{0.f, 0.f, 0.f, 0.f};
    in_down = 1.f;
    if constexpr (sizeof(TIn) == 4) {
      if (p.in_scale) in_down = *p.in_scale;  // written by the range kernels earlier on the stream
    }
    in_up = 1.f / in_down;
    if (wave >= NCW) {
      stage.init(p, lt, in_down);
      constexpr int upr = VT * sizeof(TOut) / 16;  // units per output row
      out_src = lt < OUT_UNITS ? 16 * lt : 0;
      out_dst = lt < OUT_UNITS ? ((lt / upr) * p.Hv * p.V + (lt % upr) * (16 / sizeof(TOut))) * sizeof(TOut)
                               : OUT_OF_RANGE;
    }
    lane_offsets();
  }

  // Per-lane parts of LDS addresses; everything else is a wave-uniform or
  // immediate offset. s4 is the swizzle of rows 16 m + c (bit 2 of the row).
  __device__ __forceinline__ void lane_offsets() {
    const uint32_t s4 = ((c16 >> 2) & 1) << 4;
    kp_frag = c16 * L::KPB + ((16 * g4) ^ s4);                         // row c, 16 bytes at 16 g
    sp_frag = c16 * L::SPB + ((16 * g4) ^ s4);
    kp_tile = c16 * L::KPB + ((16 * (g4 >> 1)) ^ s4) + 8 * (g4 & 1);  // row c, 8 bytes at 8 g
    sp_tile = c16 * L::SPB + ((16 * (g4 >> 1)) ^ s4) + 8 * (g4 & 1);
    // transposing reads: lanes 4k..4k+3 of group g point at row 4g + k (V)
    // or 8g + k (K), 8 bytes at 8 (c & 3)
    tr_v = (4 * g4 + (c16 >> 2)) * 32 + 8 * (c16 & 3);
    tr_k0 = (8 * g4 + (c16 >> 2)) * L::KPB + 8 * (c16 & 3);
    tr_k1 = (8 * g4 + 4 + (c16 >> 2)) * L::KPB + ((8 * (c16 & 3)) ^ 16);
  }

  template <typename T>
  __device__ __forceinline__ T ld(uint32_t off) const { return *reinterpret_cast<const T *>(lds + off); }
  template <typename T>
  __device__ __forceinline__ void st(uint32_t off, T x) const { *reinterpret_cast<T *>(lds + off) = x; }
  __device__ __forceinline__ i16x4_t ld_tr(uint32_t off) const {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t *)(lds + off));
  }

  // ------------------------------------------------------------ loader waves
  // -------------------------------------------------------- chunk stream
  // From sequence s on, the first sequence of the group with tokens (s_end if
  // none). Wave-uniform; cu_seqlens reads are scalar loads.
  __device__ __forceinline__ bool enter(Cursor &c) const {  // chunk 0 of sequence c.s, if it has tokens
    long b, e;
    seq_bounds(p, c.s, b, e);
    c.t0 = b;
    c.eos = e;
    c.rec = rec_base(b, c.s);
    c.left = static_cast<int>((e - b + CH - 1) / CH);
    c.first = true;
    return e > b;
  }
  __device__ __forceinline__ void seek(Cursor &c, int s) const {
    for (c.s = s; c.s < s_end; ++c.s) {
      if (enter(c)) return;
    }
    c.t0 = c.eos = c.rec = 0;
    c.left = 0;
    c.first = false;
  }
  __device__ __forceinline__ bool at_end(const Cursor &c) const { return c.s >= s_end; }
  __device__ __forceinline__ long len_of(const Cursor &c) const { return c.eos - c.t0; }  // 0 at the end
  // Next chunk of the stream: a few scalar adds except at a sequence's end.
  __device__ __forceinline__ void advance(Cursor &c) const {
    if constexpr (!CHAIN) {  // one sequence: past its end the loads have zero size
      c.t0 += CH;
      ++c.rec;
      return;
    }
    if (at_end(c)) return;
    if (--c.left > 0) {
      c.t0 += CH;
      ++c.rec;
      c.first = false;
    } else {
      seek(c, c.s + 1);
    }
  }
  __device__ __forceinline__ const unsigned char *rec_of(const Cursor &c) const {
    const bool none = CHAIN ? at_end(c) : c.t0 >= c.eos;
    return none ? nullptr : p.ws + (c.rec * p.Hv + h) * static_cast<long>(rec_bytes<TIn>());
  }

  // ------------------------------------------------------------ loader waves
  __device__ __forceinline__ void load_chunk(typename Stage::Regs &r, const Cursor &c) const {
    stage.load(p, r, c.t0, len_of(c), hk, h, v0, rec_of(c));
  }

  // Chained streams: the loads of this loader thread's part of the initial
  // state of the sequence whose first chunk is at cursor c (zero-size when c
  // is not a sequence's first chunk or the sequence starts from zeros), issued
  // with the chunk's own loads: 16-byte units u = lt, lt + 256 of the
  // [K][16] tile, esz = 16 / (elements per unit) units per row.
  __device__ __forceinline__ void load_h0(uint4 (&r)[2], const Cursor &c, bool first) const {
    const int esz = p.state_dtype == PBGDN_F32 ? 4 : 2;
    long bytes = 0;
    const unsigned char *base = nullptr;
    if (first && !at_end(c)) {
      const long slot = slot_of(c.s);
      if (p.h0 && in_pool(slot) && (!p.has_initial_state || p.has_initial_state[c.s])) {
        base = static_cast<const unsigned char *>(p.h0) + ((slot * p.Hv + h) * K * p.V + v0) * esz;
        bytes = (static_cast<long>(K - 1) * p.V + VT) * esz;
      }
    }
    const __amdgpu_buffer_rsrc_t rs = rsrc(base, bytes);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int u = lt + NLT * i;
      const uint32_t off = u < K * esz ? ((u / esz) * p.V + (u % esz) * (16 / esz)) * esz : OUT_OF_RANGE;
      r[i] = buf_load16(rs, off);
    }
  }
  __device__ __forceinline__ void store_h0(int buf, const uint4 (&r)[2]) const {
    const int esz = p.state_dtype == PBGDN_F32 ? 4 : 2;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int u = lt + NLT * i;
      if (u < K * esz) st(L::h0(buf) + 16 * u, r[i]);
    }
  }

  // O tile of stream chunk n (LDS buffer n & 1, at cursor oc) -> HBM, one
  // 16-byte unit per loader thread; n < 0 issues the same store with a
  // zero-size resource.
  __device__ __forceinline__ void store_out(long n) const {
    const long t0 = n >= 0 ? oc.t0 : 0;
    const long len = n >= 0 ? len_of(oc) : 0;
    const long rows = len < CH ? len : CH;
    const long bytes = rows > 0 ? ((rows - 1) * p.Hv * p.V + VT) * static_cast<long>(sizeof(TOut)) : 0;
    const __amdgpu_buffer_rsrc_t ro =
        rsrc(static_cast<TOut *>(p.o) + (t0 * p.Hv + h) * static_cast<long>(p.V) + v0, bytes);
    const uint4 x = ld<uint4>(L::ot(static_cast<int>(n & 1)) + out_src);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, x), ro, out_dst, 0, 0);
  }

  // ------------------------------------------------------------- states
  // Slot of sequence s in the state tensors (its index without state_idx);
  // a slot outside [0, num_states) starts from zeros and keeps no final state.
  __device__ __forceinline__ long slot_of(int s) const {
    return p.state_idx ? static_cast<long>(p.state_idx[s]) : static_cast<long>(s);
  }
  __device__ __forceinline__ bool in_pool(long slot) const {
    return !p.state_idx || (slot >= 0 && slot < p.num_states);
  }
  // This lane's 4 elements of key tile kt of sequence s's initial state.
  __device__ __forceinline__ float4_t initial_state(int s, int kt) const {
    float4_t x = {0.f, 0.f, 0.f, 0.f};
    const long slot = slot_of(s);
    if (p.h0 && in_pool(slot) && (!p.has_initial_state || p.has_initial_state[s])) {
      const long base = (slot * p.Hv + h) * K * p.V + v0 + c16;
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = load_elem(p.h0, base + static_cast<long>(16 * kt + 4 * g4 + i) * p.V, p.state_dtype);
    }
    return x * in_down;
  }
  __device__ __forceinline__ void final_state(int s, int kt, float4_t x) const {
    const long slot = slot_of(s);
    if (p.ht && in_pool(slot)) {
      const long base = (slot * p.Hv + h) * K * p.V + v0 + c16;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        store_elem(p.ht, base + static_cast<long>(16 * kt + 4 * g4 + i) * p.V, p.state_dtype, x[i] * in_up);
    }
  }
  // sacc -> the S^T high/low operand copies in LDS (key tile kt).
  __device__ __forceinline__ void put_state(int kt) const {
    const O4 hi = Op::from(sacc);
    st(L::SH + kp_tile + 32 * kt, hi);
    st(L::SL + kp_tile + 32 * kt, Op::from(sacc - Op::to(hi)));
  }
  // Owners, from sequence s on: pass the empty sequences' initial states to
  // their final states, and stop at the first one with tokens.
  __device__ __forceinline__ void seek_owner(Cursor &c, int s, int kt) const {
    for (c.s = s; c.s < s_end; ++c.s) {
      if (enter(c)) return;
      final_state(c.s, kt, initial_state(c.s, kt));
    }
    c.left = 0;
  }
  // Owners, phase 3 of each tick, after the state update of the cursor's
  // chunk: at a sequence's last chunk its final state goes out and the next
  // sequence's initial state (loaded first) replaces it; then the cursor
  // moves on.
  // The next sequence's initial state was staged by the loader waves with its
  // first chunk (chunk buffer nb): this lane's rows 16 kt + 4 g + i, column c.
  __device__ __forceinline__ void next_chunk(int kt, int nb) {
    if constexpr (!CHAIN) return;  // the one sequence's final state goes out after the loop
    if (--cc.left > 0) return;
    const int done = cc.s;
    const float4_t fin = sacc;
    seek_owner(cc, done + 1, kt);
    const int row0 = 16 * kt + 4 * g4;
    if (p.state_dtype == PBGDN_F32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) sacc[i] = ld<float>(L::h0(nb) + ((row0 + i) * VT + c16) * 4);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u16 x = ld<u16>(L::h0(nb) + ((row0 + i) * VT + c16) * 2);
        sacc[i] = p.state_dtype == PBGDN_BF16 ? bf16_bits_to_float(x)
                                                : static_cast<float>(__builtin_bit_cast(half_t, x));
      }
    }
    sacc *= in_down;
    final_state(done, kt, fin);
    put_state(kt);
  }

  // ------------------------------------------------------------ compute waves
  // Row float4 of a record vector (SC_GAM, SC_GSC, SC_DEC) for this lane's
  // accumulator rows 16 r + 4 g.. of the chunk in buffer b.
  // V rows 16r + 4g.. of column c of chunk buffer b (fp32 inputs: high + low parts)
  __device__ __forceinline__ float4_t v_rows(int b, int r) const {
    if constexpr (sizeof(TIn) == 4) {
      return OpOf<u16>::bits_to_float(ld_tr(L::v16(b) + 16 * r * 32 + tr_v)) +
             OpOf<u16>::bits_to_float(ld_tr(L::v16lo(b) + 16 * r * 32 + tr_v));
    } else {
      return Op::bits_to_float(ld_tr(L::v16(b) + 16 * r * 32 + tr_v));
    }
  }

  __device__ __forceinline__ float4_t rec_rows(int b, int vec, int r) const {
    return ld<float4_t>(L::rec(b) + REC_SC + vec + (16 * r + 4 * g4) * 4);
  }
  // Tb (REC_TB) or QKD (REC_QKD) fragment (r, kk) of the chunk in buffer b.
  __device__ __forceinline__ half8_t rec_frag(int b, int mat, int r, int kk) const {
    return ld<half8_t>(L::rec(b) + mat + frag_index(r, kk) * FRAG_BYTES + lane * 16);
  }
  // The second contraction step's fragment f of row tile r. Rows of tiles 0
  // and 1 vanish past column 31, so theirs is zero: every wave issues both
  // products with no branch between them and the first read of the result.
  // (With a branch around the second product, hipcc placed reads after the
  // join fewer wait states behind it than a 16x16x32 product needs, and read
  // stale result registers.)
  static __device__ __forceinline__ half8_t second_step(const half8_t &f, int r) { return r >= 2 ? f : half8_t{}; }

  // Operands are read from LDS one phase before the phase that uses them, so
  // that each phase waits only for what the previous phase produced. The two
  // compute roles run separate loops (same barrier sequence) with their own
  // registers: chain waves 0-3 (X, U for token rows 16r..) and output waves
  // 4-7 (Q S, O for rows 16r..), r = wave & 3; every wave below NKT also
  // updates its key tile of S.

  // K^T fragments of key tile kt of the chunk in buffer b: contraction slot j
  // of lane group g is token 32 ts + 8 g + j, the slot order of the dec U pair.
  __device__ __forceinline__ void fetch_kt(int b, O8 (&kt)[2]) const {
    const uint32_t kmat = L::kq(b) + 32 * wave;
#pragma unroll
    for (int ts = 0; ts < 2; ++ts) {
      const i16x4_t lo4 = ld_tr(kmat + 32 * ts * L::KPB + tr_k0);
      const i16x4_t hi4 = ld_tr(kmat + 32 * ts * L::KPB + tr_k1);
      kt[ts] = __builtin_bit_cast(O8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  }

  // A fragments of rows 16r.. of K (mat 0) or Q (mat 1) of the chunk in buffer b.
  __device__ __forceinline__ void fetch_rows(int b, int mat, O8 (&mf)[KS]) const {
    const uint32_t base = L::kq(b) + mat * L::KQ_MAT + 16 * (wave & 3) * L::KPB + kp_frag;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) mf[kk] = ld<O8>(base + 64 * kk);
  }

  // S <- gamma_63 S + K^T (dec U) for the wave's key tile (chunk in buffer b).
  __device__ __forceinline__ void update_state(int b, const O8 (&kt)[2]) {
    O8 hb[2], lb[2];
#pragma unroll
    for (int ts = 0; ts < 2; ++ts) {
      hb[ts] = ld<O8>(L::UH + sp_frag + 64 * ts);
      lb[ts] = ld<O8>(L::UL + sp_frag + 64 * ts);
    }
    float4_t acl = mma(kt[0], lb[0], float4_t{0.f, 0.f, 0.f, 0.f});
    acl = mma(kt[1], lb[1], acl);
    sacc *= ld<float>(L::rec(b) + REC_SC + SC_GAM + (CH - 1) * 4);
    sacc = mma(kt[0], hb[0], sacc);
    sacc = mma(kt[1], hb[1], sacc);
    sacc += acl;
    const O4 hi = Op::from(sacc);
    st(L::SH + kp_tile + 32 * wave, hi);
    st(L::SL + kp_tile + 32 * wave, Op::from(sacc - Op::to(hi)));
  }

  __device__ __forceinline__ void launder() {
    // Re-define the lane offsets opaquely each tick: addresses derived from
    // them are then formed where they are used instead of being hoisted out
    // of the loop, where they would hold many registers.
    asm volatile("" : "+v"(kp_frag), "+v"(sp_frag), "+v"(kp_tile), "+v"(sp_tile));
    asm volatile("" : "+v"(tr_v), "+v"(tr_k0), "+v"(tr_k1), "+v"(c16), "+v"(g4));
  }

  // Chain waves. Phase 1: X = V - gamma K S (S as a high/low pair) -> X^T;
  // Tb fragments and dec rows for phase 2. Phase 2: U = Tb X (Tb rows 16r..
  // vanish past column 16r + 15: row tiles 0, 1 need one contraction step,
  // 2, 3 two) -> U^T, (dec U)^T high/low; K^T for phase 3. Phase 3: the state
  // update, then K rows, V rows and gamma rows of the next chunk.
  template <int P>
  __device__ __forceinline__ void tick_chain(O8 (&mf)[KS], float4_t &vv, float4_t &gg) {
    launder();
    const int b = P;
    const int r = wave;
    half8_t f0, f1, fl0, fl1;  // Tb fragments (LO: and their low parts)
    float4_t dd;
    O8 kt[2];
    {
      O8 shi[KS], slo[KS];
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        shi[kk] = ld<O8>(L::SH + kp_frag + 64 * kk);
        slo[kk] = ld<O8>(L::SL + kp_frag + 64 * kk);
      }
      f0 = rec_frag(b, REC_TB, r, 0);
      f1 = second_step(rec_frag(b, REC_TB, r, 1), r);
      if constexpr (LO) {
        fl0 = ld<half8_t>(L::TBL + frag_index(r, 0) * FRAG_BYTES + lane * 16);
        fl1 = second_step(ld<half8_t>(L::TBL + frag_index(r, 1) * FRAG_BYTES + lane * 16), r);
      }
      dd = rec_rows(b, SC_DEC, r);
      float4_t acc = {0.f, 0.f, 0.f, 0.f}, acl = acc;
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        acc = mma(mf[kk], shi[kk], acc);
        acl = mma(mf[kk], slo[kk], acl);
      }
      // X of token rows 16r..: scaled into range if it leaves it (a wave vote),
      // its scale published for the U waves
      float4_t x = vv - gg * (acc + acl);
      const float xm = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
      float down = 1.f;
      if (__builtin_amdgcn_ballot_w64(xm > X_LIMIT) != 0) {
        down = range_scale(wave_max(xm));
        x *= down;
      }
      const half4_t xh = to_half4(x);
      st(L::XT + sp_tile + 32 * r, xh);
      if constexpr (LO) st(L::xtl(b) + sp_tile + 32 * r, to_half4(x - to_float4(xh)));
      if (lane == 0) st(L::RS + 4 * r, down);
    }
    sync();
    {
      const half8_t x0 = ld<half8_t>(L::XT + sp_frag);
      const half8_t x1 = ld<half8_t>(L::XT + sp_frag + 64);
      half8_t xl0, xl1;
      if constexpr (LO) {
        xl0 = ld<half8_t>(L::xtl(b) + sp_frag);
        xl1 = ld<half8_t>(L::xtl(b) + sp_frag + 64);
      }
      const float4_t downs = ld<float4_t>(L::RS);
      fetch_kt(b, kt);
      // the chunk's scale: the smallest of its tiles'; the Tb lanes that
      // multiply tile t (tokens 8g.. of step kk: tile 2 kk + g/2) take
      // d / downs[t] (a power of two, at most 1)
      const float d = fminf(fminf(downs[0], downs[1]), fminf(downs[2], downs[3]));
      const float rd = d < 1.f ? 1.f / d : 1.f;
      if (d < 1.f) {
        const int t = g4 >> 1;
        f0 *= static_cast<half_t>(d / downs[t]);
        f1 *= static_cast<half_t>(d / downs[2 + t]);
        if constexpr (LO) {
          fl0 *= static_cast<half_t>(d / downs[t]);
          fl1 *= static_cast<half_t>(d / downs[2 + t]);
        }
      }
      // no branch between the products and their first reads
      float4_t u = mfma32(f0, x0, float4_t{0.f, 0.f, 0.f, 0.f});
      if constexpr (LO) {
        u = mfma32(f0, xl0, u);
        u = mfma32(fl0, x0, u);
      }
      u = mfma32(f1, x1, u);
      if constexpr (LO) {
        u = mfma32(f1, xl1, u);
        u = mfma32(fl1, x1, u);
      }
      const uint32_t o = sp_tile + 32 * r;
      st(L::ut(b) + o, to_half4(u));  // U' = U d, for O of this chunk
      if (wave == 0 && lane == 0) st(L::RS + 16 + 4 * b, d);
      u *= rd;
      const float4_t du = u * dd;
      const O4 hi = Op::from(du);
      st(L::UH + o, hi);
      st(L::UL + o, Op::from(du - Op::to(hi)));
    }
    sync();
    {
      O8 nmf[KS];
      fetch_rows(b ^ 1, 0, nmf);
      const float4_t nvv = v_rows(b ^ 1, r);
      const float4_t ngg = rec_rows(b ^ 1, SC_GAM, r);
      update_state(b, kt);
      next_chunk(wave, b ^ 1);
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) mf[kk] = nmf[kk];
      vv = nvv;
      gg = ngg;
    }
    sync();
  }

  // Four output elements as one LDS store (8 bytes for 16-bit outputs).
  __device__ __forceinline__ void put_out4(uint32_t off, float4_t o) const {
    if constexpr (sizeof(TOut) == 4) {
      st(off, o);
    } else {
      typedef TOut out4_t __attribute__((ext_vector_type(4)));
      st(off, out4_t{out_elem<TOut>(o[0]), out_elem<TOut>(o[1]), out_elem<TOut>(o[2]), out_elem<TOut>(o[3])});
    }
  }

  // Output waves: O = scale gamma Q S + QKD U of the chunk of parity ob (its
  // U^T is in U^T buffer ob) -> O tile ob. The products are formed
  // transposed (the operands' fragments swap roles, the same registers), so
  // lane (g, c) holds O[16 r + c][4 g + i], four consecutive columns of one
  // token: one LDS store of them instead of four, 512 contiguous bytes per wave.
  __device__ __forceinline__ void out_tile(int ob, const float4_t &qs, float gs, const half8_t &f0,
                                           const half8_t &f1) {
    const int r = wave & 3;
    // U^T of the chunk holds U d (d its range scale, usually 1): O = (scale gamma Q S d + QKD U d) / d
    const float d = ld<float>(L::RS + 16 + 4 * ob);
    const float rd = (d < 1.f ? 1.f / d : 1.f) * in_up;  // powers of two: exact
    float4_t o = qs * gs;
    if (d < 1.f) o *= d;
    // no branch between the products and their first reads
    o = mfma32(ld<half8_t>(L::ut(ob) + sp_frag), f0, o);
    o = mfma32(ld<half8_t>(L::ut(ob) + sp_frag + 64), f1, o);
    o *= rd;
    put_out4(L::ot(ob) + ((16 * r + c16) * VT + 4 * g4) * sizeof(TOut), o);
  }

  // Output waves. Phase 1: (Q S)^T (high part) of chunk n. Phase 2: O of
  // chunk n-1, then this chunk's QKD fragments and its lane's scale gamma
  // (for its O in the next tick); K^T for phase 3. Phase 3: the state update
  // (K = 128), then the Q rows of the next chunk.
  template <int P>
  __device__ __forceinline__ void tick_output(long n, O8 (&mf)[KS], float4_t &qs, float4_t &qs_prev,
                                              float &gs, half8_t &f0, half8_t &f1) {
    launder();
    const int b = P;
    const int r = wave & 3;
    O8 kt[2];
    {
      O8 shi[KS];
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) shi[kk] = ld<O8>(L::SH + kp_frag + 64 * kk);
      float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) acc = mma(shi[kk], mf[kk], acc);  // (Q S)^T: columns 4 g.., token c
      qs_prev = qs;
      qs = acc;
    }
    sync();
    {
      const half8_t n0 = rec_frag(b, REC_QKD, r, 0);
      const half8_t n1 = second_step(rec_frag(b, REC_QKD, r, 1), r);
      const float ngs = ld<float>(L::rec(b) + REC_SC + SC_GSC + (16 * r + c16) * 4);
      if constexpr (NKT > 4) fetch_kt(b, kt);
      if (n > 0) out_tile(b ^ 1, qs_prev, gs, f0, f1);
      f0 = n0;
      f1 = n1;
      gs = ngs;
    }
    sync();
    {
      O8 nmf[KS];
      fetch_rows(b ^ 1, 1, nmf);
      if constexpr (NKT > 4) {
        update_state(b, kt);
        next_chunk(wave, b ^ 1);
      }
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) mf[kk] = nmf[kk];
    }
    sync();
  }

  // Tick n of a loader wave: register set P (= n mod 2) holds chunk n+1 on
  // entry; slot by slot it goes to LDS buffer 1 - P and receives chunk n+3:
  // what phase 3 reads (K, Q, V, decay vectors) in phases 1 and 2, the Tb and
  // QKD fragments in phase 3. In phase 3 the O tile of chunk n-1 (written in
  // phase 2) also goes out.
  template <int P>
  __device__ __forceinline__ void tick_loader(long n) {
    if constexpr (CHAIN) {  // chunk n + 1's initial-state units to its buffer; chunk n + 3's issued
      if (h0v[P]) store_h0(P ^ 1, h0r[P]);
      h0v[P] = lc.first && !at_end(lc);
      load_h0(h0r[P], lc, lc.first);
    }
    const long t0 = lc.t0;  // chunk n + 3
    const long len = len_of(lc);
    const unsigned char *rec = rec_of(lc);
    stage.template restage<0, Stage::SLOT_P2>(p, lds, L::kq(P ^ 1), regs[P], lt, t0, len, hk, h, v0, rec);
    sync();
    stage.template restage<Stage::SLOT_P2, Stage::SLOT_P3>(p, lds, L::kq(P ^ 1), regs[P], lt, t0, len, hk, h, v0,
                                                            rec);
    sync();
    store_out(n - 1);
    if (n > 0) advance(oc);
    stage.template restage<Stage::SLOT_P3, Stage::UPT>(p, lds, L::kq(P ^ 1), regs[P], lt, t0, len, hk, h, v0, rec);
    advance(lc);
    sync();
  }

  // Chunks of the group's sequences, summed over the whole workgroup (one
  // sequence: read directly, with no barrier before the first loads).
  __device__ __forceinline__ long group_chunks() {
    if (s_end - s_begin == 1) {
      long b, e;
      seq_bounds(p, s_begin, b, e);
      return (e - b + CH - 1) / CH;
    }
    int c = 0;
    for (int s = s_begin + tid; s < s_end; s += NT) {
      long b, e;
      seq_bounds(p, s, b, e);
      c += static_cast<int>((e - b + CH - 1) / CH);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
    int *part = reinterpret_cast<int *>(lds + L::OT);  // the O tiles are not in use yet
    if (lane == 0) part[wave] = c;
    sync();
    long total = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) total += part[w];
    sync();
    return total;
  }

  __device__ __forceinline__ void run() {
    nchunks = group_chunks();
    // Initial state of the group's first sequence with tokens (the empty ones
    // before it pass their initial states through): compute wave j owns key
    // rows 16j..16j+15.
    const int kt = wave;
    if (kt < NKT) {
      seek_owner(cc, s_begin, kt);
      if (!at_end(cc)) sacc = initial_state(cc.s, kt);
      put_state(kt);
    }
    if (wave >= NCW) {
      // Chunk 0 into buffer 0; chunks 1 and 2 in flight into register sets 0
      // and 1, each followed by a store that goes nowhere, as in a tick.
      seek(lc, s_begin);
      oc = lc;
      load_chunk(regs[1], lc);
      advance(lc);
      stage.store(lds, L::kq(0), regs[1], lt);
      if constexpr (CHAIN) {  // initial states of chunks 1 and 2, as in a tick
        h0v[0] = lc.first && !at_end(lc);
        load_h0(h0r[0], lc, lc.first);
      }
      load_chunk(regs[0], lc);
      advance(lc);
      store_out(-1);
      if constexpr (CHAIN) {
        h0v[1] = lc.first && !at_end(lc);
        load_h0(h0r[1], lc, lc.first);
      }
      load_chunk(regs[1], lc);
      advance(lc);
      store_out(-1);
      sync();
      long n = 0;
      for (; n + 1 < nchunks; n += 2) {
        tick_loader<0>(n);
        tick_loader<1>(n + 1);
      }
      if (n < nchunks) tick_loader<0>(n);
      sync();  // the O tile of the last chunk is complete
      if (nchunks > 0) store_out(nchunks - 1);
      return;
    }
    sync();
    if (wave < 4) {
      O8 mf[KS];
      fetch_rows(0, 0, mf);
      float4_t vv = v_rows(0, wave);
      float4_t gg = rec_rows(0, SC_GAM, wave);
      long n = 0;
      for (; n + 1 < nchunks; n += 2) {
        tick_chain<0>(mf, vv, gg);
        tick_chain<1>(mf, vv, gg);
      }
      if (n < nchunks) tick_chain<0>(mf, vv, gg);
      sync();
    } else {
      O8 mf[KS];
      fetch_rows(0, 1, mf);
      float4_t qs = {0.f, 0.f, 0.f, 0.f}, qs_prev = qs;
      float gs = 0.f;
      half8_t f0 = {}, f1 = {};
      long n = 0;
      for (; n + 1 < nchunks; n += 2) {
        tick_output<0>(n, mf, qs, qs_prev, gs, f0, f1);
        tick_output<1>(n + 1, mf, qs, qs_prev, gs, f0, f1);
      }
      if (n < nchunks) tick_output<0>(n, mf, qs, qs_prev, gs, f0, f1);
      if (nchunks > 0) out_tile(static_cast<int>((nchunks - 1) & 1), qs, gs, f0, f1);
      sync();
    }
    // With CHAIN, final states went out at each sequence's last chunk (next_chunk).
    if (!CHAIN && kt < NKT && !at_end(cc)) final_state(cc.s, kt, sacc);
  }
};

#ifdef PBGDN_DEBUG
// Debug builds: barrier counts of the waves of each workgroup of the last
// scan launch that used its row (blockIdx modulo AUDIT_ROWS), read by
// pbgdn_debug_scan_barriers.
constexpr int AUDIT_ROWS = 4096;
__device__ uint32_t scan_barrier_audit[AUDIT_ROWS * (NT / 64)];
#endif

template <int K, typename TIn, typename TOut, bool CHAIN>
__global__ __launch_bounds__(NT) void scan_kernel(ChunkParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  using L = ScanLayout<K, sizeof(TIn) == 4>;
  PBGDN_POISON_LDS(smem_raw, CHAIN ? L::CHAIN_BYTES : L::BYTES);
  PBGDN_POISON_SYNC();
  ScanBlock<K, TIn, TOut, CHAIN> blk(smem_raw, p);
  blk.run();
#ifdef PBGDN_DEBUG
  if ((threadIdx.x & 63) == 0) {
    scan_barrier_audit[(blockIdx.x % AUDIT_ROWS) * (NT / 64) + (threadIdx.x >> 6)] = blk.nbar;
  }
#endif
}

template <int K, typename TIn, typename TOut, bool CHAIN>
int launch_scan_kernel(const ChunkParams &p, hipStream_t stream) {
  static std::atomic<bool> configured[MAX_DEVICES];  // the attribute is set per device
  using L = ScanLayout<K, sizeof(TIn) == 4>;
  static_assert(L::CHAIN_BYTES <= 160 * 1024, "scan LDS");
  const size_t smem = CHAIN ? L::CHAIN_BYTES : L::BYTES;
  auto kernel = scan_kernel<K, TIn, TOut, CHAIN>;
  if (!smem_configured(reinterpret_cast<const void *>(kernel), smem, configured)) return PBGDN_ERR_LAUNCH;
  const int total = (p.V / VT) * p.Hv * p.seq_groups;
  hipLaunchKernelGGL(kernel, dim3(total), dim3(NT), smem, stream, p);
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}

}  // namespace

template <int K, typename TIn, typename TOut>
int launch_scan(const ChunkParams &p, hipStream_t stream) {
  if (p.num_seqs > p.seq_groups) return launch_scan_kernel<K, TIn, TOut, true>(p, stream);
  return launch_scan_kernel<K, TIn, TOut, false>(p, stream);
}

template int launch_scan<64, u16, u16>(const ChunkParams &, hipStream_t);
template int launch_scan<64, u16, float>(const ChunkParams &, hipStream_t);
template int launch_scan<64, half_t, half_t>(const ChunkParams &, hipStream_t);
template int launch_scan<64, half_t, float>(const ChunkParams &, hipStream_t);
template int launch_scan<64, float, float>(const ChunkParams &, hipStream_t);
template int launch_scan<128, u16, u16>(const ChunkParams &, hipStream_t);
template int launch_scan<128, u16, float>(const ChunkParams &, hipStream_t);
template int launch_scan<128, half_t, half_t>(const ChunkParams &, hipStream_t);
template int launch_scan<128, half_t, float>(const ChunkParams &, hipStream_t);
template int launch_scan<128, float, float>(const ChunkParams &, hipStream_t);

}  // namespace pbgdn

#ifdef PBGDN_DEBUG
// Debug builds only (no counterpart in the reference; not in the header): with
// `reset`, fill the narrow scan's barrier audit with 0xffffffff; then copy it
// (rows of 12 per-wave counts, `rows` of them at most) to host memory `out`.
// A workgroup whose waves passed different numbers of barriers shows as a row
// whose entries differ. Synchronises the device.
extern "C" int pbgdn_debug_scan_barriers(uint32_t *out, int rows, int reset) {
  using namespace pbgdn;
  constexpr size_t BYTES = sizeof(scan_barrier_audit);
  if (hipDeviceSynchronize() != hipSuccess) return PBGDN_ERR_LAUNCH;
  if (reset) {
    static uint32_t fill[AUDIT_ROWS * (NT / 64)];
    for (auto &x : fill) x = 0xffffffffu;
    if (hipMemcpyToSymbol(HIP_SYMBOL(scan_barrier_audit), fill, BYTES) != hipSuccess) return PBGDN_ERR_LAUNCH;
  }
  if (out && rows > 0) {
    const size_t n = std::min<size_t>(BYTES, static_cast<size_t>(rows) * (NT / 64) * sizeof(uint32_t));
    if (hipMemcpyFromSymbol(out, HIP_SYMBOL(scan_barrier_audit), n) != hipSuccess) return PBGDN_ERR_LAUNCH;
  }
  return PBGDN_OK;
}
#endif
