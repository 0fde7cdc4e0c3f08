// Wide scan kernel of the chunkwise prefill: the state-dependent part, chunk by
// chunk (the serial loop of delta_rule_chunked, pseudobrain/gated_deltanet.py:158-165),
// with one wave per 16-column tile of the state and a whole 128-column value
// head (8 tiles, 8 waves) per workgroup.
//
// Why wide. A chunk step needs the chunk's K and Q rows (16 KiB each at K = 128)
// and its workspace record (13 KiB) in LDS, and one CU stages at most ~25 bytes
// per clock from L2 (measured with direct-to-LDS loads, also with a single CU
// per XCD loading). A workgroup that owns one 16-column tile pays that fill for
// 16 columns of work; here the 8 waves of a workgroup own the 8 tiles of one
// (sequence, value head) and share every byte staged. Two waves per SIMD hide
// each other's LDS and dependency latency (a single wave per SIMD ran its
// chunk step at a third of its MFMA issue rate).
//
// One wave, one tile, everything in registers. The fp32 state tile S [K, 16]
// is held as K/16 MFMA accumulator tiles. The accumulator layout of a 16x16
// tile is also the B-operand layout of a contraction over its rows, so the
// chain X -> U -> S of a chunk runs without leaving the wave:
//   X   = V - diag(gamma) K S        (K rows from LDS, S as a bf16 high/low pair)
//   U   = Tb X                       (Tb fragments from the record, X as fp16)
//   S  <- gamma_63 S + K^T (dec U)   (K^T by transposing LDS reads, dec U high/low)
//   O   = scale gamma Q S + QKD U    (Q rows from LDS, S high part; QKD, U fp16)
// Contraction slots: a 32-wide contraction step kk takes accumulator tiles 2kk
// and 2kk+1 as B operand, so slot j of lane group g is row 4g + j of tile 2kk
// (j < 4) or row 4g + j - 4 of tile 2kk + 1. For the token contractions (U,
// the update, O) the A operands are read in that slot order. For the key
// contraction the state's rows are permuted instead: row 4g + i of state tile
// 2kk + p holds key 32kk + 8g + 4p + i, which makes the slots of lane group g
// keys 32kk + 8g .. + 7, one contiguous 16-byte piece of a K or Q row. The
// update's K^T reads and the state's loads and stores follow the same map.
// O is formed transposed (O^T = (Q S)^T diag(scale gamma) + U^T QKD^T: the
// same registers with the MFMA operands swapped), so a lane holds 4
// contiguous columns of a token row and stores them as one 8-byte piece.
//
// Staging. A chunk's K and Q rows (16-bit, 256 bytes at K = 128), its record
// and its V rows (128 columns) are copied HBM -> LDS by direct-to-LDS buffer
// loads (1 KiB per instruction, no registers). Rows past the end of a sequence
// read as zeros (out of the buffer resource's range): the identity steps of
// the reference's padding (gated_deltanet.py:127). K and the record, read in
// phases A to C, rotate through three buffers; Q and V, read in phase A only,
// through two.
//
// LDS banks (measured on gfx950): a 16-byte read moves about 120 bytes a
// clock; a transposing 8-byte read serves 32 lanes a clock, without conflict
// when their 8-byte pieces fall on distinct positions modulo 256 bytes. The
// 16-byte pieces of a K/Q row (256 bytes) sit at piece ^ swz(row & 15),
// swz(x) = 4 (x & 3) + (x >> 2): a transposing read of K^T (32 lanes: 8 rows
// x 4 pieces, one 8-byte half of each) then uses 16 positions twice, the
// least possible with one half per instruction. The pieces of a V row sit at
// piece ^ (2 (row & 3) + 8 ((row >> 2) & 1)), which makes its transposing reads conflict-free. Each wave issues its share of a chunk's loads (7 or 8
// instructions); a vector memory instruction holds its wave at issue until the
// CU takes it, so the two waves of a SIMD issue at different points of the
// step (waves 0-3 after the barrier, 4-7 after their state update).
//
// Step n of a workgroup (one barrier):
//   A: X and Q S of chunk n; B: U; then every wave waits for its loads of
//   chunk n+1, barrier; loads of chunk n+2 are issued (into buffers chunk n-1,
//   or for Q and V chunk n, used); C: the state update; O of chunk n, stored.
#include "chunk.hpp"
#include "layer_math.hpp"

namespace pbgdn {
namespace {

constexpr int WT = 8;          // 16-column tiles per workgroup, one wave each
constexpr int WNT = 64 * WT;   // threads per workgroup
constexpr int WCOLS = 16 * WT; // value columns per workgroup

typedef unsigned int u32x4_t_ __attribute__((ext_vector_type(4)));

template <int K>
struct WideLayout {
  static constexpr int ROW = 2 * K;                  // bytes of a staged K or Q row
  static constexpr int MAT = CH * ROW;               // one of K, Q
  static constexpr int VROW = 128 * 2;               // bytes of a staged V row (128 columns, 16-bit)
  static constexpr int VMAT = CH * VROW;
  static constexpr int K_OFF = 0;                            // [3] K
  static constexpr int Q_OFF = K_OFF + 3 * MAT;              // [2] Q
  static constexpr int R_OFF = Q_OFF + 2 * MAT;              // [3] record
  static constexpr int V_OFF = R_OFF + 3 * REC_BYTES;        // [2] V
  static constexpr int P_OFF = V_OFF + 2 * VMAT;             // epilogue: [CH tokens][WT waves] sums of squares
  static constexpr int N_OFF = P_OFF + CH * WT * 4;          // epilogue: o_norm of the 128 columns
  static constexpr int BYTES = N_OFF + WCOLS * 4;
  __device__ static constexpr int kmat(int b3) { return K_OFF + b3 * MAT; }
  __device__ static constexpr int qmat(int b2) { return Q_OFF + b2 * MAT; }
  __device__ static constexpr int rec(int b3) { return R_OFF + b3 * REC_BYTES; }
  __device__ static constexpr int vmat(int b2) { return V_OFF + b2 * VMAT; }
};

// Position of 16-byte piece u of K/Q row r is u ^ swz(r) (K = 128: 16 pieces a
// row); of V row r, u ^ vswz(r) (16 pieces).
__host__ __device__ constexpr int swz(int r) { return 4 * (r & 3) + ((r >> 2) & 3); }
__host__ __device__ constexpr int vswz(int r) { return 2 * (r & 3) + 8 * ((r >> 2) & 1); }

// The wave's per-token sums over its 16 columns: lane (g, c) holds x[r], a
// partial of token 16 r + c; returns, in lane (g, c), the sum over the four
// lane groups for token 16 g + c (a reduce-scatter: swap32 pairs lane groups
// g and g ^ 2, swap16 g and g ^ 1).
__device__ __forceinline__ float rows_reduce(const float (&x)[4]) {
  // lanes 0-31 keep tokens 16 r + c of r = 0, 1, lanes 32-63 those of r = 2, 3
  float a0 = x[0], a2 = x[2], a1 = x[1], a3 = x[3];
  swap32(a0, a2);
  swap32(a1, a3);
  float w0 = a0 + a2;  // r = 0 (lanes < 32) or 2
  float w1 = a1 + a3;  // r = 1 or 3
  swap16(w0, w1);
  return w0 + w1;
}

// The inverse movement: lane (g, c) holds y for token 16 g + c; returns in
// every lane (g, c) the four values of tokens 16 r + c, r = 0..3.
__device__ __forceinline__ void rows_gather(float y, float (&out)[4]) {
  float e = y, o = y;
  swap16(e, o);  // e: the value of group g & 2, o: of group (g & 2) + 1
  float e2 = e, o2 = o;
  swap32(e, e2);  // e: group 0, e2: group 2
  swap32(o, o2);  // o: group 1, o2: group 3
  out[0] = e;
  out[1] = o;
  out[2] = e2;
  out[3] = o2;
}

template <int K, typename TIn, typename TOut, bool EPI>
struct WideBlock {
  using L = WideLayout<K>;
  using Op = OpOf<TIn>;
  using O4 = typename Op::T4;
  using O8 = typename Op::T8;
  static constexpr int NKT = K / 16;   // state tiles
  static constexpr int KS = K / 32;    // key contraction steps
  static constexpr int DMA_KQ = L::MAT / 1024;        // 1 KiB DMA instructions per K or Q matrix
  static constexpr int DMA_REC = REC_BYTES / 1024;
  static constexpr int DMA_V = L::VMAT / 1024;
  static constexpr int OUT_STORES = 4;  // O stores a wave issues per chunk, after its loads
  // staging loads a wave issues per chunk (issue_chunk): the K, Q and V
  // instructions split evenly, the record's first DMA_REC % WT waves one more
  static constexpr int DMA_WAVE_LO = 2 * (DMA_KQ / WT) + DMA_V / WT + DMA_REC / WT;
  static_assert(DMA_REC % WT != 0, "two staging counts");
  static_assert(K == 128, "the wide scan is built for K = 128");
  static_assert(REC_BYTES % 1024 == 0 && DMA_KQ % WT == 0 && DMA_V % WT == 0, "whole DMA instructions per wave");
  static_assert(sizeof(TIn) == 2, "16-bit inputs (staged as they are)");
  static_assert(sizeof(TOut) == 2 || (EPI && sizeof(TOut) == 4), "16-bit o; hs also in float32");
  static constexpr int GATE_LOADS = EPI ? 4 : 0;  // gate loads a wave issues per chunk, at its start
  static_assert(L::BYTES <= 160 * 1024, "LDS");

  unsigned char *lds;
  const ChunkParams &p;
  int lane, c16, g4, wave, h, hk, col0, v0, seq;
  long bos, eos;
  long nchunks;
  float4_t s[NKT];  // the state tile, accumulator layout, permuted key rows

  uint32_t xa[KS];   // K/Q row fragment of row tile 0, step kk (add 16 * ROW * r)
  uint32_t tr[KS];   // K^T transposing read of state tiles 2kk + p (add 8 p), tokens 4g.. (add ROW * token)
  uint32_t vtr;      // V transposing read of row tile 0 (add 16 * VROW * r)
  uint32_t tbo0, tbo1;  // the two 8-byte halves of a Tb / QKD fragment row this lane reads
  uint32_t o_off;    // O: byte offset of this lane's piece (token c, columns v0 + 4g..) within a chunk
  uint32_t g_off;    // gate: the same piece's byte offset from the chunk's first gate row (head h)
  uint32_t dma_kq;   // source offset of this lane's piece of K/Q DMA instruction `wave` within a chunk's rows
  uint32_t dma_v;    // same for V
  // The next chunk to stage (chunks are staged in order, each once): its
  // first K/Q row, V row (column col0), record, and the tokens left from it.
  const unsigned char *kp, *qp, *vp, *rp;
  long left;

  __device__ __forceinline__ WideBlock(unsigned char *l, const ChunkParams &prm) : lds(l), p(prm) {
    const int tid = threadIdx.x;
    lane = tid & 63;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    c16 = lane & 15;
    g4 = lane >> 4;
    // Block -> (sequence, value head, column group): the column groups and the
    // value heads of one key head of one sequence share their K/Q rows; keep
    // them on one XCD (xcd_group).
    const int groups = p.V / WCOLS;
    const int per_key = groups * (p.Hv / p.Hk);
    const int total = static_cast<int>(gridDim.x);
    int kgrp, member;
    xcd_group(static_cast<int>(blockIdx.x), total / per_key, per_key, p.xcds, kgrp, member);
    seq = kgrp / p.Hk;
    hk = kgrp % p.Hk;
    h = hk * (p.Hv / p.Hk) + member / groups;
    col0 = (member % groups) * WCOLS;
    v0 = col0 + 16 * wave;
    seq_bounds(p, seq, bos, eos);
    nchunks = (eos - bos + CH - 1) / CH;

    const int sw = swz(c16);
    const int k = c16 >> 2, q = c16 & 3;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      // row c of row tile 0, piece 4kk + g
      xa[kk] = c16 * L::ROW + ((4 * kk + g4) ^ sw) * 16;
      // transposing read: lane 4k + q of group g points at token row 4g + k and
      // the 8 bytes of keys 32kk + 8q + 4p (piece 4kk + q, half p)
      tr[kk] = (4 * g4 + k) * L::ROW + ((4 * kk + q) ^ swz(4 * g4 + k)) * 16;
    }
    // V: lane 4k + q of group g points at token row 4g + k, the 8 bytes of
    // columns 16 wave + 4q .. (piece 2 wave + q/2, half q & 1)
    vtr = (4 * g4 + k) * L::VROW + (((2 * wave + (q >> 1)) ^ vswz(4 * g4 + k)) * 16) + 8 * (q & 1);
    // Tb / QKD fragment rows: lane (g, c) takes tokens 32kk + 4g.. (held by
    // fragment lane (g/2, c), half g&1) and 32kk + 16 + 4g.. (lane (2 + g/2, c))
    tbo0 = (16 * (g4 >> 1) + c16) * 16 + 8 * (g4 & 1);
    tbo1 = (16 * (2 + (g4 >> 1)) + c16) * 16 + 8 * (g4 & 1);
    o_off = (c16 * p.Hv * p.V + v0 + 4 * g4) * static_cast<uint32_t>(sizeof(TOut));
    g_off = static_cast<uint32_t>((c16 * p.gate_stride + v0 + 4 * g4) * 2);
    // K/Q DMA instruction i covers rows 4i..4i+3, lane l filling row 4i + l/16
    // at position l%16 (piece (l%16) ^ swz(row)); this wave's are i = wave +
    // WT s, rows 32 s + 4 wave + l/16 (row & 15 = 4 (wave & 3) + l/16). V rows
    // are 256 bytes too: the same shape with vswz.
    const int r = 4 * wave + (lane >> 4);
    dma_kq = static_cast<uint32_t>(r) * p.Hk * K * 2 + ((lane & 15) ^ swz(r)) * 16;
    dma_v = static_cast<uint32_t>(r) * p.Hv * p.V * 2 + ((lane & 15) ^ vswz(r)) * 16;
    const long kq0 = (bos * p.Hk + hk) * static_cast<long>(K) * 2;
    kp = static_cast<const unsigned char *>(p.k) + kq0;
    qp = static_cast<const unsigned char *>(p.q) + kq0;
    vp = static_cast<const unsigned char *>(p.v) + ((bos * p.Hv + h) * static_cast<long>(p.V) + col0) * 2;
    rp = p.ws + (rec_base(bos, seq) * p.Hv + h) * static_cast<long>(REC_BYTES);
    left = eos - bos;
  }

  template <typename T>
  __device__ __forceinline__ T ld(uint32_t off) const { return *reinterpret_cast<const T *>(lds + off); }
  __device__ __forceinline__ i16x4_t ld_tr(uint32_t off) const {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t *)(lds + off));
  }
  // Raw buffer descriptor (the words __builtin_amdgcn_make_buffer_rsrc builds):
  // base, stride 0, byte range, RSRC_WORD3.
  __device__ __forceinline__ static u32x4_t_ desc(const void *base, long bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return u32x4_t_{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xffffu,
                    static_cast<uint32_t>(bytes > 0 ? bytes : 0), static_cast<uint32_t>(RSRC_WORD3)};
  }
  // One direct-to-LDS load: 16 bytes per lane from `off` (the whole offset in
  // the VGPR, where the range check applies) to LDS lds_off + 16 lane. Written
  // as assembly: the compiler cannot tell which LDS bytes a buffer-to-LDS load
  // writes and would otherwise wait for it before every later LDS read; the
  // waits here are the explicit ones (wait_vm).
  __device__ __forceinline__ void dma(const u32x4_t_ &rs, uint32_t lds_off, uint32_t off) const {
    typedef __attribute__((address_space(3))) unsigned char lds_byte;
    const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_byte *)(lds + lds_off)));  // C-style: an address-space cast
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0), "v"(off), "s"(rs)
                 : "memory", "m0");
  }

  // ------------------------------------------------------------------ loads
  __device__ __forceinline__ long rows_of(long n) const {
    const long l = eos - (bos + n * CH);
    return l <= 0 ? 0 : (l < CH ? l : CH);
  }

  // This wave's direct-to-LDS loads of the next chunk n (zero-size resources
  // past the stream's end): K and the record into ring slot n % 3 (b3), Q and
  // V into n % 2 (b2).
  __device__ __forceinline__ void issue_chunk(int b3, int b2) {
    const long rows = left <= 0 ? 0 : (left < CH ? left : CH);
    const long kqs = static_cast<long>(p.Hk) * K * 2, vs = static_cast<long>(p.Hv) * p.V * 2;
    const u32x4_t_ rk = desc(kp, rows > 0 ? (rows - 1) * kqs + K * 2 : 0);
    const u32x4_t_ rq = desc(qp, rows > 0 ? (rows - 1) * kqs + K * 2 : 0);
    const u32x4_t_ rv = desc(vp, rows > 0 ? (rows - 1) * vs + WCOLS * 2 : 0);
    const u32x4_t_ rr = desc(rp, rows > 0 ? REC_BYTES : 0);
#pragma unroll
    for (int s_ = 0; s_ < DMA_KQ / WT; ++s_) {
      const int i = wave + WT * s_;
      const uint32_t off = dma_kq + static_cast<uint32_t>(4 * WT * s_) * static_cast<uint32_t>(kqs);
      dma(rk, L::kmat(b3) + 1024 * i, off);
      dma(rq, L::qmat(b2) + 1024 * i, off);
    }
#pragma unroll
    for (int s_ = 0; s_ < DMA_V / WT; ++s_) {
      const int i = wave + WT * s_;
      dma(rv, L::vmat(b2) + 1024 * i, dma_v + static_cast<uint32_t>(4 * WT * s_) * static_cast<uint32_t>(vs));
    }
#pragma unroll
    for (int s_ = 0; s_ < (DMA_REC + WT - 1) / WT; ++s_) {
      const int i = wave + WT * s_;
      const uint32_t roff = 1024 * i + lane * 16;  // units no scan reads: an out-of-range load stages zeros
      if (i < DMA_REC) dma(rr, L::rec(b3) + 1024 * i, rec_unused_unit(static_cast<int>(roff)) ? OUT_OF_RANGE : roff);
    }
    kp += CH * kqs;
    qp += CH * kqs;
    vp += CH * vs;
    rp += static_cast<long>(p.Hv) * REC_BYTES;
    left -= CH;
  }

  // ------------------------------------------------------------------ state I/O
  // Lane (g, c) holds rows 4g + i of state tile t = 2kk + p: key 32kk + 8g + 4p + i.
  __device__ __forceinline__ int key_of(int t, int i) const { return 32 * (t >> 1) + 8 * g4 + 4 * (t & 1) + i; }
  __device__ __forceinline__ long slot_of() const {
    return p.state_idx ? static_cast<long>(p.state_idx[seq]) : static_cast<long>(seq);
  }
  __device__ __forceinline__ bool in_pool(long slot) const {
    return !p.state_idx || (slot >= 0 && slot < p.num_states);
  }
  __device__ __forceinline__ void load_state() {
    const long slot = slot_of();
    const bool any = p.h0 && in_pool(slot) && (!p.has_initial_state || p.has_initial_state[seq]);
#pragma unroll
    for (int t = 0; t < NKT; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[t][i] = any ? load_elem(p.h0, ((slot * p.Hv + h) * K + key_of(t, i)) * static_cast<long>(p.V) + v0 + c16,
                                  p.state_dtype)
                      : 0.f;
      }
    }
  }
  __device__ __forceinline__ void store_state() const {
    const long slot = slot_of();
    if (!p.ht || !in_pool(slot)) return;
#pragma unroll
    for (int t = 0; t < NKT; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        store_elem(p.ht, ((slot * p.Hv + h) * K + key_of(t, i)) * static_cast<long>(p.V) + v0 + c16, p.state_dtype,
                   s[t][i]);
      }
    }
  }

  // ------------------------------------------------------------------ operands
  __device__ __forceinline__ O8 pair(const O4 &a, const O4 &b) const {
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  }
  __device__ __forceinline__ half8_t pairh(const half4_t &a, const half4_t &b) const {
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  }
  // A Tb / QKD fragment row in slot order is two 8-byte halves, at lane
  // offsets tbo0 and tbo1 of the fragment.
  // K^T operand of state tile t = 2kk + pp for tokens 32 ks .. + 31, from the
  // lane base tb = K slot + tr[kk]
  __device__ __forceinline__ O8 kt_frag(uint32_t tb, int pp, int ks) const {
    const uint32_t base = tb + 8 * pp + (32 * ks) * L::ROW;
    const i16x4_t lo4 = ld_tr(base);
    const i16x4_t hi4 = ld_tr(base + 16 * L::ROW);
    return __builtin_bit_cast(O8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
  }

  // Workgroup barrier; the fences keep LDS accesses on their side. Each wave
  // waits for its loads before it (wait_vm), so after it a chunk's staged
  // bytes are visible to every wave.
  __device__ __forceinline__ void barrier() const {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  }
  // Wait until at most VM of this wave's vector memory operations are
  // outstanding. They complete in issue order, so the newest VM stay in flight.
  template <int VM>
  __device__ __forceinline__ void wait_vm() const {
    static_assert(VM >= 0 && VM < 64, "vmcnt range");
    // gfx9 s_waitcnt: vmcnt[3:0] and [15:14], expcnt[6:4], lgkmcnt[11:8]
    __builtin_amdgcn_s_waitcnt((VM & 0xF) | (0x7 << 4) | (0xF << 8) | (((VM >> 4) & 3) << 14));
  }

  // An LDS byte address the compiler treats as unknown: the reads built on it
  // fold their constant parts into the instruction's offset field (the
  // compiler would otherwise hoist lane-constant sums out of the loop into
  // extra registers and add the chunk's ring slot once per read).
  __device__ __forceinline__ static uint32_t opaque(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
  }

  // The layer epilogue on O of a chunk (gated_deltanet.py:439-440): per token,
  // o rsqrt(mean over the head's V columns of o^2 + eps) o_norm SiLU(gate).
  // A token's 128 columns are spread over the 8 waves: each wave's sums go
  // through LDS, with a second barrier (the single slot is free again once
  // every wave has passed the next chunk's barrier).
  __device__ __forceinline__ void epilogue(float4_t (&o)[4], v2u32_t (&graw)[4]) const {
    float ss[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) ss[r] = o[r][0] * o[r][0] + o[r][1] * o[r][1] + o[r][2] * o[r][2] + o[r][3] * o[r][3];
    const float part = rows_reduce(ss);  // token 16 g + c, this wave's 16 columns
    const uint32_t pt = L::P_OFF + (16 * g4 + c16) * (WT * 4);
    *reinterpret_cast<float *>(lds + pt + 4 * wave) = part;
    barrier();
    const float4_t pa = ld<float4_t>(pt), pb = ld<float4_t>(pt + 16);
    const float tot = (pa[0] + pa[1]) + (pa[2] + pa[3]) + ((pb[0] + pb[1]) + (pb[2] + pb[3]));
    float rr[4];
    rows_gather(__builtin_amdgcn_rsqf(tot * (1.f / WCOLS) + p.eps), rr);
    const float4_t nrm = ld<float4_t>(L::N_OFF + (16 * wave + 4 * g4) * 4);
    // the gate loads: older than the staging loads of chunk n + 2, which stay
    // in flight (a wave's exact count: waiting on one of them costs a memory
    // latency that the barrier above passes to every wave of the next chunk)
    if (wave < DMA_REC % WT) {
      wait_vm<DMA_WAVE_LO + 1>();
    } else {
      wait_vm<DMA_WAVE_LO>();
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      v2u32_t gr = graw[r];
      asm volatile("" : "+v"(gr));  // after the wait
      const float4_t gt = Op::bits_to_float(__builtin_bit_cast(i16x4_t, gr));
#pragma unroll
      for (int i = 0; i < 4; ++i) o[r][i] *= rr[r] * nrm[i] * siluf(gt[i]);
    }
  }

  __device__ __forceinline__ void run() {
    load_state();
    if (nchunks <= 0) {
      store_state();
      return;
    }
    issue_chunk(0, 0);
    issue_chunk(1, 1);
    wait_vm<0>();
    if constexpr (EPI) {
      const int tid = threadIdx.x;
      if (tid < WCOLS) *reinterpret_cast<float *>(lds + L::N_OFF + 4 * tid) = p.o_norm[col0 + tid];
    }
    barrier();
    const bool early = wave < 4;  // issues its loads right after the barrier (else after the state update)
    // ring slots of chunks n (b3, b2) and n + 2 (i3, i2)
    int b3 = 0, b2 = 0, i3 = 2, i2 = 0;
    // O: chunk n's first row of this (value head, column range)
    unsigned char *op = static_cast<unsigned char *>(p.o) + ((bos * p.Hv + h) * static_cast<long>(p.V)) * sizeof(TOut);
    const long ostride = static_cast<long>(p.Hv) * p.V * sizeof(TOut);  // bytes per token row
    long oleft = eos - bos;
    // gate: chunk n's first row, columns of value head h
    const unsigned char *gp = EPI ? static_cast<const unsigned char *>(p.gate) +
                                        (bos * p.gate_stride + static_cast<long>(h) * p.V) * 2
                                  : nullptr;
    const long gstride = p.gate_stride * 2;  // bytes per gate row
    // Every LDS read is issued at least one group of products before its
    // first use: the scheduling fences (sched_barrier) keep the compiler from
    // moving a read down to its use, where the wave would wait out its latency.
    O8 kf[2][4], qf[2][4];  // K and Q row fragments, step kk in slot kk & 1
    {
      const uint32_t kb = opaque(L::kmat(0) + xa[0]), qb = opaque(L::qmat(0) + xa[0]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        kf[0][r] = ld<O8>(kb + 16 * r * L::ROW);
        qf[0][r] = ld<O8>(qb + 16 * r * L::ROW);
      }
    }
    for (long n = 0; n < nchunks; ++n) {
      const uint32_t km = L::kmat(b3), qm = L::qmat(b2), rc = L::rec(b3), vm = L::vmat(b2);
      // The gate of chunk n (rows 16 r + c, the lane's 4 columns), used at its
      // O: issued first, so the whole step hides its latency.
      v2u32_t graw[4];
      if constexpr (EPI) {
        const long rows = oleft < CH ? oleft : CH;
        const u32x4_t_ rg = desc(gp, (rows - 1) * gstride + p.V * 2);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t off = g_off + static_cast<uint32_t>(16 * r) * static_cast<uint32_t>(gstride);
          asm volatile("buffer_load_dwordx2 %0, %1, %2, 0 offen" : "=v"(graw[r]) : "v"(off), "s"(rg) : "memory");
        }
      }
      // lane bases of this chunk's reads
      const uint32_t rl = opaque(rc + REC_SC + 16 * g4);  // gamma, dec rows 4g..: + 64 r (+ table)
      const uint32_t rf0 = opaque(rc + tbo0), rf1 = opaque(rc + tbo1);
      // ---- A: X = V - gamma K S and (Q S)^T for the 4 row tiles, contraction
      // step kk outermost so that consecutive products go to different
      // accumulators; step kk+1's operands (after the last step, those of X
      // and U) are read before step kk's products
      float4_t ah[4], aq[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) ah[r] = aq[r] = float4_t{0.f, 0.f, 0.f, 0.f};
      i16x4_t vraw[4];
      float4_t gam[4];
      half8_t tbf[6];
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const int cur = kk & 1;
        if (kk + 1 < KS) {
          const uint32_t kb = opaque(km + xa[kk + 1]), qb = opaque(qm + xa[kk + 1]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            kf[cur ^ 1][r] = ld<O8>(kb + 16 * r * L::ROW);
            qf[cur ^ 1][r] = ld<O8>(qb + 16 * r * L::ROW);
          }
        } else {
          const uint32_t vb = opaque(vm + vtr);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            vraw[r] = ld_tr(vb + 16 * r * L::VROW);
            gam[r] = ld<float4_t>(rl + SC_GAM + 64 * r);
          }
#pragma unroll
          for (int f = 0; f < 6; ++f)
            tbf[f] = pairh(ld<half4_t>(rf0 + REC_TB + f * FRAG_BYTES), ld<half4_t>(rf1 + REC_TB + f * FRAG_BYTES));
        }
        // S as a bf16 (or fp16) high / low B operand pair: tiles 2kk, 2kk+1
        O4 h0, h1, l0, l1;
        Op::split(s[2 * kk], h0, l0);
        Op::split(s[2 * kk + 1], h1, l1);
        const O8 shi = pair(h0, h1), slo = pair(l0, l1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < 4; ++r) ah[r] = mma(kf[cur][r], shi, ah[r]);
        // (Q S)^T: S^T as the A operand (the B registers of S serve), Q as B
#pragma unroll
        for (int r = 0; r < 4; ++r) aq[r] = mma(shi, qf[cur][r], aq[r]);
#pragma unroll
        for (int r = 0; r < 4; ++r) ah[r] = mma(kf[cur][r], slo, ah[r]);
      }
      float4_t x[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = Op::bits_to_float(vraw[r]) - gam[r] * ah[r];
      // X beyond X_LIMIT anywhere in the tile (a wave vote): scale it into range
      // (range_scale); U, its products and O are restored in fp32 below.
      const bool big = __builtin_amdgcn_ballot_w64(tile_max(x) > X_LIMIT) != 0;
      float down = 1.f;
      if (big) {
        down = range_scale(wave_max(tile_max(x)));
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] *= down;
      }
      // The state update's reads of chunk n (K^T for tokens 0..31, dec, gamma_63)
      // go out before U and the barrier: chunk n has been in LDS since barrier n-1.
      O8 tf[2][NKT];
      const uint32_t tb[KS] = {opaque(km + tr[0]), opaque(km + tr[1]), opaque(km + tr[2]), opaque(km + tr[3])};
#pragma unroll
      for (int t = 0; t < NKT; ++t) tf[0][t] = kt_frag(tb[t >> 1], t & 1, 0);
      float4_t dec[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) dec[r] = ld<float4_t>(rl + SC_DEC + 64 * r);
      const float g63 = ld<float>(rl + SC_GAM + (CH - 1) * 4 - 16 * g4);
      // ---- B: U = Tb X (row tiles 0, 1 one step; 2, 3 two)
      const half8_t xb0 = pairh(to_half4(x[0]), to_half4(x[1]));
      const half8_t xb1 = pairh(to_half4(x[2]), to_half4(x[3]));
      __builtin_amdgcn_sched_barrier(0);
      float4_t u[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) u[r] = mfma32(tbf[frag_index(r, 0)], xb0, float4_t{0.f, 0.f, 0.f, 0.f});
      u[2] = mfma32(tbf[frag_index(2, 1)], xb1, u[2]);
      u[3] = mfma32(tbf[frag_index(3, 1)], xb1, u[3]);
      // ub (U' for O) is taken from the scaled U; the state update uses U itself
      half8_t ub[2];
      ub[0] = pairh(to_half4(u[0]), to_half4(u[1]));
      ub[1] = pairh(to_half4(u[2]), to_half4(u[3]));
      if (big) {
        const float up = 1.f / down;
#pragma unroll
        for (int r = 0; r < 4; ++r) u[r] *= up;
      }
      // barrier n: chunk n+1 is in LDS (each wave waited for its loads; the
      // O stores of chunk n-1, issued after them, may still be in flight),
      // every wave is past chunk n-1
      __builtin_amdgcn_sched_barrier(0);
      wait_vm<OUT_STORES + GATE_LOADS>();
      barrier();
      if (early) issue_chunk(i3, i2);
      // ---- C: S <- gamma_63 S + K^T (dec U), token step ks outermost
#pragma unroll
      for (int t = 0; t < NKT; ++t) tf[1][t] = kt_frag(tb[t >> 1], t & 1, 1);
      O8 dhi[2], dlo[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        O4 h0, h1, l0, l1;
        Op::split(u[2 * ks] * dec[2 * ks], h0, l0);
        Op::split(u[2 * ks + 1] * dec[2 * ks + 1], h1, l1);
        dhi[ks] = pair(h0, h1);
        dlo[ks] = pair(l0, l1);
      }
#pragma unroll
      for (int t = 0; t < NKT; ++t) s[t] *= g63;
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < NKT; ++t) s[t] = mma(tf[0][t], dhi[0], s[t]);
#pragma unroll
      for (int t = 0; t < NKT; ++t) s[t] = mma(tf[0][t], dlo[0], s[t]);
      // O's reads: QKD fragments, scale gamma
      half8_t qkf[6];
#pragma unroll
      for (int f = 0; f < 6; ++f)
        qkf[f] = pairh(ld<half4_t>(rf0 + REC_QKD + f * FRAG_BYTES), ld<half4_t>(rf1 + REC_QKD + f * FRAG_BYTES));
      float gsc[4];
      {
        const uint32_t rg = opaque(rc + REC_SC + SC_GSC + 4 * c16);
#pragma unroll
        for (int r = 0; r < 4; ++r) gsc[r] = ld<float>(rg + 64 * r);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < NKT; ++t) s[t] = mma(tf[1][t], dhi[1], s[t]);
#pragma unroll
      for (int t = 0; t < NKT; ++t) s[t] = mma(tf[1][t], dlo[1], s[t]);
      __builtin_amdgcn_sched_barrier(0);
      if (!early) issue_chunk(i3, i2);
      // ring slots advance: n+1 takes n's successors
      b3 = b3 == 2 ? 0 : b3 + 1;
      b2 ^= 1;
      i3 = i3 == 2 ? 0 : i3 + 1;
      i2 ^= 1;
      // the next chunk's first K and Q fragments (in LDS since barrier n)
      {
        const uint32_t kb = opaque(L::kmat(b3) + xa[0]), qb = opaque(L::qmat(b2) + xa[0]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          kf[0][r] = ld<O8>(kb + 16 * r * L::ROW);
          qf[0][r] = ld<O8>(qb + 16 * r * L::ROW);
        }
      }
      // ---- O^T = (Q S)^T diag(scale gamma) + U^T QKD^T: lane (g, c) holds
      // O[16 r + c][v0 + 4 g .. + 3], stored as one 8-byte piece
      // (with a scaled tile: O = (scale gamma Q S down + U' QKD^T) / down)
      float4_t o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        o[r] = aq[r] * (big ? gsc[r] * down : gsc[r]);
        o[r] = mfma32(ub[0], qkf[frag_index(r, 0)], o[r]);
      }
      o[2] = mfma32(ub[1], qkf[frag_index(2, 1)], o[2]);
      o[3] = mfma32(ub[1], qkf[frag_index(3, 1)], o[3]);
      if (big) {
        const float up = 1.f / down;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] *= up;
      }
      if constexpr (EPI) epilogue(o, graw);
      const long rows = oleft < CH ? oleft : CH;  // >= 1: chunk n holds tokens
      const __amdgpu_buffer_rsrc_t ro = rsrc(op, (rows - 1) * ostride + p.V * static_cast<long>(sizeof(TOut)));
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t off = o_off + 16 * r * static_cast<uint32_t>(ostride);
        if constexpr (sizeof(TOut) == 4) {
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u32_t, o[r]), ro, off, 0, 0);
        } else {
          const O4 x4 = Op::from(o[r]);
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u32_t, x4), ro, off, 0, 0);
        }
      }
      op += CH * ostride;
      oleft -= CH;
      if constexpr (EPI) gp += CH * gstride;
    }
    store_state();
  }
};

// Two waves per SIMD: 256 registers each.
template <int K, typename TIn, typename TOut, bool EPI>
__global__ __launch_bounds__(WNT) __attribute__((amdgpu_waves_per_eu(2, 2))) void wide_kernel(ChunkParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  PBGDN_POISON_LDS(smem_raw, WideLayout<K>::BYTES);
  PBGDN_POISON_SYNC();
  WideBlock<K, TIn, TOut, EPI> blk(smem_raw, p);
  blk.run();
}

}  // namespace

template <int K, typename TIn, typename TOut, bool EPI>
int launch_wide(const ChunkParams &p, hipStream_t stream) {
  static std::atomic<bool> configured[MAX_DEVICES];  // the attribute is set per device
  const size_t smem = WideLayout<K>::BYTES;
  auto kernel = wide_kernel<K, TIn, TOut, EPI>;
  if (EPI && (p.V != WCOLS || !p.gate || !p.o_norm)) return PBGDN_ERR_INVALID_ARGUMENT;
  if (!smem_configured(reinterpret_cast<const void *>(kernel), smem, configured)) return PBGDN_ERR_LAUNCH;
  const long total = static_cast<long>(p.V / WCOLS) * p.Hv * p.num_seqs;
  if (total > 0x7fffffffL) return PBGDN_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(total)), dim3(WNT), smem, stream, p);
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}

template int launch_wide<128, u16, u16, false>(const ChunkParams &, hipStream_t);
template int launch_wide<128, half_t, half_t, false>(const ChunkParams &, hipStream_t);
template int launch_wide<128, u16, u16, true>(const ChunkParams &, hipStream_t);
template int launch_wide<128, u16, float, true>(const ChunkParams &, hipStream_t);
template int launch_wide<128, half_t, half_t, true>(const ChunkParams &, hipStream_t);
template int launch_wide<128, half_t, float, true>(const ChunkParams &, hipStream_t);

}  // namespace pbgdn
