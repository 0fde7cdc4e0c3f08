// Scan kernel of the chunkwise prefill for 256-wide keys (128 < K <= 256, the
// keys zero-padded to 256 by the caller): the state-dependent part, chunk by
// chunk (the serial loop of delta_rule_chunked, pseudobrain/gated_deltanet.py:158-165),
// KH waves (1 or 2) per 16-column tile of the state and WT tiles per
// workgroup.
//
// The arithmetic and the operand layouts are the wide scan's (chunk_wide.hip)
// at twice the keys: the fp32 state tile S [256, 16] is 16 MFMA accumulator
// tiles (64 registers; 8 in each of two waves with key halves) with permuted key rows (row 4g + i of state tile
// 2kk + p holds key 32kk + 8g + 4p + i, so the slots of lane group g in key
// step kk are one contiguous 16-byte piece of a K or Q row), and a chunk step
// runs X -> U -> S and O without leaving the wave:
//   X   = V - diag(gamma) K S        (K rows from LDS, S as a high/low pair)
//   U   = Tb X                       (Tb fragments from the record, X as fp16)
//   S  <- gamma_63 S + K^T (dec U)   (K^T by transposing LDS reads, dec U high/low)
//   O^T = (Q S)^T diag(scale gamma) + U^T QKD^T
//
// What the keys change is the LDS budget. A chunk's K and Q rows take 32 KiB
// each at K = 256, so the wide scan's three K and two Q buffers (231 KiB with
// the records and V) do not fit a CU's 160 KiB. Here K and the record are
// double-buffered and Q and V single-buffered (126-130 KiB; 158 KiB with the
// key-half exchange below), with two
// barriers per step n:
//   top:  chunk n is in LDS; every wave issues its share of the K and record
//         loads of chunk n+1, into the buffers of chunk n-1
//   A:    X and (Q S)^T of chunk n: the step's reads of Q and V
//   mid:  every wave is past its reads of Q and V; the Q and V loads of
//         chunk n+1 are issued into their buffers
//   B, C, O: U, the state update and O of chunk n, O stored; each wave then
//         waits for its loads of chunk n+1 (its O stores stay in flight)
// The loads are direct-to-LDS buffer loads (1 KiB per instruction, no
// registers); rows past the end of a sequence read as zeros (out of the
// resource's range), the identity steps of the reference's padding
// (gated_deltanet.py:127), and so do the record units no scan reads
// (rec_unused_unit).
//
// WT = 2 or 4 tiles (32 or 64 columns per workgroup), one wave per SIMD: the
// LDS allows one workgroup per CU, and a wave holds more registers than two
// waves per SIMD could (eight waves spilled 52 registers). Two tiles spread
// a value head over more workgroups, and so over more CUs, at the price of
// staging the chunk's K and Q rows once per workgroup.
//
// Key halves (KH = 2, with WT = 2: four waves). At one sequence the call has
// only as many tiles as (value head, 16 columns) pairs, 512 at 32 heads of
// 256 columns, and a lone wave per SIMD keeps its MFMA pipe busy a third of
// the time. So each tile can be held by two waves, each owning 128 of the
// keys (8 state tiles): each forms its partial K S and (Q S)^T over its keys,
// writes them to LDS before the mid barrier and adds the other wave's after
// it (one addition, the same in both waves), so both hold the whole X and
// form U; each then updates its own state rows, and each forms and stores
// two of the four row tiles of O. A wave issues 90 MFMAs a step instead of
// 172; the exchange takes 32 KiB of LDS (158 KiB in all).
//
// Inputs and the state operands are 16-bit (bf16 or fp16), o in the inputs'
// type or float32.
#include "chunk.hpp"

namespace pbgdn {
namespace {

constexpr int KW = 256;  // key width of this kernel

typedef unsigned int u32x4_k __attribute__((ext_vector_type(4)));

template <int WT, int KH>
struct K256Layout {
  static constexpr int ROW = 2 * KW;                 // bytes of a staged K or Q row (512)
  static constexpr int MAT = CH * ROW;               // one chunk of K or Q (32 KiB)
  static constexpr int VROW = 32 * WT;               // bytes of a staged V row (16 WT columns, 16-bit)
  static constexpr int VMAT = CH * VROW;
  static constexpr int K_OFF = 0;                    // [2] K
  static constexpr int R_OFF = K_OFF + 2 * MAT;      // [2] record
  static constexpr int Q_OFF = R_OFF + 2 * REC_BYTES;
  static constexpr int V_OFF = Q_OFF + MAT;
  static constexpr int XCH = V_OFF + VMAT;           // KH = 2: [wave][8 fp32 tiles] partial X and (Q S)^T
  static constexpr int BYTES = XCH + (KH == 2 ? WT * KH * 8 * 1024 : 0);
  __device__ static constexpr int kmat(int b) { return K_OFF + b * MAT; }
  __device__ static constexpr int rec(int b) { return R_OFF + b * REC_BYTES; }
};

// Position of 16-byte piece u of K/Q row r is u ^ kswz(r): within the 256
// bytes a bank sweep covers, the pattern of the wide scan's 256-byte rows,
// so its fragment and transposing reads keep their bank spread.
__host__ __device__ constexpr int kswz(int r) { return 4 * (r & 3) + ((r >> 2) & 3); }
// V rows are 32 WT bytes: rows 8 / WT apart share their banks, so the piece
// index is XORed with 2 j for the j-th of the WT rows that do. A transposing
// read of V (8 token rows x 32 bytes per 32 lanes) then touches 32 distinct
// 8-byte positions modulo 256 bytes.
template <int WT>
__host__ __device__ constexpr int vswz_k(int r) {
  static_assert(WT == 2 || WT == 4, "2 or 4 tiles");
  return 2 * ((r >> (WT == 4 ? 1 : 2)) & (WT - 1));
}

template <typename TIn, typename TOut, int WT, int KH>
struct K256Block {
  using L = K256Layout<WT, KH>;
  using Op = OpOf<TIn>;
  using O4 = typename Op::T4;
  using O8 = typename Op::T8;
  static constexpr int WCOLS = 16 * WT;            // value columns per workgroup
  static constexpr int WAVES = WT * KH;            // waves per workgroup
  static constexpr int KPW = KW / KH;              // keys of a wave's state rows
  static constexpr int NKT = KPW / 16;             // state tiles of a wave
  static constexpr int KS = KPW / 32;              // key contraction steps of a wave
  static constexpr int KQ_WAVE = L::MAT / 1024 / WAVES;  // K (or Q) DMA instructions per wave
  static constexpr int NB = 8 / WAVES;             // swizzle classes of a wave's K/Q instructions
  static constexpr int DMA_REC = REC_BYTES / 1024;
  static constexpr int V_WAVE = L::VMAT / 1024 / WAVES;  // V DMA instructions per wave
  static constexpr int VRPI = 1024 / L::VROW;      // V rows per DMA instruction
  static constexpr int OROWS = 4 / KH;             // O row tiles a wave forms and stores
  static constexpr int OUT_STORES = OROWS;         // O stores a wave issues per chunk
  static_assert((WT == 2 || WT == 4) && (KH == 1 || (KH == 2 && WT == 2)), "2 or 4 waves, or 2 x 2 key halves");
  static_assert(sizeof(TIn) == 2, "16-bit inputs (staged as they are)");
  static_assert(L::BYTES <= 160 * 1024, "LDS");
  static_assert(REC_BYTES % 1024 == 0 && L::VMAT % (1024 * WAVES) == 0 && V_WAVE * KH == 2, "whole DMA instructions");

  unsigned char *lds;
  const ChunkParams &p;
  int lane, c16, g4, wave, tile, kh, h, hk, col0, v0, seq;
  long bos, eos, nchunks;
  float4_t s[NKT];  // the state tile, accumulator layout, permuted key rows

  uint32_t xa[KS];  // K/Q row fragment of row tile 0, step kk (add 16 * ROW * r)
  uint32_t tr[KS];  // K^T transposing read of state tiles 2kk + p (add 8 p), tokens 4g.. (add ROW * token)
  uint32_t vtr;     // V transposing read of row tile 0 (add 16 * VROW * r)
  uint32_t tbo0, tbo1;   // the two 8-byte halves of a Tb / QKD fragment row this lane reads
  uint32_t o_off;        // O: byte offset of this lane's piece (token c, columns v0 + 4g..) within a chunk
  uint32_t dma_kq[NB];   // source offsets of this lane's piece of the wave's K/Q instructions, by class
  uint32_t dma_v;        // same for V
  // The next chunk to stage: its first K/Q row, V row (column col0), record,
  // and the tokens left from it.
  const unsigned char *kp, *qp, *vp, *rp;
  long left;

  __device__ __forceinline__ K256Block(unsigned char *l, const ChunkParams &prm) : lds(l), p(prm) {
    const int tid = threadIdx.x;
    lane = tid & 63;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    tile = wave % WT;  // the 16-column tile of this wave
    kh = wave / WT;    // and its half of the keys (KH = 2)
    c16 = lane & 15;
    g4 = lane >> 4;
    // Block -> (sequence, value head, column group); the column groups and the
    // value heads of one key head of one sequence share K/Q rows and stay on
    // one XCD (xcd_group).
    const int groups = p.V / WCOLS;
    const int per_key = groups * (p.Hv / p.Hk);
    const int total = static_cast<int>(gridDim.x);
    int kgrp, member;
    xcd_group(static_cast<int>(blockIdx.x), total / per_key, per_key, p.xcds, kgrp, member);
    seq = kgrp / p.Hk;
    hk = kgrp % p.Hk;
    h = hk * (p.Hv / p.Hk) + member / groups;
    col0 = (member % groups) * WCOLS;
    v0 = col0 + 16 * tile;
    seq_bounds(p, seq, bos, eos);
    nchunks = (eos - bos + CH - 1) / CH;

    const int k = c16 >> 2, q = c16 & 3;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int kp = kk + KS * kh;  // the key step within the whole row
      xa[kk] = c16 * L::ROW + ((4 * kp + g4) ^ kswz(c16)) * 16;  // row c, piece 4kp + g
      // lane 4k + q of group g: token row 4g + k, keys 32kp + 8q + 4p (piece 4kp + q, half p)
      tr[kk] = (4 * g4 + k) * L::ROW + ((4 * kp + q) ^ kswz(4 * g4 + k)) * 16;
    }
    // lane 4k + q of group g: token row 4g + k, columns 16 tile + 4q.. (piece 2 tile + q/2, half q & 1)
    vtr = (4 * g4 + k) * L::VROW + (((2 * tile + (q >> 1)) ^ vswz_k<WT>(4 * g4 + k)) * 16) + 8 * (q & 1);
    // Tb / QKD fragment rows: tokens 32kk + 4g.. (fragment lane (g/2, c), half
    // g&1) and 32kk + 16 + 4g.. (lane (2 + g/2, c))
    tbo0 = (16 * (g4 >> 1) + c16) * 16 + 8 * (g4 & 1);
    tbo1 = (16 * (2 + (g4 >> 1)) + c16) * 16 + 8 * (g4 & 1);
    o_off = (c16 * p.Hv * p.V + v0 + 4 * g4) * static_cast<uint32_t>(sizeof(TOut));
    // K/Q instruction i covers token rows 2i, 2i+1: lane l fills row 2i + l/32
    // at position l%32 (piece (l%32) ^ kswz(row)). This wave's are i = wave +
    // WAVES s, rows 2 wave + 2 WAVES s + l/32: instructions 8 apart (s NB
    // apart) are 16 rows apart and share a swizzle, so class j = s % NB holds
    // the offset of s = j and the others add 16 rows per NB.
    const uint32_t kqs = static_cast<uint32_t>(p.Hk) * KW * 2;  // bytes per token row of k, q
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int r = 2 * wave + 2 * WAVES * j + (lane >> 5);
      dma_kq[j] = static_cast<uint32_t>(r) * kqs + ((lane & 31) ^ kswz(r)) * 16;
    }
    // V instruction i covers VRPI rows of 2 WT pieces: lane l fills row
    // VRPI i + l / (2 WT) at position l % (2 WT); this wave's i = wave (and
    // wave + WT when KH = 1: 32 rows on, the same swizzle).
    const int rv = wave * VRPI + lane / (2 * WT);
    dma_v = static_cast<uint32_t>(rv) * p.Hv * p.V * 2 + ((lane % (2 * WT)) ^ vswz_k<WT>(rv)) * 16;
    const long kq0 = (bos * p.Hk + hk) * static_cast<long>(KW) * 2;
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
  // Raw buffer descriptor: base, stride 0, byte range, RSRC_WORD3.
  __device__ __forceinline__ static u32x4_k desc(const void *base, long bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return u32x4_k{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xffffu,
                   static_cast<uint32_t>(bytes > 0 ? bytes : 0), static_cast<uint32_t>(RSRC_WORD3)};
  }
  // One direct-to-LDS load: 16 bytes per lane from `off` to LDS lds_off +
  // 16 lane. Assembly, so that the compiler does not wait for it before later
  // LDS reads it cannot tell apart; the waits are the explicit ones (wait_vm).
  __device__ __forceinline__ void dma(const u32x4_k &rs, uint32_t lds_off, uint32_t off) const {
    typedef __attribute__((address_space(3))) unsigned char lds_byte;
    const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_byte *)(lds + lds_off)));  // C-style: an address-space cast
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0), "v"(off), "s"(rs)
                 : "memory", "m0");
  }

  // ------------------------------------------------------------------ loads
  __device__ __forceinline__ long next_rows() const { return left <= 0 ? 0 : (left < CH ? left : CH); }
  // This wave's loads of the next chunk's K rows and record into buffer b.
  __device__ __forceinline__ void issue_kr(int b) const {
    const long rows = next_rows();
    const long kqs = static_cast<long>(p.Hk) * KW * 2;
    const u32x4_k rk = desc(kp, rows > 0 ? (rows - 1) * kqs + KW * 2 : 0);
    const u32x4_k rr = desc(rp, rows > 0 ? REC_BYTES : 0);
#pragma unroll
    for (int s_ = 0; s_ < KQ_WAVE; ++s_) {
      const uint32_t off = dma_kq[s_ % NB] + static_cast<uint32_t>(16 * (s_ / NB)) * static_cast<uint32_t>(kqs);
      dma(rk, L::kmat(b) + 1024 * (wave + WAVES * s_), off);
    }
#pragma unroll
    for (int s_ = 0; s_ < (DMA_REC + WAVES - 1) / WAVES; ++s_) {
      const int i = wave + WAVES * s_;
      const uint32_t roff = 1024 * i + lane * 16;  // units no scan reads: an out-of-range load stages zeros
      if (i < DMA_REC) dma(rr, L::rec(b) + 1024 * i, rec_unused_unit(static_cast<int>(roff)) ? OUT_OF_RANGE : roff);
    }
  }
  // This wave's loads of the next chunk's Q rows and V columns.
  __device__ __forceinline__ void issue_qv() const {
    const long rows = next_rows();
    const long kqs = static_cast<long>(p.Hk) * KW * 2, vs = static_cast<long>(p.Hv) * p.V * 2;
    const u32x4_k rq = desc(qp, rows > 0 ? (rows - 1) * kqs + KW * 2 : 0);
    const u32x4_k rv = desc(vp, rows > 0 ? (rows - 1) * vs + WCOLS * 2 : 0);
#pragma unroll
    for (int s_ = 0; s_ < KQ_WAVE; ++s_) {
      const uint32_t off = dma_kq[s_ % NB] + static_cast<uint32_t>(16 * (s_ / NB)) * static_cast<uint32_t>(kqs);
      dma(rq, L::Q_OFF + 1024 * (wave + WAVES * s_), off);
    }
#pragma unroll
    for (int s_ = 0; s_ < V_WAVE; ++s_) {
      dma(rv, L::V_OFF + 1024 * (wave + WAVES * s_), dma_v + static_cast<uint32_t>(32 * s_) * static_cast<uint32_t>(vs));
    }
  }
  __device__ __forceinline__ void advance() {
    const long kqs = static_cast<long>(p.Hk) * KW * 2, vs = static_cast<long>(p.Hv) * p.V * 2;
    kp += CH * kqs;
    qp += CH * kqs;
    vp += CH * vs;
    rp += static_cast<long>(p.Hv) * REC_BYTES;
    left -= CH;
  }

  // ------------------------------------------------------------------ state I/O
  // Lane (g, c) holds rows 4g + i of state tile t = 2kk + p: key KPW kh + 32kk + 8g + 4p + i.
  __device__ __forceinline__ int key_of(int t, int i) const {
    return KPW * kh + 32 * (t >> 1) + 8 * g4 + 4 * (t & 1) + i;
  }
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
        s[t][i] = any ? load_elem(p.h0, ((slot * p.Hv + h) * KW + key_of(t, i)) * static_cast<long>(p.V) + v0 + c16,
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
        store_elem(p.ht, ((slot * p.Hv + h) * KW + key_of(t, i)) * static_cast<long>(p.V) + v0 + c16, p.state_dtype,
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
  // K^T operand of state tile t = 2kk + pp for tokens 32 ks .. + 31, from the
  // lane base tb = K buffer + tr[kk]
  __device__ __forceinline__ O8 kt_frag(uint32_t tb, int pp, int ks) const {
    const uint32_t base = tb + 8 * pp + (32 * ks) * L::ROW;
    const i16x4_t lo4 = ld_tr(base);
    const i16x4_t hi4 = ld_tr(base + 16 * L::ROW);
    return __builtin_bit_cast(O8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
  }

  // Workgroup barrier; the fences keep LDS accesses on their side (it waits
  // for LDS operations, not for the loads in flight).
  __device__ __forceinline__ void barrier() const {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  }
  // Wait until at most VM of this wave's vector memory operations are
  // outstanding (they complete in issue order: the newest VM stay in flight).
  template <int VM>
  __device__ __forceinline__ void wait_vm() const {
    static_assert(VM >= 0 && VM < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((VM & 0xF) | (0x7 << 4) | (0xF << 8) | (((VM >> 4) & 3) << 14));
  }
  // An LDS byte address the compiler treats as unknown, so that the reads
  // built on it fold their constant parts into the instruction's offset.
  __device__ __forceinline__ static uint32_t opaque(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
  }

  __device__ __forceinline__ void run() {
    load_state();
    if (nchunks <= 0) {
      store_state();
      return;
    }
    issue_kr(0);
    issue_qv();
    advance();
    wait_vm<0>();
    barrier();
    // O: chunk n's first row of this value head
    unsigned char *op = static_cast<unsigned char *>(p.o) + ((bos * p.Hv + h) * static_cast<long>(p.V)) * sizeof(TOut);
    const long ostride = static_cast<long>(p.Hv) * p.V * sizeof(TOut);  // bytes per token row
    long oleft = eos - bos;
    for (long n = 0; n < nchunks; ++n) {
      const int b = static_cast<int>(n & 1);
      issue_kr(b ^ 1);  // chunk n+1 (zero-size resources past the end)
      const uint32_t km = L::kmat(b), rc = L::rec(b);
      const uint32_t rl = opaque(rc + REC_SC + 16 * g4);  // gamma, dec rows 4g..: + 64 r (+ table)
      const uint32_t rf0 = opaque(rc + tbo0), rf1 = opaque(rc + tbo1);
      // ---- A: X = V - gamma K S and (Q S)^T for the 4 row tiles, contraction
      // step kk outermost; step kk+1's operands (after the last step, those of
      // X and U) are read before step kk's products
      float4_t ah[4], aq[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) ah[r] = aq[r] = float4_t{0.f, 0.f, 0.f, 0.f};
      O8 kf[2][4], qf[2][4];
      {
        const uint32_t kb = opaque(km + xa[0]), qb = opaque(L::Q_OFF + xa[0]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          kf[0][r] = ld<O8>(kb + 16 * r * L::ROW);
          qf[0][r] = ld<O8>(qb + 16 * r * L::ROW);
        }
      }
      i16x4_t vraw[4];
      float4_t gam[4];
      half8_t tbf[6];
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const int cur = kk & 1;
        if (kk + 1 < KS) {
          const uint32_t kb = opaque(km + xa[kk + 1]), qb = opaque(L::Q_OFF + xa[kk + 1]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            kf[cur ^ 1][r] = ld<O8>(kb + 16 * r * L::ROW);
            qf[cur ^ 1][r] = ld<O8>(qb + 16 * r * L::ROW);
          }
        } else {
          const uint32_t vb = opaque(L::V_OFF + vtr);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            vraw[r] = ld_tr(vb + 16 * r * L::VROW);
            gam[r] = ld<float4_t>(rl + SC_GAM + 64 * r);
          }
#pragma unroll
          for (int f = 0; f < 6; ++f)
            tbf[f] = pairh(ld<half4_t>(rf0 + REC_TB + f * FRAG_BYTES), ld<half4_t>(rf1 + REC_TB + f * FRAG_BYTES));
        }
        // S as a high / low B operand pair: tiles 2kk, 2kk+1
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
      // KH = 2: this wave's partial K S and (Q S)^T (its half of the keys) to
      // LDS for the other wave of its tile
      const uint32_t xw = L::XCH + static_cast<uint32_t>(wave) * 8192 + lane * 16;
      if constexpr (KH == 2) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          *reinterpret_cast<float4_t *>(lds + xw + 1024 * r) = ah[r];
          *reinterpret_cast<float4_t *>(lds + xw + 1024 * (4 + r)) = aq[r];
        }
      }
      // mid: the step's reads of Q and V are done in every wave, and the
      // partials are in LDS; chunk n+1's Q and V go into the same buffers
      __builtin_amdgcn_sched_barrier(0);
      barrier();
      issue_qv();
      advance();
      if constexpr (KH == 2) {  // whole sums over the keys (one addition: the same in both waves)
        const uint32_t xo = L::XCH + static_cast<uint32_t>(tile + WT * (1 - kh)) * 8192 + lane * 16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          ah[r] += ld<float4_t>(xo + 1024 * r);
          aq[r] += ld<float4_t>(xo + 1024 * (4 + r));
        }
      }
      float4_t x[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = Op::bits_to_float(vraw[r]) - gam[r] * ah[r];
      // X beyond X_LIMIT anywhere in the tile (a wave vote): scale it into
      // range (range_scale); U, its products and O are restored in fp32 below.
      const bool big = __builtin_amdgcn_ballot_w64(tile_max(x) > X_LIMIT) != 0;
      float down = 1.f;
      if (big) {
        down = range_scale(wave_max(tile_max(x)));
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] *= down;
      }
      float4_t dec[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) dec[r] = ld<float4_t>(rl + SC_DEC + 64 * r);
      const float g63 = ld<float>(rl + SC_GAM + (CH - 1) * 4 - 16 * g4);
      uint32_t tb[KS];
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) tb[kk] = opaque(km + tr[kk]);
      // K^T fragments in groups of 8 state tiles: group j = (token step
      // j / GPS, tiles 8 (j % GPS) ..), group j+1 read while group j multiplies
      constexpr int GPS = NKT / 8, NG = 2 * GPS;
      O8 tf[2][8];
#pragma unroll
      for (int i = 0; i < 8; ++i) tf[0][i] = kt_frag(tb[i >> 1], i & 1, 0);
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
      // ---- C: S <- gamma_63 S + K^T (dec U)
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
#pragma unroll
      for (int j = 0; j < NG; ++j) {
        const int cur = j & 1;
        if (j + 1 < NG) {
          const int ks = (j + 1) / GPS, t0 = 8 * ((j + 1) % GPS);
#pragma unroll
          for (int i = 0; i < 8; ++i) tf[cur ^ 1][i] = kt_frag(tb[(t0 + i) >> 1], (t0 + i) & 1, ks);
        }
        __builtin_amdgcn_sched_barrier(0);
        const int ks = j / GPS, t0 = 8 * (j % GPS);
#pragma unroll
        for (int i = 0; i < 8; ++i) s[t0 + i] = mma(tf[cur][i], dhi[ks], s[t0 + i]);
#pragma unroll
        for (int i = 0; i < 8; ++i) s[t0 + i] = mma(tf[cur][i], dlo[ks], s[t0 + i]);
      }
      // ---- O^T = (Q S)^T diag(scale gamma) + U^T QKD^T: lane (g, c) holds
      // O[16 r + c][v0 + 4 g .. + 3], stored as one piece
      // (with a scaled tile: O = (scale gamma Q S down + U' QKD^T) / down)
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
      const long rows = oleft < CH ? oleft : CH;  // >= 1: chunk n holds tokens
      const __amdgpu_buffer_rsrc_t ro = rsrc(op, (rows - 1) * ostride + p.V * static_cast<long>(sizeof(TOut)));
      const float up = 1.f / down;
      auto o_row = [&](auto rconst) {  // row tile r of O, formed and stored
        constexpr int r = decltype(rconst)::value;
        float4_t o = aq[r] * (big ? gsc[r] * down : gsc[r]);
        o = mfma32(ub[0], qkf[frag_index(r, 0)], o);
        if constexpr (r >= 2) o = mfma32(ub[1], qkf[frag_index(r, 1)], o);
        if (big) o *= up;
        const uint32_t off = o_off + 16 * r * static_cast<uint32_t>(ostride);
        if constexpr (sizeof(TOut) == 4) {
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u32_t, o), ro, off, 0, 0);
        } else {
          const O4 x4 = Op::from(o);
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u32_t, x4), ro, off, 0, 0);
        }
      };
      using R0 = std::integral_constant<int, 0>;
      using R1 = std::integral_constant<int, 1>;
      using R2 = std::integral_constant<int, 2>;
      using R3 = std::integral_constant<int, 3>;
      if constexpr (KH == 1) {
        o_row(R0{});
        o_row(R1{});
        o_row(R2{});
        o_row(R3{});
      } else if (kh == 0) {  // the two waves of a tile split its rows
        o_row(R0{});
        o_row(R1{});
      } else {
        o_row(R2{});
        o_row(R3{});
      }
      op += CH * ostride;
      oleft -= CH;
      // top of n+1: this wave's loads of chunk n+1 are in LDS (its O stores,
      // issued after them, may still be in flight), and every wave's are
      // after the barrier; every wave is past chunk n's reads
      __builtin_amdgcn_sched_barrier(0);
      wait_vm<OUT_STORES>();
      barrier();
    }
    store_state();
  }
};

// One workgroup per CU (the LDS), one wave per SIMD (512 registers).
template <typename TIn, typename TOut, int WT, int KH>
__global__ __launch_bounds__(64 * WT * KH) __attribute__((amdgpu_waves_per_eu(1, 1))) void k256_kernel(ChunkParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  PBGDN_POISON_LDS(smem_raw, (K256Layout<WT, KH>::BYTES));
  PBGDN_POISON_SYNC();
  K256Block<TIn, TOut, WT, KH> blk(smem_raw, p);
  blk.run();
}

template <typename TIn, typename TOut, int WT, int KH>
int launch_k256_wt(const ChunkParams &p, hipStream_t stream) {
  static std::atomic<bool> configured[MAX_DEVICES];  // the attribute is set per device
  const size_t smem = K256Layout<WT, KH>::BYTES;
  auto kernel = k256_kernel<TIn, TOut, WT, KH>;
  if (!smem_configured(reinterpret_cast<const void *>(kernel), smem, configured)) return PBGDN_ERR_LAUNCH;
  const long total = static_cast<long>(p.V / (16 * WT)) * p.Hv * p.num_seqs;
  if (total > 0x7fffffffL) return PBGDN_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(total)), dim3(64 * WT * KH), smem, stream, p);
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}

}  // namespace

// Waves per workgroup of a call: 4 when they divide V into column groups
// and the workgroups still cover the CUs, else 2.
int k256_waves(int V, long pairs_of_seq_and_head, int cus) {
  return V % 64 == 0 && pairs_of_seq_and_head * (V / 64) >= cus ? 4 : 2;
}

template <typename TIn, typename TOut>
int launch_k256(const ChunkParams &p, int wt, int kh, hipStream_t stream) {
  if (p.V % (16 * wt) != 0) return PBGDN_ERR_UNSUPPORTED;
  if (wt == 4 && kh == 1) return launch_k256_wt<TIn, TOut, 4, 1>(p, stream);
  if (wt == 2 && kh == 1) return launch_k256_wt<TIn, TOut, 2, 1>(p, stream);
  if (wt == 2 && kh == 2) return launch_k256_wt<TIn, TOut, 2, 2>(p, stream);
  return PBGDN_ERR_UNSUPPORTED;
}

template int launch_k256<u16, u16>(const ChunkParams &, int, int, hipStream_t);
template int launch_k256<u16, float>(const ChunkParams &, int, int, hipStream_t);
template int launch_k256<half_t, half_t>(const ChunkParams &, int, int, hipStream_t);
template int launch_k256<half_t, float>(const ChunkParams &, int, int, hipStream_t);

}  // namespace pbgdn
