// Wide scan kernel of the chunkwise prefill: the state-dependent part, chunk by
// chunk (the serial loop of delta_rule_chunked, pseudobrain/gated_deltanet.py:158-165),
// with one wave per 16-column tile of the state and WT tiles per workgroup.
//
// Why wide. A chunk step needs the chunk's K and Q rows (16 KiB each at K = 128)
// and its workspace record (13 KiB) in LDS, and one CU stages at most ~25 bytes
// per clock from L2 (measured with direct-to-LDS loads, also with a single CU
// per XCD loading). A workgroup that owns one 16-column tile pays that fill for
// 16 columns of work; here the WT waves of a workgroup own WT tiles of one
// (sequence, value head) and share every byte staged.
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
//
// Staging. A chunk's K and Q rows (16-bit, 256 bytes at K = 128), its record
// and the workgroup's 64 V columns are copied HBM -> LDS by direct-to-LDS
// buffer loads (each wave moves 1 KiB per instruction, no registers). Rows
// past the end of a sequence read as zeros (out of the buffer resource's
// range): the identity steps of the reference's padding (gated_deltanet.py:127).
// K and the record, read in phases A to C, rotate through three buffers; Q and
// V, read in phase A only, through two. The 16-byte pieces of a K/Q row sit at
// piece ^ f(row & 15), f(x) = 4 (x & 3) + (x >> 2), and those of a 128-byte V
// row at piece ^ 2 ((row >> 1) & 1): the row-fragment reads (16 rows, one
// piece each) and the transposing reads (4 rows x 4 pieces per 16 lanes) then
// hit distinct bank positions. O is formed transposed (O^T = (Q S)^T diag +
// U^T QKD^T, the same registers as A and B operands swapped), so each lane
// holds 4 contiguous columns of one token row: it goes to a double-buffered
// LDS tile (pieces at u ^ ((row >> 1) & 7)) and out as whole 128-byte rows.
//
// Step n of a workgroup (one barrier):
//   A: X and Q S of chunk n; B: U; then every wave waits for its loads of
//   chunk n+1, barrier; O of chunk n-1 goes out; loads of chunk n+2 are issued
//   (into buffers chunk n-1, or for Q and V chunk n, used); C: the state update
//   and O of chunk n into the O tile.
// Vector memory operations per wave and chunk: 14 or 15 DMA loads and the O
// row stores; the issue path of a CU, not its MFMA or LDS pipes, set the pace
// of the first version, which loaded V and stored O two bytes per lane.
#include "chunk.hpp"

namespace pbgdn {
namespace {

constexpr int WT = 4;          // 16-column tiles per workgroup, one compute wave each
constexpr int WNT = 64 * WT;   // compute threads; as many loader threads follow
constexpr int WALL = 2 * WNT;  // threads per workgroup

typedef unsigned int u32x4_t_ __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ T out_elem_(float x);
template <>
__device__ __forceinline__ u16 out_elem_<u16>(float x) { return __builtin_bit_cast(u16, static_cast<bf16_t>(x)); }
template <>
__device__ __forceinline__ half_t out_elem_<half_t>(float x) { return static_cast<half_t>(x); }
template <>
__device__ __forceinline__ float out_elem_<float>(float x) { return x; }

template <int K, typename TOut>
struct WideLayout {
  static constexpr int ROW = 2 * K;                  // bytes of a staged K or Q row
  static constexpr int MAT = CH * ROW;               // one of K, Q
  static constexpr int VROW = 64 * 2;                // bytes of a staged V row (64 columns, 16-bit)
  static constexpr int VMAT = CH * VROW;
  static constexpr int OROW = 64 * static_cast<int>(sizeof(TOut));
  static constexpr int OMAT = CH * OROW;
  static constexpr int K_OFF = 0;                            // [3] K
  static constexpr int Q_OFF = K_OFF + 3 * MAT;              // [2] Q
  static constexpr int R_OFF = Q_OFF + 2 * MAT;              // [3] record
  static constexpr int V_OFF = R_OFF + 3 * REC_BYTES;        // [2] V
  static constexpr int O_OFF = V_OFF + 2 * VMAT;             // [2] O
  static constexpr int BYTES = O_OFF + 2 * OMAT;
  __device__ static constexpr int kmat(int b3) { return K_OFF + b3 * MAT; }
  __device__ static constexpr int qmat(int b2) { return Q_OFF + b2 * MAT; }
  __device__ static constexpr int rec(int b3) { return R_OFF + b3 * REC_BYTES; }
  __device__ static constexpr int vmat(int b2) { return V_OFF + b2 * VMAT; }
  __device__ static constexpr int omat(int b2) { return O_OFF + b2 * OMAT; }
};

// Position of 16-byte piece u of K/Q row r is u ^ swz(r) (K = 128: 16 pieces a
// row); of V row r, u ^ vswz(r) (8 pieces).
__host__ __device__ constexpr int swz(int r) { return 4 * (r & 3) + ((r >> 2) & 3); }
__host__ __device__ constexpr int vswz(int r) { return 2 * ((r >> 1) & 1); }
// O tile rows (64 16-bit columns, 8 pieces): piece u of row r sits at u ^ oswz(r).
__host__ __device__ constexpr int oswz(int r) { return (r >> 1) & 7; }

template <int K, typename TIn, typename TOut>
struct WideBlock {
  using L = WideLayout<K, TOut>;
  using Op = OpOf<TIn>;
  using O4 = typename Op::T4;
  using O8 = typename Op::T8;
  static constexpr int NKT = K / 16;   // state tiles
  static constexpr int KS = K / 32;    // key contraction steps
  static constexpr int DMA_KQ = L::MAT / 1024;        // 1 KiB DMA instructions per K or Q matrix
  static constexpr int DMA_REC = REC_BYTES / 1024;
  static constexpr int DMA_V = L::VMAT / 1024;
  static constexpr int OUT_UNITS = L::OMAT / 16 / WNT; // 16-byte O pieces per loader thread and chunk
  // vector memory operations a wave issues after a chunk's loads: its O row stores
  static constexpr int OUT_STORES = OUT_UNITS;
  static_assert(K == 128, "the wide scan is built for K = 128");
  static_assert(REC_BYTES % 1024 == 0 && DMA_KQ % WT == 0 && DMA_V % WT == 0, "whole DMA instructions per wave");
  static_assert(sizeof(TIn) == 2 && sizeof(TOut) == 2, "16-bit inputs (staged as they are) and outputs");
  static_assert(L::BYTES <= 160 * 1024, "LDS");

  unsigned char *lds;
  const ChunkParams &p;
  int lane, c16, g4, wave, h, hk, col0, v0, seq;
  bool compute;  // compute wave (tile `wave`) or loader wave (loader index `wave`)
  long bos, eos;
  long nchunks;
  float4_t s[NKT];  // the state tile, accumulator layout, permuted key rows

  uint32_t xa[KS];   // K/Q row fragment of row tile 0, step kk (add 16 * ROW * r)
  uint32_t tr[KS];   // K^T transposing read of state tiles 2kk + p (add 8 p), tokens 4g.. (add ROW * token)
  uint32_t vtr;      // V transposing read of row tile 0 (add 16 * VROW * r)
  uint32_t tbo0, tbo1;  // the two 8-byte halves of a Tb / QKD fragment row this lane reads

  __device__ __forceinline__ WideBlock(unsigned char *l, const ChunkParams &prm) : lds(l), p(prm) {
    const int tid = threadIdx.x;
    lane = tid & 63;
    compute = tid < WNT;
    wave = __builtin_amdgcn_readfirstlane((tid >> 6) % WT);
    c16 = lane & 15;
    g4 = lane >> 4;
    // Block -> (sequence, value head, column group): the column groups and the
    // value heads of one key head of one sequence share their K/Q rows; keep
    // them on one XCD (blocks go round-robin over the 8 XCDs).
    const int groups = p.V / (16 * WT);
    const int per_key = groups * (p.Hv / p.Hk);
    const int total = static_cast<int>(gridDim.x);
    const int L_ = static_cast<int>(blockIdx.x);
    int kgrp, member;
    if ((total / per_key) % 8 == 0) {
      kgrp = ((L_ >> 3) / per_key) * 8 + (L_ & 7);
      member = (L_ >> 3) % per_key;
    } else {
      kgrp = L_ / per_key;
      member = L_ % per_key;
    }
    seq = kgrp / p.Hk;
    hk = kgrp % p.Hk;
    h = hk * (p.Hv / p.Hk) + member / groups;
    col0 = (member % groups) * (16 * WT);
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
  // waits here are the explicit ones in sync_all().
  __device__ __forceinline__ void dma(const u32x4_t_ &r, uint32_t lds_off, uint32_t off) const {
    typedef __attribute__((address_space(3))) unsigned char lds_byte;
    const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_byte *)(lds + lds_off)));  // C-style: an address-space cast
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0), "v"(off), "s"(r)
                 : "memory", "m0");
  }

  // ------------------------------------------------------------------ loads
  __device__ __forceinline__ long rows_of(long n) const {
    const long left = eos - (bos + n * CH);
    return left <= 0 ? 0 : (left < CH ? left : CH);
  }

  // Per-lane offsets of the loader waves.
  struct LoaderLanes {
    uint32_t kq;  // source offset of this lane's piece of K/Q DMA instruction `wave` within a chunk's rows
    uint32_t v;   // same for the V tile
    uint32_t o_lds[OUT_UNITS], o_glb[OUT_UNITS];  // O row pieces this thread stores: LDS and global offsets
  };
  __device__ __forceinline__ LoaderLanes loader_lanes() const {
    LoaderLanes ll;
    // K/Q DMA instruction i covers rows 4i..4i+3, lane l filling row 4i + l/16
    // at position l%16 (piece (l%16) ^ swz(row)); this wave's are i = wave +
    // WT s, rows 16 s + 4 wave + l/16.
    const int r = 4 * wave + (lane >> 4);
    ll.kq = static_cast<uint32_t>(r) * p.Hk * K * 2 + ((lane & 15) ^ swz(r)) * 16;
    // V DMA instruction i covers rows 8i..8i+7 (8 pieces a row); this wave's
    // are i = wave + WT s, rows 32 s + 8 wave + l/8.
    const int rv = 8 * wave + (lane >> 3);
    ll.v = static_cast<uint32_t>(rv) * p.Hv * p.V * 2 + ((lane & 7) ^ vswz(rv)) * 16;
    constexpr int upr = L::OROW / 16;  // O pieces a row
#pragma unroll
    for (int u = 0; u < OUT_UNITS; ++u) {
      const int w = (static_cast<int>(threadIdx.x) - WNT) + WNT * u;
      ll.o_lds[u] = (w / upr) * L::OROW + (((w % upr) ^ oswz(w / upr)) * 16);
      ll.o_glb[u] = ((w / upr) * p.Hv * p.V) * static_cast<uint32_t>(sizeof(TOut)) + (w % upr) * 16;
    }
    return ll;
  }

  // Direct-to-LDS loads of chunk n (zero-size resources past the stream's end):
  // K and the record into ring slot n % 3, Q and V into slot n % 2.
  __device__ __forceinline__ void issue_chunk(const LoaderLanes &ll, long n) const {
    const long rows = n < nchunks ? rows_of(n) : 0;
    const long t0 = rows > 0 ? bos + n * CH : 0;
    const long kqb = rows > 0 ? ((rows - 1) * p.Hk * K + K) * 2L : 0;
    const long base = (t0 * p.Hk + hk) * static_cast<long>(K);
    const u32x4_t_ rk = desc(static_cast<const TIn *>(p.k) + base, kqb);
    const u32x4_t_ rq = desc(static_cast<const TIn *>(p.q) + base, kqb);
    const long vb = rows > 0 ? ((rows - 1) * p.Hv * p.V + 64) * 2L : 0;
    const u32x4_t_ rv = desc(static_cast<const TIn *>(p.v) + (t0 * p.Hv + h) * static_cast<long>(p.V) + col0, vb);
    const unsigned char *rp = rows > 0 ? p.ws + ((rec_base(bos, seq) + n) * p.Hv + h) * static_cast<long>(REC_BYTES)
                                       : p.ws;
    const u32x4_t_ rr = desc(rp, rows > 0 ? REC_BYTES : 0);
    const int b3 = static_cast<int>(n % 3), b2 = static_cast<int>(n & 1);
#pragma unroll
    for (int s_ = 0; s_ < DMA_KQ / WT; ++s_) {
      const int i = wave + WT * s_;
      const uint32_t off = ll.kq + static_cast<uint32_t>(16 * s_) * p.Hk * K * 2;
      dma(rk, L::kmat(b3) + 1024 * i, off);
      dma(rq, L::qmat(b2) + 1024 * i, off);
    }
#pragma unroll
    for (int s_ = 0; s_ < DMA_V / WT; ++s_) {
      const int i = wave + WT * s_;
      dma(rv, L::vmat(b2) + 1024 * i, ll.v + static_cast<uint32_t>(32 * s_) * p.Hv * p.V * 2);
    }
#pragma unroll
    for (int s_ = 0; s_ < (DMA_REC + WT - 1) / WT; ++s_) {
      const int i = wave + WT * s_;
      if (i < DMA_REC) dma(rr, L::rec(b3) + 1024 * i, 1024 * i + lane * 16);
    }
  }

  // O of chunk n from the O tile (slot n & 1) to HBM as 16-byte row pieces;
  // rows past the end are dropped by the resource's range.
  __device__ __forceinline__ void store_out(const LoaderLanes &ll, long n) const {
    const long rows = n >= 0 ? rows_of(n) : 0;  // n < 0: the same stores with a zero-size resource
    const long t0 = bos + n * CH;
    const long bytes = rows > 0 ? ((rows - 1) * p.Hv * p.V + 64) * static_cast<long>(sizeof(TOut)) : 0;
    const __amdgpu_buffer_rsrc_t ro =
        rsrc(static_cast<TOut *>(p.o) + (rows > 0 ? (t0 * p.Hv + h) * static_cast<long>(p.V) + col0 : 0), bytes);
    const int ob = static_cast<int>(n & 1);
#pragma unroll
    for (int u = 0; u < OUT_UNITS; ++u) {
      const uint4 x = ld<uint4>(L::omat(ob) + ll.o_lds[u]);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t_, x), ro, ll.o_glb[u], 0, 0);
    }
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
  // 8 fp16 of a Tb / QKD fragment row in slot order (two 8-byte halves)
  __device__ __forceinline__ half8_t frag(uint32_t base) const {
    return pairh(ld<half4_t>(base + tbo0), ld<half4_t>(base + tbo1));
  }
  // K^T operand of state tile t = 2kk + pp for tokens 32 ks .. + 31
  __device__ __forceinline__ O8 kt_frag(uint32_t km, int kk, int pp, int ks) const {
    const uint32_t base = km + tr[kk] + 8 * pp + (32 * ks) * L::ROW;
    const i16x4_t lo4 = ld_tr(base);
    const i16x4_t hi4 = ld_tr(base + 16 * L::ROW);
    return __builtin_bit_cast(O8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
  }

  // Workgroup barrier; the fences keep LDS accesses on their side. The loader
  // waves wait for their loads before it (wait_vm), so after it a chunk's
  // staged bytes are visible to every wave.
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

  // ---------------------------------------------------------------- loader waves
  // Per step n: after barrier n the loads of chunk n+2 and the O stores of
  // chunk n-1 are issued (a vector memory instruction holds its wave at issue
  // until the CU takes it, so these waves absorb the staging time), then the
  // wave waits for the loads before barrier n+1.
  __device__ __forceinline__ void run_loader() {
    const LoaderLanes ll = loader_lanes();
    issue_chunk(ll, 0);
    issue_chunk(ll, 1);
    wait_vm<0>();
    barrier();
    for (long n = 0; n < nchunks; ++n) {
      barrier();  // barrier n: chunk n+1 was waited for before it
      issue_chunk(ll, n + 2);
      store_out(ll, n - 1);
      wait_vm<OUT_STORES>();  // chunk n+2 has landed; the O stores may still be in flight
    }
    barrier();  // the last chunk's O tile is complete
    store_out(ll, nchunks - 1);
  }

  // --------------------------------------------------------------- compute waves
  __device__ __forceinline__ void run_compute() {
    barrier();
    for (long n = 0; n < nchunks; ++n) {
      const int b3 = static_cast<int>(n % 3), b2 = static_cast<int>(n & 1);
      const uint32_t km = L::kmat(b3), qm = L::qmat(b2), rc = L::rec(b3), vm = L::vmat(b2);
      // ---- A: X = V - gamma K S and Q S for the 4 row tiles, contraction
      // step kk outermost so that consecutive products go to different
      // accumulators; step kk+1's operands are read during step kk's products
      O8 kf[2][4], qf[2][4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        kf[0][r] = ld<O8>(km + xa[0] + 16 * r * L::ROW);
        qf[0][r] = ld<O8>(qm + xa[0] + 16 * r * L::ROW);
      }
      float4_t ah[4], aq[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) ah[r] = aq[r] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const int cur = kk & 1;
        // S as a bf16 (or fp16) high / low B operand pair: tiles 2kk, 2kk+1
        const O4 h0 = Op::from(s[2 * kk]), h1 = Op::from(s[2 * kk + 1]);
        const O8 shi = pair(h0, h1);
        const O8 slo = pair(Op::from(s[2 * kk] - Op::to(h0)), Op::from(s[2 * kk + 1] - Op::to(h1)));
        if (kk + 1 < KS) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            kf[cur ^ 1][r] = ld<O8>(km + xa[kk + 1] + 16 * r * L::ROW);
            qf[cur ^ 1][r] = ld<O8>(qm + xa[kk + 1] + 16 * r * L::ROW);
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) ah[r] = mma(kf[cur][r], shi, ah[r]);
        // (Q S)^T: S^T as the A operand (the B registers of S serve), Q as B
#pragma unroll
        for (int r = 0; r < 4; ++r) aq[r] = mma(shi, qf[cur][r], aq[r]);
#pragma unroll
        for (int r = 0; r < 4; ++r) ah[r] = mma(kf[cur][r], slo, ah[r]);
      }
      __builtin_amdgcn_sched_barrier(0);
      float4_t x[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float4_t vv = Op::bits_to_float(ld_tr(vm + vtr + 16 * r * L::VROW));
        const float4_t gam = ld<float4_t>(rc + REC_SC + SC_GAM + (16 * r + 4 * g4) * 4);
        x[r] = vv - gam * ah[r];
      }
      // ---- B: U = Tb X (row tiles 0, 1 one step; 2, 3 two)
      half8_t tbf[6];
#pragma unroll
      for (int f = 0; f < 6; ++f) tbf[f] = frag(rc + REC_TB + f * FRAG_BYTES);
      const half8_t xb0 = pairh(to_half4(x[0]), to_half4(x[1]));
      const half8_t xb1 = pairh(to_half4(x[2]), to_half4(x[3]));
      float4_t u[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) u[r] = mfma32(tbf[frag_index(r, 0)], xb0, float4_t{0.f, 0.f, 0.f, 0.f});
      u[2] = mfma32(tbf[frag_index(2, 1)], xb1, u[2]);
      u[3] = mfma32(tbf[frag_index(3, 1)], xb1, u[3]);
      // barrier n: chunk n+1 is in LDS, every wave is past chunk n-1
      __builtin_amdgcn_sched_barrier(0);
      barrier();
      // ---- C: S <- gamma_63 S + K^T (dec U), token step ks outermost; then
      // O = scale gamma Q S + QKD U into the O tile
      O8 tf[2][NKT];
#pragma unroll
      for (int t = 0; t < NKT; ++t) tf[0][t] = kt_frag(km, t >> 1, t & 1, 0);
      O8 dhi[2], dlo[2];
      half8_t ub[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const float4_t d0 = u[2 * ks] * ld<float4_t>(rc + REC_SC + SC_DEC + (32 * ks + 4 * g4) * 4);
        const float4_t d1 = u[2 * ks + 1] * ld<float4_t>(rc + REC_SC + SC_DEC + (32 * ks + 16 + 4 * g4) * 4);
        const O4 h0 = Op::from(d0), h1 = Op::from(d1);
        dhi[ks] = pair(h0, h1);
        dlo[ks] = pair(Op::from(d0 - Op::to(h0)), Op::from(d1 - Op::to(h1)));
        ub[ks] = pairh(to_half4(u[2 * ks]), to_half4(u[2 * ks + 1]));
      }
      const float g63 = ld<float>(rc + REC_SC + SC_GAM + (CH - 1) * 4);
#pragma unroll
      for (int t = 0; t < NKT; ++t) s[t] *= g63;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (ks == 0) {
#pragma unroll
          for (int t = 0; t < NKT; ++t) tf[1][t] = kt_frag(km, t >> 1, t & 1, 1);
        }
#pragma unroll
        for (int t = 0; t < NKT; ++t) s[t] = mma(tf[ks][t], dhi[ks], s[t]);
#pragma unroll
        for (int t = 0; t < NKT; ++t) s[t] = mma(tf[ks][t], dlo[ks], s[t]);
      }
      __builtin_amdgcn_sched_barrier(0);
      half8_t qkf[6];
#pragma unroll
      for (int f = 0; f < 6; ++f) qkf[f] = frag(rc + REC_QKD + f * FRAG_BYTES);
      // O^T = (Q S)^T diag(scale gamma) + U^T QKD^T: lane (g, c) holds
      // O[16 r + c][16 wave + 4 g .. + 3], 8 contiguous bytes of an O row
      float4_t o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        o[r] = aq[r] * ld<float>(rc + REC_SC + SC_GSC + (16 * r + c16) * 4);
        o[r] = mfma32(ub[0], qkf[frag_index(r, 0)], o[r]);
      }
      o[2] = mfma32(ub[1], qkf[frag_index(2, 1)], o[2]);
      o[3] = mfma32(ub[1], qkf[frag_index(3, 1)], o[3]);
      const uint32_t om = L::omat(b2);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t row = 16 * r + c16;
        const uint32_t piece = (2 * wave + (g4 >> 1)) ^ oswz(row);
        *reinterpret_cast<O4 *>(lds + om + row * L::OROW + piece * 16 + 8 * (g4 & 1)) = Op::from(o[r]);
      }
    }
    barrier();  // the last chunk's O tile is complete
  }

  __device__ __forceinline__ void run() {
    if (nchunks <= 0) {
      if (compute) {
        load_state();
        store_state();
      }
      return;
    }
    if (compute) {
      load_state();
      run_compute();
      store_state();
    } else {
      run_loader();
    }
  }
};

// Two waves per SIMD (a compute and a loader wave): 256 registers each.
template <int K, typename TIn, typename TOut>
__global__ __launch_bounds__(WALL) __attribute__((amdgpu_waves_per_eu(2, 2))) void wide_kernel(ChunkParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  WideBlock<K, TIn, TOut> blk(smem_raw, p);
  blk.run();
}

}  // namespace

template <int K, typename TIn, typename TOut>
int launch_wide(const ChunkParams &p, hipStream_t stream) {
  static bool configured = false;  // benign race: the attribute call is idempotent
  const size_t smem = WideLayout<K, TOut>::BYTES;
  auto kernel = wide_kernel<K, TIn, TOut>;
  if (!configured) {
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(smem)) != hipSuccess) {
      return PBGDN_ERR_LAUNCH;
    }
    configured = true;
  }
  const long total = static_cast<long>(p.V / (16 * WT)) * p.Hv * p.num_seqs;
  if (total > 0x7fffffffL) return PBGDN_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(total)), dim3(WALL), smem, stream, p);
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}

template int launch_wide<128, u16, u16>(const ChunkParams &, hipStream_t);
template int launch_wide<128, half_t, half_t>(const ChunkParams &, hipStream_t);

}  // namespace pbgdn
