// Layer-side kernels around the recurrence: the fused prologue (short causal
// convolution with its carried tail, SiLU, q/k L2 normalisation, decay and
// beta gates; pseudobrain/gated_deltanet.py:314-338, :415-429) and the fused
// epilogue (per-head RMSNorm x o_norm x SiLU(gate), :439-441). Both are one
// pass over HBM; the reference spends a torch kernel per step on each.
//
// Prologue: a workgroup of 256 threads covers 128 channels (16 lanes x 8
// channels) of TT = 128 tokens of one sequence; lane row tl (16 lanes) owns
// tokens tl*8 .. tl*8+7 and walks them with the last conv-1 input rows in
// registers. A 16-lane row holds all channels of one token, so the q/k norm
// over a key head (K/8 lanes) is a shuffle reduction inside the row. Extra
// workgroups (blockIdx.x >= channel blocks) compute the gates of the tile.
// Packed sequences run through the same kernel as one sequence; a second,
// small kernel redoes the first conv-1 tokens of each sequence against its
// own tail from a slot pool and writes the new tails, so the main pass needs
// no per-token sequence lookup.
//
// Epilogue: V/8 lanes per (token, value head) row, 8 elements each; the mean
// square over the head is a shuffle reduction inside the row group.
#include "chunk.hpp"  // buffer-resource helpers (rsrc, buf_load16, OUT_OF_RANGE)
#include "layer_math.hpp"

namespace pbgdn {
namespace {

constexpr int LNT = 256;       // threads per workgroup
constexpr int UPW = 16;        // prologue: 8-channel units per workgroup (lanes of a lane row)
constexpr int TPL = 8;         // prologue: tokens per lane row
constexpr int TT = LNT / UPW * TPL;  // prologue tokens per workgroup
constexpr int MAX_CONV = 4;          // widest filter with a kernel

// Eight consecutive elements starting at element i of a tensor of `dtype`
// (wave-uniform), as float. The addresses are 16-byte aligned when the
// tensor and its row strides are (the ABI checks this).
__device__ __forceinline__ void load8(const void *p, long i, int dtype, float (&x)[8]) {
  if (dtype == PBGDN_F32) {
    const float4_t a = *reinterpret_cast<const float4_t *>(static_cast<const float *>(p) + i);
    const float4_t b = *reinterpret_cast<const float4_t *>(static_cast<const float *>(p) + i + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = a[e];
      x[4 + e] = b[e];
    }
  } else if (dtype == PBGDN_BF16) {
    const uint4 u = *reinterpret_cast<const uint4 *>(static_cast<const u16 *>(p) + i);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = __uint_as_float(w[e] << 16);
      x[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
    }
  } else {
    const half8_t h = *reinterpret_cast<const half8_t *>(static_cast<const half_t *>(p) + i);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = static_cast<float>(h[e]);
  }
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, bf16x2_t{static_cast<__bf16>(lo), static_cast<__bf16>(hi)});
}

// A 16-byte store; STREAM: non-temporal (outputs read next by another kernel,
// far more bytes than the caches hold).
template <bool STREAM, typename T>
__device__ __forceinline__ void put16(T *dst, const T &x) {
  if constexpr (STREAM) {
    __builtin_nontemporal_store(x, dst);
  } else {
    *dst = x;
  }
}

template <bool STREAM = false>
__device__ __forceinline__ void store8(void *p, long i, int dtype, const float (&x)[8]) {
  if (dtype == PBGDN_F32) {
    put16<STREAM>(reinterpret_cast<float4_t *>(static_cast<float *>(p) + i), float4_t{x[0], x[1], x[2], x[3]});
    put16<STREAM>(reinterpret_cast<float4_t *>(static_cast<float *>(p) + i + 4), float4_t{x[4], x[5], x[6], x[7]});
  } else if (dtype == PBGDN_BF16) {
    v4u32_t u;  // v_cvt_pk_bf16_f32: round to nearest even, as float_to_bf16_bits
    u[0] = bf16_pair(x[0], x[1]);
    u[1] = bf16_pair(x[2], x[3]);
    u[2] = bf16_pair(x[4], x[5]);
    u[3] = bf16_pair(x[6], x[7]);
    put16<STREAM>(reinterpret_cast<v4u32_t *>(static_cast<u16 *>(p) + i), u);
  } else {
    half8_t h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = static_cast<half_t>(x[e]);
    put16<STREAM>(reinterpret_cast<half8_t *>(static_cast<half_t *>(p) + i), h);
  }
}

// Typed forms of load8: no run-time type switch, so a lane's loads issue back
// to back and wait only where their values are first used.
template <typename T>
__device__ __forceinline__ void load8t(const void *p, long i, float (&x)[8]);
template <>
__device__ __forceinline__ void load8t<float>(const void *p, long i, float (&x)[8]) {
  load8(p, i, PBGDN_F32, x);
}
template <>
__device__ __forceinline__ void load8t<u16>(const void *p, long i, float (&x)[8]) {
  load8(p, i, PBGDN_BF16, x);
}
template <>
__device__ __forceinline__ void load8t<half_t>(const void *p, long i, float (&x)[8]) {
  load8(p, i, PBGDN_F16, x);
}
template <typename T>
constexpr int dtype_of();
template <>
constexpr int dtype_of<float>() { return PBGDN_F32; }
template <>
constexpr int dtype_of<u16>() { return PBGDN_BF16; }
template <>
constexpr int dtype_of<half_t>() { return PBGDN_F16; }

// Eight elements of type T as loaded raw (two 16-byte pieces; the second one
// is used by fp32 only), and their float values.
struct Raw8 {
  uint4 a, b;
};
template <typename T>
__device__ __forceinline__ void decode8(const Raw8 &r, float (&x)[8]) {
  const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = __uint_as_float(w[e]);
  } else if constexpr (dtype_of<T>() == PBGDN_BF16) {
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
__device__ __forceinline__ void decode8(const Raw8 &r, int dtype, float (&x)[8]) {
  if (dtype == PBGDN_F32) {
    decode8<float>(r, x);
  } else if (dtype == PBGDN_BF16) {
    decode8<u16>(r, x);
  } else {
    decode8<half_t>(r, x);
  }
}
// Raw load of 8 elements at byte offset `off` of a buffer resource (32 bytes
// when WIDE, else 16): offsets at or past the resource's size read zeros.
// STREAM: non-temporal (inputs read once).
template <bool WIDE, bool STREAM = false>
__device__ __forceinline__ Raw8 load_raw8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  constexpr int AUX = STREAM ? 2 : 0;
  Raw8 x;
  x.a = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX));
  x.b = WIDE ? __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, AUX))
             : uint4{0u, 0u, 0u, 0u};
  return x;
}

struct PrologueParams {
  const void *qkv, *decay, *tail;
  void *tail_out;
  const float *conv_weight, *a_log, *dt_bias;
  void *q, *k, *v;
  float *g, *beta;
  long qkv_stride, decay_stride;  // elements per token row
  int in_dtype, tail_dtype, out_dtype;
  int B, T, Hk, Hv, K, V, conv, l2_mode;
  int units, ch_blocks;  // 8-channel units; channel workgroups per tile
  // Packed sequences (B = 1): cu_seqlens [N+1] over the T axis, and the tails
  // in a pool of slots, row j of channel c of slot s at element
  // s * tail_ss + j * tail_rs + c * tail_cs; slot_idx [N] (NULL: slot n),
  // has_initial [N] (NULL: all; 0: the sequence starts from a zero tail).
  const int32_t *cu_seqlens, *slot_idx;
  const uint8_t *has_initial;
  int num_seqs, num_slots;
  long tail_ss, tail_rs, tail_cs;
  // 1: rows of channels (tail_cs == 1), 2: channels of rows (tail_rs == 1,
  // tail_cs == conv-1), both 16-byte aligned in 8-element pieces, so a
  // lane's eight channels move in whole vectors; 0: element by element.
  int tail_vec;
  // The gate rows take eight heads per lane in 16-byte pieces (Hv % 8 == 0,
  // decay, g and beta 16-byte aligned, decay rows in 8-element steps).
  bool gate_vec;
};

// Where a lane's eight channels go: q, k (L2-normalised over the key head,
// K/8 lanes of a 16-lane row) or v, and the element index of its first
// channel in that output for token 0 plus the step per token.
struct OutLane {
  int kind;  // 0 q, 1 k, 2 v
  int head_lanes;
  void *ptr;
  long step, col;
  __device__ __forceinline__ OutLane(const PrologueParams &p, int u, int c0) {
    // channel c0 of a part is element c0 of its [heads x width] token row
    const int qk_units = p.Hk * p.K / 8;
    kind = u < qk_units ? 0 : u < 2 * qk_units ? 1 : 2;
    col = c0 - 8L * qk_units * kind;
    head_lanes = p.K / 8;
    const int width = kind < 2 ? p.K : p.V;
    ptr = kind == 0 ? p.q : kind == 1 ? p.k : p.v;
    step = static_cast<long>(kind < 2 ? p.Hk : p.Hv) * width;
  }
  // y = SiLU(conv) of one token: the q/k norm (every lane of a head's group
  // takes part in its sum; the q/k boundary is a multiple of the group, so
  // whole groups take the branch), then the store at element i when `store`.
  template <bool STREAM = false>
  __device__ __forceinline__ bool finish(const PrologueParams &p, float (&y)[8], bool store, long i) const {
    if (kind < 2) {
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += y[e] * y[e];
      ss = group_sum(ss, head_lanes);  // DPP: a shuffle's LDS trip and wait per step sat on every token's path
      // 1 / max(sqrt(ss), eps) ('max') or 1 / sqrt(ss + eps) ('hf') on
      // v_rsq_f32 (1 ulp): the IEEE-exact square root and division cost ~30
      // VALU operations a token
      constexpr float l2_eps = 1e-6f;
      const float n = p.l2_mode == 0 ? (ss >= l2_eps * l2_eps ? __builtin_amdgcn_rsqf(ss) : 1.f / l2_eps)
                                     : __builtin_amdgcn_rsqf(ss + l2_eps);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] *= n;
    }
    if (!store) return false;
    store8<STREAM>(ptr, i, p.out_dtype, y);
    return true;
  }
};

// Gates of a token tile, g = -exp(A_log) softplus(a + dt_bias) and
// beta = sigmoid(b), eight heads per lane: every lane's a and b pieces of a
// round are loaded before any is used, and g and beta leave in 16-byte
// stores. Rows past the tile's end read zeros and store nothing.
template <typename TIn, bool STREAM>
__device__ __forceinline__ void tile_gates_vec(const PrologueParams &p, int b, int t_tile, int tid) {
  constexpr int GU = 4;  // 8-head units per lane per round
  const int hu = p.Hv / 8;
  const int rows = min(TT, p.T - t_tile);
  const int n = rows * hu;
  const long row0 = static_cast<long>(b) * p.T + t_tile;
  const auto rd = rsrc(static_cast<const TIn *>(p.decay) + row0 * p.decay_stride,
                       (static_cast<long>(rows - 1) * p.decay_stride + 2L * p.Hv) * static_cast<long>(sizeof(TIn)));
  for (int i0 = 0; i0 < n; i0 += GU * LNT) {
    Raw8 ra[GU], rb[GU];
#pragma unroll
    for (int j = 0; j < GU; ++j) {
      const int i = i0 + tid + j * LNT;
      const int t = i / hu, hh = i - (i / hu) * hu;
      const uint32_t off = static_cast<uint32_t>((static_cast<long>(t) * p.decay_stride + 8 * hh) * sizeof(TIn));
      ra[j] = load_raw8<sizeof(TIn) == 4, STREAM>(rd, i < n ? off : OUT_OF_RANGE);
      rb[j] = load_raw8<sizeof(TIn) == 4, STREAM>(
          rd, i < n ? off + static_cast<uint32_t>(p.Hv * sizeof(TIn)) : OUT_OF_RANGE);
    }
#pragma unroll
    for (int j = 0; j < GU; ++j) {
      const int i = i0 + tid + j * LNT;
      if (i >= n) continue;
      const int t = i / hu, hh = i - (i / hu) * hu;
      float a[8], bb[8];
      decode8<TIn>(ra[j], a);
      decode8<TIn>(rb[j], bb);
      float gv[8], bv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int h = 8 * hh + e;
        gv[e] = -exp_fast(p.a_log[h]) * softplus_fast(a[e] + p.dt_bias[h]);
        bv[e] = sigmoid_fast(bb[e]);
      }
      const long o = (row0 + t) * p.Hv + 8 * hh;
      put16<STREAM>(reinterpret_cast<float4_t *>(p.g + o), float4_t{gv[0], gv[1], gv[2], gv[3]});
      put16<STREAM>(reinterpret_cast<float4_t *>(p.g + o + 4), float4_t{gv[4], gv[5], gv[6], gv[7]});
      put16<STREAM>(reinterpret_cast<float4_t *>(p.beta + o), float4_t{bv[0], bv[1], bv[2], bv[3]});
      put16<STREAM>(reinterpret_cast<float4_t *>(p.beta + o + 4), float4_t{bv[4], bv[5], bv[6], bv[7]});
    }
  }
}

// Gates of a token tile, one element per thread and step (the general form
// of tile_gates_vec).
template <typename TIn>
__device__ __forceinline__ void tile_gates(const PrologueParams &p, int b, int t_tile, int tid) {
  constexpr int IN = dtype_of<TIn>();
  const int n = min(TT, p.T - t_tile) * p.Hv;
  for (int i = tid; i < n; i += LNT) {
    const int t = t_tile + i / p.Hv;
    const int h = i % p.Hv;
    const long row = static_cast<long>(b) * p.T + t;
    const float a = load_elem(p.decay, row * p.decay_stride + h, IN);
    const float bb = load_elem(p.decay, row * p.decay_stride + p.Hv + h, IN);
    p.g[row * p.Hv + h] = -exp_fast(p.a_log[h]) * softplus_fast(a + p.dt_bias[h]);
    p.beta[row * p.Hv + h] = sigmoid_fast(bb);
  }
}

// CONV is the filter width (0: SiLU only). Every input row a lane needs (its
// TPL tokens and the CONV-1 before them) is loaded before any is used, so the
// loads of a lane overlap instead of following one another. Rows before the
// sequence's start read zeros: the first CONV-1 tokens of every sequence
// (batch row or packed sequence) are redone against the sequence's own tail by
// edge_kernel, which also writes the new tails, so this pass reads and writes
// no tail and needs no per-token sequence lookup. STREAM: non-temporal stores
// and gate loads (a call moving more bytes than the caches hold).
template <int CONV, typename TIn, bool STREAM>
__global__ __launch_bounds__(LNT) void prologue_kernel(PrologueParams p) {
  constexpr int HALO = CONV > 1 ? CONV - 1 : 0;  // rows before a lane's first token
  const int tid = threadIdx.x;
  const int b = blockIdx.z;
  const int t_tile = blockIdx.y * TT;
  if (static_cast<int>(blockIdx.x) >= p.ch_blocks) {
    if (p.gate_vec) {
      tile_gates_vec<TIn, STREAM>(p, b, t_tile, tid);
    } else {
      tile_gates<TIn>(p, b, t_tile, tid);
    }
    return;
  }
  const int u = blockIdx.x * UPW + tid % UPW;   // this lane's 8-channel unit
  const int tl = tid / UPW;                      // lane row: tokens tl*TPL ..
  const int t_first = t_tile + tl * TPL;
  if (t_first >= p.T) return;  // the whole 16-lane row: no tokens (no shuffle partner is lost)
  const bool live = u < p.units;
  const int c0 = 8 * (live ? u : 0);
  const long seq_row = static_cast<long>(b) * p.T;
  const long chans = static_cast<long>(p.units) * 8;
  // Every row this lane needs is loaded unconditionally through a buffer
  // resource that spans exactly the sequence's rows this tile reads (from
  // base_row, the tile's first halo row or the sequence's first); a row
  // outside it (or a dead lane) gets an out-of-range offset and reads zeros.
  // No load then waits on a branch merge: they all issue back to back, and
  // the offsets stay small however long the sequence.
  const int base_row = max(t_tile - HALO, 0);
  const int end_row = min(t_tile + TT, p.T);
  const auto rq = rsrc(static_cast<const TIn *>(p.qkv) + (seq_row + base_row) * p.qkv_stride,
                       (static_cast<long>(end_row - 1 - base_row) * p.qkv_stride + chans) *
                           static_cast<long>(sizeof(TIn)));
  Raw8 raw[HALO + TPL];  // rows t_first - HALO ..
  // row m at off0 + m row strides (a scalar step: one add per row); the
  // inputs are loaded cacheable, since neighbouring lane rows and tiles read
  // each other's halo rows
  const uint32_t row_bytes = static_cast<uint32_t>(p.qkv_stride * sizeof(TIn));
  const uint32_t off0 = static_cast<uint32_t>(t_first - HALO - base_row) * row_bytes + c0 * sizeof(TIn);
#pragma unroll
  for (int m = 0; m < HALO + TPL; ++m) {
    const int t = t_first - HALO + m;
    const uint32_t off = live && t >= 0 && t < p.T ? off0 + m * row_bytes : OUT_OF_RANGE;
    raw[m] = load_raw8<sizeof(TIn) == 4>(rq, off);
  }
  float xr[HALO + TPL][8];  // decoded as the token loop reaches them (fewer live registers)
#pragma unroll
  for (int m = 0; m < HALO; ++m) decode8<TIn>(raw[m], xr[m]);
  float w[8][CONV > 0 ? CONV : 1];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
#pragma unroll
    for (int j = 0; j < CONV; ++j) w[e][j] = p.conv_weight[(c0 + e) * CONV + j];
  }
  const OutLane out(p, u, c0);
  const long out0 = (seq_row + t_first) * out.step + out.col;
#pragma unroll
  for (int i = 0; i < TPL; ++i) {
    const int t = t_first + i;
    decode8<TIn>(raw[HALO + i], xr[HALO + i]);
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = CONV == 0 ? xr[HALO + i][e] : 0.f;
#pragma unroll
      for (int j = 0; j < CONV; ++j) acc += w[e][j] * xr[HALO + i - (CONV - 1) + j][e];  // tap j: row t-(CONV-1)+j
      y[e] = siluf(acc);
    }
    out.template finish<STREAM>(p, y, live && t < p.T, out0 + i * out.step);
  }
}

// A call moving more bytes than this (inputs in, outputs out) streams them
// with non-temporal hints; smaller calls keep them cacheable, since their
// inputs were most likely just written and their outputs are read next.
constexpr long STREAM_BYTES = 192L << 20;

template <typename TIn, bool STREAM>
void launch_prologue_s(int conv, dim3 grid, hipStream_t st, const PrologueParams &prm) {
  switch (conv) {
    case 0: hipLaunchKernelGGL((prologue_kernel<0, TIn, STREAM>), grid, dim3(LNT), 0, st, prm); break;
    case 1: hipLaunchKernelGGL((prologue_kernel<1, TIn, STREAM>), grid, dim3(LNT), 0, st, prm); break;
    case 2: hipLaunchKernelGGL((prologue_kernel<2, TIn, STREAM>), grid, dim3(LNT), 0, st, prm); break;
    case 3: hipLaunchKernelGGL((prologue_kernel<3, TIn, STREAM>), grid, dim3(LNT), 0, st, prm); break;
    default: hipLaunchKernelGGL((prologue_kernel<4, TIn, STREAM>), grid, dim3(LNT), 0, st, prm); break;
  }
}
template <typename TIn>
void launch_prologue(int conv, dim3 grid, hipStream_t st, const PrologueParams &prm) {
  const long in_elem = sizeof(TIn), out_elem = prm.out_dtype == PBGDN_F32 ? 4 : 2;
  const long bytes = static_cast<long>(prm.B) * prm.T *
                     (8L * prm.units * (in_elem + out_elem) + 2L * prm.Hv * (in_elem + 4));
  bytes > STREAM_BYTES ? launch_prologue_s<TIn, true>(conv, grid, st, prm)
                       : launch_prologue_s<TIn, false>(conv, grid, st, prm);
}

// After the prologue: thread (unit u, sequence s) redoes tokens 0 .. CONV-2
// of sequence s for channels 8u .. 8u+7 with the sequence's own tail (the
// prologue gave them zeros or the previous sequence's inputs), in the
// prologue's arithmetic, and writes s's new tail: the last CONV-1 rows of
// (its tail, rounded through the input dtype) ++ (its inputs). Sequence s is
// packed rows cu_seqlens[s] .. cu_seqlens[s+1]-1 of T, or without cu_seqlens
// batch row s (T rows). A thread reads every old tail row before it writes,
// and no other thread touches its channels of that slot, so tail_out may be
// the pool itself.
template <int CONV, typename TIn>
__global__ __launch_bounds__(LNT) void edge_kernel(PrologueParams p) {
  constexpr int IN = dtype_of<TIn>();
  constexpr int TAIL = CONV - 1;
  const int u = blockIdx.x * LNT + threadIdx.x;
  const int s = blockIdx.y;
  const bool live = u < p.units;
  const int c0 = 8 * (live ? u : 0);
  const long chans = static_cast<long>(p.units) * 8;
  long bos = static_cast<long>(s) * p.T, len = p.T;
  if (p.cu_seqlens) {  // clamped to the packed rows, whatever cu_seqlens holds
    bos = min(max(0L, static_cast<long>(p.cu_seqlens[s])), static_cast<long>(p.T));
    len = min(max(0L, static_cast<long>(p.cu_seqlens[s + 1]) - bos), p.T - bos);
  }
  const long slot = p.slot_idx ? static_cast<long>(p.slot_idx[s]) : static_cast<long>(s);
  // Two resources: the sequence's first TAIL rows, and its last TAIL rows
  // (from row `last0`), so the offsets stay small however long the sequence.
  const long head_rows = min(len, static_cast<long>(TAIL));
  const long last0 = max(len - TAIL, 0L);
  const auto r_head = rsrc(static_cast<const TIn *>(p.qkv) + bos * p.qkv_stride,
                           head_rows > 0 ? ((head_rows - 1) * p.qkv_stride + chans) * static_cast<long>(sizeof(TIn))
                                         : 0);
  const auto r_last = rsrc(static_cast<const TIn *>(p.qkv) + (bos + last0) * p.qkv_stride,
                           len > 0 ? ((len - 1 - last0) * p.qkv_stride + chans) * static_cast<long>(sizeof(TIn)) : 0);
  auto row_off = [&](long j) -> uint32_t {  // byte offset of row j within a resource starting at row 0 or last0
    return live && j >= 0 && j < TAIL ? static_cast<uint32_t>((j * p.qkv_stride + c0) * static_cast<long>(sizeof(TIn)))
                                      : OUT_OF_RANGE;
  };
  float old[TAIL][8], x[TAIL][8];  // the old tail; the sequence's first TAIL inputs
  // every input row this thread reads is loaded before any store (the stores
  // may alias the inputs for all the compiler knows, so a later load would
  // wait for them): the first TAIL rows, then the last TAIL (row r of the new
  // tail is row len + r of (old tail ++ inputs): input row len + r - TAIL,
  // out of range when that is an old tail row)
  Raw8 last[TAIL];
#pragma unroll
  for (int j = 0; j < TAIL; ++j) decode8<TIn>(load_raw8<sizeof(TIn) == 4>(r_head, row_off(j)), x[j]);
#pragma unroll
  for (int r = 0; r < TAIL; ++r) last[r] = load_raw8<sizeof(TIn) == 4>(r_last, row_off(len + r - TAIL - last0));
  const bool from_pool = live && slot >= 0 && slot < p.num_slots && !(p.has_initial && !p.has_initial[s]);
  if (!from_pool) {
#pragma unroll
    for (int j = 0; j < TAIL; ++j) {
#pragma unroll
      for (int e = 0; e < 8; ++e) old[j][e] = 0.f;
    }
  } else if (p.tail_vec == 1) {
#pragma unroll
    for (int j = 0; j < TAIL; ++j) load8(p.tail, slot * p.tail_ss + j * p.tail_rs + c0, p.tail_dtype, old[j]);
  } else if (p.tail_vec == 2) {  // element m of the lane's run is channel m / TAIL, row m % TAIL
#pragma unroll
    for (int m = 0; m < TAIL; ++m) {
      float v[8];
      load8(p.tail, slot * p.tail_ss + static_cast<long>(c0) * TAIL + 8 * m, p.tail_dtype, v);
#pragma unroll
      for (int k = 0; k < 8; ++k) old[(8 * m + k) % TAIL][(8 * m + k) / TAIL] = v[k];
    }
  } else {
#pragma unroll
    for (int j = 0; j < TAIL; ++j) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        old[j][e] = load_elem(p.tail, slot * p.tail_ss + j * p.tail_rs + (c0 + e) * p.tail_cs, p.tail_dtype);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < TAIL; ++j) {
#pragma unroll
    for (int e = 0; e < 8; ++e) old[j][e] = through(old[j][e], IN);  // as cat(tail.to(x.dtype), x)
  }
  float w[8][CONV];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
#pragma unroll
    for (int j = 0; j < CONV; ++j) w[e][j] = p.conv_weight[(c0 + e) * CONV + j];
  }
  const OutLane out(p, u, c0);
#pragma unroll
  for (int i = 0; i < TAIL; ++i) {  // token i: taps are rows i .. i+CONV-1 of (old tail ++ inputs)
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < CONV; ++j) acc += w[e][j] * (i + j < TAIL ? old[i + j][e] : x[i + j - TAIL][e]);
      y[e] = siluf(acc);
    }
    out.finish(p, y, live && i < len, (bos + i) * out.step + out.col);
  }
  if (!live || slot < 0 || slot >= p.num_slots) return;
  float nt[TAIL][8];  // the new tail
#pragma unroll
  for (int r = 0; r < TAIL; ++r) {
    const long e = len + r;  // row of (old tail ++ inputs)
    if (e < TAIL) {
#pragma unroll
      for (int k = 0; k < 8; ++k) nt[r][k] = old[e < TAIL ? e : 0][k];
    } else {
      decode8<TIn>(last[r], nt[r]);
    }
  }
  if (p.tail_vec == 1) {
#pragma unroll
    for (int r = 0; r < TAIL; ++r) store8(p.tail_out, slot * p.tail_ss + r * p.tail_rs + c0, p.tail_dtype, nt[r]);
  } else if (p.tail_vec == 2) {
#pragma unroll
    for (int m = 0; m < TAIL; ++m) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = nt[(8 * m + k) % TAIL][(8 * m + k) / TAIL];
      store8(p.tail_out, slot * p.tail_ss + static_cast<long>(c0) * TAIL + 8 * m, p.tail_dtype, v);
    }
  } else {
#pragma unroll
    for (int r = 0; r < TAIL; ++r) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        store_elem(p.tail_out, slot * p.tail_ss + r * p.tail_rs + (c0 + k) * p.tail_cs, p.tail_dtype, nt[r][k]);
      }
    }
  }
}

template <typename TIn>
void launch_edge(int conv, dim3 grid, hipStream_t st, const PrologueParams &prm) {
  switch (conv) {
    case 2: hipLaunchKernelGGL((edge_kernel<2, TIn>), grid, dim3(LNT), 0, st, prm); break;
    case 3: hipLaunchKernelGGL((edge_kernel<3, TIn>), grid, dim3(LNT), 0, st, prm); break;
    default: hipLaunchKernelGGL((edge_kernel<4, TIn>), grid, dim3(LNT), 0, st, prm); break;
  }
}

// The prologue pass, then (conv > 1) the edge pass over `seqs` sequences.
template <typename TIn>
void launch_prologue_and_edges(const PrologueParams &prm, dim3 grid, int seqs, hipStream_t st) {
  if (prm.T > 0) launch_prologue<TIn>(prm.conv, grid, st, prm);
  if (prm.conv > 1) {
    const dim3 egrid(static_cast<unsigned>((prm.units + LNT - 1) / LNT), static_cast<unsigned>(seqs));
    launch_edge<TIn>(prm.conv, egrid, st, prm);
  }
}

struct EpilogueParams {
  const void *o, *gate;
  const float *o_norm;
  void *out;
  long gate_stride;  // elements per token row
  int o_dtype, gate_dtype, out_dtype;
  long rows;         // B * T * Hv
  int Hv, V;
  float eps;
};

// ROWS (token, head) rows per lane: a lane group of V/8 lanes takes rows
// g, g + G, ... (G = groups per workgroup); all loads issue before any use.
constexpr int EPI_ROWS = 1;


template <typename TO, typename TG, int V, bool STREAM>
__global__ __launch_bounds__(LNT) void epilogue_kernel(EpilogueParams p) {
  constexpr int LANES = V / 8;             // lanes per (token, head) row
  constexpr int GROUPS = LNT / LANES;      // row groups per workgroup
  const int tid = threadIdx.x;
  const int c0 = 8 * (tid % LANES);
  // The workgroup's rows, from its first (r0) and its first token (tk0): the
  // buffer offsets stay small however many rows the call has.
  const long r0 = static_cast<long>(blockIdx.x) * GROUPS * EPI_ROWS;
  const long r_end = min(r0 + GROUPS * EPI_ROWS, p.rows);
  const long tk0 = r0 / p.Hv;
  const long row0 = r0 + tid / LANES;
  const auto ro = rsrc(static_cast<const TO *>(p.o) + r0 * V, (r_end - r0) * V * static_cast<long>(sizeof(TO)));
  const auto rg = rsrc(static_cast<const TG *>(p.gate) + tk0 * p.gate_stride,
                       ((r_end - 1) / p.Hv - tk0 + 1) * p.gate_stride * static_cast<long>(sizeof(TG)));
  Raw8 ro8[EPI_ROWS], rg8[EPI_ROWS];
#pragma unroll
  for (int j = 0; j < EPI_ROWS; ++j) {
    const long row = row0 + static_cast<long>(j) * GROUPS;
    const bool live = row < p.rows;
    const long token = row / p.Hv;
    const long h = row - token * p.Hv;
    ro8[j] = load_raw8<sizeof(TO) == 4, STREAM>(
        ro, live ? static_cast<uint32_t>(((row - r0) * V + c0) * sizeof(TO)) : OUT_OF_RANGE);
    rg8[j] = load_raw8<sizeof(TG) == 4, STREAM>(
        rg, live ? static_cast<uint32_t>(((token - tk0) * p.gate_stride + h * V + c0) * sizeof(TG)) : OUT_OF_RANGE);
  }
  float nrm[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) nrm[e] = p.o_norm[c0 + e];
#pragma unroll
  for (int j = 0; j < EPI_ROWS; ++j) {
    const long row = row0 + static_cast<long>(j) * GROUPS;
    float o[8], gt[8];
    decode8<TO>(ro8[j], o);
    decode8<TG>(rg8[j], gt);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += o[e] * o[e];
    ss = group_sum(ss, LANES);
    const float r = rsqrtf(ss * (1.f / V) + p.eps);
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = o[e] * r * nrm[e] * siluf(gt[e]);
    if (row < p.rows) store8<STREAM>(p.out, row * V + c0, p.out_dtype, y);
  }
}

template <typename TO, int V, bool STREAM>
void launch_epilogue_v(int gate_dtype, dim3 grid, hipStream_t st, const EpilogueParams &prm) {
  switch (gate_dtype) {
    case PBGDN_F32: hipLaunchKernelGGL((epilogue_kernel<TO, float, V, STREAM>), grid, dim3(LNT), 0, st, prm); break;
    case PBGDN_BF16: hipLaunchKernelGGL((epilogue_kernel<TO, u16, V, STREAM>), grid, dim3(LNT), 0, st, prm); break;
    default: hipLaunchKernelGGL((epilogue_kernel<TO, half_t, V, STREAM>), grid, dim3(LNT), 0, st, prm); break;
  }
}
template <typename TO>
void launch_epilogue(int gate_dtype, dim3 grid, hipStream_t st, const EpilogueParams &prm) {
  const long elem_out = prm.out_dtype == PBGDN_F32 ? 4 : 2, elem_gate = gate_dtype == PBGDN_F32 ? 4 : 2;
  const bool stream = prm.rows * prm.V * (static_cast<long>(sizeof(TO)) + elem_gate + elem_out) > STREAM_BYTES;
  if (prm.V == 64) {
    stream ? launch_epilogue_v<TO, 64, true>(gate_dtype, grid, st, prm)
           : launch_epilogue_v<TO, 64, false>(gate_dtype, grid, st, prm);
  } else {
    stream ? launch_epilogue_v<TO, 128, true>(gate_dtype, grid, st, prm)
           : launch_epilogue_v<TO, 128, false>(gate_dtype, grid, st, prm);
  }
}

bool valid_dtype(int d) { return d == PBGDN_F32 || d == PBGDN_BF16 || d == PBGDN_F16; }

// Debug builds: q, k, v, g and beta of `rows` token rows start as NaN.
void poison_prologue_outputs(const PrologueParams &prm, long rows, hipStream_t st) {
  const long osz = prm.out_dtype == PBGDN_F32 ? 4 : 2;
  debug_poison(prm.q, static_cast<size_t>(rows * prm.Hk * prm.K * osz), st);
  debug_poison(prm.k, static_cast<size_t>(rows * prm.Hk * prm.K * osz), st);
  debug_poison(prm.v, static_cast<size_t>(rows * prm.Hv * prm.V * osz), st);
  debug_poison(prm.g, static_cast<size_t>(rows * prm.Hv * 4), st);
  debug_poison(prm.beta, static_cast<size_t>(rows * prm.Hv * 4), st);
}
bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
// The gate rows move in 16-byte pieces of eight heads: tile_gates_vec's
// conditions, and its 32-bit offsets within a tile's decay rows.
bool gates_vectorize(const void *decay, long decay_stride, long in_elem, const float *g, const float *beta, int Hv) {
  return Hv % 8 == 0 && decay_stride % 8 == 0 && aligned16(decay) && aligned16(g) && aligned16(beta) &&
         static_cast<long>(TT) * decay_stride * in_elem <= 0x7ffffff0L - 64;
}

}  // namespace
}  // namespace pbgdn

extern "C" int pbgdn_prologue_fwd(const void *qkv, long qkv_stride, const void *decay, long decay_stride,
                                  int in_dtype, const void *tail, void *tail_out, int tail_dtype,
                                  const float *conv_weight, int conv, const float *a_log, const float *dt_bias,
                                  void *q, void *k, void *v, int out_dtype, float *g, float *beta, int B, int T,
                                  int Hk, int Hv, int K, int V, int l2_mode, void *stream) {
  using namespace pbgdn;
  if (B < 0 || T < 0 || Hk <= 0 || Hv <= 0 || K <= 0 || V <= 0 || Hv % Hk != 0 || conv < 0) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype) || !valid_dtype(tail_dtype) ||
      !(l2_mode == 0 || l2_mode == 1)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!(K == 64 || K == 128) || V % 8 != 0 || conv > MAX_CONV) return PBGDN_ERR_UNSUPPORTED;
  const long channels = 2L * Hk * K + static_cast<long>(Hv) * V;
  if (qkv_stride < channels || decay_stride < 2L * Hv || qkv_stride % 8 != 0) return PBGDN_ERR_INVALID_ARGUMENT;
  // A tile's rows (and the ends of a sequence) are addressed with 32-bit byte
  // offsets from their first row, below the out-of-range marker.
  const long in_elem = in_dtype == PBGDN_F32 ? 4 : 2;
  if (static_cast<long>(TT + MAX_CONV) * qkv_stride * in_elem > 0x7ffffff0L - 64) return PBGDN_ERR_UNSUPPORTED;
  if (static_cast<long>(B) * T == 0) return PBGDN_OK;
  const bool has_tail = conv > 1;
  if (!qkv || !decay || !a_log || !dt_bias || !q || !k || !v || !g || !beta || (conv > 0 && !conv_weight) ||
      (has_tail && (!tail || !tail_out))) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!aligned16(qkv) || !aligned16(q) || !aligned16(k) || !aligned16(v) ||
      (has_tail && (!aligned16(tail) || !aligned16(tail_out)))) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (channels / 8 > 0x7fffffffL / 16 || static_cast<long>(T) + TT > 0x7fffffffL) return PBGDN_ERR_UNSUPPORTED;
  PrologueParams prm{qkv, decay, tail, tail_out, conv_weight, a_log, dt_bias, q, k, v, g, beta, qkv_stride,
                     decay_stride, in_dtype, tail_dtype, out_dtype, B, T, Hk, Hv, K, V, conv, l2_mode,
                     static_cast<int>(channels / 8), static_cast<int>((channels / 8 + UPW - 1) / UPW),
                     nullptr, nullptr, nullptr, B, B, (conv - 1) * channels, channels, 1, 1, false};
  prm.gate_vec = gates_vectorize(decay, decay_stride, in_elem, g, beta, Hv);
  const dim3 grid(prm.ch_blocks + 1, (T + TT - 1) / TT, B);
  if (grid.y > 0x7fffffffu || B > 65535 || grid.y > 65535u) return PBGDN_ERR_UNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  poison_prologue_outputs(prm, static_cast<long>(B) * T, st);
  if (has_tail && tail_out != tail) {
    debug_poison(tail_out, static_cast<size_t>(static_cast<long>(B) * (conv - 1) * channels *
                                               (tail_dtype == PBGDN_F32 ? 4 : 2)), st);
  }
  switch (in_dtype) {  // tails: row-major [B, conv-1, C], batch row b in slot b
    case PBGDN_F32: launch_prologue_and_edges<float>(prm, grid, B, st); break;
    case PBGDN_BF16: launch_prologue_and_edges<u16>(prm, grid, B, st); break;
    default: launch_prologue_and_edges<half_t>(prm, grid, B, st); break;
  }
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}

extern "C" int pbgdn_prologue_varlen_fwd(const void *qkv, long qkv_stride, const void *decay, long decay_stride,
                                         int in_dtype, const int32_t *cu_seqlens, int num_seqs, const void *tail,
                                         void *tail_out, int tail_dtype, long tail_slot_stride, long tail_row_stride,
                                         long tail_chan_stride, const int32_t *slot_idx,
                                         const uint8_t *has_initial_state, int num_slots, const float *conv_weight,
                                         int conv, const float *a_log, const float *dt_bias, void *q, void *k,
                                         void *v, int out_dtype, float *g, float *beta, int T, int Hk, int Hv,
                                         int K, int V, int l2_mode, void *stream) {
  using namespace pbgdn;
  if (T < 0 || num_seqs < 0 || num_slots < 0 || Hk <= 0 || Hv <= 0 || K <= 0 || V <= 0 || Hv % Hk != 0 ||
      conv < 0) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype) || !valid_dtype(tail_dtype) ||
      !(l2_mode == 0 || l2_mode == 1)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!(K == 64 || K == 128) || V % 8 != 0 || conv > MAX_CONV) return PBGDN_ERR_UNSUPPORTED;
  const long channels = 2L * Hk * K + static_cast<long>(Hv) * V;
  if (qkv_stride < channels || decay_stride < 2L * Hv || qkv_stride % 8 != 0) return PBGDN_ERR_INVALID_ARGUMENT;
  const long in_elem = in_dtype == PBGDN_F32 ? 4 : 2;
  if (static_cast<long>(TT + MAX_CONV) * qkv_stride * in_elem > 0x7ffffff0L - 64) return PBGDN_ERR_UNSUPPORTED;
  if (num_seqs == 0) return T == 0 ? PBGDN_OK : PBGDN_ERR_INVALID_ARGUMENT;
  const bool has_tail = conv > 1;
  if (!cu_seqlens || !qkv || !decay || !a_log || !dt_bias || !q || !k || !v || !g || !beta ||
      (conv > 0 && !conv_weight) ||
      (has_tail && (!tail || !tail_out || tail_slot_stride < 0 || tail_row_stride < 0 || tail_chan_stride < 0))) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!aligned16(qkv) || !aligned16(q) || !aligned16(k) || !aligned16(v)) return PBGDN_ERR_INVALID_ARGUMENT;
  if (channels / 8 > 0x7fffffffL / 16 || static_cast<long>(T) + TT > 0x7fffffffL) return PBGDN_ERR_UNSUPPORTED;
  PrologueParams prm{qkv, decay, tail, tail_out, conv_weight, a_log, dt_bias, q, k, v, g, beta, qkv_stride,
                     decay_stride, in_dtype, tail_dtype, out_dtype, 1, T, Hk, Hv, K, V, conv, l2_mode,
                     static_cast<int>(channels / 8), static_cast<int>((channels / 8 + UPW - 1) / UPW), cu_seqlens,
                     slot_idx, has_initial_state, num_seqs, num_slots, tail_slot_stride, tail_row_stride,
                     tail_chan_stride, 0, false};
  prm.gate_vec = gates_vectorize(decay, decay_stride, in_elem, g, beta, Hv);
  if (has_tail && tail_slot_stride % 8 == 0 && aligned16(tail) && aligned16(tail_out)) {
    if (tail_chan_stride == 1 && tail_row_stride % 8 == 0) prm.tail_vec = 1;
    if (tail_row_stride == 1 && tail_chan_stride == conv - 1) prm.tail_vec = 2;
  }
  const dim3 grid(prm.ch_blocks + 1, (T + TT - 1) / TT, 1);
  if (grid.y > 65535u || num_seqs > 65535) return PBGDN_ERR_UNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  poison_prologue_outputs(prm, T, st);
  switch (in_dtype) {
    case PBGDN_F32: launch_prologue_and_edges<float>(prm, grid, num_seqs, st); break;
    case PBGDN_BF16: launch_prologue_and_edges<u16>(prm, grid, num_seqs, st); break;
    default: launch_prologue_and_edges<half_t>(prm, grid, num_seqs, st); break;
  }
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}

extern "C" int pbgdn_epilogue_fwd(const void *o, int o_dtype, const void *gate, long gate_stride, int gate_dtype,
                                  const float *o_norm, float eps, void *out, int out_dtype, int B, int T, int Hv,
                                  int V, void *stream) {
  using namespace pbgdn;
  if (B < 0 || T < 0 || Hv <= 0 || V <= 0 || !(eps >= 0.f)) return PBGDN_ERR_INVALID_ARGUMENT;
  if (!valid_dtype(o_dtype) || !valid_dtype(gate_dtype) || !valid_dtype(out_dtype)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!(V == 64 || V == 128)) return PBGDN_ERR_UNSUPPORTED;
  if (gate_stride < static_cast<long>(Hv) * V || gate_stride % 8 != 0) return PBGDN_ERR_INVALID_ARGUMENT;
  const long rows = static_cast<long>(B) * T * Hv;
  if (rows == 0) return PBGDN_OK;
  if (!o || !gate || !o_norm || !out || !aligned16(o) || !aligned16(gate) || !aligned16(out)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  // 32-bit byte offsets below the out-of-range marker for a workgroup's gate
  // rows: its LNT / (V / 8) rows span at most that many tokens plus one
  const long wg_tokens = LNT / (V / 8) + 1;
  if (wg_tokens * gate_stride * (gate_dtype == PBGDN_F32 ? 4 : 2) > 0x7ffffff0L - 64) return PBGDN_ERR_UNSUPPORTED;
  EpilogueParams prm{o, gate, o_norm, out, gate_stride, o_dtype, gate_dtype, out_dtype, rows, Hv, V, eps};
  const long rows_per_wg = LNT / (V / 8) * EPI_ROWS;
  const long blocks = (rows + rows_per_wg - 1) / rows_per_wg;
  if (blocks > 0x7fffffffL) return PBGDN_ERR_UNSUPPORTED;
  const dim3 grid(static_cast<unsigned>(blocks));
  hipStream_t st = static_cast<hipStream_t>(stream);
  debug_poison(out, static_cast<size_t>(rows * V * (out_dtype == PBGDN_F32 ? 4 : 2)), st);  // debug builds: NaN first
  switch (o_dtype) {
    case PBGDN_F32: launch_epilogue<float>(gate_dtype, grid, st, prm); break;
    case PBGDN_BF16: launch_epilogue<u16>(gate_dtype, grid, st, prm); break;
    default: launch_epilogue<half_t>(gate_dtype, grid, st, prm); break;
  }
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}
