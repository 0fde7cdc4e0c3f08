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
//
// Epilogue: V/8 lanes per (token, value head) row, 8 elements each; the mean
// square over the head is a shuffle reduction inside the row group.
#include "chunk.hpp"  // buffer-resource helpers (rsrc, buf_load16, OUT_OF_RANGE)
#include "layer_math.hpp"

namespace pbgdn {
namespace {

constexpr int LNT = 256;       // threads per workgroup
constexpr int TT = 128;        // prologue tokens per workgroup
constexpr int TPL = TT / 16;   // tokens per lane row
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

__device__ __forceinline__ void store8(void *p, long i, int dtype, const float (&x)[8]) {
  if (dtype == PBGDN_F32) {
    *reinterpret_cast<float4_t *>(static_cast<float *>(p) + i) = float4_t{x[0], x[1], x[2], x[3]};
    *reinterpret_cast<float4_t *>(static_cast<float *>(p) + i + 4) = float4_t{x[4], x[5], x[6], x[7]};
  } else if (dtype == PBGDN_BF16) {
    uint4 u;  // v_cvt_pk_bf16_f32: round to nearest even, as float_to_bf16_bits
    u.x = bf16_pair(x[0], x[1]);
    u.y = bf16_pair(x[2], x[3]);
    u.z = bf16_pair(x[4], x[5]);
    u.w = bf16_pair(x[6], x[7]);
    *reinterpret_cast<uint4 *>(static_cast<u16 *>(p) + i) = u;
  } else {
    half8_t h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = static_cast<half_t>(x[e]);
    *reinterpret_cast<half8_t *>(static_cast<half_t *>(p) + i) = h;
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
template <bool WIDE>
__device__ __forceinline__ Raw8 load_raw8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  Raw8 x;
  x.a = buf_load16(r, off);
  x.b = WIDE ? buf_load16(r, off + 16) : uint4{0u, 0u, 0u, 0u};
  return x;
}

// Sum over groups of `width` lanes (a power of two up to 16), inside a
// 16-lane row.
__device__ __forceinline__ float group_sum(float x, int width) {
  for (int off = 1; off < width; off <<= 1) x += __shfl_xor(x, off, 64);
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
};

// CONV is the filter width (0: SiLU only). Every input row a lane needs (its
// TPL tokens and the CONV-1 before them) is loaded before any is used, so the
// loads of a lane overlap instead of following one another.
template <int CONV, typename TIn>
__global__ __launch_bounds__(LNT) void prologue_kernel(PrologueParams p) {
  constexpr int IN = dtype_of<TIn>();
  constexpr int TAIL = CONV > 1 ? CONV - 1 : 0;  // rows of the carried tail
  constexpr int HALO = CONV > 1 ? CONV - 1 : 0;  // rows before a lane's first token
  const int tid = threadIdx.x;
  const int b = blockIdx.z;
  const int t_tile = blockIdx.y * TT;
  if (static_cast<int>(blockIdx.x) >= p.ch_blocks) {
    // Gates of the tile: g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b).
    const int n = min(TT, p.T - t_tile) * p.Hv;
    for (int i = tid; i < n; i += LNT) {
      const int t = t_tile + i / p.Hv;
      const int h = i % p.Hv;
      const long row = static_cast<long>(b) * p.T + t;
      const float a = load_elem(p.decay, row * p.decay_stride + h, IN);
      const float bb = load_elem(p.decay, row * p.decay_stride + p.Hv + h, IN);
      p.g[row * p.Hv + h] = -expf(p.a_log[h]) * softplusf(a + p.dt_bias[h]);
      p.beta[row * p.Hv + h] = sigmoidf(bb);
    }
    return;
  }
  const int u = blockIdx.x * 16 + (tid & 15);   // this lane's 8-channel unit
  const int tl = tid >> 4;                       // lane row: tokens tl*TPL ..
  const int t_first = t_tile + tl * TPL;
  if (t_first >= p.T) return;  // the whole 16-lane row: no tokens (no shuffle partner is lost)
  const bool live = u < p.units;
  const int c0 = 8 * (live ? u : 0);
  const int qk_units = p.Hk * p.K / 8;
  const long seq_row = static_cast<long>(b) * p.T;
  const long tail_base = static_cast<long>(b) * TAIL;
  const long chans = static_cast<long>(p.units) * 8;
  // Every row this lane needs is loaded unconditionally through buffer
  // resources that span exactly this sequence's rows and its carried tail; a
  // row outside them (or a dead lane) gets an out-of-range offset and reads
  // zeros. No load then waits on a branch merge: they all issue back to back.
  const auto rq = rsrc(static_cast<const TIn *>(p.qkv) + seq_row * p.qkv_stride,
                       (static_cast<long>(p.T - 1) * p.qkv_stride + chans) * static_cast<long>(sizeof(TIn)));
  const int tail_elem = p.tail_dtype == PBGDN_F32 ? 4 : 2;
  const auto rt = rsrc(static_cast<const unsigned char *>(p.tail) + tail_base * chans * tail_elem,
                       TAIL > 0 ? static_cast<long>(TAIL) * chans * tail_elem : 0);
  Raw8 raw[HALO + TPL], raw_tail[HALO > 0 ? HALO : 1];  // rows t_first - HALO ..
#pragma unroll
  for (int m = 0; m < HALO + TPL; ++m) {
    const int t = t_first - HALO + m;
    const uint32_t off = live && t >= 0 && t < p.T
                             ? (static_cast<uint32_t>(t) * static_cast<uint32_t>(p.qkv_stride) + c0) * sizeof(TIn)
                             : OUT_OF_RANGE;
    raw[m] = load_raw8<sizeof(TIn) == 4>(rq, off);
  }
#pragma unroll
  for (int m = 0; m < HALO; ++m) {  // tail rows: only the first lane row of the first tile has any
    const int t = t_first - HALO + m;
    const uint32_t off = live && t < 0 && t >= -TAIL
                             ? (static_cast<uint32_t>(TAIL + t) * static_cast<uint32_t>(chans) + c0) * tail_elem
                             : OUT_OF_RANGE;
    raw_tail[m] = load_raw8<true>(rt, off);  // 32 bytes whatever the tail's type: no branch
  }
  float xr[HALO + TPL][8];
#pragma unroll
  for (int m = 0; m < HALO + TPL; ++m) {
    decode8<TIn>(raw[m], xr[m]);
    if (m < HALO && t_first - HALO + m < 0) {
      // the carried tail, rounded through the input dtype as in cat(tail.to(x.dtype), x)
      float xt[8];
      decode8(raw_tail[m < HALO ? m : 0], p.tail_dtype, xt);
#pragma unroll
      for (int e = 0; e < 8; ++e) xr[m][e] = through(xt[e], IN);
    }
  }
  auto input_row = [&](int t, float (&x)[8]) {  // used only for the old-tail rows of the new tail
    if (live && t < 0 && t >= -TAIL) {
      load8(p.tail, (tail_base + TAIL + t) * chans + c0, p.tail_dtype, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = through(x[e], IN);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = 0.f;
    }
  };
  float w[8][CONV > 0 ? CONV : 1];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
#pragma unroll
    for (int j = 0; j < CONV; ++j) w[e][j] = p.conv_weight[(c0 + e) * CONV + j];
  }
  // The new tail: the last CONV-1 rows of tail ++ x. Rows that still come
  // from the old tail (T < CONV-1) are written once, by lane row 0 of the
  // first tile.
  if (TAIL > 0 && live && t_tile == 0 && tl == 0) {
    for (int r = 0; r + p.T < TAIL; ++r) {
      float x[8];
      input_row(p.T + r - TAIL, x);
      store8(p.tail_out, (tail_base + r) * chans + c0, p.tail_dtype, x);
    }
  }
  int kind = 2, head = 0, off = 0;  // 0 q, 1 k, 2 v
  if (u < qk_units) {
    kind = 0;
    head = c0 / p.K;
    off = c0 % p.K;
  } else if (u < 2 * qk_units) {
    kind = 1;
    head = (c0 - 8 * qk_units) / p.K;
    off = (c0 - 8 * qk_units) % p.K;
  } else {
    head = (c0 - 16 * qk_units) / p.V;
    off = (c0 - 16 * qk_units) % p.V;
  }
  const int head_lanes = p.K / 8;
  // Output element index of token t_first and the step per token.
  const int out_heads = kind < 2 ? p.Hk : p.Hv;
  const int out_width = kind < 2 ? p.K : p.V;
  void *const out_ptr = kind == 0 ? p.q : kind == 1 ? p.k : p.v;
  const long out_step = static_cast<long>(out_heads) * out_width;
  const long out0 = (seq_row + t_first) * out_step + static_cast<long>(head) * out_width + off;
  const float l2_eps = 1e-6f;
#pragma unroll
  for (int i = 0; i < TPL; ++i) {
    const int t = t_first + i;
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = CONV == 0 ? xr[HALO + i][e] : 0.f;
#pragma unroll
      for (int j = 0; j < CONV; ++j) acc += w[e][j] * xr[HALO + i - (CONV - 1) + j][e];  // tap j: row t-(CONV-1)+j
      y[e] = siluf(acc);
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += y[e] * y[e];
    ss = group_sum(ss, head_lanes);  // every lane of the row takes part
    if (live && t < p.T) {
      if (kind < 2) {
        const float n = p.l2_mode == 0 ? 1.f / fmaxf(sqrtf(ss), l2_eps) : rsqrtf(ss + l2_eps);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] *= n;
      }
      store8(out_ptr, out0 + i * out_step, p.out_dtype, y);
      if (TAIL > 0 && t >= p.T - TAIL) {
        store8(p.tail_out, (tail_base + t - (p.T - TAIL)) * chans + c0, p.tail_dtype, xr[HALO + i]);
      }
    }
  }
}

template <typename TIn>
void launch_prologue(int conv, dim3 grid, hipStream_t st, const PrologueParams &prm) {
  switch (conv) {
    case 0: hipLaunchKernelGGL((prologue_kernel<0, TIn>), grid, dim3(LNT), 0, st, prm); break;
    case 1: hipLaunchKernelGGL((prologue_kernel<1, TIn>), grid, dim3(LNT), 0, st, prm); break;
    case 2: hipLaunchKernelGGL((prologue_kernel<2, TIn>), grid, dim3(LNT), 0, st, prm); break;
    case 3: hipLaunchKernelGGL((prologue_kernel<3, TIn>), grid, dim3(LNT), 0, st, prm); break;
    default: hipLaunchKernelGGL((prologue_kernel<4, TIn>), grid, dim3(LNT), 0, st, prm); break;
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

template <typename TO, typename TG, int V>
__global__ __launch_bounds__(LNT) void epilogue_kernel(EpilogueParams p) {
  constexpr int LANES = V / 8;             // lanes per (token, head) row
  constexpr int GROUPS = LNT / LANES;      // row groups per workgroup
  const int tid = threadIdx.x;
  const int c0 = 8 * (tid % LANES);
  const long row0 = static_cast<long>(blockIdx.x) * GROUPS * EPI_ROWS + tid / LANES;
  const auto ro = rsrc(p.o, p.rows * V * static_cast<long>(sizeof(TO)));
  const auto rg = rsrc(p.gate, (p.rows / p.Hv) * p.gate_stride * static_cast<long>(sizeof(TG)));
  Raw8 ro8[EPI_ROWS], rg8[EPI_ROWS];
#pragma unroll
  for (int j = 0; j < EPI_ROWS; ++j) {
    const long row = row0 + static_cast<long>(j) * GROUPS;
    const bool live = row < p.rows;
    const uint32_t token = static_cast<uint32_t>(row) / static_cast<uint32_t>(p.Hv);
    const uint32_t h = static_cast<uint32_t>(row) - token * static_cast<uint32_t>(p.Hv);
    ro8[j] = load_raw8<sizeof(TO) == 4>(ro, live ? static_cast<uint32_t>((row * V + c0) * sizeof(TO)) : OUT_OF_RANGE);
    rg8[j] = load_raw8<sizeof(TG) == 4>(
        rg, live ? static_cast<uint32_t>((token * p.gate_stride + h * V + c0) * sizeof(TG)) : OUT_OF_RANGE);
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
    if (row < p.rows) store8(p.out, row * V + c0, p.out_dtype, y);
  }
}

template <typename TO, int V>
void launch_epilogue_v(int gate_dtype, dim3 grid, hipStream_t st, const EpilogueParams &prm) {
  switch (gate_dtype) {
    case PBGDN_F32: hipLaunchKernelGGL((epilogue_kernel<TO, float, V>), grid, dim3(LNT), 0, st, prm); break;
    case PBGDN_BF16: hipLaunchKernelGGL((epilogue_kernel<TO, u16, V>), grid, dim3(LNT), 0, st, prm); break;
    default: hipLaunchKernelGGL((epilogue_kernel<TO, half_t, V>), grid, dim3(LNT), 0, st, prm); break;
  }
}
template <typename TO>
void launch_epilogue(int gate_dtype, dim3 grid, hipStream_t st, const EpilogueParams &prm) {
  if (prm.V == 64) {
    launch_epilogue_v<TO, 64>(gate_dtype, grid, st, prm);
  } else {
    launch_epilogue_v<TO, 128>(gate_dtype, grid, st, prm);
  }
}

bool valid_dtype(int d) { return d == PBGDN_F32 || d == PBGDN_BF16 || d == PBGDN_F16; }
bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

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
  // A sequence's rows are addressed with 32-bit byte offsets below the out-of-range marker.
  const long in_elem = in_dtype == PBGDN_F32 ? 4 : 2;
  if (static_cast<long>(T) * qkv_stride * in_elem > 0x7ffffff0L - 64) return PBGDN_ERR_UNSUPPORTED;
  if (static_cast<long>(B) * T == 0) return PBGDN_OK;
  const bool has_tail = conv > 1;
  if (!qkv || !decay || !a_log || !dt_bias || !q || !k || !v || !g || !beta || (conv > 0 && !conv_weight) ||
      (has_tail && (!tail || !tail_out || tail == tail_out))) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!aligned16(qkv) || !aligned16(q) || !aligned16(k) || !aligned16(v) ||
      (has_tail && (!aligned16(tail) || !aligned16(tail_out)))) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (channels / 8 > 0x7fffffffL / 16 || static_cast<long>(T) + TT > 0x7fffffffL) return PBGDN_ERR_UNSUPPORTED;
  PrologueParams prm{qkv, decay, tail, tail_out, conv_weight, a_log, dt_bias, q, k, v, g, beta, qkv_stride,
                     decay_stride, in_dtype, tail_dtype, out_dtype, B, T, Hk, Hv, K, V, conv, l2_mode,
                     static_cast<int>(channels / 8), static_cast<int>((channels / 8 + 15) / 16)};
  const dim3 grid(prm.ch_blocks + 1, (T + TT - 1) / TT, B);
  if (grid.y > 0x7fffffffu || B > 65535 || grid.y > 65535u) return PBGDN_ERR_UNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (in_dtype) {
    case PBGDN_F32: launch_prologue<float>(conv, grid, st, prm); break;
    case PBGDN_BF16: launch_prologue<u16>(conv, grid, st, prm); break;
    default: launch_prologue<half_t>(conv, grid, st, prm); break;
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
  // 32-bit byte offsets below the out-of-range marker for o and the gate rows
  const long o_bytes = rows * V * (o_dtype == PBGDN_F32 ? 4 : 2);
  const long g_bytes = static_cast<long>(B) * T * gate_stride * (gate_dtype == PBGDN_F32 ? 4 : 2);
  if (o_bytes > 0x7ffffff0L - 64 || g_bytes > 0x7ffffff0L - 64) return PBGDN_ERR_UNSUPPORTED;
  EpilogueParams prm{o, gate, o_norm, out, gate_stride, o_dtype, gate_dtype, out_dtype, rows, Hv, V, eps};
  const long rows_per_wg = LNT / (V / 8) * EPI_ROWS;
  const long blocks = (rows + rows_per_wg - 1) / rows_per_wg;
  if (blocks > 0x7fffffffL) return PBGDN_ERR_UNSUPPORTED;
  const dim3 grid(static_cast<unsigned>(blocks));
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (o_dtype) {
    case PBGDN_F32: launch_epilogue<float>(gate_dtype, grid, st, prm); break;
    case PBGDN_BF16: launch_epilogue<u16>(gate_dtype, grid, st, prm); break;
    default: launch_epilogue<half_t>(gate_dtype, grid, st, prm); break;
  }
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}
