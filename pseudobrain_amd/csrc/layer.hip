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
#include "common.hpp"

namespace pbgdn {
namespace {

constexpr int LNT = 256;       // threads per workgroup
constexpr int TT = 128;        // prologue tokens per workgroup
constexpr int TPL = TT / 16;   // tokens per lane row
constexpr int MAX_CONV = 4;

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

__device__ __forceinline__ void store8(void *p, long i, int dtype, const float (&x)[8]) {
  if (dtype == PBGDN_F32) {
    *reinterpret_cast<float4_t *>(static_cast<float *>(p) + i) = float4_t{x[0], x[1], x[2], x[3]};
    *reinterpret_cast<float4_t *>(static_cast<float *>(p) + i + 4) = float4_t{x[4], x[5], x[6], x[7]};
  } else if (dtype == PBGDN_BF16) {
    uint4 u;
    u.x = float_to_bf16_bits(x[0]) | (static_cast<uint32_t>(float_to_bf16_bits(x[1])) << 16);
    u.y = float_to_bf16_bits(x[2]) | (static_cast<uint32_t>(float_to_bf16_bits(x[3])) << 16);
    u.z = float_to_bf16_bits(x[4]) | (static_cast<uint32_t>(float_to_bf16_bits(x[5])) << 16);
    u.w = float_to_bf16_bits(x[6]) | (static_cast<uint32_t>(float_to_bf16_bits(x[7])) << 16);
    *reinterpret_cast<uint4 *>(static_cast<u16 *>(p) + i) = u;
  } else {
    half8_t h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = static_cast<half_t>(x[e]);
    *reinterpret_cast<half8_t *>(static_cast<half_t *>(p) + i) = h;
  }
}

// The value a float takes after a round trip through `dtype` (the reference
// casts the carried tail to the input's dtype before the convolution).
__device__ __forceinline__ float through(float x, int dtype) {
  if (dtype == PBGDN_BF16) return bf16_bits_to_float(float_to_bf16_bits(x));
  if (dtype == PBGDN_F16) return static_cast<float>(static_cast<half_t>(x));
  return x;
}

__device__ __forceinline__ float sigmoidf(float x) { return 1.f / (1.f + expf(-x)); }
__device__ __forceinline__ float siluf(float x) { return x * sigmoidf(x); }
// torch.nn.functional.softplus with beta 1, threshold 20
__device__ __forceinline__ float softplusf(float x) { return x > 20.f ? x : log1pf(expf(x)); }

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

__global__ __launch_bounds__(LNT) void prologue_kernel(PrologueParams p) {
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
      const float a = load_elem(p.decay, row * p.decay_stride + h, p.in_dtype);
      const float bb = load_elem(p.decay, row * p.decay_stride + p.Hv + h, p.in_dtype);
      p.g[row * p.Hv + h] = -expf(p.a_log[h]) * softplusf(a + p.dt_bias[h]);
      p.beta[row * p.Hv + h] = sigmoidf(bb);
    }
    return;
  }
  const int u = blockIdx.x * 16 + (tid & 15);   // this lane's 8-channel unit
  const int tl = tid >> 4;                       // lane row: tokens tl*TPL ..
  const bool live = u < p.units;
  const int c0 = 8 * (live ? u : 0);
  const int conv = p.conv;
  const int tail_rows = conv > 1 ? conv - 1 : 0;
  const int qk_units = p.Hk * p.K / 8;
  float w[8][MAX_CONV];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
#pragma unroll
    for (int j = 0; j < MAX_CONV; ++j) w[e][j] = (conv > 0 && j < conv) ? p.conv_weight[(c0 + e) * conv + j] : 0.f;
  }
  const long seq_row = static_cast<long>(b) * p.T;
  const long tail_base = static_cast<long>(b) * tail_rows;
  const long chans = static_cast<long>(p.units) * 8;
  // Input row t of this sequence (t < 0: the carried tail, rounded through
  // the input dtype as in cat(tail.to(x.dtype), x)).
  auto input_row = [&](int t, float (&x)[8]) {
    if (!live) {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = 0.f;
    } else if (t >= 0) {
      load8(p.qkv, (seq_row + t) * p.qkv_stride + c0, p.in_dtype, x);
    } else {
      load8(p.tail, (tail_base + tail_rows + t) * chans + c0, p.tail_dtype, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = through(x[e], p.in_dtype);
    }
  };
  const int t_first = t_tile + tl * TPL;
  float prev[MAX_CONV - 1][8];  // rows t-3, t-2, t-1
#pragma unroll
  for (int m = 0; m < MAX_CONV - 1; ++m) {
    const int t = t_first - (MAX_CONV - 1) + m;
    if (t >= -tail_rows && t < p.T) {  // rows past T: this lane row has no tokens
      input_row(t, prev[m]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) prev[m][e] = 0.f;
    }
  }
  // The new tail: the last conv-1 rows of tail ++ x. Rows that still come
  // from the old tail (T < conv-1) are written once, by lane row 0 of the
  // first tile.
  if (live && tail_rows > 0 && t_tile == 0 && tl == 0) {
    for (int r = 0; r + p.T < tail_rows; ++r) {
      float x[8];
      input_row(p.T + r - tail_rows, x);
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
#pragma unroll 1
  for (int i = 0; i < TPL; ++i) {
    const int t = t_first + i;
    if (t_tile + tl * TPL >= p.T) break;  // uniform over the 16-lane row
    const bool valid = t < p.T;
    float x[8];
    if (valid) {
      input_row(t, x);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = 0.f;
    }
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (conv == 0) {
        y[e] = x[e];
      } else {
        float acc = w[e][conv - 1] * x[e];
#pragma unroll
        for (int j = 0; j < MAX_CONV - 1; ++j) {
          // tap j of a width-conv filter reads row t - (conv - 1) + j
          if (j < conv - 1) acc += w[e][j] * prev[MAX_CONV - conv + j][e];
        }
        y[e] = acc;
      }
      y[e] = siluf(y[e]);
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += y[e] * y[e];
    ss = group_sum(ss, head_lanes);  // every lane of the row takes part
    if (live && valid) {
      if (kind < 2) {
        const float n = p.l2_mode == 0 ? 1.f / fmaxf(sqrtf(ss), 1e-6f) : rsqrtf(ss + 1e-6f);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] *= n;
        const long dst = ((seq_row + t) * p.Hk + head) * static_cast<long>(p.K) + off;
        store8(kind == 0 ? p.q : p.k, dst, p.out_dtype, y);
      } else {
        store8(p.v, ((seq_row + t) * p.Hv + head) * static_cast<long>(p.V) + off, p.out_dtype, y);
      }
      if (t >= p.T - tail_rows) store8(p.tail_out, (tail_base + t - (p.T - tail_rows)) * chans + c0, p.tail_dtype, x);
    }
#pragma unroll
    for (int m = 0; m < MAX_CONV - 2; ++m) {
#pragma unroll
      for (int e = 0; e < 8; ++e) prev[m][e] = prev[m + 1][e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) prev[MAX_CONV - 2][e] = x[e];
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

__global__ __launch_bounds__(LNT) void epilogue_kernel(EpilogueParams p) {
  const int lanes = p.V / 8;            // lanes per (token, head) row
  const int rows_per_wg = LNT / lanes;
  const long row = static_cast<long>(blockIdx.x) * rows_per_wg + threadIdx.x / lanes;
  const int c0 = 8 * (threadIdx.x % lanes);
  const bool live = row < p.rows;
  float o[8];
  if (live) {
    load8(p.o, row * p.V + c0, p.o_dtype, o);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.f;
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += o[e] * o[e];
  ss = group_sum(ss, lanes);
  if (!live) return;
  const float r = rsqrtf(ss / p.V + p.eps);
  const long token = row / p.Hv;
  const int h = static_cast<int>(row % p.Hv);
  float gt[8];
  load8(p.gate, token * p.gate_stride + static_cast<long>(h) * p.V + c0, p.gate_dtype, gt);
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = o[e] * r * p.o_norm[c0 + e] * siluf(gt[e]);
  store8(p.out, row * p.V + c0, p.out_dtype, y);
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
  hipLaunchKernelGGL(prologue_kernel, grid, dim3(LNT), 0, static_cast<hipStream_t>(stream), prm);
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
  EpilogueParams prm{o, gate, o_norm, out, gate_stride, o_dtype, gate_dtype, out_dtype, rows, Hv, V, eps};
  const long rows_per_wg = LNT / (V / 8);
  const long blocks = (rows + rows_per_wg - 1) / rows_per_wg;
  if (blocks > 0x7fffffffL) return PBGDN_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(epilogue_kernel, dim3(static_cast<unsigned>(blocks)), dim3(LNT), 0,
                     static_cast<hipStream_t>(stream), prm);
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}
