// Fused decode step of a Gated DeltaNet layer for gfx950: one token per
// sequence, from the input projection to the gated, normed output, with the
// conv tail and the recurrent state updated in place in their slot pools.
//
// Reference: GatedDeltaNetLayer.forward at T = 1, pseudobrain/gated_deltanet.py:415-441:
// short_convolution (:314-338), l2_normalize (:59-70), the gates (:425-427),
// delta_rule_sequential (:93-107; select_kernel picks it for T <= 4) and the
// epilogue (:439-441). q, k and v stay float32 from the convolution into the
// recurrence, as on the reference's sequential path (no cast to the matmul
// precision there).
//
// One workgroup of 256 threads per (sequence, key head). It first forms every
// input of the step in LDS (q and k of its key head; v, SiLU(gate) and the
// gates of the Hv/Hk value heads that read them), then runs the recurrent
// step and the epilogue of each of those value heads. It alone reads and writes
// the conv-tail channels of its heads, so each tail shifts in place with no
// race (a thread reads its channel's rows before it writes them). The state
// step is the one-token step of the recurrent kernel: the state in registers
// (packed as loaded when it is 16-bit), float32 arithmetic, buffer I/O; no
// input work is left to hold registers while a state is in them.
#include "layer_math.hpp"
#include "state_io.hpp"
#include "device.hpp"

namespace pbgdn {
namespace {

constexpr int DNT = 256;
constexpr int DECODE_MAX_CONV = 4;
constexpr int DECODE_MAX_GROUP = 8;  // value heads per key head

struct DecodeLayerParams {
  const void *z;  // [B, z_stride] rows: q | k | v | gate | a | b
  long z_stride;
  int in_dtype;
  void *conv_state;  // (slot, row j, channel c) at slot*conv_ss + j*conv_rs + c*conv_cs
  int conv_dtype;
  long conv_ss, conv_rs, conv_cs;
  const float *conv_weight;  // [channels, conv]
  int conv;
  const float *a_log, *dt_bias;
  int l2_mode;
  void *state;  // [num_states, Hv, K, V], state_dtype (the kernel's TS)
  const int32_t *state_idx;
  int num_states;
  const float *o_norm;
  float eps;
  void *hs;  // [B, Hv * V], out_dtype
  int out_dtype;
  int Hk, Hv;
  float scale;
};

// SiLU of the causal convolution of channel c at the current token: the
// conv-1 rows of the slot's tail (rounded through the input dtype, as the
// reference joins the tail to the input) then the input x, summed in the
// reference's tap order; the tail then shifts by one row in place (the new
// last row is x).
__device__ float conv_channel(const DecodeLayerParams &p, long slot, long c, float x) {
  if (p.conv == 0) return siluf(x);
  const float *w = p.conv_weight + c * p.conv;
  const long base = slot * p.conv_ss + c * p.conv_cs;
  float t[DECODE_MAX_CONV - 1];
#pragma unroll
  for (int j = 0; j < DECODE_MAX_CONV - 1; ++j) {
    t[j] = j < p.conv - 1 ? through(load_elem(p.conv_state, base + j * p.conv_rs, p.conv_dtype), p.in_dtype) : 0.f;
  }
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < DECODE_MAX_CONV - 1; ++j) {
    if (j < p.conv - 1) acc += w[j] * t[j];
  }
  acc += w[p.conv - 1] * x;
#pragma unroll
  for (int j = 0; j < DECODE_MAX_CONV - 1; ++j) {
    if (j < p.conv - 1) store_elem(p.conv_state, base + j * p.conv_rs, p.conv_dtype, j + 1 < p.conv - 1 ? t[j + 1] : x);
  }
  return siluf(acc);
}

// conv_channel for a bf16 input and DECODE_MAX_CONV taps: the tail rows
// (oldest first, already rounded through bf16) and x, summed in
// conv_channel's order.
__device__ __forceinline__ float conv4(const float *w, float a, float b, float c, float x) {
  float acc = 0.f;
  acc += w[0] * a;
  acc += w[1] * b;
  acc += w[2] * c;
  acc += w[3] * x;
  return siluf(acc);
}

// A tail element of type TC (bf16 bits or float) as conv_channel reads it
// for a bf16 input (rounded through bf16), and a value stored back as
// store_elem would store it.
template <typename TC>
__device__ __forceinline__ float tail_in(TC x) {
  if constexpr (std::is_same<TC, u16>::value) {
    return bf16_bits_to_float(x);
  } else {
    return bf16_bits_to_float(float_to_bf16_bits(x));
  }
}
template <typename TC>
__device__ __forceinline__ TC tail_out(float x) {
  if constexpr (std::is_same<TC, u16>::value) {
    return float_to_bf16_bits(x);
  } else {
    return x;
  }
}

// CP: the state's cache policy (state_io.hpp).
template <int K, int V, typename TS, int CP>
__global__ __launch_bounds__(DNT, (sizeof(TS) == 2 ? 5 : 4)) void decode_layer_kernel(DecodeLayerParams p) {
  constexpr bool PACKED = sizeof(TS) == 2;
  constexpr int NW = DNT / 64;
  constexpr int CG = V / 4;    // float4 column groups
  constexpr int RG = DNT / CG;  // row groups
  constexpr int RPT = K / RG;  // rows per thread
  static_assert(CG <= 64 && 64 % CG == 0 && RG * RPT == K, "head widths 64 or 128");
  using IO = StateIO<TS>;
  constexpr uint32_t ROW_STEP = RG * V * sizeof(TS);
  constexpr uint32_t STATE_BYTES = K * V * sizeof(TS);

  const int hk = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int cg = tid % CG;
  const int rg = tid / CG;
  const int group = p.Hv / p.Hk;
  const long qk_width = static_cast<long>(p.Hk) * K;
  const long channels = 2 * qk_width + static_cast<long>(p.Hv) * V;
  const long zrow = b * p.z_stride;
  const long hs_row = static_cast<long>(b) * p.Hv * V;

  __shared__ float sk[K];
  __shared__ float sq[K];
  __shared__ float sv[DECODE_MAX_GROUP * V];
  __shared__ float sgate[DECODE_MAX_GROUP * V];  // SiLU(gate)
  __shared__ float salpha[DECODE_MAX_GROUP];
  __shared__ float sbeta[DECODE_MAX_GROUP];
  __shared__ float4_t red_k[NW][CG];
  __shared__ float4_t red_q[NW][CG];
  __shared__ float part[2][NW];
  PBGDN_POISON_LDS(sk, sizeof(sk));
  PBGDN_POISON_LDS(sq, sizeof(sq));
  PBGDN_POISON_LDS(sv, sizeof(sv));
  PBGDN_POISON_LDS(sgate, sizeof(sgate));
  PBGDN_POISON_LDS(salpha, sizeof(salpha));
  PBGDN_POISON_LDS(sbeta, sizeof(sbeta));
  PBGDN_POISON_LDS(red_k, sizeof(red_k));
  PBGDN_POISON_LDS(red_q, sizeof(red_q));
  PBGDN_POISON_LDS(part, sizeof(part));
  PBGDN_POISON_SYNC();

  const long slot = p.state_idx ? static_cast<long>(p.state_idx[b]) : static_cast<long>(b);
  if (slot < 0 || slot >= p.num_states) {  // padded entry: nothing is read or written but a zero output
    for (int i = tid; i < group * V; i += DNT) store_elem(p.hs, hs_row + static_cast<long>(hk) * group * V + i, p.out_dtype, 0.f);
    return;
  }

  const uint32_t voff = (rg * V + 4 * cg) * sizeof(TS);
  typename IO::Raw raw[PACKED ? RPT : 1];
  float4_t s[PACKED ? 1 : RPT];
  auto state_rsrc = [&](int h) {
    return rsrc(static_cast<TS *>(p.state) + (slot * p.Hv + h) * static_cast<long>(K) * V, STATE_BYTES);
  };
  auto load_state = [&](int h) {
    const __amdgpu_buffer_rsrc_t r = state_rsrc(h);
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      if constexpr (PACKED) {
        raw[j] = IO::template load<CP>(r, voff, j * ROW_STEP);
      } else {
        s[j] = IO::widen(IO::template load<CP>(r, voff, j * ROW_STEP));
      }
    }
  };
  auto row = [&](int j) -> float4_t {
    if constexpr (PACKED) {
      return IO::widen(raw[j]);
    } else {
      return s[j];
    }
  };

  // Every input of the step first, before any state is in registers: q and
  // k of the key head (convolution, SiLU, L2 norm over the head), then v,
  // SiLU(gate) and the decay/beta gates of each value head of the group.
  float yq = 0.f, yk = 0.f;
  const long v0 = 2 * qk_width + static_cast<long>(hk) * group * V;  // the group's v channels
  // The serving cases, a bf16 projection with a bf16 or float32 tail of
  // DECODE_MAX_CONV taps: a channel's loads (typed, no branch on a runtime
  // dtype between them) all issue before their first use, so a thread waits
  // once per channel group instead of once per load. Same values as the
  // general path below.
  auto typed_inputs = [&](auto tag) {
    using TC = decltype(tag);
    const u16 *z16 = static_cast<const u16 *>(p.z);
    TC *cs = static_cast<TC *>(p.conv_state);
    const long rs = p.conv_rs;
    if (tid < K) {
      const long cq = static_cast<long>(hk) * K + tid, ck = qk_width + cq;
      const long bq = slot * p.conv_ss + cq * p.conv_cs, bk = slot * p.conv_ss + ck * p.conv_cs;
      const u16 zq = z16[zrow + cq], zk = z16[zrow + ck];
      const TC q0 = cs[bq], q1 = cs[bq + rs], q2 = cs[bq + 2 * rs];
      const TC k0 = cs[bk], k1 = cs[bk + rs], k2 = cs[bk + 2 * rs];
      const float xq = bf16_bits_to_float(zq), xk = bf16_bits_to_float(zk);
      const float fq1 = tail_in(q1), fq2 = tail_in(q2), fk1 = tail_in(k1), fk2 = tail_in(k2);
      yq = conv4(p.conv_weight + cq * DECODE_MAX_CONV, tail_in(q0), fq1, fq2, xq);
      yk = conv4(p.conv_weight + ck * DECODE_MAX_CONV, tail_in(k0), fk1, fk2, xk);
      cs[bq] = tail_out<TC>(fq1);
      cs[bq + rs] = tail_out<TC>(fq2);
      cs[bq + 2 * rs] = tail_out<TC>(xq);
      cs[bk] = tail_out<TC>(fk1);
      cs[bk + rs] = tail_out<TC>(fk2);
      cs[bk + 2 * rs] = tail_out<TC>(xk);
    }
    for (int e = tid; e < group * V; e += DNT) {
      const long cv = v0 + e, bv = slot * p.conv_ss + cv * p.conv_cs;
      const u16 zv = z16[zrow + cv], zg = z16[zrow + channels + static_cast<long>(hk) * group * V + e];
      const TC a0 = cs[bv], a1 = cs[bv + rs], a2 = cs[bv + 2 * rs];
      const float xv = bf16_bits_to_float(zv), f1 = tail_in(a1), f2 = tail_in(a2);
      sv[e] = conv4(p.conv_weight + cv * DECODE_MAX_CONV, tail_in(a0), f1, f2, xv);
      sgate[e] = siluf(bf16_bits_to_float(zg));
      cs[bv] = tail_out<TC>(f1);
      cs[bv + rs] = tail_out<TC>(f2);
      cs[bv + 2 * rs] = tail_out<TC>(xv);
    }
    if (tid < group) {
      const int h = hk * group + tid;
      const long ab = zrow + channels + static_cast<long>(p.Hv) * V + h;
      const float za = bf16_bits_to_float(z16[ab]), zb = bf16_bits_to_float(z16[ab + p.Hv]);
      salpha[tid] = expf(-expf(p.a_log[h]) * softplusf(za + p.dt_bias[h]));
      sbeta[tid] = sigmoidf(zb);
    }
  };
  const bool typed = p.in_dtype == PBGDN_BF16 && p.conv == DECODE_MAX_CONV;
  if (typed && p.conv_dtype == PBGDN_BF16) {
    typed_inputs(u16{});
  } else if (typed && p.conv_dtype == PBGDN_F32) {
    typed_inputs(float{});
  } else {
    if (tid < K) {
      const long cq = static_cast<long>(hk) * K + tid;
      const long ck = qk_width + cq;
      yq = conv_channel(p, slot, cq, load_elem(p.z, zrow + cq, p.in_dtype));
      yk = conv_channel(p, slot, ck, load_elem(p.z, zrow + ck, p.in_dtype));
    }
    for (int e = tid; e < group * V; e += DNT) {
      sv[e] = conv_channel(p, slot, v0 + e, load_elem(p.z, zrow + v0 + e, p.in_dtype));
      sgate[e] = siluf(load_elem(p.z, zrow + channels + static_cast<long>(hk) * group * V + e, p.in_dtype));
    }
    if (tid < group) {
      const int h = hk * group + tid;
      const long ab = zrow + channels + static_cast<long>(p.Hv) * V + h;
      salpha[tid] = expf(-expf(p.a_log[h]) * softplusf(load_elem(p.z, ab, p.in_dtype) + p.dt_bias[h]));
      sbeta[tid] = sigmoidf(load_elem(p.z, ab + p.Hv, p.in_dtype));
    }
  }
  const float pq2 = wave_sum(yq * yq);
  const float pk2 = wave_sum(yk * yk);
  if (lane == 0) {
    part[0][wave] = pq2;
    part[1][wave] = pk2;
  }
  __syncthreads();
  float ssq = 0.f, ssk = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    ssq += part[0][w];
    ssk += part[1][w];
  }
  constexpr float L2_EPS = 1e-6f;  // gated_deltanet.py:56
  const float nq = p.l2_mode == 0 ? 1.f / fmaxf(sqrtf(ssq), L2_EPS) : rsqrtf(ssq + L2_EPS);
  const float nk = p.l2_mode == 0 ? 1.f / fmaxf(sqrtf(ssk), L2_EPS) : rsqrtf(ssk + L2_EPS);
  if (tid < K) {
    sq[tid] = yq * nq * p.scale;
    sk[tid] = yk * nk;
  }
  __syncthreads();
  float kq = 0.f;
  for (int e = lane; e < K; e += 64) kq += sk[e] * sq[e];
  kq = wave_sum(kq);

  for (int i = 0; i < group; ++i) {
    const int h = hk * group + i;
    load_state(h);
    const float alpha = salpha[i];
    const float bt = sbeta[i];
    const float4_t vv = {sv[i * V + 4 * cg], sv[i * V + 4 * cg + 1], sv[i * V + 4 * cg + 2], sv[i * V + 4 * cg + 3]};

    float4_t pk = {0.f, 0.f, 0.f, 0.f};
    float4_t pq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const float4_t sj = row(j);
      pk += sj * sk[rg + RG * j];
      pq += sj * sq[rg + RG * j];
    }
    if constexpr (PACKED) {
      // Widen again in the second sweep rather than keep the widened rows alive.
#pragma unroll
      for (int j = 0; j < RPT; ++j) asm volatile("" : "+v"(raw[j]));
    }
    // the wave's row groups (lanes congruent modulo CG), on the VALU
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      pk[c] = sum_mod_lanes<CG>(pk[c]);
      pq[c] = sum_mod_lanes<CG>(pq[c]);
    }
    if (lane < CG) {  // lane % CG == cg, and lane < CG selects the wave's first row group
      red_k[wave][lane] = pk;
      red_q[wave][lane] = pq;
    }
    __syncthreads();
    float4_t tk = red_k[0][cg];
    float4_t tq = red_q[0][cg];
#pragma unroll
    for (int w = 1; w < NW; ++w) {
      tk += red_k[w][cg];
      tq += red_q[w][cg];
    }
    const float4_t u = bt * (vv - alpha * tk);
    const float4_t out = alpha * tq + u * kq;
    const __amdgpu_buffer_rsrc_t rout = state_rsrc(h);
#pragma unroll
    for (int j = 0; j < RPT; ++j) IO::template store<CP>(rout, voff, j * ROW_STEP, alpha * row(j) + sk[rg + RG * j] * u);

    // Epilogue: RMSNorm over the head's V outputs (the CG lanes of a row
    // group hold them), times o_norm, times SiLU(gate).
    float ss = out[0] * out[0] + out[1] * out[1] + out[2] * out[2] + out[3] * out[3];
    ss = group_sum(ss, CG < 16 ? CG : 16);  // the row group's CG consecutive lanes
    if constexpr (CG == 32) ss = add_xor16(ss);
    static_assert(CG <= 32, "a row group within half a wave");
    const float r = rsqrtf(ss * (1.f / V) + p.eps);
    if (rg == 0) {
      const long o_base = hs_row + static_cast<long>(h) * V + 4 * cg;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        store_elem(p.hs, o_base + c, p.out_dtype, out[c] * r * p.o_norm[4 * cg + c] * sgate[i * V + 4 * cg + c]);
      }
    }
    __syncthreads();  // the partials are rewritten by the next head
  }
}

// Keeps the state cached or streams it past the cache as the caller names it,
// as the decode step does (pbgdn_recurrent_fwd).
template <int K, int V, typename TS>
int launch_decode_layer(const DecodeLayerParams &p, int B, int policy, hipStream_t stream) {
  const long moved = static_cast<long>(B) * p.Hv * K * V * static_cast<long>(sizeof(TS));
  if (policy == PBGDN_STATE_RESIDENT && moved <= STATE_CACHE_BYTES) {
    hipLaunchKernelGGL((decode_layer_kernel<K, V, TS, STATE_CACHED>), dim3(p.Hk, B), dim3(DNT), 0, stream, p);
  } else {
    hipLaunchKernelGGL((decode_layer_kernel<K, V, TS, state_streamed<TS>()>), dim3(p.Hk, B), dim3(DNT), 0, stream, p);
  }
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}

template <typename TS>
int dispatch_decode_layer(const DecodeLayerParams &p, int B, int K, int V, int policy, hipStream_t stream) {
  if (K == 64 && V == 64) return launch_decode_layer<64, 64, TS>(p, B, policy, stream);
  if (K == 64 && V == 128) return launch_decode_layer<64, 128, TS>(p, B, policy, stream);
  if (K == 128 && V == 64) return launch_decode_layer<128, 64, TS>(p, B, policy, stream);
  if (K == 128 && V == 128) return launch_decode_layer<128, 128, TS>(p, B, policy, stream);
  return PBGDN_ERR_UNSUPPORTED;
}

bool valid_dtype(int d) { return d == PBGDN_F32 || d == PBGDN_BF16 || d == PBGDN_F16; }

}  // namespace
}  // namespace pbgdn

extern "C" int pbgdn_decode_layer_fwd(const void *z, long z_stride, int in_dtype, void *conv_state, int conv_dtype,
                                      long conv_slot_stride, long conv_row_stride, long conv_chan_stride,
                                      const float *conv_weight, int conv, const float *a_log, const float *dt_bias,
                                      int l2_mode, void *state, int state_dtype, const int32_t *state_idx,
                                      int num_states, const float *o_norm, float eps, void *hs, int out_dtype, int B,
                                      int Hk, int Hv, int K, int V, float scale, int state_policy,
                                      void *stream) {
  using pbgdn::valid_dtype;
  if (!(state_policy == PBGDN_STATE_STREAM || state_policy == PBGDN_STATE_RESIDENT)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (B < 0 || Hk <= 0 || Hv <= 0 || K <= 0 || V <= 0 || Hv % Hk != 0 || num_states < 0) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!valid_dtype(in_dtype) || !valid_dtype(state_dtype) || !valid_dtype(out_dtype) ||
      (conv > 1 && !valid_dtype(conv_dtype))) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (conv < 0 || conv > pbgdn::DECODE_MAX_CONV || !(l2_mode == 0 || l2_mode == 1) || !(eps >= 0.f)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!state_idx && num_states < B) return PBGDN_ERR_INVALID_ARGUMENT;
  if (Hv / Hk > pbgdn::DECODE_MAX_GROUP) return PBGDN_ERR_UNSUPPORTED;
  if (B == 0) return PBGDN_OK;
  const long width = 2L * Hk * K + 2L * Hv * V + 2L * Hv;
  if (!z || z_stride < width || !state || !a_log || !dt_bias || !o_norm || !hs) return PBGDN_ERR_INVALID_ARGUMENT;
  if (conv >= 1 && !conv_weight) return PBGDN_ERR_INVALID_ARGUMENT;
  if (conv > 1 && (!conv_state || conv_slot_stride < 0 || conv_row_stride < 0 || conv_chan_stride < 0)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  const uintptr_t align = state_dtype == PBGDN_F32 ? 15u : 7u;  // the state moves in pieces of 4 elements
  if (reinterpret_cast<uintptr_t>(state) & align) return PBGDN_ERR_INVALID_ARGUMENT;
  if (B > 65535) return PBGDN_ERR_UNSUPPORTED;
  pbgdn::DecodeLayerParams p{z, z_stride, in_dtype, conv_state, conv_dtype, conv_slot_stride, conv_row_stride,
                             conv_chan_stride, conv_weight, conv, a_log, dt_bias, l2_mode, state, state_idx,
                             num_states, o_norm, eps, hs, out_dtype, Hk, Hv, scale};
  hipStream_t s = static_cast<hipStream_t>(stream);
  // debug builds: hs starts as NaN (the pools are updated in place)
  pbgdn::debug_poison(hs, static_cast<size_t>(static_cast<long>(B) * Hv * V * (out_dtype == PBGDN_F32 ? 4 : 2)), s);
  switch (state_dtype) {
    case PBGDN_F32: return pbgdn::dispatch_decode_layer<float>(p, B, K, V, state_policy, s);
    case PBGDN_BF16: return pbgdn::dispatch_decode_layer<pbgdn::u16>(p, B, K, V, state_policy, s);
    default: return pbgdn::dispatch_decode_layer<pbgdn::half_t>(p, B, K, V, state_policy, s);
  }
}
