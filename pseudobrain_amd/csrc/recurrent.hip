// Fused recurrent Gated DeltaNet steps (decode) for gfx950.
//
// Reference: delta_rule_sequential, pseudobrain/gated_deltanet.py:93-107. Per
// token t and value head h, with S = S[h] stored [K, V]:
//   S <- a S;  u = b (v - S^T k);  S <- S + k u^T;  o = S^T (q scale),  a = exp(g).
// One workgroup owns one (sequence, value head) state of K*V floats. Each of
// the 256 threads holds RPT rows x 4 columns of it in registers, so the state is
// read from HBM once and written once however many tokens the call carries.
// Per token the two column reductions S^T k and S^T q are formed together in one
// sweep over the registers (wavefront shuffles, then 4 partials per column
// through LDS), and then the update and o = a S^T q + u (k.q) need no second
// sweep. The kernel is HBM-bound: K*V*8 bytes of state traffic per head.
// In verify mode (speculative decoding) the state after every token is also
// written, to a slot per token, so that the state after the last accepted
// draft token can be kept.
#include "common.hpp"

namespace pbgdn {

struct RecurrentParams {
  const void *q, *k, *v;
  int in_dtype;
  const float *g;
  const void *beta;
  int beta_dtype;
  const float *state_in;
  float *state_out;
  const int32_t *state_idx;
  const int32_t *token_state_idx;  // [B, T] slot of the state after each token, or NULL
  int num_states;
  void *o;
  int out_dtype;
  int T, Hk, Hv;
  float scale;
};

template <int K, int V>
__global__ __launch_bounds__(256) void recurrent_kernel(RecurrentParams p) {
  constexpr int NT = 256;
  constexpr int NW = NT / 64;
  constexpr int CG = V / 4;    // float4 column groups
  constexpr int RG = NT / CG;  // row groups
  constexpr int RPT = K / RG;  // rows per thread
  static_assert(CG >= 1 && CG <= 64 && 64 % CG == 0, "V/4 must divide 64");
  static_assert(RPT >= 1 && RG * RPT == K, "K must be a multiple of the row groups");

  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int cg = tid % CG;
  const int rg = tid / CG;
  const int hk = h / (p.Hv / p.Hk);

  __shared__ float sk[K];
  __shared__ float sq[K];
  __shared__ float4_t red_k[NW][CG];
  __shared__ float4_t red_q[NW][CG];

  const long slot = p.state_idx ? static_cast<long>(p.state_idx[b]) : static_cast<long>(b);
  if (slot < 0 || slot >= p.num_states) {  // padded entry: no state, zero output
    if (rg == 0) {
      for (int t = 0; t < p.T; ++t) {
        const long o_base = ((static_cast<long>(b) * p.T + t) * p.Hv + h) * V + 4 * cg;
#pragma unroll
        for (int c = 0; c < 4; ++c) store_elem(p.o, o_base + c, p.out_dtype, 0.f);
      }
    }
    return;
  }
  const long state_off = (slot * p.Hv + h) * static_cast<long>(K) * V;
  const float *sin = p.state_in + state_off;
  float *sout = p.state_out + state_off;

  float4_t s[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    s[j] = *reinterpret_cast<const float4_t *>(sin + static_cast<long>(rg + RG * j) * V + 4 * cg);
  }

  for (int t = 0; t < p.T; ++t) {
    const long tok = static_cast<long>(b) * p.T + t;
    const long qk_base = (tok * p.Hk + hk) * K;
    for (int i = tid; i < K; i += NT) {
      sk[i] = load_elem(p.k, qk_base + i, p.in_dtype);
      sq[i] = load_elem(p.q, qk_base + i, p.in_dtype) * p.scale;
    }
    const long v_base = (tok * p.Hv + h) * V + 4 * cg;
    float4_t vv;
#pragma unroll
    for (int c = 0; c < 4; ++c) vv[c] = load_elem(p.v, v_base + c, p.in_dtype);
    const long gb = tok * p.Hv + h;
    const float alpha = expf(p.g[gb]);
    const float bt = load_elem(p.beta, gb, p.beta_dtype);
    __syncthreads();

    float kq = 0.f;
    for (int i = lane; i < K; i += 64) kq += sk[i] * sq[i];
    kq = wave_sum(kq);

    float4_t pk = {0.f, 0.f, 0.f, 0.f};
    float4_t pq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const float kr = sk[rg + RG * j];
      const float qr = sq[rg + RG * j];
      pk += s[j] * kr;
      pq += s[j] * qr;
    }
#pragma unroll
    for (int off = CG; off < 64; off <<= 1) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        pk[c] += __shfl_xor(pk[c], off, 64);
        pq[c] += __shfl_xor(pq[c], off, 64);
      }
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
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const float kr = sk[rg + RG * j];
      s[j] = alpha * s[j] + kr * u;
    }
    if (rg == 0) {
      const long o_base = (tok * p.Hv + h) * V + 4 * cg;
#pragma unroll
      for (int c = 0; c < 4; ++c) store_elem(p.o, o_base + c, p.out_dtype, out[c]);
    }
    if (p.token_state_idx) {  // verify mode: the state after this token goes to its own slot
      const long ts = p.token_state_idx[tok];
      if (ts >= 0 && ts < p.num_states) {
        float *dst = p.state_out + (ts * p.Hv + h) * static_cast<long>(K) * V;
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
          *reinterpret_cast<float4_t *>(dst + static_cast<long>(rg + RG * j) * V + 4 * cg) = s[j];
        }
      }
    }
    __syncthreads();  // sk, sq and the partials are rewritten by the next token
  }

  if (!p.token_state_idx) {
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      *reinterpret_cast<float4_t *>(sout + static_cast<long>(rg + RG * j) * V + 4 * cg) = s[j];
    }
  }
}

template <int K, int V>
static int launch_recurrent(const RecurrentParams &p, int B, hipStream_t stream) {
  hipLaunchKernelGGL((recurrent_kernel<K, V>), dim3(p.Hv, B), dim3(256), 0, stream, p);
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}

template <int K>
static int dispatch_v(const RecurrentParams &p, int B, int V, hipStream_t stream) {
  switch (V) {
    case 32: return launch_recurrent<K, 32>(p, B, stream);
    case 64: return launch_recurrent<K, 64>(p, B, stream);
    case 128: return launch_recurrent<K, 128>(p, B, stream);
    case 256: return launch_recurrent<K, 256>(p, B, stream);
    default: return PBGDN_ERR_UNSUPPORTED;
  }
}

int recurrent_fwd(const RecurrentParams &p, int B, int K, int V, hipStream_t stream) {
  switch (K) {
    case 32: return dispatch_v<32>(p, B, V, stream);
    case 64: return dispatch_v<64>(p, B, V, stream);
    case 128: return dispatch_v<128>(p, B, V, stream);
    case 256: return dispatch_v<256>(p, B, V, stream);
    default: return PBGDN_ERR_UNSUPPORTED;
  }
}

}  // namespace pbgdn

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
static bool valid_dtype(int d) { return d == PBGDN_F32 || d == PBGDN_BF16 || d == PBGDN_F16; }

extern "C" int pbgdn_recurrent_fwd(const void *q, const void *k, const void *v, int in_dtype,
                                   const float *g, const void *beta, int beta_dtype,
                                   const float *state_in, float *state_out,
                                   const int32_t *state_idx, int num_states, void *o,
                                   int out_dtype, int B,
                                   int T, int Hk, int Hv, int K, int V, float scale,
                                   void *stream) {
  if (B < 0 || T < 0 || Hk <= 0 || Hv <= 0 || K <= 0 || V <= 0 || Hv % Hk != 0) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype) ||
      !(beta_dtype == PBGDN_F32 || beta_dtype == in_dtype)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (B == 0 || Hv == 0) return PBGDN_OK;
  if (!state_in || !state_out || num_states < 0) return PBGDN_ERR_INVALID_ARGUMENT;
  if (!state_idx && num_states < B) return PBGDN_ERR_INVALID_ARGUMENT;
  if (T > 0 && (!q || !k || !v || !g || !beta || !o)) return PBGDN_ERR_INVALID_ARGUMENT;
  if (B > 65535) return PBGDN_ERR_UNSUPPORTED;
  pbgdn::RecurrentParams p{q, k, v, in_dtype, g, beta, beta_dtype, state_in, state_out,
                           state_idx, nullptr, num_states, o, out_dtype, T, Hk, Hv, scale};
  return pbgdn::recurrent_fwd(p, B, K, V, static_cast<hipStream_t>(stream));
}

extern "C" int pbgdn_recurrent_verify_fwd(const void *q, const void *k, const void *v, int in_dtype,
                                          const float *g, const void *beta, int beta_dtype,
                                          const float *state_in, float *states,
                                          const int32_t *state_idx, const int32_t *token_state_idx,
                                          int num_states, void *o, int out_dtype, int B, int T, int Hk,
                                          int Hv, int K, int V, float scale, void *stream) {
  if (B < 0 || T < 0 || Hk <= 0 || Hv <= 0 || K <= 0 || V <= 0 || Hv % Hk != 0) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype) ||
      !(beta_dtype == PBGDN_F32 || beta_dtype == in_dtype)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (B == 0 || T == 0) return PBGDN_OK;
  if (!state_in || !states || !token_state_idx || num_states < 0) return PBGDN_ERR_INVALID_ARGUMENT;
  if (!state_idx && num_states < B) return PBGDN_ERR_INVALID_ARGUMENT;
  if (!q || !k || !v || !g || !beta || !o) return PBGDN_ERR_INVALID_ARGUMENT;
  if (B > 65535) return PBGDN_ERR_UNSUPPORTED;
  pbgdn::RecurrentParams p{q, k, v, in_dtype, g, beta, beta_dtype, state_in, states,
                           state_idx, token_state_idx, num_states, o, out_dtype, T, Hk, Hv, scale};
  return pbgdn::recurrent_fwd(p, B, K, V, static_cast<hipStream_t>(stream));
}
