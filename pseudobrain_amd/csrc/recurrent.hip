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
// sweep. The kernel is HBM-bound: K*V*8 bytes of state traffic per head for a
// float32 state, K*V*4 for a bf16 or fp16 one (serving caches often keep the
// state in the model's dtype); the arithmetic is float32 either way.
// In verify mode (speculative decoding) the state after every token is also
// written, to a slot per token, so that the state after the last accepted
// draft token can be kept.
//
// The state moves through buffer loads and stores: one VGPR of lane offset,
// and the row steps as constant SGPR offsets. For a one-token step over a
// 16-bit state (the serving decode) the registers hold the state as loaded,
// two elements a register, and widen it in each sweep: half the registers, so
// twice the workgroups per CU and as many state bytes in flight as a float32
// state has. The arithmetic is the same float32 either way.
#include "state_io.hpp"
#include "device.hpp"

namespace pbgdn {

struct RecurrentParams {
  const void *q, *k, *v;
  int in_dtype;
  const float *g;
  const void *beta;
  int beta_dtype;
  const void *state_in;
  void *state_out;
  const int32_t *state_idx;
  const int32_t *token_state_idx;  // [B, T] slot of the state after each token, or NULL
  int num_states;
  void *o;
  int out_dtype;
  int T, Hk, Hv;
  float scale;
};

// Workgroups per CU for the one-token step: 4 (128 VGPRs) where a thread's
// state is at most 64 floats, 6 (80 VGPRs) for the packed 16-bit form of the
// same. The token loop and the larger head shapes take what the compiler
// gives them (a bound there would spill).
template <int K, int V, bool ONE, bool PACKED>
constexpr int recurrent_wg_per_cu() {
  return ONE && K * V / 256 <= 32 ? (PACKED ? 10 : 8) : ONE && K * V / 256 <= 64 ? (PACKED ? 6 : 4) : 1;
}

// ONE: a single token and no verify slots (the decode step), with no token
// loop; then a 16-bit state stays packed in the registers as loaded.
// CP: the state's cache policy (state_io.hpp). VW: the value columns of one
// workgroup (V / VW workgroups share a state: its column ranges are
// independent, every reduction runs over the key rows).
template <int K, int V, int VW, typename TS, bool ONE, int CP>
__global__ __launch_bounds__(256, (recurrent_wg_per_cu<K, VW, ONE, ONE && sizeof(TS) == 2>())) void recurrent_kernel(
    RecurrentParams p) {
  constexpr bool PACKED = ONE && sizeof(TS) == 2;
  constexpr int NT = 256;
  constexpr int NW = NT / 64;
  constexpr int CG = VW / 4;   // float4 column groups
  constexpr int RG = NT / CG;  // row groups
  constexpr int RPT = K / RG;  // rows per thread
  static_assert(CG >= 1 && CG <= 64 && 64 % CG == 0, "V/4 must divide 64");
  static_assert(RPT >= 1 && RG * RPT == K, "K must be a multiple of the row groups");
  using IO = StateIO<TS>;
  constexpr uint32_t ROW_STEP = RG * V * sizeof(TS);         // bytes between a thread's rows
  constexpr uint32_t STATE_BYTES = K * V * sizeof(TS);

  const int h = blockIdx.x / (V / VW);
  const int col0 = (blockIdx.x % (V / VW)) * VW;
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
  PBGDN_POISON_LDS(sk, sizeof(sk));
  PBGDN_POISON_LDS(sq, sizeof(sq));
  PBGDN_POISON_LDS(red_k, sizeof(red_k));
  PBGDN_POISON_LDS(red_q, sizeof(red_q));
  PBGDN_POISON_SYNC();

  const long slot = p.state_idx ? static_cast<long>(p.state_idx[b]) : static_cast<long>(b);
  if (slot < 0 || slot >= p.num_states) {  // padded entry: no state, zero output
    if (rg == 0) {
      for (int t = 0; t < p.T; ++t) {
        const long o_base = ((static_cast<long>(b) * p.T + t) * p.Hv + h) * V + col0 + 4 * cg;
#pragma unroll
        for (int c = 0; c < 4; ++c) store_elem(p.o, o_base + c, p.out_dtype, 0.f);
      }
    }
    return;
  }
  const long state_off = (slot * p.Hv + h) * static_cast<long>(K) * V;
  const __amdgpu_buffer_rsrc_t rin = rsrc(static_cast<const TS *>(p.state_in) + state_off, STATE_BYTES);
  const __amdgpu_buffer_rsrc_t rout = rsrc(static_cast<TS *>(p.state_out) + state_off, STATE_BYTES);
  const uint32_t voff = (rg * V + col0 + 4 * cg) * sizeof(TS);

  // A token's inputs, as loaded: the same load instructions for every input
  // dtype (the elements are picked out of the loaded words afterwards), so no
  // branches sit around loads and no per-dtype addresses are kept. Thread
  // i < K takes element i of the q and k rows; every thread takes v columns
  // 4cg..4cg+3 (two 8-byte loads; the second is sent out of range for 16-bit
  // inputs, which need only the first).
  const int esz = p.in_dtype == PBGDN_F32 ? 4 : 2;
  const int besz = p.beta_dtype == PBGDN_F32 ? 4 : 2;
  const uint32_t qk_off = (tid * esz) & ~3u;
  const uint32_t v_off0 = (col0 + 4 * cg) * esz;
  const uint32_t v_off1 = esz == 4 ? v_off0 + 8 : OUT_OF_RANGE;
  struct Inputs {
    uint32_t wq, wk, wb;
    v2u32_t wv0, wv1;
    float g;
  };
  auto fetch = [&](long tok) {
    Inputs in;
    const long qk_row = (tok * p.Hk + hk) * K * esz;
    const __amdgpu_buffer_rsrc_t rq = rsrc(static_cast<const char *>(p.q) + qk_row, K * esz);
    const __amdgpu_buffer_rsrc_t rk = rsrc(static_cast<const char *>(p.k) + qk_row, K * esz);
    in.wq = __builtin_amdgcn_raw_buffer_load_b32(rq, qk_off, 0, 0);
    in.wk = __builtin_amdgcn_raw_buffer_load_b32(rk, qk_off, 0, 0);
    const __amdgpu_buffer_rsrc_t rv = rsrc(static_cast<const char *>(p.v) + (tok * p.Hv + h) * V * esz, V * esz);
    in.wv0 = __builtin_amdgcn_raw_buffer_load_b64(rv, v_off0, 0, 0);
    in.wv1 = __builtin_amdgcn_raw_buffer_load_b64(rv, v_off1, 0, 0);
    const long gb = tok * p.Hv + h;
    in.g = p.g[gb];
    // The aligned word holding beta (for a 16-bit beta with an odd count, the
    // last word reaches 2 bytes past the end, inside the same aligned word).
    in.wb = *reinterpret_cast<const uint32_t *>(static_cast<const char *>(p.beta) + ((gb * besz) & ~3L));
    return in;
  };
  const long tok0 = static_cast<long>(b) * p.T;
  Inputs in = {};
  if (ONE || p.T > 0) in = fetch(tok0);  // with T = 0 the input pointers may be null
  // Keep the inputs' loads ahead of the state's: the wait for the inputs then
  // leaves the state loads in flight.
  asm volatile("" ::: "memory");

  typename IO::Raw raw[PACKED ? RPT : 1];
  float4_t s[PACKED ? 1 : RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    if constexpr (PACKED) {
      raw[j] = IO::template load<CP>(rin, voff, j * ROW_STEP);
    } else {
      s[j] = IO::widen(IO::template load<CP>(rin, voff, j * ROW_STEP));
    }
  }
  auto row = [&](int j) -> float4_t {
    if constexpr (PACKED) {
      return IO::widen(raw[j]);
    } else {
      return s[j];
    }
  };

  const int T = ONE ? 1 : p.T;
  for (int t = 0; t < T; ++t) {
    const long tok = tok0 + t;
    if (t > 0) in = fetch(tok);
    if (tid < K) {
      sk[tid] = widen_word(in.wk, tid & 1, p.in_dtype);
      sq[tid] = widen_word(in.wq, tid & 1, p.in_dtype) * p.scale;
    }
    const float4_t vv = widen_words(in.wv0, in.wv1, p.in_dtype);
    const float alpha = expf(in.g);
    const float bt = widen_word(in.wb, static_cast<int>((tok * p.Hv + h) & 1), p.beta_dtype);
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
      const float4_t sj = row(j);
      pk += sj * kr;
      pq += sj * qr;
    }
    if constexpr (PACKED) {
      // Widen again in the second sweep rather than keep the widened rows
      // alive across the reduction (which would undo the packing).
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
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const float kr = sk[rg + RG * j];
      if constexpr (PACKED) {
        IO::template store<CP>(rout, voff, j * ROW_STEP, alpha * row(j) + kr * u);
      } else {
        s[j] = alpha * s[j] + kr * u;
      }
    }
    if (rg == 0) {
      const long o_base = (tok * p.Hv + h) * V + col0 + 4 * cg;
#pragma unroll
      for (int c = 0; c < 4; ++c) store_elem(p.o, o_base + c, p.out_dtype, out[c]);
    }
    if (!ONE && p.token_state_idx) {  // verify mode: the state after this token goes to its own slot
      const long ts = p.token_state_idx[tok];
      if (ts >= 0 && ts < p.num_states) {
        const __amdgpu_buffer_rsrc_t rts =
            rsrc(static_cast<TS *>(p.state_out) + (ts * p.Hv + h) * static_cast<long>(K) * V, STATE_BYTES);
#pragma unroll
        for (int j = 0; j < RPT; ++j) IO::store(rts, voff, j * ROW_STEP, row(j));
      }
    }
    __syncthreads();  // sk, sq and the partials are rewritten by the next token
  }

  if (!PACKED && (ONE || !p.token_state_idx)) {
#pragma unroll
    for (int j = 0; j < RPT; ++j) IO::template store<CP>(rout, voff, j * ROW_STEP, row(j));
  }
}

// The decode step's state loads and stores take the cache policy the caller
// names (cached or streamed past the last-level cache); token loops move each
// state once per call and keep the cached policy.
template <int K, int V, int VW, typename TS>
static void launch_step(const RecurrentParams &p, int B, bool cached, hipStream_t stream) {
  const dim3 grid(p.Hv * (V / VW), B);
  if (cached) {
    hipLaunchKernelGGL((recurrent_kernel<K, V, VW, TS, true, STATE_CACHED>), grid, dim3(256), 0, stream, p);
  } else {
    hipLaunchKernelGGL((recurrent_kernel<K, V, VW, TS, true, state_streamed<TS>()>), grid, dim3(256), 0, stream, p);
  }
}

// The decode step keeps its state cached when the caller declares it resident
// (PBGDN_STATE_RESIDENT: the same pool is stepped again before much else
// passes through the cache) and the call moves at most STATE_CACHE_BYTES of
// state; otherwise it streams the state past the cache. The launch shape
// follows from the call's shape alone, so equal inputs give equal results
// whatever the policy: a float32 step over 4,096 or more head states splits
// each state's columns over two workgroups (streamed, at B = 256, Hv = 32:
// 71% of HBM against 67% whole; at B = 64 the whole state is faster).
template <int K, int V, typename TS>
static int launch_recurrent(const RecurrentParams &p, int B, int policy, hipStream_t stream) {
  if (p.T == 1 && !p.token_state_idx) {
    const long moved = static_cast<long>(B) * p.Hv * K * V * static_cast<long>(sizeof(TS));
    const bool cached = policy == PBGDN_STATE_RESIDENT && moved <= STATE_CACHE_BYTES;
    if constexpr (sizeof(TS) == 4 && V >= 128 && V % 64 == 0) {
      if (static_cast<long>(B) * p.Hv >= 4096) {
        launch_step<K, V, 64, TS>(p, B, cached, stream);
        return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
      }
    }
    launch_step<K, V, V, TS>(p, B, cached, stream);
  } else {
    hipLaunchKernelGGL((recurrent_kernel<K, V, V, TS, false, STATE_CACHED>), dim3(p.Hv, B), dim3(256), 0, stream, p);
  }
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}

template <int K, typename TS>
static int dispatch_v(const RecurrentParams &p, int B, int V, int policy, hipStream_t stream) {
  switch (V) {
    case 32: return launch_recurrent<K, 32, TS>(p, B, policy, stream);
    case 64: return launch_recurrent<K, 64, TS>(p, B, policy, stream);
    case 128: return launch_recurrent<K, 128, TS>(p, B, policy, stream);
    case 256: return launch_recurrent<K, 256, TS>(p, B, policy, stream);
    default: return PBGDN_ERR_UNSUPPORTED;
  }
}

template <typename TS>
static int dispatch_k(const RecurrentParams &p, int B, int K, int V, int policy, hipStream_t stream) {
  switch (K) {
    case 32: return dispatch_v<32, TS>(p, B, V, policy, stream);
    case 64: return dispatch_v<64, TS>(p, B, V, policy, stream);
    case 128: return dispatch_v<128, TS>(p, B, V, policy, stream);
    case 256: return dispatch_v<256, TS>(p, B, V, policy, stream);
    default: return PBGDN_ERR_UNSUPPORTED;
  }
}

int recurrent_fwd(const RecurrentParams &p, int state_dtype, int B, int K, int V, int policy, hipStream_t stream) {
  switch (state_dtype) {
    case PBGDN_F32: return dispatch_k<float>(p, B, K, V, policy, stream);
    case PBGDN_BF16: return dispatch_k<u16>(p, B, K, V, policy, stream);
    case PBGDN_F16: return dispatch_k<half_t>(p, B, K, V, policy, stream);
    default: return PBGDN_ERR_INVALID_ARGUMENT;
  }
}

}  // namespace pbgdn

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
static bool valid_dtype(int d) { return d == PBGDN_F32 || d == PBGDN_BF16 || d == PBGDN_F16; }

// The kernel moves the state in pieces of 4 elements, and reads q, k, v in
// aligned words (16-byte aligned tensors, as pbgdn_chunk_fwd takes them) and
// g and beta in 4-byte words.
static bool state_aligned(const void *p, int dtype) {
  return (reinterpret_cast<uintptr_t>(p) & (dtype == PBGDN_F32 ? 15u : 7u)) == 0;
}
static bool inputs_aligned(const void *q, const void *k, const void *v, const void *g, const void *beta) {
  auto a = [](const void *x, uintptr_t m) { return (reinterpret_cast<uintptr_t>(x) & m) == 0; };
  return a(q, 15) && a(k, 15) && a(v, 15) && a(g, 3) && a(beta, 3);
}

extern "C" int pbgdn_recurrent_fwd(const void *q, const void *k, const void *v, int in_dtype,
                                   const float *g, const void *beta, int beta_dtype,
                                   const void *state_in, void *state_out, int state_dtype,
                                   const int32_t *state_idx, int num_states, void *o,
                                   int out_dtype, int B,
                                   int T, int Hk, int Hv, int K, int V, float scale,
                                   int state_policy, void *stream) {
  if (B < 0 || T < 0 || Hk <= 0 || Hv <= 0 || K <= 0 || V <= 0 || Hv % Hk != 0) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!(state_policy == PBGDN_STATE_STREAM || state_policy == PBGDN_STATE_RESIDENT)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype) || !valid_dtype(state_dtype) ||
      !(beta_dtype == PBGDN_F32 || beta_dtype == in_dtype)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (B == 0 || Hv == 0) return PBGDN_OK;
  if (!state_in || !state_out || num_states < 0) return PBGDN_ERR_INVALID_ARGUMENT;
  if (!state_aligned(state_in, state_dtype) || !state_aligned(state_out, state_dtype)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!state_idx && num_states < B) return PBGDN_ERR_INVALID_ARGUMENT;
  if (T > 0 && (!q || !k || !v || !g || !beta || !o)) return PBGDN_ERR_INVALID_ARGUMENT;
  if (!inputs_aligned(q, k, v, g, beta)) return PBGDN_ERR_INVALID_ARGUMENT;
  if (B > 65535) return PBGDN_ERR_UNSUPPORTED;
  pbgdn::RecurrentParams p{q, k, v, in_dtype, g, beta, beta_dtype, state_in, state_out,
                           state_idx, nullptr, num_states, o, out_dtype, T, Hk, Hv, scale};
  {  // debug builds: the outputs start as NaN (in-place states excepted)
    hipStream_t s = static_cast<hipStream_t>(stream);
    pbgdn::debug_poison(o, static_cast<size_t>(static_cast<long>(B) * T * Hv * V * (out_dtype == PBGDN_F32 ? 4 : 2)), s);
    if (state_out != state_in && !state_idx) {
      pbgdn::debug_poison(state_out, static_cast<size_t>(static_cast<long>(B) * Hv * K * V * (state_dtype == PBGDN_F32 ? 4 : 2)), s);
    }
  }
  return pbgdn::recurrent_fwd(p, state_dtype, B, K, V, state_policy, static_cast<hipStream_t>(stream));
}

extern "C" int pbgdn_recurrent_verify_fwd(const void *q, const void *k, const void *v, int in_dtype,
                                          const float *g, const void *beta, int beta_dtype,
                                          const void *state_in, void *states, int state_dtype,
                                          const int32_t *state_idx, const int32_t *token_state_idx,
                                          int num_states, void *o, int out_dtype, int B, int T, int Hk,
                                          int Hv, int K, int V, float scale, void *stream) {
  if (B < 0 || T < 0 || Hk <= 0 || Hv <= 0 || K <= 0 || V <= 0 || Hv % Hk != 0) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype) || !valid_dtype(state_dtype) ||
      !(beta_dtype == PBGDN_F32 || beta_dtype == in_dtype)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (B == 0 || T == 0) return PBGDN_OK;
  if (!state_in || !states || !token_state_idx || num_states < 0) return PBGDN_ERR_INVALID_ARGUMENT;
  if (!state_aligned(state_in, state_dtype) || !state_aligned(states, state_dtype)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!state_idx && num_states < B) return PBGDN_ERR_INVALID_ARGUMENT;
  if (!q || !k || !v || !g || !beta || !o) return PBGDN_ERR_INVALID_ARGUMENT;
  if (!inputs_aligned(q, k, v, g, beta)) return PBGDN_ERR_INVALID_ARGUMENT;
  if (B > 65535) return PBGDN_ERR_UNSUPPORTED;
  pbgdn::RecurrentParams p{q, k, v, in_dtype, g, beta, beta_dtype, state_in, states,
                           state_idx, token_state_idx, num_states, o, out_dtype, T, Hk, Hv, scale};
  pbgdn::debug_poison(o, static_cast<size_t>(static_cast<long>(B) * T * Hv * V * (out_dtype == PBGDN_F32 ? 4 : 2)),
                      static_cast<hipStream_t>(stream));  // debug builds: o starts as NaN
  return pbgdn::recurrent_fwd(p, state_dtype, B, K, V, PBGDN_STATE_STREAM, static_cast<hipStream_t>(stream));
}
