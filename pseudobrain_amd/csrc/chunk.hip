// Chunkwise Gated DeltaNet prefill for gfx950 (CDNA4).
//
// Reference algorithm: delta_rule_chunked, pseudobrain/gated_deltanet.py:110-165.
// Within a chunk of C = 64 tokens with inclusive cumulative log decay c_t:
//   A  = strict_lower(b_t (k_t . k_i) exp(c_t - c_i))            (:143-146)
//   T  = (I + A)^-1                                               (:147-149)
//   W  = T diag(b exp(c)) K,  U' = T diag(b) V                    (:150-152)
//   U  = U' - W S;  O = diag(exp(c) scale) Q S + (Q K^T o D) U;    (:158-163)
//   S <- exp(c_C) S + K^T diag(exp(c_C - c)) U
// Every exponent is <= 0 (g <= 0), as in the reference.
//
// Decomposition. The recurrence is separable along the value columns, so a
// workgroup owns one (sequence, value head, 16-column tile of V): grid =
// V/16 x Hv x N, 256 threads (4 waves), one workgroup per CU (about 128 KB of
// LDS). The fp32 state tile S [K, 16] lives in MFMA accumulator registers for
// the whole sequence (each wave owns K/64 16x16 key tiles) and never leaves the
// CU until the final state is written. The chunk-local work that does not
// depend on S (K K^T, Q K^T, the triangular inverse, W) is recomputed by every
// column tile of a head; it is the price of keeping S resident.
//
// Arithmetic. Products run on v_mfma_f32_16x16x32_f16 / 16x16x16_f16 with fp32
// accumulation. Operands are fp16, not bf16: the intermediate operands
// (T, W, S, U) need the 11-bit fp16 significand to keep the fp32 final state
// within 1e-3 of an fp32 evaluation (8-bit bf16 operands miss it by about 3x).
// bf16 inputs convert to fp16 exactly (for |x| >= 2^-14). Scalings are applied
// where they cost no extra rounding: decays and beta fold into T's columns
// (diag(b) and diag(b exp(c))), the query scale and exp(c) multiply the fp32
// accumulator of Q S, and the state update uses exp(c_C - c) U split into an
// fp16 high and low part (two MFMAs), so the state sees fp32-accurate U.
//
// Register chaining. MFMA output tiles hold 4 rows x 1 column per lane; an A or
// B fragment holds 8 contraction slots x 1 row/column per lane. Two output
// tiles stacked along the contraction index therefore form one fragment with
// the slot order (4g..4g+3 of tile 2j, then of tile 2j+1); the partner operand
// is read from LDS in the same order. W^T is computed (not W) so that its
// output tiles are directly the A fragments of W S.
#include "common.hpp"

namespace pbgdn {

constexpr int CH = 64;   // chunk length (CHUNK, gated_deltanet.py:49)
constexpr int VT = 16;   // value columns per workgroup
constexpr int NT = 256;  // threads per workgroup

struct ChunkParams {
  const void *q, *k, *v;
  const float *g;
  const void *beta;
  int beta_dtype;
  const float *h0;
  float *ht;
  const int32_t *cu_seqlens;
  void *o;
  int out_dtype;
  int T, Hk, Hv, V, num_seqs;
  float scale;
};

template <int K>
struct ChunkSmem {
  static constexpr int KP = K + 8;   // pitch (halfs) of [t][key] rows
  static constexpr int CP = CH + 8;  // pitch (halfs) of [.][t] rows
  static constexpr int FP = CH + 4;  // pitch (floats) of the fp32 64x64 matrices
  alignas(16) half_t kn[CH][KP];     // K chunk, [t][key]
  alignas(16) half_t kt[K][CP];      // K chunk transposed, [key][t]
  alignas(16) half_t qn[CH][KP];     // Q chunk, [t][key]
  alignas(16) half_t vt[VT][CP];     // V column tile transposed, [v][t]
  alignas(16) float am[CH][FP];      // A (strictly lower), fp32
  alignas(16) float tm[CH][FP];      // T = (I + A)^-1, fp32
  alignas(16) half_t tb[CH][CP];     // T diag(b)
  alignas(16) half_t tbg[CH][CP];    // T diag(b exp(c))
  alignas(16) half_t qkd[CH][CP];    // (Q K^T o D) * scale, lower incl. diagonal
  alignas(16) float cum[CH];         // inclusive cumsum of g
  alignas(16) float gam[CH];         // exp(cum)
  alignas(16) float dec[CH];         // exp(cum[C-1] - cum)
  alignas(16) float bet[CH];         // beta
  alignas(16) half4_t sd[K / 16][64];   // S tiles (fp16, output layout) for the next chunk
  alignas(16) half4_t ud[CH / 16][64];  // U tiles (fp16)
  alignas(16) half4_t uh[CH / 16][64];  // exp(c_C - c) U, fp16 high part
  alignas(16) half4_t ul[CH / 16][64];  // exp(c_C - c) U, fp16 low part
};

// 8 consecutive input elements as fp16.
template <typename TIn>
__device__ __forceinline__ half8_t load8(const TIn *p);

template <>
__device__ __forceinline__ half8_t load8<u16>(const u16 *p) {  // bf16
  const uint4 raw = *reinterpret_cast<const uint4 *>(p);
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  half8_t out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = static_cast<half_t>(__uint_as_float(w[i] << 16));
    out[2 * i + 1] = static_cast<half_t>(__uint_as_float(w[i] & 0xffff0000u));
  }
  return out;
}

template <>
__device__ __forceinline__ half8_t load8<half_t>(const half_t *p) {
  return *reinterpret_cast<const half8_t *>(p);
}

template <>
__device__ __forceinline__ half8_t load8<float>(const float *p) {
  const float4_t a = *reinterpret_cast<const float4_t *>(p);
  const float4_t b = *reinterpret_cast<const float4_t *>(p + 4);
  return half8_t{static_cast<half_t>(a[0]), static_cast<half_t>(a[1]), static_cast<half_t>(a[2]),
                 static_cast<half_t>(a[3]), static_cast<half_t>(b[0]), static_cast<half_t>(b[1]),
                 static_cast<half_t>(b[2]), static_cast<half_t>(b[3])};
}

template <typename TIn>
__device__ __forceinline__ half4_t load4(const TIn *p);

template <>
__device__ __forceinline__ half4_t load4<u16>(const u16 *p) {
  const uint2 raw = *reinterpret_cast<const uint2 *>(p);
  return half4_t{static_cast<half_t>(__uint_as_float(raw.x << 16)),
                 static_cast<half_t>(__uint_as_float(raw.x & 0xffff0000u)),
                 static_cast<half_t>(__uint_as_float(raw.y << 16)),
                 static_cast<half_t>(__uint_as_float(raw.y & 0xffff0000u))};
}

template <>
__device__ __forceinline__ half4_t load4<half_t>(const half_t *p) {
  return *reinterpret_cast<const half4_t *>(p);
}

template <>
__device__ __forceinline__ half4_t load4<float>(const float *p) {
  const float4_t a = *reinterpret_cast<const float4_t *>(p);
  return half4_t{static_cast<half_t>(a[0]), static_cast<half_t>(a[1]), static_cast<half_t>(a[2]),
                 static_cast<half_t>(a[3])};
}

// Block index -> (sequence, value head, column tile). All column tiles of the
// value heads that share one query/key head of one sequence form a group; a
// group is kept on one XCD (workgroups are dispatched round-robin over the 8
// XCDs) so that its q/k chunks are fetched into that XCD's L2 once.
__device__ __forceinline__ void decode_block(int L, int total, int nv, int group_heads, int Hk,
                                             int &seq, int &h, int &vtile) {
  const int gsize = nv * group_heads;
  const int ngroups = total / gsize;
  int grp, in;
  if (ngroups % 8 == 0) {
    const int xcd = L & 7;
    const int slot = L >> 3;
    grp = (slot / gsize) * 8 + xcd;
    in = slot % gsize;
  } else {
    grp = L / gsize;
    in = L % gsize;
  }
  const int hk = grp % Hk;
  seq = grp / Hk;
  h = hk * group_heads + in / nv;
  vtile = in % nv;
}

template <int K, typename TIn>
__global__ __launch_bounds__(NT) void chunk_kernel(ChunkParams p) {
  static_assert(K % 32 == 0 && K <= 128, "K must be 32, 64, 96 or 128");
  constexpr int NKT = K / 16;           // key tiles
  constexpr int SPW = (NKT + 3) / 4;    // key tiles of S per wave
  constexpr int KS = K / 32;            // contraction steps over keys
  using Smem = ChunkSmem<K>;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Smem &sm = *reinterpret_cast<Smem *>(smem_raw);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c16 = lane & 15;
  const int g4 = lane >> 4;

  const int nv = p.V / VT;
  const int group_heads = p.Hv / p.Hk;
  const int total = gridDim.x;
  int seq, h, vtile;
  decode_block(blockIdx.x, total, nv, group_heads, p.Hk, seq, h, vtile);
  const int hk = h / group_heads;
  const int v0 = vtile * VT;

  long bos, eos;
  if (p.cu_seqlens) {
    bos = p.cu_seqlens[seq];
    eos = p.cu_seqlens[seq + 1];
  } else {
    bos = static_cast<long>(seq) * p.T;
    eos = bos + p.T;
  }

  const TIn *qg = static_cast<const TIn *>(p.q);
  const TIn *kg = static_cast<const TIn *>(p.k);
  const TIn *vg = static_cast<const TIn *>(p.v);

  // Regions read but never written by the chunk loop start at zero: the
  // strictly upper blocks of T, of A and of QKD.
  for (int i = tid; i < CH * Smem::FP; i += NT) (&sm.am[0][0])[i] = 0.f;
  for (int i = tid; i < CH * Smem::FP; i += NT) (&sm.tm[0][0])[i] = 0.f;
  for (int i = tid; i < CH * Smem::CP; i += NT) (&sm.qkd[0][0])[i] = static_cast<half_t>(0.f);

  // Initial state: wave w owns key tiles w, w + 4, ...
  float4_t sacc[SPW];
  const long state_base = (static_cast<long>(seq) * p.Hv + h) * K * p.V + v0 + c16;
#pragma unroll
  for (int m = 0; m < SPW; ++m) {
    const int kt = wave + 4 * m;
    sacc[m] = float4_t{0.f, 0.f, 0.f, 0.f};
    if (kt < NKT) {
      if (p.h0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sacc[m][i] = p.h0[state_base + static_cast<long>(16 * kt + 4 * g4 + i) * p.V];
      }
      sm.sd[kt][lane] = to_half4(sacc[m]);
    }
  }

  const long nchunks = (eos - bos + CH - 1) / CH;
  for (long ci = 0; ci < nchunks; ++ci) {
    const long t0 = bos + ci * CH;
    const int len = static_cast<int>(min(static_cast<long>(CH), eos - t0));

    // ---- Phase L: chunk inputs into LDS --------------------------------
    {
      constexpr int PER_ROW = K / 8;
      for (int it = tid; it < CH * PER_ROW; it += NT) {
        const int t = it / PER_ROW;
        const int kc = (it % PER_ROW) * 8;
        half8_t kx = {}, qx = {};
        if (t < len) {
          const long off = ((t0 + t) * p.Hk + hk) * static_cast<long>(K) + kc;
          kx = load8<TIn>(kg + off);
          qx = load8<TIn>(qg + off);
        }
        *reinterpret_cast<half8_t *>(&sm.kn[t][kc]) = kx;
        *reinterpret_cast<half8_t *>(&sm.qn[t][kc]) = qx;
#pragma unroll
        for (int j = 0; j < 8; ++j) sm.kt[kc + j][t] = kx[j];
      }
      for (int it = tid; it < CH * (VT / 4); it += NT) {
        const int t = it / (VT / 4);
        const int vc = (it % (VT / 4)) * 4;
        half4_t vx = {};
        if (t < len) vx = load4<TIn>(vg + ((t0 + t) * p.Hv + h) * static_cast<long>(p.V) + v0 + vc);
#pragma unroll
        for (int j = 0; j < 4; ++j) sm.vt[vc + j][t] = vx[j];
      }
      if (wave == 0) {
        float gv = 0.f, bv = 0.f;
        if (lane < len) {
          const long gi = (t0 + lane) * p.Hv + h;
          gv = p.g[gi];
          bv = load_elem(p.beta, gi, p.beta_dtype);
        }
        float x = gv;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const float y = __shfl_up(x, off, 64);
          if (lane >= off) x += y;
        }
        const float last = __shfl(x, 63, 64);
        sm.cum[lane] = x;
        sm.gam[lane] = __expf(x);
        sm.dec[lane] = __expf(last - x);
        sm.bet[lane] = bv;
      }
    }
    __syncthreads();

    // ---- Phase A: K K^T (row tile = wave) and Q K^T (row tile = 3 - wave) ----
    {
      const int ra = wave;
      for (int s = 0; s <= ra; ++s) {
        float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
          const half8_t a = *reinterpret_cast<const half8_t *>(&sm.kn[16 * ra + c16][32 * kk + 8 * g4]);
          const half8_t b = *reinterpret_cast<const half8_t *>(&sm.kn[16 * s + c16][32 * kk + 8 * g4]);
          acc = mfma32(a, b, acc);
        }
        const int j = 16 * s + c16;
        const float cj = sm.cum[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * ra + 4 * g4 + i;
          sm.am[t][j] = (j < t) ? sm.bet[t] * acc[i] * __expf(sm.cum[t] - cj) : 0.f;
        }
      }
      const int rq = 3 - wave;
      for (int s = 0; s <= rq; ++s) {
        float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
          const half8_t a = *reinterpret_cast<const half8_t *>(&sm.qn[16 * rq + c16][32 * kk + 8 * g4]);
          const half8_t b = *reinterpret_cast<const half8_t *>(&sm.kn[16 * s + c16][32 * kk + 8 * g4]);
          acc = mfma32(a, b, acc);
        }
        const int j = 16 * s + c16;
        const float cj = sm.cum[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * rq + 4 * g4 + i;
          const float val = (j <= t) ? p.scale * acc[i] * __expf(sm.cum[t] - cj) : 0.f;
          sm.qkd[t][j] = static_cast<half_t>(val);
        }
      }
    }
    __syncthreads();

    // ---- Phase T1: 16x16 diagonal blocks of T by forward substitution ----
    if (lane < 16) {
      const int r0 = 16 * wave;
      float x[16];
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        float acc = (t == lane) ? 1.f : 0.f;
#pragma unroll
        for (int i = 0; i < t; ++i) acc -= sm.am[r0 + t][r0 + i] * x[i];
        x[t] = acc;
      }
#pragma unroll
      for (int t = 0; t < 16; ++t) sm.tm[r0 + t][r0 + lane] = x[t];
    }
    __syncthreads();

    // ---- Phase T2: off-diagonal blocks, T_rs = -T_rr sum_{s<=j<r} A_rj T_js ----
#pragma unroll
    for (int d = 1; d < 4; ++d) {
      if (wave >= d) {
        const int r = wave, s = wave - d;
        float4_t x = {0.f, 0.f, 0.f, 0.f};
        for (int j = s; j < r; ++j) {
          const float4_t af = *reinterpret_cast<const float4_t *>(&sm.am[16 * r + c16][16 * j + 4 * g4]);
          float4_t bf;
#pragma unroll
          for (int i = 0; i < 4; ++i) bf[i] = sm.tm[16 * j + 4 * g4 + i][16 * s + c16];
          x = mfma16(to_half4(af), to_half4(bf), x);
        }
        const float4_t tf = *reinterpret_cast<const float4_t *>(&sm.tm[16 * r + c16][16 * r + 4 * g4]);
        const float4_t y = mfma16(to_half4(tf), to_half4(x), float4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int i = 0; i < 4; ++i) sm.tm[16 * r + 4 * g4 + i][16 * s + c16] = -y[i];
      }
      __syncthreads();
    }

    // ---- Phase T3: T diag(b) and T diag(b exp(c)) in fp16 ----
    for (int it = tid; it < CH * CH; it += NT) {
      const int t = it / CH;
      const int s = it % CH;
      const float tv = sm.tm[t][s] * sm.bet[s];
      sm.tb[t][s] = static_cast<half_t>(tv);
      sm.tbg[t][s] = static_cast<half_t>(tv * sm.gam[s]);
    }
    __syncthreads();

    // ---- Phase W/U: wave w owns token rows 16w..16w+15 ----
    const int w = wave;
    const int nks = (16 * w + 16 + 31) / 32;  // contraction steps over tokens s <= t
    float4_t wt[NKT];                         // W^T tiles [key tile][t tile w]
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
      wt[kt] = float4_t{0.f, 0.f, 0.f, 0.f};
      for (int ks = 0; ks < nks; ++ks) {
        const half8_t a = *reinterpret_cast<const half8_t *>(&sm.kt[16 * kt + c16][32 * ks + 8 * g4]);
        const half8_t b = *reinterpret_cast<const half8_t *>(&sm.tbg[16 * w + c16][32 * ks + 8 * g4]);
        wt[kt] = mfma32(a, b, wt[kt]);
      }
    }
    float4_t u = {0.f, 0.f, 0.f, 0.f};  // U' rows 16w.., then U
    for (int ks = 0; ks < nks; ++ks) {
      const half8_t a = *reinterpret_cast<const half8_t *>(&sm.tb[16 * w + c16][32 * ks + 8 * g4]);
      const half8_t b = *reinterpret_cast<const half8_t *>(&sm.vt[c16][32 * ks + 8 * g4]);
      u = mfma32(a, b, u);
    }
    float4_t o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      const half8_t sb = cat8(sm.sd[2 * j][lane], sm.sd[2 * j + 1][lane]);
      const half8_t wa = cat8(to_half4(-wt[2 * j]), to_half4(-wt[2 * j + 1]));
      u = mfma32(wa, sb, u);
      const half4_t qlo = *reinterpret_cast<const half4_t *>(&sm.qn[16 * w + c16][32 * j + 4 * g4]);
      const half4_t qhi = *reinterpret_cast<const half4_t *>(&sm.qn[16 * w + c16][32 * j + 16 + 4 * g4]);
      o = mfma32(cat8(qlo, qhi), sb, o);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * w + 4 * g4 + i;
      o[i] *= sm.gam[t] * p.scale;
    }
    {
      sm.ud[w][lane] = to_half4(u);
      float4_t us;
#pragma unroll
      for (int i = 0; i < 4; ++i) us[i] = u[i] * sm.dec[16 * w + 4 * g4 + i];
      const half4_t hi = to_half4(us);
      sm.uh[w][lane] = hi;
      sm.ul[w][lane] = to_half4(us - to_float4(hi));
    }
    __syncthreads();

    // ---- Phase O: O rows 16w.. += (Q K^T o D) U ----
    for (int ks = 0; ks <= (w >> 1); ++ks) {
      const half4_t alo = *reinterpret_cast<const half4_t *>(&sm.qkd[16 * w + c16][32 * ks + 4 * g4]);
      const half4_t ahi = *reinterpret_cast<const half4_t *>(&sm.qkd[16 * w + c16][32 * ks + 16 + 4 * g4]);
      const half8_t b = cat8(sm.ud[2 * ks][lane], sm.ud[2 * ks + 1][lane]);
      o = mfma32(cat8(alo, ahi), b, o);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * w + 4 * g4 + i;
      if (t < len) {
        store_elem(p.o, ((t0 + t) * p.Hv + h) * static_cast<long>(p.V) + v0 + c16, p.out_dtype, o[i]);
      }
    }

    // ---- Phase S: S <- exp(c_C) S + K^T (exp(c_C - c) U) ----
    {
      const float gc = sm.gam[CH - 1];
#pragma unroll
      for (int m = 0; m < SPW; ++m) {
        const int kt = wave + 4 * m;
        if (kt < NKT) {
          sacc[m] *= gc;
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const half4_t alo = *reinterpret_cast<const half4_t *>(&sm.kt[16 * kt + c16][32 * ks + 4 * g4]);
            const half4_t ahi = *reinterpret_cast<const half4_t *>(&sm.kt[16 * kt + c16][32 * ks + 16 + 4 * g4]);
            const half8_t a = cat8(alo, ahi);
            sacc[m] = mfma32(a, cat8(sm.uh[2 * ks][lane], sm.uh[2 * ks + 1][lane]), sacc[m]);
            sacc[m] = mfma32(a, cat8(sm.ul[2 * ks][lane], sm.ul[2 * ks + 1][lane]), sacc[m]);
          }
          sm.sd[kt][lane] = to_half4(sacc[m]);
        }
      }
    }
    __syncthreads();
  }

  if (p.ht) {
#pragma unroll
    for (int m = 0; m < SPW; ++m) {
      const int kt = wave + 4 * m;
      if (kt < NKT) {
#pragma unroll
        for (int i = 0; i < 4; ++i) p.ht[state_base + static_cast<long>(16 * kt + 4 * g4 + i) * p.V] = sacc[m][i];
      }
    }
  }
}

template <int K, typename TIn>
static int launch_chunk(const ChunkParams &p, hipStream_t stream) {
  const size_t smem = sizeof(ChunkSmem<K>);
  auto kernel = chunk_kernel<K, TIn>;
  if (hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(smem)) != hipSuccess) {
    return PBGDN_ERR_LAUNCH;
  }
  const int total = (p.V / VT) * p.Hv * p.num_seqs;
  hipLaunchKernelGGL(kernel, dim3(total), dim3(NT), smem, stream, p);
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}

template <int K>
static int dispatch_in(const ChunkParams &p, int in_dtype, hipStream_t stream) {
  switch (in_dtype) {
    case PBGDN_BF16: return launch_chunk<K, u16>(p, stream);
    case PBGDN_F16: return launch_chunk<K, half_t>(p, stream);
    case PBGDN_F32: return launch_chunk<K, float>(p, stream);
    default: return PBGDN_ERR_INVALID_ARGUMENT;
  }
}

}  // namespace pbgdn

static bool valid_dtype(int d) { return d == PBGDN_F32 || d == PBGDN_BF16 || d == PBGDN_F16; }

extern "C" int pbgdn_chunk_fwd(const void *q, const void *k, const void *v, int in_dtype,
                               const float *g, const void *beta, int beta_dtype, const float *h0,
                               float *ht, const int32_t *cu_seqlens, int num_seqs, void *o,
                               int out_dtype, int B, int T, int Hk, int Hv, int K, int V,
                               float scale, int chunk, void *stream) {
  if (B < 0 || T < 0 || Hk <= 0 || Hv <= 0 || K <= 0 || V <= 0 || Hv % Hk != 0 || num_seqs < 0) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype) ||
      !(beta_dtype == PBGDN_F32 || beta_dtype == in_dtype)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (cu_seqlens ? B != 1 : num_seqs != B) return PBGDN_ERR_INVALID_ARGUMENT;
  if (chunk != pbgdn::CH) return PBGDN_ERR_UNSUPPORTED;
  if (!(K == 64 || K == 128) || V % pbgdn::VT != 0) return PBGDN_ERR_UNSUPPORTED;
  if (num_seqs == 0) return PBGDN_OK;
  if (T > 0 && (!q || !k || !v || !g || !beta || !o)) return PBGDN_ERR_INVALID_ARGUMENT;
  const long total = static_cast<long>(V / pbgdn::VT) * Hv * num_seqs;
  if (total > 0x7fffffffL) return PBGDN_ERR_UNSUPPORTED;
  pbgdn::ChunkParams p{q, k, v, g, beta, beta_dtype, h0, ht, cu_seqlens, o, out_dtype,
                       T, Hk, Hv, V, num_seqs, scale};
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (K) {
    case 64: return pbgdn::dispatch_in<64>(p, in_dtype, s);
    case 128: return pbgdn::dispatch_in<128>(p, in_dtype, s);
    default: return PBGDN_ERR_UNSUPPORTED;
  }
}
