// The residuals that pseudobrain::gated_delta_chunk returns beside o and the
// final state (pseudobrain/gated_deltanet.py:200-217, fla's chunk forward with
// 64-token chunks): gc, the inclusive cumulative sum of g within each chunk,
// and A, the chunk's
//
//   T = (I + strict_lower(beta_t (k_t . k_s) exp(gc_t - gc_s)))^-1
//
// (the `solve` of delta_rule_chunked, gated_deltanet.py:141-149) stored by
// rows: A[b, t, h, :] = row t mod 64 of its chunk's T. The prefill kernels
// never form T itself (they fold diag(beta) into it and keep fp16 MFMA
// fragments), so these come from a kernel of their own, in float32 like the
// reference's chunked path: one workgroup per (chunk, value head), K K^T by
// per-thread dot products over LDS slabs of k, and T by forward substitution
// with one thread per column (each column of a unit lower-triangular inverse
// depends only on itself). Also here: the inverse map gc -> g that the
// backward with fla's residuals needs.
#include <algorithm>

#include "common.hpp"
#include "device.hpp"

namespace pbgdn {
namespace {

constexpr int RC = 64;        // chunk length (fla's chunk_size)
constexpr int RNT = 256;      // threads per workgroup
constexpr int SLAB = 32;      // k columns per LDS slab
constexpr int LA = RC + 1;    // padded rows of the C x C tiles

struct ResidualParams {
  const void *k;
  int k_dtype;
  const float *g;
  const void *beta;
  int beta_dtype;
  float *gc;
  void *a;
  int a_dtype;
  int B, T, Hk, Hv, K;
};

__global__ __launch_bounds__(RNT) void residuals_kernel(ResidualParams p) {
  __shared__ float sk[RC][SLAB + 1];
  __shared__ float sa[RC][LA];  // beta_t (k_t . k_s) e^{gc_t - gc_s}, strict lower
  __shared__ float st[RC][LA];  // T
  __shared__ float sc[RC], sb[RC];
  PBGDN_POISON_LDS(sk, sizeof(sk));
  PBGDN_POISON_LDS(sa, sizeof(sa));
  PBGDN_POISON_LDS(st, sizeof(st));
  PBGDN_POISON_LDS(sc, sizeof(sc));
  PBGDN_POISON_LDS(sb, sizeof(sb));
  PBGDN_POISON_SYNC();
  const int i = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int hk = h / (p.Hv / p.Hk);
  const long t0 = static_cast<long>(i) * RC;
  const int len = static_cast<int>(min(static_cast<long>(RC), p.T - t0));
  const long row0 = static_cast<long>(b) * p.T + t0;  // the chunk's first token row
  if (tid < RC) {
    sb[tid] = tid < len ? load_elem(p.beta, (row0 + tid) * p.Hv + h, p.beta_dtype) : 0.f;
  }
  if (tid == 0) {  // in token order, as a sequential cumulative sum rounds
    float c = 0.f;
    for (int t = 0; t < RC; ++t) {
      if (t < len) c += p.g[(row0 + t) * p.Hv + h];
      sc[t] = c;
    }
  }
  // K K^T: thread (row t = tid / 4, columns 16 (tid % 4) ..) accumulates 16 dot products
  const int tr = tid >> 2, s0 = 16 * (tid & 3);
  float acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.f;
  for (int k0 = 0; k0 < p.K; k0 += SLAB) {
    __syncthreads();  // the previous slab's readers are done
    for (int e = tid; e < RC * SLAB; e += RNT) {
      const int t = e / SLAB, kk = e % SLAB;
      sk[t][kk] = t < len && k0 + kk < p.K
                      ? load_elem(p.k, ((row0 + t) * p.Hk + hk) * static_cast<long>(p.K) + k0 + kk, p.k_dtype)
                      : 0.f;
    }
    __syncthreads();
    for (int kk = 0; kk < SLAB; ++kk) {
      const float x = sk[tr][kk];
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[j] += x * sk[s0 + j][kk];
    }
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int s = s0 + j;
    sa[tr][s] = s < tr ? sb[tr] * acc[j] * expf(sc[tr] - sc[s]) : 0.f;
  }
  __syncthreads();
  // T = (I + A)^-1: column j by forward substitution, T[t][j] = [t == j] - sum_{j <= s < t} A[t][s] T[s][j]
  if (tid < RC) {
    const int j = tid;
    for (int t = 0; t < RC; ++t) {
      float x = t == j ? 1.f : 0.f;
      for (int s = j; s < t; ++s) x -= sa[t][s] * st[s][j];
      st[t][j] = x;
    }
  }
  __syncthreads();
  for (int e = tid; e < RC * RC; e += RNT) {
    const int t = e / RC, s = e % RC;
    if (t < len && p.a) store_elem(p.a, ((row0 + t) * p.Hv + h) * static_cast<long>(RC) + s, p.a_dtype, st[t][s]);
  }
  if (tid < len && p.gc) p.gc[(row0 + tid) * p.Hv + h] = sc[tid];
}

// g_t = gc_t - gc_{t-1} within each chunk (gc_t at a chunk's first token).
__global__ __launch_bounds__(RNT) void decumulate_kernel(const float *gc, float *g, long rows, int T, int H) {
  for (long e = static_cast<long>(blockIdx.x) * RNT + threadIdx.x; e < rows * H;
       e += static_cast<long>(gridDim.x) * RNT) {
    const long bt = e / H;
    const long t = bt % T;
    g[e] = t % RC == 0 ? gc[e] : gc[e] - gc[e - H];
  }
}

bool valid_dtype(int d) { return d == PBGDN_F32 || d == PBGDN_BF16 || d == PBGDN_F16; }

}  // namespace
}  // namespace pbgdn

extern "C" int pbgdn_chunk_residuals(const void *k, int k_dtype, const float *g, const void *beta, int beta_dtype,
                                     float *gc, void *a, int a_dtype, int B, int T, int Hk, int Hv, int K,
                                     void *stream) {
  using namespace pbgdn;
  if (B < 0 || T < 0 || Hk <= 0 || Hv <= 0 || K <= 0 || Hv % Hk != 0) return PBGDN_ERR_INVALID_ARGUMENT;
  if (!valid_dtype(k_dtype) || !valid_dtype(a_dtype) || !valid_dtype(beta_dtype)) return PBGDN_ERR_INVALID_ARGUMENT;
  if (static_cast<long>(B) * T == 0 || (!gc && !a)) return PBGDN_OK;
  if (!k || !g || !beta) return PBGDN_ERR_INVALID_ARGUMENT;
  if (B > 65535 || Hv > 65535) return PBGDN_ERR_UNSUPPORTED;
  const long chunks = (static_cast<long>(T) + RC - 1) / RC;
  if (chunks > 0x7fffffffL) return PBGDN_ERR_UNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const long rows = static_cast<long>(B) * T * Hv;
  if (gc) debug_poison(gc, static_cast<size_t>(rows * 4), st);  // debug builds: NaN first
  if (a) debug_poison(a, static_cast<size_t>(rows * RC * (a_dtype == PBGDN_F32 ? 4 : 2)), st);
  ResidualParams p{k, k_dtype, g, beta, beta_dtype, gc, a, a_dtype, B, T, Hk, Hv, K};
  hipLaunchKernelGGL(residuals_kernel, dim3(static_cast<unsigned>(chunks), Hv, B), dim3(RNT), 0, st, p);
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}

extern "C" int pbgdn_chunk_decumulate(const float *gc, float *g, int B, int T, int Hv, void *stream) {
  using namespace pbgdn;
  if (B < 0 || T < 0 || Hv <= 0) return PBGDN_ERR_INVALID_ARGUMENT;
  const long rows = static_cast<long>(B) * T;
  if (rows == 0) return PBGDN_OK;
  if (!gc || !g || gc == g) return PBGDN_ERR_INVALID_ARGUMENT;
  const long blocks = std::min<long>((rows * Hv + RNT - 1) / RNT, 65535L);
  hipLaunchKernelGGL(decumulate_kernel, dim3(static_cast<unsigned>(blocks)), dim3(RNT), 0,
                     static_cast<hipStream_t>(stream), gc, g, rows, T, Hv);
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}
