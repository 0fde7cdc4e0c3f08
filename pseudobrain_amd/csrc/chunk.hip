// C ABI of the chunkwise prefill: argument checks, the workspace size, and
// the two launches on the caller's stream: the prep kernel (every chunk's
// state-independent part, chunk_prep.hip), then the scan kernel (the serial
// state recurrence, chunk_scan.hip). The workspace carries the prep kernel's
// records to the scan kernel; see chunk.hpp for the algorithm and the record
// format.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "chunk.hpp"

// Scratch of pbgdn_chunk_fwd_noalloc: the prep kernel's workspace records for
// callers that cannot allocate. Each GPU the library runs on holds its own copy
// until the process ends. In host code `scratch` names a host-side stand-in,
// not a device address: kernels and copies take the address that
// hipGetSymbolAddress returns for the current device (scratch_for_stream).
static __device__ __align__(256) unsigned char scratch[PBGDN_NOALLOC_SCRATCH_BYTES];

namespace pbgdn {
namespace {

// The scan kernel of a call. The wide scan (chunk_wide.hip: all 128 columns
// of a (sequence, value head) per workgroup, one wave per 16-column tile)
// takes 16-bit inputs and outputs at K = 128 with V a multiple of 128. It
// stages each chunk once for eight tiles, so it wins whenever its workgroups
// number at least half the CUs (measured at the Qwen3-Next head shape, 32,768
// tokens: 4 x 8,192 0.53 vs 0.72 ms, 8 x 4,096 0.39 vs 0.73 ms, 1024 x 32
// 1.76 vs 2.68 ms); one or two sequences of that shape have 32 or 64 of them
// and run faster on the narrow scan, which spreads each head over 8
// workgroups (1 x 32,768: 0.78 vs 1.69 ms). PBGDN_SCAN=narrow|wide in the
// environment forces a choice (for measurements).
inline int scan_choice() {
  static const int choice = [] {
    const char *e = getenv("PBGDN_SCAN");
    if (!e) return 0;
    return strcmp(e, "narrow") == 0 ? 1 : strcmp(e, "wide") == 0 ? 2 : 0;
  }();
  return choice;
}

template <int K, typename TIn>
bool wide_eligible(const ChunkParams &p) {
  if constexpr (K != 128 || sizeof(TIn) != 2) {
    return false;
  } else {
    if (p.V % 128 != 0 || scan_choice() == 1) return false;
    return scan_choice() == 2 || static_cast<long>(p.num_seqs) * p.Hv * (p.V / 128) >= p.cus / 2;
  }
}

template <int K, typename TIn>
int run_chunk(const ChunkParams &p, long records, int out_dtype, hipStream_t s) {
  const int st = launch_prep<K, TIn>(p, records, s);
  if (st != PBGDN_OK) return st;
  if constexpr (K == 128 && sizeof(TIn) == 2) {
    if (out_dtype != PBGDN_F32 && wide_eligible<K, TIn>(p)) return launch_wide<K, TIn, TIn, false>(p, s);
  }
  if (out_dtype == PBGDN_F32) return launch_scan<K, TIn, float>(p, s);
  return launch_scan<K, TIn, TIn>(p, s);  // out_dtype == in_dtype, checked by the caller
}

template <int K>
int dispatch_in(const ChunkParams &p, long records, int in_dtype, int out_dtype, hipStream_t s) {
  switch (in_dtype) {
    case PBGDN_BF16: return run_chunk<K, u16>(p, records, out_dtype, s);
    case PBGDN_F16: return run_chunk<K, half_t>(p, records, out_dtype, s);
    case PBGDN_F32: return run_chunk<K, float>(p, records, out_dtype, s);
    default: return PBGDN_ERR_INVALID_ARGUMENT;
  }
}

// 256-wide keys, 16-bit inputs: the prep kernel, then the k256 scan with the
// tiles per workgroup of k256_waves (two waves per tile, each a half of the
// keys, with two tiles). PBGDN_K256_WAVES=2|4 and PBGDN_K256_SPLIT=1|2 in the
// environment force them (for measurements) where they apply.
inline int env_choice(const char *name, int a, int b) {
  const char *e = getenv(name);
  const int w = e ? atoi(e) : 0;
  return (w == a || w == b) ? w : 0;
}

template <typename TIn>
int run_chunk_k256(const ChunkParams &p, long records, int out_dtype, hipStream_t s) {
  static const int forced_wt = env_choice("PBGDN_K256_WAVES", 2, 4);
  static const int forced_kh = env_choice("PBGDN_K256_SPLIT", 1, 2);
  const int st = launch_prep<256, TIn>(p, records, s);
  if (st != PBGDN_OK) return st;
  int wt = k256_waves(p.V, static_cast<long>(p.num_seqs) * p.Hv, p.cus);
  if (forced_wt && p.V % (16 * forced_wt) == 0) wt = forced_wt;
  int kh = wt == 2 ? 2 : 1;
  if (forced_kh && (forced_kh == 1 || wt == 2)) kh = forced_kh;
  if (out_dtype == PBGDN_F32) return launch_k256<TIn, float>(p, wt, kh, s);
  return launch_k256<TIn, TIn>(p, wt, kh, s);  // out_dtype == in_dtype, checked by the caller
}

// The prefill with the layer epilogue in the wide scan (p.o is hs).
template <typename TIn>
int run_chunk_epilogue(const ChunkParams &p, long records, int hs_dtype, hipStream_t s) {
  const int st = launch_prep<128, TIn>(p, records, s);
  if (st != PBGDN_OK) return st;
  if (hs_dtype == PBGDN_F32) return launch_wide<128, TIn, float, true>(p, s);
  return launch_wide<128, TIn, TIn, true>(p, s);  // hs_dtype == in_dtype, checked by the caller
}

bool valid_dtype(int d) { return d == PBGDN_F32 || d == PBGDN_BF16 || d == PBGDN_F16; }

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The dtypes and widths for which the wide scan can apply the layer epilogue
// (then it does whenever it takes the call: wide_eligible).
bool layer_fusable(int in_dtype, int gate_dtype, int hs_dtype, long gate_stride, int K, int V) {
  return K == 128 && V == 128 && (in_dtype == PBGDN_BF16 || in_dtype == PBGDN_F16) && gate_dtype == in_dtype &&
         (hs_dtype == PBGDN_F32 || hs_dtype == in_dtype) && static_cast<long>(CH) * gate_stride * 2 <= 0x7fffffffL;
}

// Device address of `scratch` per device ordinal, resolved once per device
// (with that device current) on the first no-allocation call there.
constexpr int MAX_DEVICES = 64;
std::atomic<unsigned char *> scratch_ptr[MAX_DEVICES];
std::mutex scratch_mu;

// This call's scratch: the copy on the current device, which must be the
// device of `stream` (the kernels run on the stream's device).
int scratch_for_stream(hipStream_t stream, unsigned char **out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return PBGDN_ERR_LAUNCH;
  if (dev >= MAX_DEVICES) return PBGDN_ERR_UNSUPPORTED;
  if (stream) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess || sdev != dev) return PBGDN_ERR_INVALID_ARGUMENT;
  }
  unsigned char *ptr = scratch_ptr[dev].load(std::memory_order_acquire);
  if (!ptr) {
    std::lock_guard<std::mutex> lock(scratch_mu);
    ptr = scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!ptr) {
      void *addr = nullptr;
      if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || !addr) return PBGDN_ERR_LAUNCH;
      ptr = static_cast<unsigned char *>(addr);
      scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return PBGDN_OK;
}

}  // namespace
}  // namespace pbgdn

namespace pbgdn {
namespace {

// float32 inputs enter the kernels' products as fp16-based operands (q, k as
// fp16, v and the state as bf16 or fp16 high/low pairs), so v and the initial
// states are brought within RANGE_LIMIT by a power of two first: the
// recurrence is linear in (v, h0), and o and the final states of the scaled
// inputs are the scaled results, exactly. range_max_kernel writes
// RANGE_BLOCKS partial maxima into the workspace's tail; the prep kernel's
// first wave reduces them into the scale after them, which the scan reads.
constexpr long RANGE_TAIL_BYTES = 4096;
static_assert((RANGE_BLOCKS + 1) * 4 <= RANGE_TAIL_BYTES, "range tail");

struct RangeParams {
  const float *v;
  long nv;                      // elements of v
  const void *h0;               // initial states or a pool of them (may be NULL)
  int state_dtype;
  const int32_t *state_idx;     // as ChunkParams
  const uint8_t *has_initial_state;
  int num_states, num_seqs;
  long state_elems;             // Hv K V
  float *part;                  // [RANGE_BLOCKS]
};

// Partial maxima of |v| and of |the initial states the call reads| (NaNs
// are passed over; an infinity makes the scale 1).
__global__ __launch_bounds__(256) void range_max_kernel(RangeParams p) {
  __shared__ float wm[4];
  PBGDN_POISON_LDS(wm, sizeof(wm));
  PBGDN_POISON_SYNC();
  float m = 0.f;
  const long stride = static_cast<long>(gridDim.x) * 256;
  for (long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x; i < p.nv; i += stride) m = fmaxf(m, fabsf(p.v[i]));
  if (p.h0) {
    for (int n = 0; n < p.num_seqs; ++n) {
      const long slot = p.state_idx ? static_cast<long>(p.state_idx[n]) : static_cast<long>(n);
      if ((p.state_idx && (slot < 0 || slot >= p.num_states)) || (p.has_initial_state && !p.has_initial_state[n])) {
        continue;
      }
      for (long e = static_cast<long>(blockIdx.x) * 256 + threadIdx.x; e < p.state_elems; e += stride) {
        m = fmaxf(m, fabsf(load_elem(p.h0, slot * p.state_elems + e, p.state_dtype)));
      }
    }
  }
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) p.part[blockIdx.x] = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
}

}  // namespace
}  // namespace pbgdn

extern "C" size_t pbgdn_chunk_workspace_size(int B, int T, int Hv, int num_seqs, int in_dtype) {
  if (B < 0 || T < 0 || Hv <= 0 || num_seqs < 0 || !pbgdn::valid_dtype(in_dtype)) return 0;
  const long records = pbgdn::chunk_records(static_cast<long>(B) * T, num_seqs);
  return static_cast<size_t>(records) * Hv * pbgdn::rec_bytes_of(in_dtype) + pbgdn::RANGE_TAIL_BYTES;
}

namespace pbgdn {
namespace {

// Argument checks of pbgdn_chunk_fwd and its launch parameters: PBGDN_OK with
// *empty set when there is nothing to launch.
int chunk_setup(const void *q, const void *k, const void *v, int in_dtype, const float *g, const void *beta,
                int beta_dtype, const void *h0, void *ht, int state_dtype, const int32_t *state_idx,
                const uint8_t *has_initial_state, int num_states, const int32_t *cu_seqlens, int num_seqs, void *o,
                int out_dtype, int B, int T, int Hk, int Hv, int K, int V, float scale, int chunk, void *workspace,
                size_t workspace_bytes, ChunkParams &p, long &records, bool &empty) {
  empty = false;
  if (B < 0 || T < 0 || Hk <= 0 || Hv <= 0 || K <= 0 || V <= 0 || Hv % Hk != 0 || num_seqs < 0) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype) || !valid_dtype(state_dtype) ||
      !(beta_dtype == PBGDN_F32 || beta_dtype == in_dtype)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (state_idx && num_states < 0) return PBGDN_ERR_INVALID_ARGUMENT;
  if (cu_seqlens ? B != 1 : num_seqs != B) return PBGDN_ERR_INVALID_ARGUMENT;
  if (chunk != pbgdn::CH) return PBGDN_ERR_UNSUPPORTED;
  if (!(K == 64 || K == 128 || K == 256) || V % pbgdn::VT != 0) return PBGDN_ERR_UNSUPPORTED;
  // 256-wide keys (chunk_k256.hip): 16-bit inputs, V a multiple of 32
  if (K == 256 && (in_dtype == PBGDN_F32 || V % 32 != 0)) return PBGDN_ERR_UNSUPPORTED;
  if (!(out_dtype == PBGDN_F32 || out_dtype == in_dtype)) return PBGDN_ERR_UNSUPPORTED;
  // Per-chunk buffer ranges and per-lane offsets are 32-bit byte counts.
  if (static_cast<long>(pbgdn::CH) * Hv * V * 4 > 0x7fffffffL ||
      static_cast<long>(pbgdn::CH) * Hk * K * 4 > 0x7fffffffL) {
    return PBGDN_ERR_UNSUPPORTED;
  }
  if (num_seqs == 0) {
    empty = true;
    return PBGDN_OK;
  }
  if (T > 0 && (!q || !k || !v || !g || !beta || !o)) return PBGDN_ERR_INVALID_ARGUMENT;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v)) return PBGDN_ERR_INVALID_ARGUMENT;
  if (!workspace || !aligned16(workspace) ||
      workspace_bytes < pbgdn_chunk_workspace_size(B, T, Hv, num_seqs, in_dtype)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  const long total = static_cast<long>(V / pbgdn::VT) * Hv * num_seqs;
  if (total > 0x7fffffffL) return PBGDN_ERR_UNSUPPORTED;
  records = chunk_records(static_cast<long>(B) * T, num_seqs);
  // The scan's sequence groups (scan_groups): a chained workgroup pays
  // ~1 µs per sequence boundary instead of a pipeline fill and drain, and the
  // unchained kernel's step is ~10% shorter.
  DeviceShape shape;
  if (!device_shape(shape)) return PBGDN_ERR_LAUNCH;
  const int pairs = (V / VT) * Hv;
  const int groups = scan_groups(static_cast<long>(B) * T, num_seqs, pairs, shape.cus);
  p = ChunkParams{q, k, v, g, beta, beta_dtype, h0, ht, state_dtype, state_idx, has_initial_state,
                  num_states, cu_seqlens, o, static_cast<unsigned char *>(workspace), T, Hk, Hv, V,
                  num_seqs, groups, scale, shape.cus, shape.xcds, nullptr, 0, nullptr, 0.f, nullptr, nullptr};
  return PBGDN_OK;
}

}  // namespace
}  // namespace pbgdn

extern "C" int pbgdn_chunk_fwd(const void *q, const void *k, const void *v, int in_dtype, const float *g,
                               const void *beta, int beta_dtype, const void *h0, void *ht, int state_dtype,
                               const int32_t *state_idx, const uint8_t *has_initial_state, int num_states,
                               const int32_t *cu_seqlens, int num_seqs, void *o, int out_dtype, int B, int T,
                               int Hk, int Hv, int K, int V, float scale, int chunk, void *workspace,
                               size_t workspace_bytes, void *stream) {
  pbgdn::ChunkParams p;
  long records = 0;
  bool empty = false;
  const int st = pbgdn::chunk_setup(q, k, v, in_dtype, g, beta, beta_dtype, h0, ht, state_dtype, state_idx,
                                    has_initial_state, num_states, cu_seqlens, num_seqs, o, out_dtype, B, T, Hk,
                                    Hv, K, V, scale, chunk, workspace, workspace_bytes, p, records, empty);
  if (st != PBGDN_OK || empty) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  {  // debug builds: every element the call writes starts as NaN, so do the records the scan reads
    const long esz = out_dtype == PBGDN_F32 ? 4 : 2, ssz = state_dtype == PBGDN_F32 ? 4 : 2;
    pbgdn::debug_poison(o, static_cast<size_t>(static_cast<long>(B) * T * Hv * V * esz), s);
    if (ht && ht != h0 && !state_idx) {
      pbgdn::debug_poison(ht, static_cast<size_t>(static_cast<long>(num_seqs) * Hv * K * V * ssz), s);
    }
    pbgdn::debug_poison(workspace, workspace_bytes, s);
  }
  if (in_dtype == PBGDN_F32) {  // the range scale of v and the initial states, into the workspace's tail
    float *part = reinterpret_cast<float *>(static_cast<unsigned char *>(workspace) +
                                            records * Hv * pbgdn::rec_bytes_of(PBGDN_F32));
    pbgdn::RangeParams rp{static_cast<const float *>(v), static_cast<long>(B) * T * Hv * V, h0, state_dtype,
                          state_idx, has_initial_state, num_states, num_seqs, static_cast<long>(Hv) * K * V, part};
    hipLaunchKernelGGL(pbgdn::range_max_kernel, dim3(pbgdn::RANGE_BLOCKS), dim3(256), 0, s, rp);
    if (hipGetLastError() != hipSuccess) return PBGDN_ERR_LAUNCH;
    p.range_part = part;
    p.in_scale = part + pbgdn::RANGE_BLOCKS;
  }
  switch (K) {
    case 64: return pbgdn::dispatch_in<64>(p, records, in_dtype, out_dtype, s);
    case 128: return pbgdn::dispatch_in<128>(p, records, in_dtype, out_dtype, s);
    case 256:
      return in_dtype == PBGDN_BF16 ? pbgdn::run_chunk_k256<pbgdn::u16>(p, records, out_dtype, s)
                                    : pbgdn::run_chunk_k256<pbgdn::half_t>(p, records, out_dtype, s);
    default: return PBGDN_ERR_UNSUPPORTED;
  }
}

// The prefill followed by the layer epilogue. Where the wide scan takes the
// call (16-bit inputs, K = V = 128, enough workgroups) and the gate is in the
// inputs' dtype and hs in it or float32, the scan applies the epilogue to each
// chunk's O and writes hs; o is not touched. Otherwise o receives the
// operator's output (in the inputs' dtype) and pbgdn_epilogue_fwd runs after.
extern "C" int pbgdn_chunk_layer_fwd(const void *q, const void *k, const void *v, int in_dtype, const float *g,
                                     const void *beta, int beta_dtype, const void *h0, void *ht, int state_dtype,
                                     const int32_t *state_idx, const uint8_t *has_initial_state, int num_states,
                                     const int32_t *cu_seqlens, int num_seqs, const void *gate, long gate_stride,
                                     int gate_dtype, const float *o_norm, float eps, void *hs, int hs_dtype,
                                     void *o, int B, int T, int Hk, int Hv, int K, int V, float scale, int chunk,
                                     void *workspace, size_t workspace_bytes, void *stream) {
  using pbgdn::aligned16;
  using pbgdn::valid_dtype;
  if (!valid_dtype(gate_dtype) || !valid_dtype(hs_dtype) || !(eps >= 0.f)) return PBGDN_ERR_INVALID_ARGUMENT;
  if (Hv > 0 && V > 0 && (gate_stride < static_cast<long>(Hv) * V || gate_stride % 8 != 0)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (!(V == 64 || V == 128)) return PBGDN_ERR_UNSUPPORTED;  // the epilogue's value widths
  if (static_cast<long>(B) * T == 0) {  // no tokens: the final states only (h0 carried over)
    return pbgdn_chunk_fwd(q, k, v, in_dtype, g, beta, beta_dtype, h0, ht, state_dtype, state_idx,
                           has_initial_state, num_states, cu_seqlens, num_seqs, o, in_dtype, B, T, Hk, Hv, K, V,
                           scale, chunk, workspace, workspace_bytes, stream);
  }
  if (!gate || !o_norm || !hs || !aligned16(gate) || !aligned16(hs)) return PBGDN_ERR_INVALID_ARGUMENT;
  const bool fusable = pbgdn::layer_fusable(in_dtype, gate_dtype, hs_dtype, gate_stride, K, V);
  pbgdn::ChunkParams p;
  long records = 0;
  bool empty = false;
  if (fusable) {
    const int st = pbgdn::chunk_setup(q, k, v, in_dtype, g, beta, beta_dtype, h0, ht, state_dtype, state_idx,
                                      has_initial_state, num_states, cu_seqlens, num_seqs, hs, in_dtype, B, T, Hk,
                                      Hv, K, V, scale, chunk, workspace, workspace_bytes, p, records, empty);
    if (st != PBGDN_OK || empty) return st;
    if (in_dtype == PBGDN_BF16 ? pbgdn::wide_eligible<128, pbgdn::u16>(p)
                               : pbgdn::wide_eligible<128, pbgdn::half_t>(p)) {
      p.gate = gate;
      p.gate_stride = gate_stride;
      p.o_norm = o_norm;
      p.eps = eps;
      hipStream_t s = static_cast<hipStream_t>(stream);
      {  // debug builds: the outputs start as NaN (as in pbgdn_chunk_fwd)
        const long hsz = hs_dtype == PBGDN_F32 ? 4 : 2, ssz = state_dtype == PBGDN_F32 ? 4 : 2;
        pbgdn::debug_poison(hs, static_cast<size_t>(static_cast<long>(B) * T * Hv * V * hsz), s);
        if (ht && ht != h0 && !state_idx) {
          pbgdn::debug_poison(ht, static_cast<size_t>(static_cast<long>(num_seqs) * Hv * K * V * ssz), s);
        }
        pbgdn::debug_poison(workspace, workspace_bytes, s);
      }
      return in_dtype == PBGDN_BF16 ? pbgdn::run_chunk_epilogue<pbgdn::u16>(p, records, hs_dtype, s)
                                    : pbgdn::run_chunk_epilogue<pbgdn::half_t>(p, records, hs_dtype, s);
    }
  }
  // Two passes: o in the inputs' dtype, then the epilogue.
  if (!o || !aligned16(o)) return PBGDN_ERR_INVALID_ARGUMENT;
  pbgdn::debug_poison(hs, static_cast<size_t>(static_cast<long>(B) * T * Hv * V * (hs_dtype == PBGDN_F32 ? 4 : 2)),
                      static_cast<hipStream_t>(stream));
  const int st = pbgdn_chunk_fwd(q, k, v, in_dtype, g, beta, beta_dtype, h0, ht, state_dtype, state_idx,
                                 has_initial_state, num_states, cu_seqlens, num_seqs, o, in_dtype, B, T, Hk, Hv, K,
                                 V, scale, chunk, workspace, workspace_bytes, stream);
  if (st != PBGDN_OK) return st;
  return pbgdn_epilogue_fwd(o, in_dtype, gate, gate_stride, gate_dtype, o_norm, eps, hs, hs_dtype, B, T, Hv, V,
                            stream);
}

extern "C" int pbgdn_chunk_layer_fuses(int in_dtype, int gate_dtype, int hs_dtype, long gate_stride, int num_seqs,
                                       int Hv, int K, int V) {
  using pbgdn::valid_dtype;
  if (!valid_dtype(in_dtype) || !valid_dtype(gate_dtype) || !valid_dtype(hs_dtype) || num_seqs < 0 || Hv <= 0 ||
      !(V == 64 || V == 128) || !(K == 64 || K == 128 || K == 256)) {
    return -1;
  }
  if (!pbgdn::layer_fusable(in_dtype, gate_dtype, hs_dtype, gate_stride, K, V)) return 0;
  pbgdn::DeviceShape shape;
  if (!pbgdn::device_shape(shape)) return -1;
  pbgdn::ChunkParams p{};
  p.V = V;
  p.Hv = Hv;
  p.num_seqs = num_seqs;
  p.cus = shape.cus;
  const bool wide = in_dtype == PBGDN_BF16 ? pbgdn::wide_eligible<128, pbgdn::u16>(p)
                                           : pbgdn::wide_eligible<128, pbgdn::half_t>(p);
  return wide ? 1 : 0;
}

// The prefill of pbgdn_chunk_fwd with the workspace taken from this device's
// `scratch` array: nothing is allocated (no hipMalloc, hipFree or allocating
// library call), so callers under graph capture or in allocation-free loops
// can use it. Calls on one GPU share its array; calls whose work overlaps on
// one GPU (two streams, or two threads) race on it.
extern "C" int pbgdn_chunk_fwd_noalloc(const void *q, const void *k, const void *v, int in_dtype, const float *g,
                                       const void *beta, int beta_dtype, const void *h0, void *ht,
                                       int state_dtype, const int32_t *state_idx,
                                       const uint8_t *has_initial_state, int num_states,
                                       const int32_t *cu_seqlens, int num_seqs, void *o, int out_dtype, int B,
                                       int T, int Hk, int Hv, int K, int V, float scale, int chunk,
                                       void *stream) {
  if (!pbgdn::valid_dtype(in_dtype)) return PBGDN_ERR_INVALID_ARGUMENT;
  if (pbgdn_chunk_workspace_size(B, T, Hv, num_seqs, in_dtype) > PBGDN_NOALLOC_SCRATCH_BYTES) return PBGDN_ERR_SCRATCH;
  unsigned char *ws = nullptr;
  const int st = pbgdn::scratch_for_stream(static_cast<hipStream_t>(stream), &ws);
  if (st != PBGDN_OK) return st;
  // the records need no initialisation: the prep kernel writes every record the scan reads
  return pbgdn_chunk_fwd(q, k, v, in_dtype, g, beta, beta_dtype, h0, ht, state_dtype, state_idx,
                         has_initial_state, num_states, cu_seqlens, num_seqs, o, out_dtype, B, T, Hk, Hv, K, V,
                         scale, chunk, ws, PBGDN_NOALLOC_SCRATCH_BYTES, stream);
}
