// Prep kernel of the chunkwise prefill: the state-independent part of every
// (chunk, value head), computed in parallel over all chunks of all sequences.
//
// Reference: delta_rule_chunked, pseudobrain/gated_deltanet.py:139-157 (cumsum
// of g, decay D, A = strict_lower(beta K K^T o D), the unit-lower-triangular
// solve, Q K^T o D). For chunk record r and value head h it writes the
// workspace record (chunk.hpp):
//   Tb  = (I + A)^-1 diag(beta)                  as 16x16x32 fp16 A fragments
//   QKD = scale (Q K^T o D), D inclusive        as 16x16x32 fp16 A fragments
//   exp(c_t), scale exp(c_t), exp(c_63 - c_t)  fp32
//   Tb - fp16(Tb)                               float32 inputs: the low part, as Tb
//
// A persistent grid of 4-wave workgroups walks the items: a chunk record and
// HPI value heads that share a key head (HPI = 2 when the value heads per key
// head are even, else 1). The inputs of a workgroup's next item are loaded
// into registers while it works on the current one, and items are numbered so
// that neighbours share an XCD.
//
// Per item (barrier-separated stages):
//   stage   K, Q -> LDS (bf16/fp16 kept, fp32 rounded to fp16); waves 3, 2
//           scan g of heads 0, 1 into their decay tables
//   tiles   the 10 lower 16x16 tile pairs of K K^T and Q K^T (bf16/fp16
//           16x16x32 MFMA, fp32 accumulate) once for the key head, kept in
//           registers, formed transposed so each lane holds 4 consecutive
//           elements of a row
// then for each value head:
//   decay   A = beta K K^T o D, QKD = scale Q K^T o D; off-diagonal tiles take
//           the decay as u_t W_R[s] (two multiplies, no masks), diagonal tiles
//           exp(c_t - c_s) with the triangular masks, in fp32 for the inverse
//   diag    the 4 diagonal blocks of T as (I+M)(I+M^2)(I+M^4)(I+M^8), M = -A_ww
//           strictly lower (nilpotent), on fp16 high/low MFMAs (~22-bit products)
//   offdiag the off-diagonal blocks of T by block forward substitution
//           T_rs = -D_r sum_{s<=j<r} A_rj T_js in three independent chains
//   out     Tb and QKD fragments and the decay vectors -> the record
#include "chunk.hpp"

namespace pbgdn {
namespace {

constexpr int PNT = 256;          // threads per prep workgroup
// Resident workgroups per CU: three when the registers allow it (16-bit
// inputs); fp32 inputs hold more registers and keep two, and so do 256-wide
// keys (their K and Q rows take twice the LDS).
template <int K, typename TIn>
constexpr int prep_wg_per_cu() { return sizeof(TIn) == 4 || K == 256 ? 2 : 3; }

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// LDS layout (byte offsets); (swz) as in chunk.hpp. K and Q are read only by
// the tiles stage, and Tb, QKD, A16, AT (and with LO Tb's low part) live from
// the decay stage to the record stores, so the two groups share bytes (a
// barrier separates the two uses); the decay tables follow the larger of the
// two.
template <int K, bool LO>
struct PrepLayout {
  static constexpr int KPB = 2 * K + 32;
  static constexpr int SPB = 2 * CH + 32;
  static constexpr int ATP = 4 * 16 + 16;               // fp32 16-column rows + pad
  static constexpr int KQ_MAT = CH * KPB;
  static constexpr int KQ = 0;                          // [K, Q][64 t][K] operand type (swz)
  static constexpr int TB = 0;                          // [64 t][64 s] fp16 Tb (swz), over K
  static constexpr int QKD = TB + CH * SPB;             // [64 t][64 s] fp16 (swz)
  static constexpr int A16 = QKD + CH * SPB;            // [64 t][64 s] fp16: off-diagonal A, diagonal D (swz)
  static constexpr int AT = A16 + CH * SPB;             // [4 tiles][16][16] fp32 diagonal tiles of A
  static constexpr int AT_END = AT + 4 * 16 * ATP;
  static constexpr int TBL = AT_END;                    // LO: [64 t][64 s] fp16 low part of Tb (swz)
  static constexpr int TBL_END = LO ? TBL + CH * SPB : AT_END;
  static constexpr int SC = TBL_END > 2 * KQ_MAT ? TBL_END : 2 * KQ_MAT;  // [2 heads][11][64] fp32 decay tables
  static constexpr int SC_HEAD = 11 * CH * 4;
  static constexpr int CUM = 0, GAM = 256, DEC = 512, BET = 768, CUM4 = 1024, BET4 = 1280, BU4 = 1536,
                       SU4 = 1792, W1 = 2048;
  static constexpr int BYTES = SC + 2 * SC_HEAD;
};

template <int K, typename TIn>
struct PrepBlock {
  // float32 inputs also store Tb's low fp16 part, so that the scan forms U = Tb X
  // from high/low pairs
  static constexpr bool LO = sizeof(TIn) == 4;
  static constexpr int RB = rec_bytes<TIn>();
  using L = PrepLayout<K, LO>;
  using Op = OpOf<TIn>;
  using O8 = typename Op::T8;
  using Inputs = ChunkInputs<K, TIn, PNT, L, false, true>;
  static constexpr int KS = K / 32;  // contraction steps over keys
  static_assert(K == 64 || K == 128 || (K == 256 && sizeof(TIn) == 2), "K must be 64 or 128, or 256 (16-bit)");
  static_assert(L::TBL_END <= L::SC, "Tb's low part before the decay tables");
  static_assert(L::BYTES * prep_wg_per_cu<K, TIn>() <= 160 * 1024, "prep LDS");

  unsigned char *lds;
  const ChunkParams &p;
  int tid, lane, c16, g4, wave, group_heads, hpi, hgroups, jscan;
  bool nt = false;  // record stores non-temporal (a large call)
  Inputs in;
  float4_t rk[3], rq[3];  // raw K K^T and Q K^T of this wave's tile pairs
  uint32_t kp_frag, sp_frag, sp_tile, at_lane, tr_a;

  __device__ PrepBlock(unsigned char *l, const ChunkParams &prm) : lds(l), p(prm) {
    tid = threadIdx.x;
    lane = tid & 63;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    c16 = lane & 15;
    g4 = lane >> 4;
    group_heads = p.Hv / p.Hk;
    hpi = (group_heads % 2 == 0) ? 2 : 1;
    hgroups = p.Hv / hpi;
    jscan = (3 - wave) < hpi ? 3 - wave : 0;  // head whose g this wave loads (waves 3, 2 scan)
    in.init(p, tid, lane);
    const uint32_t s4 = ((c16 >> 2) & 1) << 4;
    kp_frag = c16 * L::KPB + ((16 * g4) ^ s4);                         // row c, 16 bytes at 16 g
    sp_frag = c16 * L::SPB + ((16 * g4) ^ s4);
    sp_tile = c16 * L::SPB + ((16 * (g4 >> 1)) ^ s4) + 8 * (g4 & 1);  // row c, 8 bytes at 8 g
    at_lane = c16 * L::ATP + 16 * g4;
    // transposing read of a [16][16] fp16 tile: lanes 4k..4k+3 of group g point
    // at row 4g + k, 8 bytes at 8 (c & 3)
    tr_a = (4 * g4 + (c16 >> 2)) * L::SPB + ((8 * (c16 & 3)) ^ ((g4 & 1) << 4));
  }

  template <typename T>
  __device__ T ld(uint32_t off) const { return *reinterpret_cast<const T *>(lds + off); }
  template <typename T>
  __device__ void st(uint32_t off, T x) const { *reinterpret_cast<T *>(lds + off) = x; }
  __device__ i16x4_t ld_tr(uint32_t off) const {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t *)(lds + off));
  }

  // Item = (chunk record, group of hpi value heads) -> first head, sequence,
  // first token, tokens left.
  // Returns false for a record that no sequence's chunk maps to. Everything
  // here is wave-uniform and kept in scalar registers (readfirstlane), so the
  // lookups are scalar loads that do not wait for outstanding vector memory
  // operations.
  __device__ bool locate(int item, int &h, long &rec, long &t0, long &len) const {
    const int r32 = __builtin_amdgcn_readfirstlane(item / hgroups);
    rec = r32;
    h = __builtin_amdgcn_readfirstlane((item - r32 * hgroups) * hpi);  // first value head of the item
    int lo = 0, hi = p.num_seqs - 1;  // largest s with rec_base(s) <= rec
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      long b, e;
      seq_bounds(p, mid, b, e);
      if (rec_base(b, mid) <= rec) lo = mid; else hi = mid - 1;
    }
    long bos, eos;
    seq_bounds(p, lo, bos, eos);
    const long j = rec - rec_base(bos, lo);
    t0 = bos + j * CH;
    len = eos - t0;
    return j >= 0 && len > 0;
  }

  // First valid item at or after `item` on this workgroup's stride.
  __device__ int next_valid(int item, int stride, int items, int &h, long &rec, long &t0, long &len) const {
    for (; item < items; item += stride) {
      if (locate(item, h, rec, t0, len)) return item;
    }
    return items;
  }

  // Raw products of tile pair (R, S), S <= R, formed transposed (rows s from
  // K_S, columns t from K_R and Q_R): lane (g, c) holds row t = 16R + c,
  // columns s = 16S + 4g..4g+3 of K K^T (ak) and Q K^T (aq).
  __device__ void raw_pair(int R, int S, float4_t &ak, float4_t &aq) const {
    const uint32_t kmat = L::KQ + kp_frag;
    const uint32_t qmat = kmat + L::KQ_MAT;
    O8 kr[KS], qr[KS], ks[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      kr[kk] = ld<O8>(kmat + 16 * R * L::KPB + 64 * kk);
      qr[kk] = ld<O8>(qmat + 16 * R * L::KPB + 64 * kk);
      ks[kk] = ld<O8>(kmat + 16 * S * L::KPB + 64 * kk);
    }
    ak = float4_t{0.f, 0.f, 0.f, 0.f};
    aq = ak;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      ak = mma(ks[kk], kr[kk], ak);
      aq = mma(ks[kk], qr[kk], aq);
    }
  }

  // Tile pair i of the list (3,0) (3,1) (3,2) (3,3) (2,0) (2,1) (2,2) (1,0)
  // (1,1) (0,0); wave w takes i = w, w + 4, w + 8 (3, 3, 2, 2 pairs).
  __device__ static int pair_r(int i) { return (i < 4) ? 3 : (i < 7) ? 2 : (i < 9) ? 1 : 0; }
  __device__ static int pair_s(int i) { return i - ((i < 4) ? 0 : (i < 7) ? 4 : (i < 9) ? 7 : 9); }

  __device__ void tiles() {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int i = wave + 4 * j;
      if (i < 10) raw_pair(pair_r(i), pair_s(i), rk[j], rq[j]);
    }
  }

  // Decays of value head jh on the raw tile pairs: tile (R, S) of
  // A = strict_lower(b_t K K^T o D) and QKD = scale (Q K^T o D) (inclusive).
  // Off the diagonal, s < 16R <= t and exp(c_t - c_s) = u_t W_R[s], both
  // factors <= 1 (an underflow only drops a product that is itself below the
  // fp32 range). Diagonal tiles go to AT (fp32, for the inverse), off-diagonal
  // A tiles to A16.
  __device__ void decay(int jh) const {
    const uint32_t sc = L::SC + jh * L::SC_HEAD;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int i = wave + 4 * j;
      if (i >= 10) continue;
      const int R = pair_r(i), S = pair_s(i);
      const int s0 = 16 * S + 4 * g4;
      const uint32_t qkd_out = L::QKD + 16 * R * L::SPB + 32 * S + sp_tile;
      if (R == S) {
        const int t = 16 * R + c16;
        const float ct = pick(ld<float4_t>(sc + L::CUM4 + c16 * 16), R);
        const float bt = pick(ld<float4_t>(sc + L::BET4 + c16 * 16), R);
        const float4_t cs = ld<float4_t>(sc + L::CUM + s0 * 4);
        float4_t av, qv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float d = __expf(ct - cs[e]);
          av[e] = (s0 + e < t) ? bt * rk[j][e] * d : 0.f;
          qv[e] = (s0 + e <= t) ? p.scale * rq[j][e] * d : 0.f;
        }
        st(L::AT + 16 * R * L::ATP + at_lane, av);
        st(qkd_out, to_half4(qv));
      } else {
        const float bu = pick(ld<float4_t>(sc + L::BU4 + c16 * 16), R);
        const float su = pick(ld<float4_t>(sc + L::SU4 + c16 * 16), R);
        const float4_t w = ld<float4_t>(sc + L::W1 + ((R - 1) * CH + s0) * 4);
        st(L::A16 + 16 * R * L::SPB + 32 * S + sp_tile, to_half4(rk[j] * bu * w));
        st(qkd_out, to_half4(rq[j] * su * w));
      }
    }
  }

  // fp16 high/low pair of an fp32 tile, and c + a b from pairs (3 MFMAs, the
  // low*low term dropped): a product accurate to ~22 bits.
  struct Pair16 {
    half4_t h, l;
  };
  __device__ static Pair16 split16(float4_t x) {
    Pair16 r;
    r.h = to_half4(x);
    r.l = to_half4(x - to_float4(r.h));
    return r;
  }
  __device__ static float4_t mul3(const Pair16 &a, const Pair16 &b, float4_t c) {
    c = mfma16(a.h, b.h, c);
    c = mfma16(a.h, b.l, c);
    return mfma16(a.l, b.h, c);
  }

  // Diagonal block D_w = (I + A_ww)^-1 (w = this wave). A_ww is strictly lower
  // triangular (nilpotent), so with M = -A_ww
  //   D = (I + M)(I + M^2)(I + M^4)(I + M^8).
  // Keeping P_k = M^k both as tile(P_k) and tile(P_k^T) gives every operand
  // in registers; tile(M) comes from tile(M^T) as MFMA(tile(M^T), tile(I)).
  // Y = D is built transposed: Y^T <- Y^T + P_k^T Y^T. D goes to A16 (fp16)
  // for the off-diagonal blocks, D diag(beta) to the diagonal block of Tb.
  __device__ void diag(int jh) {
    const int w = wave;
    const float4_t z = {0.f, 0.f, 0.f, 0.f};
    const float4_t p1t = -ld<float4_t>(L::AT + 16 * w * L::ATP + at_lane);  // tile(M^T)
    const float4_t bw = ld<float4_t>(L::SC + jh * L::SC_HEAD + L::BET + (16 * w + 4 * g4) * 4);
    half4_t eye;
#pragma unroll
    for (int j = 0; j < 4; ++j) eye[j] = static_cast<half_t>((4 * g4 + j == c16) ? 1.f : 0.f);
    float4_t yt = p1t;  // tile((I + M)^T)
#pragma unroll
    for (int i = 0; i < 4; ++i) yt[i] += (4 * g4 + i == c16) ? 1.f : 0.f;
    const Pair16 s1t = split16(p1t);
    Pair16 s1;  // tile(M), exactly, from the pair of tile(M^T)
    s1.h = to_half4(mfma16(s1t.h, eye, z));
    s1.l = to_half4(mfma16(s1t.l, eye, z));
    const Pair16 s2 = split16(mul3(s1t, s1, z)), s2t = split16(mul3(s1, s1t, z));  // M^2, (M^2)^T
    yt = mul3(s2, split16(yt), yt);
    const Pair16 s4 = split16(mul3(s2t, s2, z)), s4t = split16(mul3(s2, s2t, z));  // M^4, (M^4)^T
    yt = mul3(s4, split16(yt), yt);
    const Pair16 s8 = split16(mul3(s4t, s4, z));                                    // M^8
    yt = mul3(s8, split16(yt), yt);
    // yt = tile(D^T): lane (g, c) holds D[c][4g + i], row c of D at columns 4g..
    const uint32_t o = 16 * w * L::SPB + 32 * w + sp_tile;
    st(L::A16 + o, to_half4(yt));
    put_tb(o, yt * bw);
  }

  // A tile of Tb (fp32) -> the fp16 Tb tile, and with LO its low part.
  __device__ void put_tb(uint32_t o, float4_t tb) const {
    const half4_t hi = to_half4(tb);
    st(L::TB + o, hi);
    if constexpr (LO) st(L::TBL + o, to_half4(tb - to_float4(hi)));
  }

  // Off-diagonal blocks of T:
  //   T_rs = -D_r Y_rs,  Y_rs = sum_{s<=j<r} A_rj T_js,  T_ss = D_s,
  // with A_rj and D_r from A16 (fp16). Blocks needed by later products are
  // formed as tiles (tile(D_r Y) = MFMA(A op D_r, tile(Y))); every block is
  // also formed transposed (MFMA(tile(Y), A op D_r) = tile((D_r Y)^T)) and
  // written as Tb rows T_rs diag(beta). Chains: T10 -> T20 -> T30; T21 -> T31;
  // T32.
  __device__ void offdiag(int chain, int jh) {
    const float4_t z = {0.f, 0.f, 0.f, 0.f};
    auto aop = [&](int r, int s) { return ld<half4_t>(L::A16 + 16 * r * L::SPB + 32 * s + sp_tile); };
    auto dop = [&](int s) {  // tile(D_s) via a transposing read
      return __builtin_bit_cast(half4_t, ld_tr(L::A16 + 16 * s * L::SPB + 32 * s + tr_a));
    };
    auto put = [&](int r, int s, float4_t mt) {  // mt = tile((D_r Y_rs)^T) = -tile(T_rs^T)
      const float4_t bs = ld<float4_t>(L::SC + jh * L::SC_HEAD + L::BET + (16 * s + 4 * g4) * 4);
      put_tb(16 * r * L::SPB + 32 * s + sp_tile, -mt * bs);
    };
    if (chain == 0) {
      const half4_t a10 = aop(1, 0), a20 = aop(2, 0), a21 = aop(2, 1);
      const half4_t a30 = aop(3, 0), a31 = aop(3, 1), a32 = aop(3, 2);
      const half4_t d1 = aop(1, 1), d2 = aop(2, 2), d3 = aop(3, 3), d0 = dop(0);
      const half4_t y10 = to_half4(mfma16(a10, d0, z));
      const half4_t t10 = to_half4(-mfma16(d1, y10, z));
      put(1, 0, mfma16(y10, d1, z));
      const half4_t y20 = to_half4(mfma16(a21, t10, mfma16(a20, d0, z)));
      const half4_t t20 = to_half4(-mfma16(d2, y20, z));
      put(2, 0, mfma16(y20, d2, z));
      const half4_t y30 = to_half4(mfma16(a32, t20, mfma16(a31, t10, mfma16(a30, d0, z))));
      put(3, 0, mfma16(y30, d3, z));
    } else if (chain == 1) {
      const half4_t a21 = aop(2, 1), a31 = aop(3, 1), a32 = aop(3, 2);
      const half4_t d2 = aop(2, 2), d3 = aop(3, 3), d1 = dop(1);
      const half4_t y21 = to_half4(mfma16(a21, d1, z));
      const half4_t t21 = to_half4(-mfma16(d2, y21, z));
      put(2, 1, mfma16(y21, d2, z));
      const half4_t y31 = to_half4(mfma16(a32, t21, mfma16(a31, d1, z)));
      put(3, 1, mfma16(y31, d3, z));
    } else {
      const half4_t a32 = aop(3, 2), d3 = aop(3, 3), d2 = dop(2);
      put(3, 2, mfma16(to_half4(mfma16(a32, d2, z)), d3, z));
    }
  }

  // Fragments f = wave + 4 j of Tb (f < 6), QKD (6 <= f < 12) and with LO
  // Tb's low part (12 <= f < 18) but for their units no scan reads
  // (rec_unused_unit), and the decay vectors of waves 0-2 -> the workspace
  // record. Every wave issues the same stores (past
  // the last fragment to an offset out of range); rec < 0 issues them with a
  // zero-size resource.
  __device__ void out(long rec, int h, int jh) const {
    const __amdgpu_buffer_rsrc_t rr = rsrc(p.ws + (rec * p.Hv + h) * static_cast<long>(RB), rec >= 0 ? RB : 0);
    constexpr int NF = (LO ? 3 : 2) * NFRAG;
#pragma unroll
    for (int j = 0; j < (NF + 3) / 4; ++j) {
      const int f = wave + 4 * j;
      const int m = f < NF ? f / NFRAG : 0;  // 0 Tb, 1 QKD, 2 Tb low
      const int fi = f < NF ? f - m * NFRAG : 0;
      const int r = fi < 2 ? fi : 2 + ((fi - 2) >> 1);
      const int kk = fi < 2 ? 0 : ((fi - 2) & 1);
      const uint32_t src = (m == 0 ? L::TB : m == 1 ? L::QKD : L::TBL) + 16 * r * L::SPB + sp_frag + 64 * kk;
      // the units no scan reads are not stored
      const uint32_t at = (m == 0 ? REC_TB : m == 1 ? REC_QKD : REC_TBL) + fi * FRAG_BYTES + lane * 16;
      const uint32_t dst = f < NF && !rec_unused_unit(static_cast<int>(at)) ? at : OUT_OF_RANGE;
      const u32x4_t x = __builtin_bit_cast(u32x4_t, ld<half8_t>(src));
      if (nt) {
        __builtin_amdgcn_raw_buffer_store_b128(x, rr, dst, 0, 2);
      } else {
        __builtin_amdgcn_raw_buffer_store_b128(x, rr, dst, 0, 0);
      }
    }
    const uint32_t sc = L::SC + jh * L::SC_HEAD;
    const float gam = ld<float>(sc + L::GAM + lane * 4);
    const float val = wave == 0 ? gam
                      : wave == 1 ? p.scale * gam
                      : ld<float>(sc + (wave == 2 ? L::DEC : L::CUM) + lane * 4);
    const uint32_t dst = wave < 3 ? REC_SC + 256 * wave + lane * 4 : OUT_OF_RANGE;  // SC_GAM, SC_GSC, SC_DEC
    if (nt) {
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, val), rr, dst, 0, 2);
    } else {
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, val), rr, dst, 0, 0);
    }
  }

  // Blocks (0, 1) and (2, 3) of Tb and QKD (and of Tb's low part) lie above
  // the diagonal inside the fragments the record holds and must read as
  // zero; the staging of K and Q overwrote them, so each wave clears one of
  // the four per item (and one of Tb's low part).
  __device__ void clear_upper() const {
    const int r = (wave & 1) ? 2 : 0;
    const uint32_t base = (wave & 2) ? L::QKD : L::TB;
    st(base + 16 * r * L::SPB + 32 * (r + 1) + sp_tile, half4_t{});
    if constexpr (LO) st(L::TBL + 16 * r * L::SPB + 32 * (r + 1) + sp_tile, half4_t{});  // waves 0, 2 and 1, 3 alike
  }

  // Items of this workgroup (prep_share, schedule.hpp).
  __device__ void share(int items, int &first, int &stride, int &end) const {
    const PrepShare sh = prep_share(items, static_cast<int>(gridDim.x), static_cast<int>(blockIdx.x), p.cus, p.xcds);
    first = sh.first;
    stride = sh.stride;
    end = sh.end;
  }

  __device__ void run(int items) {
    int first, stride, end;
    share(items, first, stride, end);
    int h;
    long rec, t0, len;
    int item = next_valid(first, stride, end, h, rec, t0, len);
    if (item >= end) return;
    // Every wave issues the same memory operations on every path (loads of an
    // absent next item have zero length; the stores before the first item go
    // nowhere), so waits for the item's inputs never cover newer stores.
    in.load(p, t0, len, h / group_heads, h + jscan, 0);
    out(-1, 0, 0);
    while (true) {
      int h_n = 0;
      long rec_n = 0, t0_n = 0, len_n = 0;
      const int next = next_valid(item + stride, stride, end, h_n, rec_n, t0_n, len_n);
      block_sync();  // the previous item's readers of K, Q, the tables and Tb/QKD are done
      in.store(lds, 0, tid, lane, wave >= 4 - hpi, p.scale, jscan * L::SC_HEAD);
      in.load(p, t0_n, next < end ? len_n : 0, h_n / group_heads, h_n + jscan, 0);
      block_sync();
      tiles();
      block_sync();  // K, Q are read; Tb, QKD, A16, AT take their bytes
      clear_upper();
      for (int jh = 0; jh < hpi; ++jh) {
        if (jh > 0) block_sync();  // out() of the previous head has read Tb, QKD
        decay(jh);
        block_sync();
        diag(jh);
        block_sync();
        if (wave < 3) offdiag(wave, jh);
        block_sync();
        out(rec, h + jh, jh);
      }
      if (next >= end) break;
      item = next;
      h = h_n;
      rec = rec_n;
      t0 = t0_n;
      len = len_n;
    }
  }
};

template <int K, typename TIn>
__global__ __launch_bounds__(PNT, (prep_wg_per_cu<K, TIn>())) void prep_kernel(ChunkParams p, int items, int nt) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  PBGDN_POISON_LDS(smem_raw, (PrepLayout<K, sizeof(TIn) == 4>::BYTES));
  PBGDN_POISON_SYNC();
  if constexpr (sizeof(TIn) == 4) {  // the range scale the scan reads (prep reads none of v)
    if (p.range_part && blockIdx.x == 0 && threadIdx.x < 64) {
      range_scale_wave(p.range_part, const_cast<float *>(p.in_scale));
    }
  }
  PrepBlock<K, TIn> blk(smem_raw, p);
  blk.nt = nt != 0;
  blk.run(items);
}

}  // namespace

constexpr long REC_STREAM_BYTES = 64L << 20;

template <int K, typename TIn>
int launch_prep(const ChunkParams &p, long records, hipStream_t stream) {
  static std::atomic<bool> configured[MAX_DEVICES];  // the attribute is set per device
  const size_t smem = PrepLayout<K, sizeof(TIn) == 4>::BYTES;
  auto kernel = prep_kernel<K, TIn>;
  if (!smem_configured(reinterpret_cast<const void *>(kernel), smem, configured)) return PBGDN_ERR_LAUNCH;
  const int hpi = ((p.Hv / p.Hk) % 2 == 0) ? 2 : 1;  // value heads per item (PrepBlock::hpi)
  const long items = records * (p.Hv / hpi);
  if (items > 0x3fffffffL) return PBGDN_ERR_UNSUPPORTED;  // item numbers are 32-bit
  const long grid = prep_grid(items, p.cus, prep_wg_per_cu<K, TIn>(), p.xcds);
  // Records of a large call are written non-temporally: measured on the
  // 32,768-token call, the whole call is 2% faster than with cached stores
  // (0.663-0.666 against 0.673-0.676 ms with the 160 MB of records stored
  // now; the same with the 213 MB stored before).
  const int nt = records * p.Hv * static_cast<long>(rec_bytes<TIn>()) > REC_STREAM_BYTES ? 1 : 0;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(PNT), smem, stream, p, static_cast<int>(items), nt);
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}

template int launch_prep<64, u16>(const ChunkParams &, long, hipStream_t);
template int launch_prep<64, half_t>(const ChunkParams &, long, hipStream_t);
template int launch_prep<64, float>(const ChunkParams &, long, hipStream_t);
template int launch_prep<128, u16>(const ChunkParams &, long, hipStream_t);
template int launch_prep<128, half_t>(const ChunkParams &, long, hipStream_t);
template int launch_prep<128, float>(const ChunkParams &, long, hipStream_t);
template int launch_prep<256, u16>(const ChunkParams &, long, hipStream_t);
template int launch_prep<256, half_t>(const ChunkParams &, long, hipStream_t);

}  // namespace pbgdn
