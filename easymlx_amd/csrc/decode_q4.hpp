// Single-token paged decode over 4-bit affine pages, head_dim 128, on the
// 16-block 4x4x4 MFMA (v_mfma_f32_4x4x4_16b_f16), group size 64 or 128.
//
// Replaces the reference's per-(seq, q_head) serial key loop
// (lib/python/easymlx/operations/kernels/unified_attention.py:467-609) and its
// split-K variant (page_attention.py:1718-2059) for int4 pages.  Work
// decomposition, split-K partials and the in-kernel merge are those of
// decode_affine_d128 (decode_affine.hpp); only the per-item math differs.
//
// Per item (64 tokens of one (sequence, kv_head); lane L = 0..63):
//   QK^T : A = K codes, lane L holds token L's row (MFMA row = token),
//          B = query, column = head (4 heads of a head quad), broadcast to all
//          16 blocks from one 16-lane group (blgp 4..7), so 8 VGPR pairs hold
//          the query operands of all 32 k-steps.  Output: lane L holds head
//          L%4 of tokens 4*(L/4) .. +3, every output element a live score.
//          One accumulator per quantization group; the affine scale and bias
//          are applied per (token, group) after the MFMAs:
//            s = sum_g scale[t,g] * C_g + bias[t,g] * sum_{d in g} q_d
//   softmax: online, base 2, fp32; the per-head max and sum run over the 16
//          lanes of a head (DPP row rotations, then two cross-row shuffles).
//   PV   : A = P' = p * v_scale[t, g] in fp16 (its rounding error folded into the fp32 bias term at the
//          centre code 8), lane layout exactly as the QK
//          output; block tau of A is broadcast to all blocks (cbsz 4, abid
//          tau), so no transpose is needed.  B = V codes, lane L holds dims L
//          and 64 + L (one group half each).  Output: lane L holds dims L and
//          64 + L of the 4 heads.  sum_t p_t * v_bias[t, g] is kept in fp32.
//
// Codes enter the MFMA as exact fp16 subnormals: for a word x of eight 4-bit
// codes, x & 0x000F000F and x & 0x00F000F0 (and the same for x >> 8) are the
// code pairs of nibbles (0,4), (1,5)*16, (2,6), (3,7)*16.  The factor 16 is
// taken out of the other operand (query / P' elements 2, 3 of each k-step).
// Value words interleave tokens (token k at nibble (k >> 1) | ((k & 1) << 2)),
// so each k-step of PV covers 4 consecutive tokens, the token quad of one QK
// output block.
#pragma once

#include <utility>

#include "decode_affine.hpp"

namespace emx {

typedef h16 h16x4 __attribute__((ext_vector_type(4)));

template <int CBSZ, int ABID, int BLGP>
__device__ __forceinline__ f32x4 mfma4(const h16x4 a, const h16x4 b, const f32x4 c) {
  return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, CBSZ, ABID, BLGP);
}

template <class F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
// f(std::integral_constant<int, i>) for i = 0 .. N-1, with i usable as a constant.
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Code pairs (nibbles 0,4) and (1,5)*16 of x as one 4-element MFMA operand.
__device__ __forceinline__ h16x4 nib_pairs(const uint32_t x) {
  return __builtin_bit_cast(h16x4, u32x2{x & 0x000F000Fu, x & 0x00F000F0u});
}

__device__ __forceinline__ float half_of(const uint32_t (&w)[2], const int i) {
  const uint32_t x = w[i >> 1];
  return (float)__builtin_bit_cast(h16, (uint16_t)((i & 1) ? (x >> 16) : (x & 0xFFFFu)));
}

template <int GS, int HQ>
struct Q4Cfg {
  static constexpr int D = 128;
  static constexpr int G = D / GS;  // quantization groups per head
  static constexpr int NT = 64;     // tokens per work item
  static constexpr int W = 16;      // K code words per token
  static_assert(GS == 64 || GS == 128, "a value half (64 dims) must lie in one quantization group");
};

// Register image of one item's loads.
template <int GS, int HQ>
struct Q4Loads {
  static constexpr int G = Q4Cfg<GS, HQ>::G;
  static constexpr int NSEG = 4 * G;                 // (array, group) segments of 64 tokens, 128 B each
  static constexpr int SNI = NSEG * 8 > 64 ? NSEG * 8 / 64 : 1;  // 16-byte scale pieces per lane
  uint32_t k[16];       // K codes of token L (128 dims)
  uint32_t v[2][8];     // V codes of dims L and 64 + L, 64 tokens
  u32x4 sraw[SNI];      // scale pieces as loaded: piece 64i + L = segment (64i + L) / 8, tokens 8 * ((64i + L) % 8) ..
  uint32_t s[4][G][2];  // after staging: k_scale, k_bias, v_scale, v_bias of tokens 4*(L/4) .. +3, per group
};

// Per-lane base pointers of the scale pieces: piece P = 64i + L is segment
// seg = P / 8 = (array seg / G, group seg % G), tokens 8 * (P % 8) .. + 7.
template <int GS>
struct Q4ScalePtrs {
  static constexpr int G = 128 / GS, NSEG = 4 * G, SNI = NSEG * 8 > 64 ? NSEG * 8 / 64 : 1;
  const h16* p[SNI];
};

template <int GS>
__device__ __forceinline__ Q4ScalePtrs<GS> q4_scale_ptrs(const DecodeArgs& a, const int lane) {
  using SP = Q4ScalePtrs<GS>;
  SP r;
#pragma unroll
  for (int i = 0; i < SP::SNI; ++i) {
    const int P = (64 * i + lane) % (SP::NSEG * 8);  // G = 1: lanes 32..63 repeat 0..31
    const int seg = P / 8, arr = seg / SP::G, g = seg % SP::G;
    const h16* base = arr == 0 ? a.ks : arr == 1 ? a.kb : arr == 2 ? a.vs : a.vb;
    r.p[i] = base + (size_t)g * a.bs + 8 * (P % 8);
  }
  return r;
}

// Scale pieces -> per-lane token-quad values, through this wave's LDS region
// [16 quads][NSEG] of 8 bytes.
template <int GS, int HQ>
__device__ __forceinline__ void q4_stage_scales(Q4Loads<GS, HQ>& L, u32x2* region, const int lane) {
  using LD = Q4Loads<GS, HQ>;
  constexpr int G = LD::G, NSEG = LD::NSEG;
#pragma unroll
  for (int i = 0; i < LD::SNI; ++i) {
    const int P = 64 * i + lane;
    if (NSEG * 8 >= 64 || P < NSEG * 8) {
      const int seg = P / 8, pc = P % 8;
      region[(2 * pc) * NSEG + seg] = u32x2{L.sraw[i][0], L.sraw[i][1]};
      region[(2 * pc + 1) * NSEG + seg] = u32x2{L.sraw[i][2], L.sraw[i][3]};
    }
  }
#pragma unroll
  for (int seg = 0; seg < NSEG; ++seg) {
    const u32x2 y = region[(lane >> 2) * NSEG + seg];
    L.s[seg / G][seg % G][0] = y[0];
    L.s[seg / G][seg % G][1] = y[1];
  }
}

template <int GS, int HQ>
__device__ __forceinline__ void q4_issue_loads(Q4Loads<GS, HQ>& L, const TileRsrc& rs, const Q4ScalePtrs<GS>& sp,
                                               const size_t soff, const int it, const int lane, const int bs) {
  constexpr int G = Q4Cfg<GS, HQ>::G;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rs.k, lane * 64 + 16 * v, it * 64 * 64, kLoadAux);
#pragma unroll
    for (int e = 0; e < 4; ++e) L.k[4 * v + e] = x[e];
  }
#pragma unroll
  for (int c = 0; c < 2; ++c) {
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const u32x4 x =
          __builtin_amdgcn_raw_buffer_load_b128(rs.v, (64 * c + lane) * 32 + 16 * v, it * 128 * 8 * 4, kLoadAux);
#pragma unroll
      for (int e = 0; e < 4; ++e) L.v[c][4 * v + e] = x[e];
    }
  }
  (void)bs;
#pragma unroll
  for (int i = 0; i < Q4Loads<GS, HQ>::SNI; ++i)
    L.sraw[i] = *reinterpret_cast<const u32x4*>(sp.p[i] + soff + it * 64);
}

// One wave-item's loads over pages of PS = 16, 32 or 64 tokens: the 64-token slice
// spans NSUB = 64 / PS pages pg[0 .. NSUB-1] (an invalid id reads page 0; its tokens
// are masked by the compute).  K: lane L holds token L's row from page pg[L / PS]
// (per-lane address).  V: a page holds one tile of PS tokens per dim (PS / 8 words,
// v_word_index), so dim lane d takes PS / 8 words from each page.  Scales: piece
// 64i + L (8 tokens of one (array, group) run) from the page of its tokens.  The
// register image is the big-page one (q4_issue_loads).
template <int GS, int PS>
__device__ __forceinline__ void q4_issue_loads_small(Q4Loads<GS, 1>& L, const DecodeArgs& a, const int (&pg)[64 / PS],
                                                     const int kh, const int lane) {
  constexpr int NSUB = 64 / PS, G = Q4Cfg<GS, 1>::G, D = 128, VW = PS / 8;
  auto page = [&](int j) { return (unsigned)pg[j] < (unsigned)a.nb ? pg[j] : 0; };
  {
    int pl = page(0);
#pragma unroll
    for (int j = 1; j < NSUB; ++j) pl = lane / PS == j ? page(j) : pl;
    const uint32_t* kp = a.kc + ((size_t)pl * a.Hkv + kh) * (PS * 16) + (lane % PS) * 16;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const u32x4 x = *reinterpret_cast<const u32x4*>(kp + 4 * v);
#pragma unroll
      for (int e = 0; e < 4; ++e) L.k[4 * v + e] = x[e];
    }
  }
#pragma unroll
  for (int c = 0; c < 2; ++c) {
#pragma unroll
    for (int j = 0; j < NSUB; ++j) {
      const uint32_t* vp = a.vc + (((size_t)page(j) * a.Hkv + kh) * D + 64 * c + lane) * VW;
      if constexpr (VW == 2) {
        const u32x2 x = *reinterpret_cast<const u32x2*>(vp);
        L.v[c][2 * j] = x[0];
        L.v[c][2 * j + 1] = x[1];
      } else {
#pragma unroll
        for (int h = 0; h < VW / 4; ++h) {
          const u32x4 x = *reinterpret_cast<const u32x4*>(vp + 4 * h);
#pragma unroll
          for (int e = 0; e < 4; ++e) L.v[c][VW * j + 4 * h + e] = x[e];
        }
      }
    }
  }
  using LD = Q4Loads<GS, 1>;
  const h16* sb[4] = {a.ks, a.kb, a.vs, a.vb};
#pragma unroll
  for (int i = 0; i < LD::SNI; ++i) {
    const int P = (64 * i + lane) % (LD::NSEG * 8);
    const int seg = P / 8, arr = seg / G, g = seg % G, t0 = 8 * (P % 8);
    int pj = page(0);
#pragma unroll
    for (int j = 1; j < NSUB; ++j) pj = t0 / PS == j ? page(j) : pj;
    const h16* base = arr == 0 ? sb[0] : arr == 1 ? sb[1] : arr == 2 ? sb[2] : sb[3];
    L.sraw[i] = *reinterpret_cast<const u32x4*>(base + (((size_t)pj * a.Hkv + kh) * G + g) * PS + t0 % PS);
  }
}

// Per-lane softmax / accumulator state of one head quad.
struct Q4State {
  f32x4 o[2];   // dims L, 64 + L of the quad's 4 heads (2^-24 units)
  float m;      // running max of this lane's head (scaled log2 units)
  float l;      // this lane's share of the softmax denominator
  float pb[2];  // this lane's share of sum_t p_t * v_bias[t, g]
};

// Reduce over the 16 lanes holding one head (lanes L, L^4, L^8, ... within
// rows of 16, then across rows).
__device__ __forceinline__ float head_sum(float v) {
  v += row_ror<4>(v);
  v += row_ror<8>(v);
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

__device__ __forceinline__ float head_max(float v) {
  v = fmaxf(v, row_ror<4>(v));
  v = fmaxf(v, row_ror<8>(v));
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}

// One 64-token item.  `full`: every token of the item is inside [start_k, kv_len).
// sub_ok (small pages, PS tokens each): bit j set when page j of the slice is valid.
template <int GS, int HQ, int PS = 0>
__device__ __forceinline__ void q4_compute(Q4Loads<GS, HQ>& L, const bool full, const int lane, const int tok_base,
                                           const int start_k, const int kv_len, const h16x4 (&qB)[HQ][8],
                                           const float (&qs)[HQ][2], const float sc_l2, Q4State (&st)[HQ],
                                           const int sub_ok = 1) {
  constexpr int G = Q4Cfg<GS, HQ>::G;

  // ---- S = K Q^T, one accumulator per (head quad, group)
  f32x4 acc[HQ][G];
#pragma unroll
  for (int hq = 0; hq < HQ; ++hq)
#pragma unroll
    for (int g = 0; g < G; ++g) acc[hq][g] = f32x4{0.f, 0.f, 0.f, 0.f};
  static_for<16>([&](auto M) {
    constexpr int m = decltype(M)::value;  // K word m = dims 8m .. 8m+7
    constexpr int g = (8 * m) / GS;
    const uint32_t x = L.k[m];
    const h16x4 a0 = nib_pairs(x), a1 = nib_pairs(x >> 8);
#pragma unroll
    for (int hq = 0; hq < HQ; ++hq) {
      acc[hq][g] = mfma4<0, 0, 4 + (2 * m) % 4>(a0, qB[hq][(2 * m) / 4], acc[hq][g]);
      acc[hq][g] = mfma4<0, 0, 4 + (2 * m + 1) % 4>(a1, qB[hq][(2 * m + 1) / 4], acc[hq][g]);
    }
  });

  // ---- dead tokens (outside [start_k, kv_len)): score -inf, value scale / bias 0
  const int t0 = tok_base + 4 * (lane >> 2);
  bool live[4] = {true, true, true, true};
  if (!full) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      live[i] = t0 + i >= start_k && t0 + i < kv_len;
      if constexpr (PS != 0) live[i] = live[i] && ((sub_ok >> ((t0 + i - tok_base) / PS)) & 1);
    }
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t keep = (live[2 * w] ? 0x0000FFFFu : 0u) | (live[2 * w + 1] ? 0xFFFF0000u : 0u);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        L.s[2][g][w] &= keep;
        L.s[3][g][w] &= keep;
      }
    }
  }

#pragma unroll
  for (int hq = 0; hq < HQ; ++hq) {
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) v = fmaf(acc[hq][g][i], half_of(L.s[0][g], i), fmaf(half_of(L.s[1][g], i), qs[hq][g], v));
      sc[i] = live[i] ? v : -INFINITY;
    }
    // ---- online softmax in base 2 (scores scaled by sc_l2 = softmax_scale * log2(e) * 2^24)
    const float tmax = head_max(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
    const float m_new = fmaxf(st[hq].m, tmax * sc_l2);
    if (__any(m_new != st[hq].m)) {
      const float alpha = __builtin_amdgcn_exp2f(st[hq].m - m_new);  // lane's head; 0 while m is -inf
      st[hq].l *= alpha;
      st[hq].pb[0] *= alpha;
      st[hq].pb[1] *= alpha;
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // lane i holds head i of the quad
        const float ai = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), i));
        st[hq].o[0][i] *= ai;
        st[hq].o[1][i] *= ai;
      }
      st[hq].m = m_new;
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = __builtin_amdgcn_exp2f(fmaf(sc[i], sc_l2, -fmaxf(st[hq].m, -3.0e38f)));  // 0 for a dead score
      st[hq].l += p[i];
    }
    // ---- O += P' V, P' = p * v_scale (elements 2, 3 of each quad / 16: their codes enter * 16)
    // rounded once to fp16; its rounding error e is folded into the fp32 bias term at
    // the centre code 8 (sum P' * c = sum fp16(P') * c + sum e * 8 + sum e * (c - 8)),
    // so the loss is e * (c - 8), |c - 8| <= 8, instead of e * c.  One fp16 P' alone put
    // outputs near zero (sum P' * code cancelling sum p * v_bias) up to 1.02x the
    // tolerance on short-context batches; with the centre 0.44x (float64 model of this
    // arithmetic on the same seeds); a second MFMA pass over the lo part of P' gave
    // ~1e-4x at twice the PV matrix work.
    h16x4 pv[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        st[hq].pb[g] = fmaf(p[i], half_of(L.s[3][g], i), st[hq].pb[g]);
        const float x = (i < 2 ? p[i] : p[i] * 0.0625f) * half_of(L.s[2][g], i);
        pv[g][i] = (h16)x;
        st[hq].pb[g] = fmaf(x - (float)pv[g][i], i < 2 ? 8.f : 128.f, st[hq].pb[g]);
      }
    }
    static_for<8>([&](auto Wd) {
      constexpr int w = decltype(Wd)::value;  // V word w = tokens 8w .. 8w+7 of the item
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const uint32_t x = L.v[c][w];
        const int g = (64 * c) / GS;
        st[hq].o[c] = mfma4<4, 2 * w, 0>(pv[g], nib_pairs(x), st[hq].o[c]);
        st[hq].o[c] = mfma4<4, 2 * w + 1, 0>(pv[g], nib_pairs(x >> 8), st[hq].o[c]);
      }
    });
  }
}

// Work decomposition of decode_q4_d128.  The unit of work is a workgroup of
// four waves; a workgroup item is TW = 64 * 4 / HQ consecutive tokens of one
// (sequence, kv_head) unit, wave k taking head quad k % HQ of the 64-token
// slice k / HQ.  Items are ordered unit-major; workgroup w of NWG takes the
// contiguous range [w*I/NWG, (w+1)*I/NWG), so only the first and the last unit
// of a range can be shared with other workgroups.
//   * unit end: the waves' (o, m, l) of the unit are combined in LDS (one
//     barrier); a unit inside the range is written to the output directly;
//   * a shared unit leaves one fp32 partial per workgroup (slot = w + unit),
//     written with device-coherent (SC1) stores; at the end of its range the
//     workgroup waits for its stores, counts its arrival on the unit's
//     counter, and the workgroup that arrives last merges the partials
//     (page_attention.py:2006-2059) and resets the counter.
template <int HG>
struct Q4Geom {
  static constexpr int HQ = (HG + 3) / 4;  // head quads (4 heads each, padded)
  static constexpr int NSL = 4 / HQ;       // 64-token slices per workgroup item
  static constexpr int TW = 64 * NSL;      // tokens per workgroup item
  static_assert(HQ == 1 || HQ == 2 || HQ == 4, "GQA ratio 1, 2, 4, 8 or 16");
};

// Cost-balanced ranges.  A workgroup's time grows with its items (kCostItem
// each), with the units it touches (kCostUnit each: the unit-end reductions,
// combine and stores, and the split-K partial and merge of a shared unit) and,
// for a workgroup that starts in the second slot of a compute unit, by a start
// delay (kCostLag: its first loads queue behind the first workgroup's).  With
//   C(x) = kCostItem * x + kCostUnit * #{unit starts <= x}   (units with items)
// workgroup w starts at b_w = min{x : NWG * C(x) >= T_w}, where
//   T_w = w * P                    for w <= N1 (first-slot workgroups),
//   T_w = N1 * P + (w - N1) * Q    after,  P = C(I) + Le * (NWG - N1), Q = P - NWG * Le,
// so every range gets an equal share of C, the second-slot ones Le less, and
// T_NWG = NWG * C(I).  A target inside the step of C at a unit start lands on
// that start, so ranges prefer to end at unit boundaries.  Only wave-uniform
// integer multiplications and float estimates corrected by exact comparisons: no
// 64-bit division.  c2: equal item ranges 27.2 us, these 26.1 us (kCostUnit 20..32
// and kCostLag 31..48 all within 0.2 us of each other); the same ranges handed in
// from the host measured 24.9-25.1 us, the difference being this search on every
// workgroup's critical path (~2 us from kv_lens to the boundaries).  The weights:
// per-workgroup end clocks of the c2 decode (s_memrealtime, 40 launches) fit
// end = 1.0 + 2.02 items + 2.54 units + 5.31 (second slot) us, i.e. a unit ~1.26
// items and the second slot's lag ~2.6 items; unit 16 / lag 40 measured 24.17 us
// against 24.58 for 24 / 48 (20 / 42: 24.23; 12 / 40: 24.19; 16 / 36: 24.31).
constexpr int kCostItem = 16, kCostUnit = 16, kCostLag = 40;

struct Q4Balance {
  long long P, Q;
  int NWG, N1;
  __device__ __forceinline__ long long target(const int w) const {
    return w <= N1 ? (long long)w * P : (long long)N1 * P + (long long)(w - N1) * Q;
  }
  // The workgroup whose range holds an item x with NWG * C(x) = X: max{w < NWG : T_w <= X}.
  __device__ __forceinline__ int wg_of(const long long X) const {
    const long long XN = (long long)N1 * P;
    int w = X < XN ? (int)((float)X / (float)P) : N1 + (int)((float)(X - XN) / (float)Q);
    w = min(max(w, 0), NWG - 1);
    while (w + 1 < NWG && target(w + 1) <= X) ++w;
    while (w > 0 && target(w) > X) --w;
    return w;
  }
};

// Q4Balance::wg_of with one lane per candidate around the float estimate (one
// ballot); the scalar correction loop only if the estimate were off by > 31.
__device__ __forceinline__ int wg_of_lanes(const Q4Balance& bl, const long long X, const int lane) {
  const long long XN = (long long)bl.N1 * bl.P;
  const int est = X < XN ? (int)((float)X * __builtin_amdgcn_rcpf((float)bl.P))
                         : bl.N1 + (int)((float)(X - XN) * __builtin_amdgcn_rcpf((float)bl.Q));
  const int w = est - 31 + lane;
  const unsigned long long pb = __ballot(w <= 0 || (w < bl.NWG && bl.target(w) <= X));
  if (pb != ~0ull && (pb & 1ull)) return min(max(est - 31 + 63 - __builtin_clzll(pb), 0), bl.NWG - 1);
  return bl.wg_of(X);
}

// Plan cache.  A decode step runs the same batch through every layer: the same
// kv_lens, so the same item counts, workgroup ranges and first items; and from
// one step to the next each kv_len grows by one token, which leaves a
// sequence's item count unchanged except when it crosses a TW boundary.  The
// ranges are a function of the item counts alone (and of the shape).  A pure
// decode call (no mixed batch) keeps, in a region of the caller's workspace, the
// plan it computed: per workgroup {g0, g1, pk_first, pk_last, first sequence,
// kv head, token base, -, page of each 64-token slice of the first item}, plus a
// copy of the per-sequence item counts and a header {generation, S, Hkv, NWG,
// window, first_slot, kernel kind, kv_len cap}.  The next call on the workspace
// loads its entry, the header and the copy in its first memory round trip, sends
// the first item's query and page loads out at once, and uses the cached ranges
// when the header matches its shape and the copy matches its item counts
// (compared during the table scan); its first item's sequence, head, token base
// and pages are checked against this call's own (the block table may change
// under the same counts, a sliding window moves the first item) and loaded
// again if they differ.  Tokens past kv_len are masked from this call's kv_lens.
// Otherwise it computes the ranges itself and writes its own plan into the
// other slot; the workgroup counted last on header[15] then publishes it (every
// workgroup of the call has read the old header by then, so none of them reads a
// slot while it is written).  Zero-filled: no plan (generation 0).
constexpr int kPlanMaxWG = 1024;  // workgroup entries per slot
constexpr int kPlanSlotInts = kMaxSeqs + 16 * kPlanMaxWG;
constexpr int kPlanInts = 16 + 2 * kPlanSlotInts;
__host__ __device__ constexpr int q4_plan_kvl(const int slot) { return 16 + slot * kPlanSlotInts; }
__host__ __device__ constexpr int q4_plan_entry(const int slot, const int w) {
  return q4_plan_kvl(slot) + kMaxSeqs + 16 * w;
}

constexpr int kTableCache = 4096;  // block-table entries a workgroup keeps in LDS
constexpr int kSnapItems = 2;     // unit length (items) up to which ranges end on unit starts ...
constexpr int kSnapRange = 4;     // ... when the ranges average at most this many items

// The kernel body as workgroup `bid` of `nblocks` (a grid of its own, or the
// decode part of a mixed batch's single launch, unified_q4).
template <int GS, int HG, int PS = 0>
__device__ __forceinline__ void decode_q4_body(const DecodeArgs& a, const int bid, const int nblocks, int* const plan,
                                               const int32_t* const kv_lens, const int32_t* const block_tables,
                                               const int S, const int max_blocks) {
  using Geo = Q4Geom<HG>;
  constexpr int HQ = Geo::HQ, NSL = Geo::NSL, TW = Geo::TW;
  constexpr int D = 128, G = Q4Cfg<GS, 1>::G;
  // pages of a 64-token slice: one (big pages, a multiple of 128 tokens) or 64 / PS
  static_assert(PS == 0 || PS == 16 || PS == 32 || PS == 64, "small pages of 16, 32 or 64 tokens");
  constexpr int NSUB = PS ? 64 / PS : 1;

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int quad = wv % HQ, slice = wv / HQ;
  const int hl = 4 * quad + (lane & 3);  // head of this lane's query operand and scores

  // LDS, carved from the shared arena
  constexpr int oCum = 0, oKvl = lds_next(oCum, 4 * (kMaxSeqs + 1)), oQrw = lds_next(oKvl, 4 * kMaxSeqs);
  constexpr int oSo = lds_next(oQrw, 4 * kMaxSeqs), oSml = lds_next(oSo, 4 * 2 * 4 * 4 * D);
  constexpr int oSlast = lds_next(oSml, 4 * 2 * 4 * 4 * 2), oSbt = lds_next(oSlast, 4 * 2);
  constexpr int oSst = lds_next(oSbt, 4 * kTableCache), oXb = lds_next(oSst, 8 * 4 * 16 * 4 * G);
  constexpr int oEnd = lds_next(oXb, 64);
  static_assert(oEnd <= kArenaBytes, "LDS arena too small");
  int(&cum)[kMaxSeqs + 1] = lds_at<int[kMaxSeqs + 1]>(oCum);
  int(&kvl)[kMaxSeqs] = lds_at<int[kMaxSeqs]>(oKvl);
  int(&qrw)[kMaxSeqs] = lds_at<int[kMaxSeqs]>(oQrw);
  float(&so)[2][4][4][D] = lds_at<float[2][4][4][D]>(oSo);  // two slot sets; per wave: o * 2^24 + bias term of its 4 heads
  float(&sml)[2][4][4][2] = lds_at<float[2][4][4][2]>(oSml);  // per wave: (m, l) of its 4 heads
  int(&slast)[2] = lds_at<int[2]>(oSlast);
  // Block tables of up to kTableCache entries are read into LDS together with
  // kv_lens (one memory round trip for both), larger ones from global memory.
  int(&sbt)[kTableCache] = lds_at<int[kTableCache]>(oSbt);
  const int Hkv = a.Hkv;
  // LDS table entries read at a wave-uniform index are moved to SGPRs (uru), so the
  // per-item scheduling arithmetic stays scalar
  auto uru = [](int v) { return __builtin_amdgcn_readfirstlane(v); };
  const int nbt = S * max_blocks;
  const bool bt_lds = nbt <= kTableCache;

  // ---- query operand of a unit (this wave's head quad).  Lane L (head 4*quad + L%4,
  // 16-lane group n = L/16) holds, in VGPR pair r, the operand of k-step 4r + n: K word
  // m = 2r + n/2, dims 8m + (n even ? {0,4,1,5} : {2,6,3,7}), the last two / 16.
  const int n16 = lane >> 4;
  const int qhalf = n16 & 1;
  uint32_t qraw[8][2];
  auto issue_q = [&](int row, int kh) {
    const uint32_t* qp = reinterpret_cast<const uint32_t*>(
        a.q + ((size_t)row * a.Hq + (size_t)kh * HG + (hl < HG ? hl : 0)) * D);
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int m = 2 * r + (n16 >> 1);
      qraw[r][0] = qp[4 * m + qhalf];      // dims 8m + 2*qhalf + {0, 1}
      qraw[r][1] = qp[4 * m + qhalf + 2];  // dims 8m + 2*qhalf + {4, 5}
    }
  };
  h16x4 qB[1][8];
  float qs[1][2];
  auto build_q = [&]() {
    const bool ok = hl < HG;
    float gsum[2] = {0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int m = 2 * r + (n16 >> 1);
      const h16 d0 = __builtin_bit_cast(h16, (uint16_t)(qraw[r][0] & 0xFFFFu));
      const h16 d1 = __builtin_bit_cast(h16, (uint16_t)(qraw[r][0] >> 16));
      const h16 d4 = __builtin_bit_cast(h16, (uint16_t)(qraw[r][1] & 0xFFFFu));
      const h16 d5 = __builtin_bit_cast(h16, (uint16_t)(qraw[r][1] >> 16));
      // element order (nibble 0,4 | 1,5) of the word pair; with qhalf the dims are offset by 2
      const h16x4 v = {d0, d4, (h16)((float)d1 * 0.0625f), (h16)((float)d5 * 0.0625f)};
      qB[0][r] = ok ? v : h16x4{(h16)0.f, (h16)0.f, (h16)0.f, (h16)0.f};
      const float sum = ok ? ((float)d0 + (float)d1) + ((float)d4 + (float)d5) : 0.f;
      if (G == 1 || (8 * m) / GS == 0)
        gsum[0] += sum;
      else
        gsum[1] += sum;
    }
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      float x = gsum[g];
      x += __shfl_xor(x, 16, 64);
      x += __shfl_xor(x, 32, 64);
      qs[0][g] = x * (1.0f / kTwo24);  // bias term in the 2^-24 units of the MFMA output
    }
  };


  // descriptors of this wave's slice at token t of page b (zero-size, reading nothing, when b is
  // invalid), and the element offset of the page-head's scales (page 0 when b is invalid)
  auto tile_of = [&](int b, int kh, int t, size_t& soff) {
    const bool ok = (unsigned)b < (unsigned)a.nb;
    const int off = t & (a.bs - 1) & ~127;  // page sizes are powers of two here
    const size_t ph = (size_t)(ok ? b : 0) * a.Hkv + kh;
    const int RW = a.bs * 4 / 32;
    TileRsrc r;
    r.k = uniform_rsrc(a.kc + (ph * a.bs + off) * 16, ok ? 128 * 16 * 4 : 0);
    r.v = uniform_rsrc(a.vc + ph * D * RW + (off / 64) * D * 8, ok ? (D * RW - (off / 64) * D * 8) * 4 : 0);
    soff = ph * G * a.bs + off;
    return r;
  };
  // LDS reads are per lane to the compiler: 64-bit values go back to scalar registers
  auto uru64 = [](long long v) {
    return (long long)(((unsigned long long)(unsigned)__builtin_amdgcn_readfirstlane((int)(v >> 32)) << 32) |
                       (unsigned)__builtin_amdgcn_readfirstlane((int)v));
  };

  // ---- the plan cache (Q4Plan): lanes 0-15 load this workgroup's entry in slot 0, lanes
  // 16-31 its entry in slot 1, lanes 32-47 the header -- in the memory round trip that
  // also brings kv_lens and the block tables.
  int pl = 0;
  if (plan) pl = plan[lane < 32 ? q4_plan_entry(lane >> 4, bid) + (lane & 15) : (lane & 15)];
  // Block tables of up to kTableCache entries are read into LDS together with
  // kv_lens (one memory round trip for both), larger ones from global memory.
  int btv[kTableCache / 256];
  if (bt_lds) {
#pragma unroll
    for (int k = 0; k < kTableCache / 256; ++k) {
      const int i = threadIdx.x + 256 * k;
      btv[k] = i < nbt ? block_tables[i] : -1;
    }
  }
  // per-sequence loads (sequences ch*t .. ch*t+ch-1 of thread t): kv_len, the mixed
  // batch's query row, and the plan's copies of the item counts
  constexpr int kSeqPT = kMaxSeqs / 256;
  const int ch = (S + 255) / 256;
  const int sq0 = threadIdx.x * ch;
  // (A load whose destination another path writes with a plain move makes the
  // compiler wait for every load in flight there, so the optional query_start_loc is
  // loaded into registers of its own and selected afterwards.)
  int klr[kSeqPT], qlo[kSeqPT] = {}, qhi[kSeqPT] = {}, kc[2][kSeqPT] = {};
  const bool mixed = a.qsl != nullptr;
#pragma unroll
  for (int i = 0; i < kSeqPT; ++i) {
    const int si = sq0 + i;
    if (i < ch && si < S) {
      klr[i] = kv_lens[si];
      if (mixed) {
        qlo[i] = a.qsl[si];
        qhi[i] = a.qsl[si + 1];
      }
      if (plan) {
        kc[0][i] = plan[q4_plan_kvl(0) + si];
        kc[1][i] = plan[q4_plan_kvl(1) + si];
      }
    }
  }

  // ---- header and entry: when a plan is committed for this shape, the first item's
  // query and pages go out now, before the tables are scanned (checked below)
  Q4Loads<GS, 1> bufA, bufB;
  const Q4ScalePtrs<GS> sptr = q4_scale_ptrs<GS>(a, lane);
  const int pgen = plan ? uru(__builtin_amdgcn_readlane(pl, 32)) : 0;
  const int kind = GS | (HG << 8) | (__builtin_ctz(a.bs) << 16);
  const int kv_cap = max_blocks * a.bs;
  const bool hdr_ok = pgen > 0 && __builtin_amdgcn_readlane(pl, 33) == S && __builtin_amdgcn_readlane(pl, 34) == Hkv &&
                      __builtin_amdgcn_readlane(pl, 36) == a.window &&
                      __builtin_amdgcn_readlane(pl, 37) == a.first_slot && __builtin_amdgcn_readlane(pl, 38) == kind &&
                      __builtin_amdgcn_readlane(pl, 39) == kv_cap;
  const int pslot = pgen & 1;  // the committed slot
  auto pe = [&](const int k) { return uru(__builtin_amdgcn_readlane(pl, 16 * pslot + k)); };
  const int spec_s = pe(4), spec_kvh = pe(5), spec_tb = pe(6) + 64 * slice, spec_blk = pe(8 + slice);
  // Only entries below the header's NWG belong to the committed plan (the others are
  // left from older plans); the sequence and kv head are bounds-checked as well, so the
  // loads stay inside q and the pools whatever the entry holds (pages: tile_of).
  const bool spec = PS == 0 && hdr_ok && bid < __builtin_amdgcn_readlane(pl, 35) && pe(0) < pe(1) &&
                    (unsigned)spec_s < (unsigned)S && (unsigned)spec_kvh < (unsigned)Hkv && spec_tb >= 0;
  if (spec) {
    issue_q(spec_s, spec_kvh);  // a plan exists only for pure decode calls: row = sequence
    size_t so;
    const TileRsrc rs = tile_of(spec_blk, spec_kvh, spec_tb, so);
    q4_issue_loads(bufA, rs, sptr, so, (spec_tb & 127) / 64, lane, a.bs);
  }

  // ---- block-wide exclusive prefix of the live item counts (cum[s]), clamped
  // kv_lens (kvl[s], -1 for rows a mixed batch runs elsewhere), query rows (qrw[s]),
  // and whether the item counts differ from the committed plan's copy
  int tsum = 0, mis = 0;
#pragma unroll
  for (int i = 0; i < kSeqPT; ++i) {
    const int si = sq0 + i;
    if (i < ch && si < S) {
      const int kl = max(min(klr[i], kv_cap), 0);
      const bool dec = !mixed || qhi[i] - qlo[i] == 1;  // in a mixed batch only single-token rows decode here
      qrw[si] = mixed ? qlo[i] : si;
      kvl[si] = dec ? kl : -1;
      int n = 0;
      if (dec && kl > 0) {
        const int sk = a.window > 0 ? max(0, kl - a.window) : 0;
        n = (kl - 1) / TW - sk / TW + 1;
      }
      cum[si] = n;  // temporarily the count
      tsum += n;
      mis |= plan && kc[pslot][i] != n;
    }
  }
  {
    int x = tsum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    int(&wsum)[8] = lds_at<int[8]>(oXb + 32);
    const bool wmis = __ballot(mis) != 0ull;  // every lane votes (not under the lane test below)
    if (lane == 63) wsum[wv] = x;
    if (lane == 0) wsum[4 + wv] = wmis;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wv; ++w) base += wsum[w];
    mis = wsum[4] | wsum[5] | wsum[6] | wsum[7];
    int run = base + x - tsum;
#pragma unroll
    for (int i = 0; i < kSeqPT; ++i) {
      const int si = sq0 + i;
      if (i < ch && si < S) {
        const int n = cum[si];
        cum[si] = run;
        run += n;
      }
    }
    if (threadIdx.x == 255) cum[S] = base + x;
    if (bt_lds) {
#pragma unroll
      for (int k = 0; k < kTableCache / 256; ++k) sbt[threadIdx.x + 256 * k] = btv[k];
    }
    __syncthreads();
  }
  if (wv >= 2) {  // decoded sequences without a live token produce zeros (the reference's l == 0 case);
                  // waves 2-3, while waves 0-1 find the workgroup's range (below)
    const int per_seq = a.Hq * D / 8;
    for (int i = bid * 128 + threadIdx.x - 128; i < S * per_seq; i += nblocks * 128) {
      const int si = i / per_seq;
      if (kvl[si] >= 0 && cum[si + 1] == cum[si])
        reinterpret_cast<u32x4*>(a.out)[(size_t)qrw[si] * per_seq + i % per_seq] = u32x4{0u, 0u, 0u, 0u};
    }
  }

  const long long I = (long long)Hkv * uru(cum[S]);
  const int NWG = (int)min((long long)nblocks, I);  // every range non-empty (before snapping, below)
  const int wg = bid;
  if (wg >= NWG) return;
  // The committed plan holds when its shape and its copy of the item counts match this call's.
  const bool pvalid = hdr_ok && __builtin_amdgcn_readlane(pl, 35) == NWG && uru(mis) == 0;
  const bool pwrite = plan && !pvalid;  // otherwise this call commits its own plan (slot pgen + 1)
  const int wslot = (pgen + 1) & 1;
  long long g0, g1;
  int pk_first, pk_last;  // pieces (wf | np << 16, both below kMaxWaves) of the units the range
                          // shares: its first (begun before g0) and its last (going on past g1)
  if (pvalid) {
    g0 = pe(0);
    g1 = pe(1);
    pk_first = pe(2);
    pk_last = pe(3);
  } else {
    long long(&xb)[2] = lds_at<long long[2]>(oXb);
  int(&xpk)[2] = lds_at<int[2]>(oXb + 16);
  if (wv < 2) {
    int ne_tot = 0;  // sequences with items
    for (int c = 0; c < S; c += 64) {
      const int si = c + lane;
      ne_tot += __builtin_popcountll(__ballot(si < S && cum[si + 1] > cum[si]));
    }
    ne_tot = uru(ne_tot);
    const long long Ctot = (long long)kCostItem * I + (long long)kCostUnit * Hkv * ne_tot;
    const int N1 = a.first_slot > 0 ? min(a.first_slot, NWG) : NWG;
    int Le = 0;
    if (N1 < NWG) {  // Q >= NWG * kCostItem keeps ranges inside a unit non-empty
      Le = min(kCostLag, max(0, (int)((float)Ctot / (float)NWG) - kCostItem));
      while (Le > 0 && Ctot - (long long)Le * N1 < (long long)NWG * kCostItem) --Le;
    }
    const Q4Balance bl{Ctot + (long long)Le * (NWG - N1), Ctot - (long long)Le * N1, NWG, N1};
    // b = min{x in [0, I] : NWG * C(x) >= T}: the last sequence with items whose start
    // lies below T (ballot over 64 sequences at a time), its last unit below T, then
    // the item inside that unit.  A boundary inside a unit also yields that unit's
    // pieces, pk = wf | np << 16 (the workgroups holding its first and last item).
    const int w = wg + wv;
    long long b = w == 0 ? 0 : I;
    int pk = 1 << 16;
    if (w > 0 && w < NWG) {
      const long long T = bl.target(w);
      int sb = -1, sne = 0, ne_run = 0;
      for (int c = 0; c < S; c += 64) {
        const int si = c + lane;
        const int n = si < S ? cum[si + 1] - cum[si] : 0;
        const unsigned long long live = __ballot(n > 0);
        const int ne = ne_run + __builtin_popcountll(live & ((1ull << lane) - 1ull));
        const long long Cs =
            (long long)kCostItem * Hkv * (si < S ? cum[si] : 0) + (long long)kCostUnit * ((long long)Hkv * ne + 1);
        const bool below = n > 0 && (long long)NWG * Cs < T;
        const unsigned long long pb = __ballot(below);
        if (pb) {
          const int Lb = 63 - __builtin_clzll(pb);
          sb = c + Lb;
          sne = __builtin_amdgcn_readlane(ne, Lb);
        }
        ne_run += __builtin_popcountll(live);
        if (__ballot(n > 0 && !below)) break;
      }
      b = 0;
      if (sb >= 0) {
        sb = uru(sb);
        sne = uru(sne);
        const int n = uru(cum[sb + 1]) - uru(cum[sb]);
        const long long st0 = (long long)Hkv * uru(cum[sb]);
        const long long C0 = (long long)kCostItem * st0 + (long long)kCostUnit * ((long long)Hkv * sne + 1);
        const long long slope = (long long)kCostItem * n + kCostUnit;  // C between consecutive unit starts
        // lane-parallel from here (a wave's serial scalar chain runs at a few hundred
        // instructions per microsecond, and this is on every workgroup's critical path):
        // the unit h = last with NWG * C(start of h) < T, one lane per unit ...
        int h = 0;
        for (int c = 0; c < Hkv; c += 64) {
          const int hh = c + lane;
          const unsigned long long pb = __ballot(hh < Hkv && (long long)NWG * (C0 + (long long)hh * slope) < T);
          if (pb) h = c + 63 - __builtin_clzll(pb);
          if (!(pb >> 63)) break;
        }
        h = uru(h);
        const long long Cu = C0 + (long long)h * slope;
        // ... then jj = 1 + #{j in [1, n) : NWG * (Cu + kCostItem * j) < T}, one lane per j
        // (jj = n: the next unit start, whose step of C reaches T)
        int jj = 1;
        for (int c = 1; c < n; c += 64) {
          const int j = c + lane;
          const unsigned long long pb = __ballot(j < n && (long long)NWG * (Cu + (long long)kCostItem * j) < T);
          jj += __builtin_popcountll(pb);
          if (!(pb >> 63)) break;
        }
        jj = uru(jj);
        b = st0 + (long long)h * n + jj;
        if (jj < n) {  // the range boundary cuts the unit: its pieces
          const int wf = wg_of_lanes(bl, (long long)NWG * Cu, lane);
          const int np = wg_of_lanes(bl, (long long)NWG * (Cu + (long long)kCostItem * (n - 1)), lane) - wf + 1;
          pk = wf | (np << 16);
        }
      }
    }
    if (lane == 0) {
      xb[wv] = b;
      xpk[wv] = pk;
    }
  }
  __syncthreads();
    g0 = uru64(xb[0]);
    g1 = uru64(xb[1]);
    pk_first = uru(xpk[0]);
    pk_last = uru(xpk[1]);
  int max_items = kSnapItems + 1;
  if (I <= (long long)kSnapRange * NWG) {  // longest unit, by every wave for itself (no barrier)
    max_items = 0;
    for (int si = lane; si < S; si += 64) max_items = max(max_items, cum[si + 1] - cum[si]);
    for (int o = 1; o < 64; o <<= 1) max_items = max(max_items, __shfl_xor(max_items, o, 64));
  }
  if (uru(max_items) <= kSnapItems) {
    auto unit_start = [&](long long x) -> long long {  // first unit start >= x
      if (x >= I) return I;
      int lo = 0, hi = S - 1;  // the sequence holding item x
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if ((long long)Hkv * cum[mid + 1] > x)
          hi = mid;
        else
          lo = mid + 1;
      }
      const long long base = (long long)Hkv * cum[lo];
      const int n = cum[lo + 1] - cum[lo];
      return base + (long long)((((int)(x - base)) + n - 1) / n) * n;
    };
    g0 = uru64(wg == 0 ? 0 : unit_start(g0));
    g1 = uru64(wg + 1 == NWG ? I : unit_start(g1));
  }
  }
  if (pwrite && wv == 0 && lane == 0) {  // this workgroup's range into the plan being written
    int* e = plan + q4_plan_entry(wslot, wg);
    e[0] = (int)g0;
    e[1] = (int)g1;
    e[2] = pk_first;
    e[3] = pk_last;
  }
  if (pwrite && wg == 0) {  // the item counts of this call
#pragma unroll
    for (int i = 0; i < kSeqPT; ++i) {
      const int si = sq0 + i;
      if (i < ch && si < S) plan[q4_plan_kvl(wslot) + si] = cum[si + 1] - cum[si];
    }
  }
  if (g0 < g1) {
  const int bs_log2 = __builtin_ctz(a.bs);

  // ---- item g -> (sequence, kv_head, item j of the unit)
  auto seq_of = [&](long long g, int s_from) {  // first s >= s_from with Hkv*cum[s+1] > g
    int si = s_from;
    while (si + 1 < S && (long long)Hkv * cum[si + 1] <= g) ++si;
    return si;
  };
  auto lo_of = [&](int si) { return (a.window > 0 ? max(0, kvl[si] - a.window) : 0) / TW; };
  int s = 0;
  for (int c = 0; c < S; c += 64) {
    const int si = c + lane;
    s += __builtin_popcountll(__ballot(si < S && (long long)Hkv * cum[si + 1] <= g0));
  }
  s = __builtin_amdgcn_readfirstlane(s);

  // ---- page of this wave's slice for every item of the range, one item per lane
  // (64 items per chunk); -1 where the slice holds no token below kv_len
  // (small pages: the NSUB pages of the slice; -1 past kv_len or past the table row)
  auto blk_chunk = [&](long long gb, int (&b)[NSUB]) {
    const long long g = gb + lane;
#pragma unroll
    for (int q = 0; q < NSUB; ++q) b[q] = -1;
    if (g < g1) {
      const int si = seq_of(g, s);
      const int n = cum[si + 1] - cum[si];
      const int jn = (int)(g - (long long)Hkv * cum[si]) % n;
      const int t = (lo_of(si) + jn) * TW + 64 * slice;
#pragma unroll
      for (int q = 0; q < NSUB; ++q) {
        const int tq = t + q * (PS ? PS : 0);
        if (tq < kvl[si] && (tq >> bs_log2) < max_blocks) {
          const size_t bi = (size_t)si * max_blocks + (tq >> bs_log2);
          b[q] = bt_lds ? sbt[bi] : block_tables[bi];
        }
      }
    }
  };
  int blkv[NSUB];
  blk_chunk(g0, blkv);

  int n_s = uru(cum[s + 1]) - uru(cum[s]);
  int kvh, j;
  {
    const int r = (int)(g0 - (long long)Hkv * uru(cum[s]));
    kvh = r / n_s;
    j = r % n_s;
  }
  int kv_len = uru(kvl[s]);
  int start_k = a.window > 0 ? max(0, kv_len - a.window) : 0;
  int it_lo = start_k / TW;
  const float sc_l2 = a.scale_log2 * kTwo24;
  u32x2(&sst)[4][16 * 4 * G] = lds_at<u32x2[4][16 * 4 * G]>(oSst);  // per wave: scale staging [16 quads][4 * G segments]

  // ---- first item's query and pages: already in flight when the plan held and its
  // pages are this call's (the block tables may have changed under the same item counts)
  int tb = (it_lo + j) * TW + 64 * slice;
  int blk[NSUB];
#pragma unroll
  for (int q = 0; q < NSUB; ++q) blk[q] = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(blkv[q], 0));
  if (pwrite && lane == 0) {
    int* e = plan + q4_plan_entry(wslot, wg);
    if (wv == 0) {
      e[4] = s;
      e[5] = kvh;
      e[6] = (it_lo + j) * TW;
    }
    if (wv % HQ == 0) e[8 + slice] = blk[0];
  }
  // this wave's slice of one item: loads of pages blk_ at token base t_
  auto issue_item = [&](Q4Loads<GS, 1>& buf, const int (&blk_)[NSUB], const int kh, const int t_) {
    if constexpr (PS == 0) {
      size_t so;
      const TileRsrc rs = tile_of(blk_[0], kh, t_, so);
      q4_issue_loads(buf, rs, sptr, so, (t_ & 127) / 64, lane, a.bs);
    } else {
      q4_issue_loads_small<GS, PS>(buf, a, blk_, kh, lane);
    }
  };
  if (!(spec && pvalid && s == spec_s && kvh == spec_kvh && tb == spec_tb && blk[0] == spec_blk)) {
    issue_q(uru(qrw[s]), kvh);  // the query first: loads return in order
    issue_item(bufA, blk, kvh, tb);
  }
  build_q();

  Q4State st[1];
  auto reset = [&]() {
    st[0].o[0] = f32x4{0.f, 0.f, 0.f, 0.f};
    st[0].o[1] = f32x4{0.f, 0.f, 0.f, 0.f};
    st[0].m = -INFINITY;
    st[0].l = 0.f;
    st[0].pb[0] = 0.f;
    st[0].pb[1] = 0.f;
  };
  reset();
  long long unit_first = (long long)Hkv * cum[s] + (long long)kvh * n_s;  // first item of the current unit

  // shared units awaiting their arrival (at most the range's first and last unit)
  int npend = 0;
  int nue = 0;  // unit ends passed (uniform across the workgroup)
  int pend_u[2], pend_row[2], pend_kvh[2], pend_wf[2], pend_np[2];
  auto pieces = [&](const int u, const int wf, const int np) {
    PieceInfo pi;
    pi.np = __builtin_amdgcn_readfirstlane(np);
    pi.slot0 = __builtin_amdgcn_readfirstlane(wf + u);  // the pieces of unit u sit in slots wf+u .. wl+u
    pi.me = __builtin_amdgcn_readfirstlane(wg - wf);
    pi.ro = uniform_rsrc(a.ws_o + (size_t)pi.slot0 * (HG * D), pi.np * HG * D * 4);
    pi.rm = uniform_rsrc(a.ws_ml + (size_t)pi.slot0 * (HG * 2), pi.np * HG * 2 * 4);
    return pi;
  };

  auto step = [&](Q4Loads<GS, 1>& cur, Q4Loads<GS, 1>& nxt, const long long g) {
    // ---- next item (the state is wave-uniform: scalar registers and branches)
    s = uru(s);
    kvh = uru(kvh);
    j = uru(j);
    n_s = uru(n_s);
    kv_len = uru(kv_len);
    it_lo = uru(it_lo);
    int s1 = s, kvh1 = kvh, j1 = j + 1, n1 = n_s, kl1 = kv_len, lo1 = it_lo;
    if (j1 == n_s) {
      j1 = 0;
      if (++kvh1 == Hkv) {
        kvh1 = 0;
        do {
          ++s1;
        } while (s1 < S && uru(cum[s1 + 1]) == uru(cum[s1]));
        if (s1 < S) {
          n1 = uru(cum[s1 + 1]) - uru(cum[s1]);
          kl1 = uru(kvl[s1]);
          lo1 = (a.window > 0 ? max(0, kl1 - a.window) : 0) / TW;
        }
      }
    }
    const bool has_next = g + 1 < g1;
    const bool unit_end = !has_next || s1 != s || kvh1 != kvh;
    int blk1[NSUB];
#pragma unroll
    for (int q = 0; q < NSUB; ++q) blk1[q] = -1;
    const int tb1 = (lo1 + j1) * TW + 64 * slice;
    if (has_next) {
      const int k1 = (int)(g + 1 - g0);
      if ((k1 & 63) == 0) blk_chunk(g + 1, blkv);
#pragma unroll
      for (int q = 0; q < NSUB; ++q)
        blk1[q] = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(blkv[q], k1 & 63));
    }
    // The next unit's query first: loads return in order, so building its
    // operand at this unit's end does not wait for the next item's pages.
    if (has_next && unit_end) issue_q(uru(qrw[s1]), kvh1);
    // Issued on every path (an empty descriptor returns zeros without touching
    // memory), so the wait before this item's compute leaves them in flight.
    issue_item(nxt, blk1, kvh1, tb1);

    // ---- compute this wave's slice of the item.  A slice without a live token or
    // with an invalid page (skipped by the reference's Metal kernel) is computed
    // with every token dead, so it adds nothing: a branch around it left the
    // compiler unable to order this item's loads against the next item's, and
    // it waited for all of them before issuing the next page loads.
    {
      int sub_ok = 0;
#pragma unroll
      for (int q = 0; q < NSUB; ++q) sub_ok |= ((unsigned)blk[q] < (unsigned)a.nb) << q;
      const bool ok = sub_ok != 0;
      q4_stage_scales<GS, 1>(cur, sst[wv], lane);
      const bool full = sub_ok == (1 << NSUB) - 1 && tb >= start_k && tb + 64 <= kv_len;
      q4_compute<GS, 1, PS>(cur, full, lane, tb, start_k, ok ? kv_len : 0, qB, qs, sc_l2, st, sub_ok);
    }

    // ---- unit finished (or range ends): the waves' (o, m, l) meet in LDS and, after one
    // workgroup barrier, all four combine them into the output or the workgroup's
    // partial.  Unit ends alternate between two slot sets: a set is written again two
    // unit ends later, after every wave has passed the barrier of the unit end between,
    // so its reads are done.  (Measured against a last-arriver protocol with an arrival
    // counter: c2 28.4 -> 27.4 us, batch 128 81.2 -> 78.1 us.)
    if (unit_end) {
      const bool whole = unit_first >= g0 && unit_first + n_s <= g1;
      const int u = s * Hkv + kvh;
      const int par = nue & 1;
      const int row = uru(qrw[s]);
      {
        const float l = head_sum(st[0].l);
        float pbs[2];
#pragma unroll
        for (int g = 0; g < G; ++g) pbs[g] = head_sum(st[0].pb[g]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // lane i holds head i's sums
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const float pbi =
                __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pbs[(64 * c) / GS]), i));
            so[par][wv][i][64 * c + lane] = st[0].o[c][i] * kTwo24 + pbi;
          }
        }
        if (lane < 4) {
          sml[par][wv][lane][0] = st[0].m;
          sml[par][wv][lane][1] = l;
        }
      }
      int wf = 0, np = 1;
      {
        // every wave has its (o, m, l) of the unit in LDS: all four combine it together
        __syncthreads();
        PieceInfo pi;
        if (!whole) {  // the range's first unit (begun before g0) or its last (going on past g1)
          const int pk = unit_first < g0 ? pk_first : pk_last;
          wf = pk & 0xFFFF;
          np = pk >> 16;
          pi = pieces(u, wf, np);
        }
        // Two adjacent dims per thread, so a thread issues one 4-byte output store
        // (or one 8-byte partial store): the stores wait for room in the memory
        // queue the page loads keep full, and one element per store made this
        // combine ~0.9 us per unit end.  A fixed number of store instructions lets
        // the compiler still count the loads in flight past them.
#pragma unroll
        for (int k = 0; k < (HG * D / 2 + 255) / 256; ++k) {
          const int e = 2 * (threadIdx.x + 256 * k);
          if (HG * D % 512 != 0 && e >= HG * D) break;
          const int h = e / D, d = e % D, q = h / 4, i = h % 4;
          float M = -INFINITY;
#pragma unroll
          for (int sl = 0; sl < NSL; ++sl) M = fmaxf(M, sml[par][q + HQ * sl][i][0]);
          f32x2 O = {0.f, 0.f};
          float L = 0.f;
#pragma unroll
          for (int sl = 0; sl < NSL; ++sl) {
            const float m = sml[par][q + HQ * sl][i][0];
            const float f = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
            const f32x2 x = *reinterpret_cast<const f32x2*>(&so[par][q + HQ * sl][i][d]);
            O[0] = fmaf(f, x[0], O[0]);
            O[1] = fmaf(f, x[1], O[1]);
            L = fmaf(f, sml[par][q + HQ * sl][i][1], L);
          }
          if (whole) {
            const h16 r0 = (h16)(L > 0.f ? O[0] / L : 0.f), r1 = (h16)(L > 0.f ? O[1] / L : 0.f);
            *reinterpret_cast<uint32_t*>(a.out + ((size_t)row * a.Hq + (size_t)kvh * HG + h) * D + d) =
                (uint32_t)__builtin_bit_cast(uint16_t, r0) | ((uint32_t)__builtin_bit_cast(uint16_t, r1) << 16);
          } else {
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, O), pi.ro, (h * D + d) * 4,
                                                  pi.me * HG * D * 4, kCoherent);
            if (d == 0)
              __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f32x2{M, L}), pi.rm, h * 8,
                                                    pi.me * HG * 8, kCoherent);
          }
        }
      }
      ++nue;
      if (!whole) {
        pend_u[npend] = u;
        pend_row[npend] = row;
        pend_kvh[npend] = kvh;
        pend_wf[npend] = wf;
        pend_np[npend] = np;
        ++npend;
      }
      reset();
      if (has_next) {
        unit_first = g + 1;
        build_q();
      }
    }

    // ---- advance
    if (s1 != s) {
      kv_len = kl1;
      start_k = a.window > 0 ? max(0, kv_len - a.window) : 0;
    }
    s = s1;
    kvh = kvh1;
    j = j1;
    n_s = n1;
    it_lo = lo1;
    tb = tb1;
#pragma unroll
    for (int q = 0; q < NSUB; ++q) blk[q] = blk1[q];
  };
  for (long long g = g0; g < g1; g += 2) {
    step(bufA, bufB, g);
    if (g + 1 >= g1) break;
    step(bufB, bufA, g + 1);
  }

  // ---- arrivals of the shared units; the last workgroup to arrive merges
  if (npend > 0) {
    __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are complete ...
    __syncthreads();                // ... and so are the workgroup's
    if (threadIdx.x < npend) {  // one thread per shared unit: both arrivals in flight together
      const int p = threadIdx.x;
      const int np = pend_np[p];
      const int old = __hip_atomic_fetch_add(a.ws_cnt + pend_u[p], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = old == np - 1;
      if (last) __hip_atomic_store(a.ws_cnt + pend_u[p], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      slast[p] = last;
    }
    __syncthreads();
    // Merge (page_attention.py:2006-2059): with two units to merge, waves 0-1 take
    // the first and waves 2-3 the second, so both units' loads are in flight
    // together; a thread owns float4 f of the unit's HG*D values and loads only
    // the pieces that exist, up to eight at once.
    const bool mg0 = slast[0] != 0, mg1 = npend > 1 && slast[1] != 0;
    if (mg0 || mg1) {
      const int T = mg0 && mg1 ? 128 : 256;
      const int p = mg0 && mg1 ? (wv >> 1) : (mg0 ? 0 : 1);
      const int t = threadIdx.x & (T - 1);
      const PieceInfo pi = pieces(pend_u[p], pend_wf[p], pend_np[p]);
      h16* out = a.out + ((size_t)pend_row[p] * a.Hq + (size_t)pend_kvh[p] * HG) * D;
      constexpr int NF4 = HG * D / 4;
      for (int f = t; f < NF4; f += T) {
        const int h = 4 * f / D;
        float M = -INFINITY, L = 0.f;
        f32x4 O = {0.f, 0.f, 0.f, 0.f};
        for (int p0 = 0; p0 < pi.np; p0 += 8) {
          f32x4 o[8];
          f32x2 ml[8];
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            if (p0 + c < pi.np) {
              o[c] = __builtin_bit_cast(
                  f32x4, __builtin_amdgcn_raw_buffer_load_b128(pi.ro, f * 16, (p0 + c) * HG * D * 4, kCoherent));
              ml[c] = __builtin_bit_cast(
                  f32x2, __builtin_amdgcn_raw_buffer_load_b64(pi.rm, h * 8, (p0 + c) * HG * 8, kCoherent));
            }
          }
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            if (p0 + c >= pi.np || ml[c].x == -INFINITY) continue;  // a piece may hold no live token
            const float Mn = fmaxf(M, ml[c].x);
            const float fo = __builtin_amdgcn_exp2f(M - Mn);  // 0 while M is -inf
            const float fp = __builtin_amdgcn_exp2f(ml[c].x - Mn);
            O = O * fo + o[c] * fp;
            L = L * fo + ml[c].y * fp;
            M = Mn;
          }
        }
        const float inv = L > 0.f ? 1.f / L : 0.f;
        const h16x4 r = {(h16)(O[0] * inv), (h16)(O[1] * inv), (h16)(O[2] * inv), (h16)(O[3] * inv)};
        *reinterpret_cast<u32x2*>(out + 4 * f) = __builtin_bit_cast(u32x2, r);
      }
    }
  }
  }  // g0 < g1

  // ---- a call that wrote a plan commits it: the workgroup counted last (every
  // workgroup of the call has read the old header by then) publishes the header,
  // which the next call on this workspace reads
  if (pwrite && threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(plan + 15, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == NWG - 1) {
      plan[1] = S;
      plan[2] = Hkv;
      plan[3] = NWG;
      plan[4] = a.window;
      plan[5] = a.first_slot;
      plan[6] = kind;
      plan[7] = kv_cap;
      plan[0] = pgen + 1;
      __hip_atomic_store(plan + 15, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// The values the first loads need lead the argument list: the library is built with
// kernel-argument preloading, so they arrive in SGPRs with the wave instead of
// after a scalar load from the kernel-argument buffer.
template <int GS, int HG, int PS = 0>
__global__ __launch_bounds__(256, 2) void decode_q4_d128(int* plan, const int32_t* kv_lens,
                                                         const int32_t* block_tables, int S, int max_blocks,
                                                         DecodeArgs a) {
  decode_q4_body<GS, HG, PS>(a, blockIdx.x, gridDim.x, plan, kv_lens, block_tables, S, max_blocks);
}

}  // namespace emx
