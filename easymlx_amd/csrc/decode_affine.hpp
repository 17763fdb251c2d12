// Single-token paged decode over affine-quantized pages, head_dim 128, MFMA.
//
// Replaces the reference's per-(seq, q_head) serial key loop
// (lib/python/easymlx/operations/kernels/unified_attention.py:467-609) and its
// split-K variant (page_attention.py:1718-2059) for affine int4/int8 pages.
//
// Work decomposition (persistent, one resident round of waves)
//   A work item is one NT-token iteration (64 tokens at 4-bit, 32 at 8-bit) of
//   one unit = (sequence, kv_head); items are ordered unit-major, and the live
//   items of every unit are counted on the device from kv_lens.  Wave w of NW
//   takes the contiguous item range [w*I/NW, (w+1)*I/NW) and streams it with a
//   two-stage pipeline (the loads of item i+1 are in flight while item i
//   computes).  All Hq/Hkv query heads of the GQA group are served from one
//   read of each K/V byte.  A unit that lies inside one wave's range is written
//   straight to the output.  A unit cut by range boundaries leaves one fp32
//   partial per wave (slot wave + unit, unique because ranges are monotone),
//   written with device-coherent (SC1) vector stores; once they are complete
//   the wave bumps the unit's arrival counter, and the wave that arrives last
//   reads the partials back with SC1 loads, merges them (page_attention.py:
//   2006-2059) and resets the counter.  One launch, and no cache write-back or
//   invalidate fences: only the partials travel device-coherently.
//
// Per iteration (lane l: col = l%16, jj = l/16)
//   QK^T : NT/16 token sub-tiles x 4 k-slices of v_mfma_f32_16x16x32_f16.
//          A = K codes as exact fp16 subnormals (code * 2^-24); row rho of
//          sub-tile a is token TPL*(rho/4) + 4a + rho%4.  B = query columns:
//          column h + (16/G)*g holds query head h restricted to quantization
//          group g (zeros elsewhere), so one MFMA yields per-group partial dots
//          and the affine scale / bias are applied per (token, group):
//            s = 2^24 * sum_g scale[t,g] * C[t,(h,g)] + bias[t,g] * sum_{d in g} q_hd
//          The group sum is a DPP row rotation.
//   softmax: online, base 2, fp32.
//   PV   : 8 dim sub-tiles x NT/32 token k-slices.  A = V codes (V tiles are
//          dim-major, so a lane's uint32 holds consecutive tokens of one dim),
//          B = p * v_scale[t, g] in fp16; sum_t p_t * v_bias[t, g] is kept in fp32.
//   Scales and biases of the iteration are staged through a per-wave LDS slot.
#pragma once

#include "common.hpp"

namespace emx {

struct DecodeArgs {
  const h16* q;               // [S, Hq, 128]
  const uint32_t* kc;         // [nb, Hkv, bs, 128*BITS/32]
  const h16* ks;              // [nb, Hkv, G, bs]
  const h16* kb;              // [nb, Hkv, G, bs]
  const uint32_t* vc;         // [nb, Hkv, bs/NT, 128, 8] (NT-token tiles, dim-major, 32 B per dim)
  const h16* vs;              // [nb, Hkv, G, bs]
  const h16* vb;              // [nb, Hkv, G, bs]
  const int32_t* block_tables;  // [S, max_blocks]
  const int32_t* kv_lens;       // [S]
  const int32_t* qsl;           // [S + 1] query rows of a mixed batch, or null: row s is sequence s
  h16* out;                   // [rows, Hq, 128]
  int* ws_cnt;                // [kMaxUnits] per-unit arrival counters: zero before and after every launch
  int* ws_cnt_grp;            // [kMaxUnits + kMaxWaves] per-group arrival counters (indexed by slot), likewise
  float* ws_o;                // [num_waves + S*Hkv, HG, 128] partial accumulators, slot = wave + unit
  float* ws_ml;               // [num_waves + S*Hkv, HG, 2]   partial (max, sum)
  int S, Hq, Hkv, bs, nb, max_blocks;
  float scale_log2;           // softmax_scale * log2(e)
  int window;                 // sliding window, 0 = off
  int num_waves;              // waves of the persistent decode grid
  int nt;                     // tokens per work item (64 at 4-bit, 32 at 8-bit and FP8)
  int* plan = nullptr;        // 4-bit kernel, pure decode: the workspace's plan cache (decode_q4.hpp)
  int first_slot = 0;         // 4-bit kernel: workgroups that start in the first slot of a compute unit
                              // (the rest start later; 0 = all start together)
  const float* kps;           // FP8 pages only: key / value scale per page [nb]
  const float* vps;
};

constexpr int kMaxSeqs = 2048;    // per-sequence table held in LDS
constexpr int kMaxUnits = 65536;  // (sequence, kv_head) units with an arrival counter
constexpr int kMaxWaves = 4096;   // waves of the persistent grid

// DPP row_ror:N -- rotate within each row of 16 lanes.
template <int N>
__device__ __forceinline__ float row_ror(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x120 + N, 0xF, 0xF,
                                                               false));
}

template <int BITS, int GS, int HG>
struct DecodeCfg {
  static constexpr int D = 128;
  static constexpr int G = D / GS;           // quantization groups per head
  static constexpr int GSTRIDE = 16 / G;     // MFMA column of (head h, group g) = h + GSTRIDE * g
  static constexpr int TPL = 64 / BITS;      // tokens per lane group per iteration
  static constexpr int NT = 4 * TPL;         // tokens per iteration (64 at 4-bit, 32 at 8-bit)
  static constexpr int NIT = 128 / NT;       // iterations per 128-token tile
  static constexpr int NA = TPL / 4;         // 16-token MFMA sub-tiles per iteration
  static constexpr int KW = BITS;            // K code words a lane holds per sub-tile (32 dims)
  static constexpr int NWS = TPL / 8;        // PV k-slices (8 tokens each) per iteration
  static constexpr int W = D * BITS / 32;    // code words per token
  static constexpr int SPIECES = G * NT / 2; // dwords of one staged (scale|bias) array per iteration
  static constexpr int SK = (SPIECES + 63) / 64;
  static constexpr int SHALVES = 4 * G * NT;
  static_assert(HG <= GSTRIDE, "GQA group x quant groups must fit 16 MFMA columns");
  static_assert(SK <= 2, "staging assumes <= 2 dwords per lane per array");
};

// Buffer resources of one 128-token tile of one (page, kv_head), held in SGPRs:
// every per-lane address is then a single 32-bit offset.
struct TileRsrc {
  __amdgpu_buffer_rsrc_t k, v, s[4];
};

template <int BITS, int GS, int HG>
__device__ __forceinline__ TileRsrc make_tile_rsrc(const DecodeArgs& a, const int blk, const int kvh, const int off,
                                                   const bool live = true) {
  using C = DecodeCfg<BITS, GS, HG>;
  const int RW = a.bs * BITS / 32;
  const size_t ph = (size_t)blk * a.Hkv + kvh;
  TileRsrc rs;  // live = false: zero-size descriptors (loads read nothing and return zeros)
  rs.k = uniform_rsrc(a.kc + (ph * a.bs + off) * C::W, live ? 128 * C::W * 4 : 0);
  rs.v = uniform_rsrc(a.vc + ph * C::D * RW + (off / C::NT) * C::D * 8,
                      live ? (C::D * RW - (off / C::NT) * C::D * 8) * 4 : 0);
  const h16* sp[4] = {a.ks, a.kb, a.vs, a.vb};
#pragma unroll
  for (int arr = 0; arr < 4; ++arr)
    rs.s[arr] = uniform_rsrc(sp[arr] + ph * C::G * a.bs + off, live ? (C::G * a.bs - off) * 2 : 0);
  return rs;
}

// Register image of one iteration's loads.
template <int BITS, int GS, int HG>
struct IterLoads {
  using C = DecodeCfg<BITS, GS, HG>;
  uint32_t kw[C::NA][C::KW];
  uint32_t vw[8][2];
  uint32_t sw[4][C::SK];
};

template <int BITS, int GS, int HG>
__device__ __forceinline__ void issue_loads(IterLoads<BITS, GS, HG>& L, const TileRsrc& rs, const int RW,
                                            const int it_, const int lk, const int lv, const int (&ls)[2]) {
  using C = DecodeCfg<BITS, GS, HG>;
  const int it = __builtin_amdgcn_readfirstlane(it_);  // wave-uniform: the loads' scalar offsets
#pragma unroll
  for (int at = 0; at < C::NA; ++at) {
#pragma unroll
    for (int v = 0; v < C::KW / 4; ++v) {
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rs.k, lk + (4 * at * C::W + 4 * v) * 4,
                                                            it * C::NT * C::W * 4, kLoadAux);
      L.kw[at][4 * v + 0] = x[0];
      L.kw[at][4 * v + 1] = x[1];
      L.kw[at][4 * v + 2] = x[2];
      L.kw[at][4 * v + 3] = x[3];
    }
  }
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 x =
        __builtin_amdgcn_raw_buffer_load_b64(rs.v, lv, dt * 16 * 8 * 4 + it * C::D * 8 * 4, kLoadAux);
    L.vw[dt][0] = x[0];
    L.vw[dt][1] = x[1];
  }
#pragma unroll
  for (int arr = 0; arr < 4; ++arr) {
#pragma unroll
    for (int k = 0; k < C::SK; ++k) {
      if (C::SPIECES % 64 == 0 || ls[k] >= 0)
        L.sw[arr][k] = __builtin_amdgcn_raw_buffer_load_b32(rs.s[arr], ls[k], it * C::NT * 2, kLoadAux);
    }
  }
}

// One NT-token iteration of one wave.  `full`: every token of the iteration is
// inside [start_k, kv_len) (all but the first / last iteration of a sequence).
template <int BITS, int GS, int HG>
__device__ __forceinline__ void compute_iteration(IterLoads<BITS, GS, HG>& L, const bool full, const int (&lsd)[2],
                                                  const int jj, const bool col_ok, const int gg, const int tok_base,
                                                  const int start_k, const int kv_len, const h16x8 (&qB)[4],
                                                  const float qs, const float sc_l2, h16* stage, float& m_run,
                                                  float& l_part, float& pb, f32x4 (&acc)[8]) {
  using C = DecodeCfg<BITS, GS, HG>;
  constexpr int G = C::G, TPL = C::TPL, NT = C::NT, NA = C::NA, NWS = C::NWS, SK = C::SK;

  // ---- stage this iteration's scales / biases (dead tokens' may be garbage: zero them)
  if (!full) {
#pragma unroll
    for (int k = 0; k < SK; ++k) {
      const int pos = tok_base + (lsd[k] >= 0 ? lsd[k] % NT : 0);
      const uint32_t keep = (pos >= start_k && pos < kv_len ? 0x0000FFFFu : 0u) |
                            (pos + 1 >= start_k && pos + 1 < kv_len ? 0xFFFF0000u : 0u);
#pragma unroll
      for (int arr = 0; arr < 4; ++arr) L.sw[arr][k] &= keep;
    }
  }
#pragma unroll
  for (int arr = 0; arr < 4; ++arr) {
#pragma unroll
    for (int k = 0; k < SK; ++k) {
      if (C::SPIECES % 64 == 0 || lsd[k] >= 0)
        *reinterpret_cast<uint32_t*>(stage + arr * G * NT + lsd[k]) = L.sw[arr][k];
    }
  }

  // ---- S = Q K^T: lane holds tokens TPL*jj + 4*at + r of the iteration, column (hh, gg)
  const h16* sks = stage + (0 * G + gg) * NT + TPL * jj;
  const h16* skb = stage + (1 * G + gg) * NT + TPL * jj;
  float sc[NA][4];
#pragma unroll
  for (int at = 0; at < NA; ++at) {
    f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const h16x8 A = BITS == 4 ? unpack4(L.kw[at][w]) : unpack8(L.kw[at][2 * w], L.kw[at][2 * w + 1]);
      c = mfma16x16x32(A, qB[w], c);
    }
    typedef h16 h16x4 __attribute__((ext_vector_type(4)));
    const h16x4 ks4 = *reinterpret_cast<const h16x4*>(sks + 4 * at);
    const h16x4 kb4 = *reinterpret_cast<const h16x4*>(skb + 4 * at);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = fmaf(c[r], (float)ks4[r], (float)kb4[r] * qs);
      if constexpr (G >= 2) v += row_ror<8>(v);
      if constexpr (G >= 4) v += row_ror<4>(v);
      sc[at][r] = v;
    }
  }

  // ---- online softmax in base 2 (scores scaled by sc_l2 = softmax_scale * log2(e) * 2^24)
  if (!full) {
#pragma unroll
    for (int at = 0; at < NA; ++at) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int pos = tok_base + TPL * jj + 4 * at + r;
        if (pos < start_k || pos >= kv_len) sc[at][r] = -INFINITY;
      }
    }
  }
  float tmax = -INFINITY;
#pragma unroll
  for (int at = 0; at < NA; ++at) {
#pragma unroll
    for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, sc[at][r]);
  }
  tmax = rows4_max(tmax);
  const float m_new = fmaxf(m_run, tmax * sc_l2);
  if (__any(m_new != m_run)) {
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    l_part *= alpha;
    pb *= alpha;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;
    m_run = m_new;
  }
#pragma unroll
  for (int at = 0; at < NA; ++at) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float p = __builtin_amdgcn_exp2f(fmaf(sc[at][r], sc_l2, -m_run));
      sc[at][r] = p;
      l_part += p;
    }
  }

  // ---- O += P V: B = P' = p * v_scale rounded once to fp16, bias term accumulated on
  // the side in fp32.  The rounding error e of P' is folded into the bias term at the
  // centre code 2^(BITS-1): sum P' * c = sum fp16(P') * c + sum e * C0 + sum e * (c - C0),
  // so only e * (c - C0), |c - C0| <= 2^(BITS-1), is lost instead of e * c.  (One fp16
  // P' alone put outputs near zero, where sum P' * c cancels against the bias term,
  // up to 1.14x the tolerance on short-context batches; with the centre at most 0.45x,
  // measured by a float64 model of this arithmetic on the same seeds; a second MFMA
  // pass over the lo part of P' gave ~1e-4x at twice the matrix work.)
  const h16* svs = stage + (2 * G + gg) * NT + TPL * jj;
  const h16* svb = stage + (3 * G + gg) * NT + TPL * jj;
#pragma unroll
  for (int w = 0; w < NWS; ++w) {
    const h16x8 vs8 = *reinterpret_cast<const h16x8*>(svs + 8 * w);
    const h16x8 vb8 = *reinterpret_cast<const h16x8*>(svb + 8 * w);
    h16x8 pB;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = 8 * w + i;  // unpacked value element i is token i of the word
      const float p = sc[j >> 2][j & 3];
      const float x = col_ok ? p * (float)vs8[i] : 0.f;
      pB[i] = (h16)x;
      pb = fmaf(p, (float)vb8[i], pb);
      pb = fmaf(x - (float)pB[i], (float)(1 << (BITS - 1)), pb);
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const h16x8 A = BITS == 4 ? unpack4(L.vw[dt][w]) : unpack8(L.vw[dt][0], L.vw[dt][1]);
      acc[dt] = mfma16x16x32(A, pB, acc[dt]);
    }
  }
}

// Block-wide exclusive prefix of per-sequence live item counts into LDS.
// cum[s] = sum_{s' < s} n(s'), cum[S] = total; kvl[s] = clamped kv_len.
__device__ __forceinline__ void seq_table(const DecodeArgs& a, int* cum, int* kvl, int* qrw) {
  const int S = a.S;
  const int ch = (S + 255) / 256;
  const int s0 = threadIdx.x * ch;
  int tsum = 0;
  for (int i = 0; i < ch; ++i) {
    const int s = s0 + i;
    if (s < S) {
      int kl = min(a.kv_lens[s], a.max_blocks * a.bs);
      kl = max(kl, 0);
      // in a mixed batch only sequences with exactly one query token are decoded here
      const bool dec = a.qsl == nullptr || a.qsl[s + 1] - a.qsl[s] == 1;
      qrw[s] = a.qsl == nullptr ? s : a.qsl[s];
      kvl[s] = dec ? kl : -1;
      int n = 0;
      if (dec && kl > 0) {
        const int start_k = a.window > 0 ? max(0, kl - a.window) : 0;
        n = (kl - 1) / a.nt - start_k / a.nt + 1;
      }
      cum[s] = n;  // temporarily the count
      tsum += n;
    }
  }
  // inclusive scan of tsum over the block
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int x = tsum;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  __shared__ int wsum[4];
  if (lane == 63) wsum[wv] = x;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wv; ++w) base += wsum[w];
  int run = base + x - tsum;
  for (int i = 0; i < ch; ++i) {
    const int s = s0 + i;
    if (s < S) {
      const int n = cum[s];
      cum[s] = run;
      run += n;
    }
  }
  if (threadIdx.x == 255) cum[S] = base + x;
  __syncthreads();
}

// Wave containing item g of I items split over NW waves as [w*I/NW, (w+1)*I/NW):
// the w with start(w) <= g < start(w+1), start(w) = floor(w*I/NW).  A float
// estimate corrected with multiplications only (64-bit division is a long
// software sequence): start(w) <= g  <=>  w*I < (g+1)*NW.
__device__ __forceinline__ int wave_of_item(long long g, long long I, int NW) {
  int w = (int)((float)g * ((float)NW / (float)I));
  w = min(max(w, 0), NW - 1);
  const long long lim = (g + 1) * (long long)NW;
  while (w + 1 < NW && (long long)(w + 1) * I < lim) ++w;
  while (w > 0 && (long long)w * I >= lim) --w;
  return w;
}

constexpr int kCoherent = 16;  // cache policy SC1: device-coherent access
constexpr int kGroup = 4;       // pieces merged together at the first level ...
constexpr int kSingle = 8;      // ... when a unit has more pieces than this (c4: 16 pieces per unit merge
                                // as 4 groups in parallel, then 4 group results; 71.0 -> 66.6 us)

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Store 16 bytes as two 8-byte stores.  A VALU write to the data VGPRs of a
// wider vector-memory store right after its issue has been seen (gfx950, as
// scheduled by this compiler) to corrupt the stored data.
__device__ __forceinline__ void store_f32x4(const f32x4 v, const __amdgpu_buffer_rsrc_t r, const int voff,
                                            const int soff) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f32x2{v[0], v[1]}), r, voff, soff, kCoherent);
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f32x2{v[2], v[3]}), r, voff + 8, soff, kCoherent);
}

// Combine `count` partials (slots first, first + stride, ...) of one unit:
// O = sum_p 2^(m_p - M) o_p, L = sum_p 2^(m_p - M) l_p, M = max_p m_p.  To the
// fp16 output (out != nullptr: O / L) or back into slot `dst` as a partial.
// Lane owns float4 f = lane + 64k of the unit's HG*D values (head 4f/128).
// The loads of NB pieces (all of a lane's float4s) are in flight together:
// each batch costs one round trip to the coherent cache.
template <int HG>
__device__ __forceinline__ void merge_range(const __amdgpu_buffer_rsrc_t ro, const __amdgpu_buffer_rsrc_t rm,
                                            const int first, const int count, const int stride, h16* out,
                                            const int dst, const int lane) {
  constexpr int D = 128;
  constexpr int NF4 = HG * D / 4;
  constexpr int PL = (NF4 + 63) / 64;
  constexpr int KC = PL <= 2 ? PL : 2;  // float4s per lane merged together
  constexpr int NB = 8 / KC / (PL <= 2 ? 1 : 2);  // pieces per batch (fewer with more values: no spills)
  // lanes past the unit's values (HG = 1) read inside the buffer and write nothing
  auto fidx = [&](int k) { return NF4 % 64 == 0 ? lane + 64 * k : min(lane + 64 * k, NF4 - 1); };
#pragma unroll 1
  for (int k0 = 0; k0 < PL; k0 += KC) {
    float M[KC], L[KC];
    f32x4 O[KC];
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      M[k] = -INFINITY;
      L[k] = 0.f;
      O[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int p0 = 0; p0 < count; p0 += NB) {
      f32x4 o[NB][KC];
      f32x2 ml[NB][KC];
#pragma unroll
      for (int c = 0; c < NB; ++c) {
        const int p = first + min(p0 + c, count - 1) * stride;
#pragma unroll
        for (int k = 0; k < KC; ++k) {
          const int f = fidx(k0 + k), h = 4 * f / D;
          o[c][k] = __builtin_bit_cast(f32x4,
                                       __builtin_amdgcn_raw_buffer_load_b128(ro, f * 16, p * HG * D * 4, kCoherent));
          ml[c][k] =
              __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(rm, h * 8, p * HG * 8, kCoherent));
        }
      }
#pragma unroll
      for (int c = 0; c < NB; ++c) {
        if (p0 + c >= count) break;
#pragma unroll
        for (int k = 0; k < KC; ++k) {
          if (ml[c][k].x == -INFINITY) continue;  // a piece may hold no live token (invalid pages)
          const float Mn = fmaxf(M[k], ml[c][k].x);
          const float fo = __builtin_amdgcn_exp2f(M[k] - Mn);  // 0 while M is -inf
          const float fp = __builtin_amdgcn_exp2f(ml[c][k].x - Mn);
          O[k] = O[k] * fo + o[c][k] * fp;
          L[k] = L[k] * fo + ml[c][k].y * fp;
          M[k] = Mn;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      const int f = lane + 64 * (k0 + k);
      if (NF4 % 64 != 0 && f >= NF4) break;
      const int h = 4 * f / D;
      if (out != nullptr) {
        const float inv = L[k] > 0.f ? 1.f / L[k] : 0.f;
        typedef h16 h16x4 __attribute__((ext_vector_type(4)));
        *reinterpret_cast<h16x4*>(out + 4 * f) = h16x4{(h16)(O[k][0] * inv), (h16)(O[k][1] * inv),
                                                        (h16)(O[k][2] * inv), (h16)(O[k][3] * inv)};
      } else {
        store_f32x4(O[k], ro, f * 16, dst * HG * D * 4);
        if ((4 * f) % D == 0)
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f32x2{M[k], L[k]}), rm, h * 8,
                                                dst * HG * 8, kCoherent);
      }
    }
  }
}

// Count one arrival on a counter (lane 0); true on the `expected`-th arrival.
__device__ __forceinline__ bool arrive_last(int* cnt, const int expected, const int lane) {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's stores are complete before it is counted
  int old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __builtin_amdgcn_readfirstlane(old);
  if (old != expected - 1) return false;
  if (lane == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // zero for the next call
  return true;
}

// Pieces of unit u (items [unit_first, unit_first + n) of the I items split
// over NW waves): np pieces, partial slots slot0 .. slot0 + np - 1, wave W's
// piece is `me`; ro / rm address the pieces' accumulators and (max, sum) pairs.
struct PieceInfo {
  int slot0, np, me;
  __amdgpu_buffer_rsrc_t ro, rm;
};

// Number of pieces of a unit (lane-local: callers may pass per-lane units).
__device__ __forceinline__ int piece_count(const long long unit_first, const int n, const long long I, const int NW) {
  return wave_of_item(unit_first + n - 1, I, NW) - wave_of_item(unit_first, I, NW) + 1;
}

// Wave-uniform arguments only.
template <int HG>
__device__ __forceinline__ PieceInfo piece_info(const DecodeArgs& a, const int W, const int u,
                                                const long long unit_first, const int n, const long long I,
                                                const int NW) {
  constexpr int D = 128;
  PieceInfo pi;
  const int wf = wave_of_item(unit_first, I, NW);
  const int wl = wave_of_item(unit_first + n - 1, I, NW);
  // wave-uniform by construction; readfirstlane keeps the descriptors in SGPRs
  pi.np = __builtin_amdgcn_readfirstlane(wl - wf + 1);
  pi.slot0 = __builtin_amdgcn_readfirstlane(wf + u);  // the pieces of unit u sit in slots wf+u .. wl+u
  pi.me = __builtin_amdgcn_readfirstlane(W - wf);
  pi.ro = uniform_rsrc(a.ws_o + (size_t)pi.slot0 * (HG * D), pi.np * HG * D * 4);
  pi.rm = uniform_rsrc(a.ws_ml + (size_t)pi.slot0 * (HG * 2), pi.np * HG * 2 * 4);
  return pi;
}

// After storing its partial (o = unnormalized accumulator, m, l) in piece slot
// `me` with device-coherent stores: pieces are merged in groups of kGroup by
// the last arrival of each group (counter per group, indexed by the group's
// first slot); with more than one group, the group result replaces the group's
// first partial and the last group to finish merges the groups into the fp16
// output (counter per unit).  The reduce of page_attention.py:2006-2059.
template <int HG>
__device__ __forceinline__ void merge_pieces(const DecodeArgs& a, const PieceInfo& pi, const int u, const int row,
                                             const int kvh, const int lane) {
  constexpr int D = 128;
  const int np = pi.np;
  // one level up to kSingle pieces; beyond, groups of kGroup first
  const int gsz = np <= kSingle ? np : kGroup;
  const int grp = pi.me / gsz, ngrp = (np + gsz - 1) / gsz;
  const int gfirst = grp * gsz, gcount = min(gsz, np - gfirst);
  if (!arrive_last(a.ws_cnt_grp + pi.slot0 + gfirst, gcount, lane)) return;
  h16* out = a.out + ((size_t)row * a.Hq + (size_t)kvh * HG) * D;
  if (ngrp == 1) {
    merge_range<HG>(pi.ro, pi.rm, 0, np, 1, out, 0, lane);
    return;
  }
  merge_range<HG>(pi.ro, pi.rm, gfirst, gcount, 1, nullptr, gfirst, lane);
  if (!arrive_last(a.ws_cnt + u, ngrp, lane)) return;
  merge_range<HG>(pi.ro, pi.rm, 0, ngrp, gsz, out, 0, lane);
}

// Stores a wave's partial (HG x 128 floats, head-major, already in the wave's
// LDS slot xw) with 8-byte stores of 64 consecutive lanes: every store
// instruction writes 512 contiguous bytes, whole lines instead of scattered pieces.
template <int HG>
__device__ __forceinline__ void store_partial_lds(const float* xw, const __amdgpu_buffer_rsrc_t ro, const int me,
                                                  const int lane) {
  constexpr int D = 128;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int b = 0; b < HG * D; b += 128) {
    const f32x2 v = *reinterpret_cast<const f32x2*>(xw + b + 2 * lane);
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), ro, (b + 2 * lane) * 4, me * HG * D * 4,
                                          kCoherent);
  }
}

// Wave W finished its piece of unit u: store its partial (through the wave's
// LDS slot xw), then merge.
template <int GS, int HG>
__device__ __forceinline__ void merge_piece(const DecodeArgs& a, const int W, const int u, const long long unit_first,
                                            const int n, const long long I, const int NW, const int row, const int kvh,
                                            const f32x4 (&acc)[8], const float pbs, const float m_run, const float l,
                                            const bool col_ok, const int gg, const int jj, const int hh,
                                            const int lane, float* xw) {
  constexpr int D = 128;
  const PieceInfo pi = piece_info<HG>(a, W, u, unit_first, n, I, NW);
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {  // lane (hh, gg, jj) owns dims 16*dt + 4*jj .. +3 when they lie in group gg
    const int d = 16 * dt + 4 * jj;
    if (col_ok && d / GS == gg) *reinterpret_cast<f32x4*>(xw + hh * D + d) = acc[dt] * kTwo24 + pbs;
  }
  store_partial_lds<HG>(xw, pi.ro, pi.me, lane);
  if (col_ok && gg == 0 && jj == 0)
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f32x2{m_run, l}), pi.rm, hh * 8,
                                          pi.me * HG * 8, kCoherent);
  merge_pieces<HG>(a, pi, u, row, kvh, lane);
}

// The kernel body as workgroup `bid` of `nblocks` (a grid of its own, or the
// decode part of a mixed batch's single launch, unified_affine); a.num_waves is
// the number of waves the ranges are split over.
template <int BITS, int GS, int HG>
__device__ __forceinline__ void decode_affine_body(const DecodeArgs& a, const int bid, const int nblocks) {
  using C = DecodeCfg<BITS, GS, HG>;
  constexpr int D = C::D, G = C::G, GSTRIDE = C::GSTRIDE, NT = C::NT;

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int jj = lane >> 4;
  const int hh = col % GSTRIDE;
  const int gg = col / GSTRIDE;
  const bool col_ok = hh < HG;

  // LDS, carved from the shared arena
  constexpr int oCum = 0, oKvl = lds_next(oCum, 4 * (kMaxSeqs + 1)), oQrw = lds_next(oKvl, 4 * kMaxSeqs);
  constexpr int oStage = lds_next(oQrw, 4 * kMaxSeqs), oXst = lds_next(oStage, 2 * 4 * C::SHALVES);
  constexpr int oEnd = lds_next(oXst, 4 * 4 * HG * 128);
  static_assert(oEnd <= kArenaBytes, "LDS arena too small");
  int(&cum)[kMaxSeqs + 1] = lds_at<int[kMaxSeqs + 1]>(oCum);
  int(&kvl)[kMaxSeqs] = lds_at<int[kMaxSeqs]>(oKvl);
  int(&qrw)[kMaxSeqs] = lds_at<int[kMaxSeqs]>(oQrw);
  h16(&stage_all)[4][C::SHALVES] = lds_at<h16[4][C::SHALVES]>(oStage);
  float(&xst)[4][HG * 128] = lds_at<float[4][HG * 128]>(oXst);  // per wave: a partial, head-major
  seq_table(a, cum, kvl, qrw);
  {  // decoded sequences without a live token produce zeros (the reference's l == 0 case)
    const int per_seq = a.Hq * D / 8;
    for (int i = bid * 256 + threadIdx.x; i < a.S * per_seq; i += nblocks * 256) {
      const int si = i / per_seq;
      if (kvl[si] >= 0 && cum[si + 1] == cum[si])
        reinterpret_cast<u32x4*>(a.out)[(size_t)qrw[si] * per_seq + i % per_seq] = u32x4{0u, 0u, 0u, 0u};
    }
  }

  const int S = a.S, Hkv = a.Hkv;
  // LDS table entries read at a wave-uniform index are moved to SGPRs (uru), so the
  // per-item scheduling arithmetic and the load offsets stay scalar
  auto uru = [](int v) { return __builtin_amdgcn_readfirstlane(v); };
  const long long I = (long long)Hkv * uru(cum[S]);
  const int NW = (int)min((long long)a.num_waves, I);  // every wave range non-empty
  const int W = bid * 4 + wv;
  if (W >= NW) return;
  const long long g0 = ((long long)W * I) / NW;
  const long long g1 = ((long long)(W + 1) * I) / NW;

  // ---- item g -> (sequence, kv_head, live iteration j, token base)
  auto seq_of = [&](long long g, int s_from) {  // first s >= s_from with Hkv*cum[s+1] > g
    int si = s_from;
    while (si + 1 < S && (long long)Hkv * cum[si + 1] <= g) ++si;
    return si;
  };
  auto lo_of = [&](int si) { return (a.window > 0 ? max(0, kvl[si] - a.window) : 0) / NT; };
  int s = 0;
  for (int c = 0; c < S; c += 64) {
    const int si = c + lane;
    s += __builtin_popcountll(__ballot(si < S && (long long)Hkv * cum[si + 1] <= g0));
  }
  s = __builtin_amdgcn_readfirstlane(s);

  // ---- block id of every item of the range, one item per lane (64 items per chunk)
  auto blk_chunk = [&](long long gb) {
    const long long g = gb + lane;
    int b = -1;
    if (g < g1) {
      const int si = seq_of(g, s);
      const int n = cum[si + 1] - cum[si];
      const int jn = (int)(g - (long long)Hkv * cum[si]) % n;
      b = a.block_tables[(size_t)si * a.max_blocks + ((lo_of(si) + jn) * NT) / a.bs];
    }
    return b;
  };
  int blkv = blk_chunk(g0);

  // ---- query operand of a unit: lane holds dims 32*jj .. 32*jj+31 of head hh, zero outside group gg
  u32x4 qraw[4];
  auto issue_q = [&](int seq, int kh) {
    const u32x4* qp = reinterpret_cast<const u32x4*>(
        a.q + ((size_t)qrw[seq] * a.Hq + (size_t)kh * HG + (col_ok ? hh : 0)) * D + 32 * jj);
#pragma unroll
    for (int i = 0; i < 4; ++i) qraw[i] = qp[i];
  };
  h16x8 qB[4];
  float qs = 0.f;
  auto build_q = [&]() {
    const h16* qv = reinterpret_cast<const h16*>(qraw);
    float qsum = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int dl = 8 * w + slot_perm<BITS>(i);
        const int dim = 32 * jj + dl;
        const h16 v = (col_ok && dim / GS == gg) ? qv[dl] : (h16)0.0f;
        qB[w][i] = v;
        qsum += (float)v;
      }
    }
    qsum += __shfl_xor(qsum, 16, 64);
    qsum += __shfl_xor(qsum, 32, 64);
    qs = qsum * (1.0f / kTwo24);  // bias term in the 2^-24 units of the MFMA output
  };

  int n_s = uru(cum[s + 1]) - uru(cum[s]);
  int kvh, j;
  {
    const int r = (int)(g0 - (long long)Hkv * uru(cum[s]));
    kvh = r / n_s;
    j = r % n_s;
  }
  issue_q(s, kvh);
  int kv_len = uru(kvl[s]);
  int start_k = a.window > 0 ? max(0, kv_len - a.window) : 0;
  int it_lo = start_k / NT;

  const int RW = a.bs * BITS / 32;
  const int lk = ((C::TPL * (col >> 2) + (col & 3)) * C::W + C::KW * jj) * 4;
  const int lv = (col * 8 + C::TPL * jj * BITS / 32) * 4;
  int ls[2], lsd[2];  // staged scale/bias dword: global byte offset and LDS half index (-1 = none)
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int pc = lane + 64 * k;
    const int g = pc / (NT / 2), c2 = pc % (NT / 2);
    const bool ok = pc < G * NT / 2;
    ls[k] = ok ? (g * a.bs + 2 * c2) * 2 : -1;
    lsd[k] = ok ? g * NT + 2 * c2 : -1;
  }
  h16* stage = stage_all[wv];
  const float sc_l2 = a.scale_log2 * kTwo24;

  // ---- first item's loads (its query is already in flight)
  int tb = (it_lo + j) * NT;
  int blk = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(blkv, 0));
  const TileRsrc rs_first =
      make_tile_rsrc<BITS, GS, HG>(a, (unsigned)blk < (unsigned)a.nb ? blk : 0, kvh, (tb & ~127) % a.bs);
  // two load buffers used alternately, so the wait before an item's compute
  // never covers the following item's loads
  IterLoads<BITS, GS, HG> bufA, bufB;
  issue_loads(bufA, rs_first, RW, (tb & 127) / NT, lk, lv, ls);
  build_q();

  float m_run = -INFINITY, l_part = 0.f, pb = 0.f;
  f32x4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  long long unit_first = (long long)Hkv * cum[s] + (long long)kvh * n_s;  // first item of the current unit

  auto step = [&](IterLoads<BITS, GS, HG>& cur, IterLoads<BITS, GS, HG>& nxt, const long long g) {
    // ---- next item
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
          lo1 = (a.window > 0 ? max(0, kl1 - a.window) : 0) / NT;
        }
      }
    }
    const bool has_next = g + 1 < g1;
    const bool unit_end = !has_next || s1 != s || kvh1 != kvh;
    int blk1 = blk, tb1 = (lo1 + j1) * NT;
    if (has_next) {
      const int k1 = (int)(g + 1 - g0);
      if ((k1 & 63) == 0) blkv = blk_chunk(g + 1);
      blk1 = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(blkv, k1 & 63));
    }
    // built from scalar inputs every step (a descriptor carried or selected between
    // steps ends up in VGPRs, which wraps each load in a per-lane loop)
    const TileRsrc rs_nxt = make_tile_rsrc<BITS, GS, HG>(a, (unsigned)blk1 < (unsigned)a.nb ? blk1 : 0, kvh1,
                                                         (tb1 & ~127) % a.bs, has_next);
    // Issued on every path (an empty descriptor returns zeros without touching
    // memory): the compiler's wait before this item's compute then counts these
    // loads as younger and leaves them in flight, instead of draining them.
    issue_loads(nxt, rs_nxt, RW, (tb1 & 127) / NT, lk, lv, ls);
    if (has_next && unit_end) issue_q(s1, kvh1);

    // ---- compute the current item (an invalid page is skipped like the reference's Metal kernel)
    if ((unsigned)blk < (unsigned)a.nb) {
      const bool full = tb >= start_k && tb + NT <= kv_len;
      compute_iteration<BITS, GS, HG>(cur, full, lsd, jj, col_ok, gg, tb, start_k, kv_len, qB, qs, sc_l2, stage,
                                      m_run, l_part, pb, acc);
    }

    // ---- unit finished (or range ends): write output / partial, reset
    if (unit_end) {
      float l = l_part + __shfl_xor(l_part, 16, 64);
      l += __shfl_xor(l, 32, 64);
      float pbs = pb + __shfl_xor(pb, 16, 64);
      pbs += __shfl_xor(pbs, 32, 64);
      const bool whole = unit_first >= g0 && unit_first + n_s <= g1;
      const int u = s * Hkv + kvh;
      if (whole) {
        h16* out = a.out + ((size_t)qrw[s] * a.Hq + (size_t)kvh * HG + hh) * D;
        const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int d = 16 * dt + 4 * jj + r;
            if (col_ok && d / GS == gg) out[d] = (h16)((acc[dt][r] * kTwo24 + pbs) * inv);
          }
      } else {
        merge_piece<GS, HG>(a, W, u, unit_first, n_s, I, NW, qrw[s], kvh, acc, pbs, m_run, l, col_ok, gg, jj, hh,
                            lane, xst[wv]);
      }
      m_run = -INFINITY;
      l_part = 0.f;
      pb = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
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
    blk = blk1;
  };
  for (long long g = g0; g < g1; g += 2) {
    step(bufA, bufB, g);
    if (g + 1 >= g1) break;
    step(bufB, bufA, g + 1);
  }
}

template <int BITS, int GS, int HG>
__global__ __launch_bounds__(256, 2) void decode_affine_d128(DecodeArgs a) {
  decode_affine_body<BITS, GS, HG>(a, blockIdx.x, gridDim.x);
}

}  // namespace emx
