// Single-token paged decode over affine-quantized pages, head_dim 128, MFMA.
//
// Replaces the reference's per-(seq, q_head) serial key loop
// (lib/python/easymlx/operations/kernels/unified_attention.py:467-609) and its
// split-K variant (page_attention.py:1718-2059) for affine int4/int8 pages.
//
// Work decomposition
//   workgroup = (seq, kv_head, split) with 4 waves; a split is a run of
//   `tiles_per_split` 128-token tiles, wave w takes tiles w, w+4, ... of it.
//   All Hq/Hkv query heads of the GQA group are served from one read of each
//   K/V byte.  Splits of one (seq, kv_head) write fp32 partials that
//   decode_merge_d128 combines (no cross-workgroup fences in the hot kernel).
//
// Per 128-token tile and wave (lane l: col = l%16, jj = l/16)
//   QK^T : 8 token sub-tiles x 4 k-slices of v_mfma_f32_16x16x32_f16.
//          A = K codes as fp16 subnormals (row rho of sub-tile a is token
//          32*(rho/4) + 4a + rho%4), B = query columns: column c holds query
//          head c % HG restricted to quantization group c / HG (zeros elsewhere),
//          so one MFMA produces per-group partial dots and the affine scale /
//          bias is applied per (token, group) afterwards:
//            s = sum_g 2^24 * scale[t,g] * C[t,(h,g)] + bias[t,g] * sum_{d in g} q_hd
//   softmax: online, base-2, fp32; row max over the lane's 32 tokens then
//          across the 4 lane groups.
//   PV   : 8 dim sub-tiles x 4 token k-slices.  A = V codes (V pages are stored
//          dim-major, so a lane's uint32 is 8 consecutive tokens of one dim),
//          B = p * v_scale[t, g(col)] in fp16; the bias term
//          sum_t p_t * v_bias[t,g] is accumulated in fp32 on the side.
#pragma once

#include "common.hpp"

namespace emx {

struct DecodeArgs {
  const h16* q;               // [S, Hq, 128]
  const uint32_t* kc;         // [nb, Hkv, bs, 128*BITS/32]
  const h16* ks;              // [nb, Hkv, G, bs]
  const h16* kb;              // [nb, Hkv, G, bs]
  const uint32_t* vc;         // [nb, Hkv, 128, bs*BITS/32]
  const h16* vs;              // [nb, Hkv, G, bs]
  const h16* vb;              // [nb, Hkv, G, bs]
  const int32_t* block_tables;  // [S, max_blocks]
  const int32_t* kv_lens;       // [S]
  h16* out;                   // [S, Hq, 128]
  float* ws_o;                // [S, Hkv, max_splits, HG, 128]
  float* ws_ml;               // [S, Hkv, max_splits, HG, 2]
  int S, Hq, Hkv, bs, nb, max_blocks;
  float scale_log2;           // softmax_scale * log2(e)
  int window;                 // sliding window, 0 = off
  int tiles_per_split;
  int max_splits;
};

// Rotate within each row of 16 lanes (DPP row_ror:N); sums over lanes c, c+N, ...
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
  static constexpr int NA = TPL / 4;         // 16-token MFMA sub-tiles per iteration
  static constexpr int KW = BITS;            // K code words a lane holds per sub-tile (32 dims)
  static constexpr int NWS = TPL / 8;        // PV k-slices (8 tokens each) per iteration
  static constexpr int W = D * BITS / 32;    // code words per token
  static constexpr int SROW = NT;            // halves per staged (array, group) row
  static constexpr int SHALVES = 4 * G * NT; // staged ks, kb, vs, vb halves per iteration
  static_assert(HG <= GSTRIDE, "GQA group x quant groups must fit 16 MFMA columns");
};

// Buffer resources of one 128-token tile of one (page, kv_head); built in SGPRs
// per tile, so every per-lane load address is a single 32-bit offset.
struct TileRsrc {
  __amdgpu_buffer_rsrc_t k, v, s[4];
};

constexpr int kRsrcFlags = 0x00020000;  // raw 32-bit buffer, gfx9 family
constexpr int kLoadAux = 0;             // default cache policy

// One NT-token iteration of one wave.  `full`: every token of the iteration is
// inside [start_k, kv_len) (all but the first / last iteration of a sequence).
template <int BITS, int GS, int HG>
__device__ __forceinline__ void decode_iteration(const bool full, const TileRsrc& rs, const int RW, const int it, const int lk,
                                                 const int lv, const int (&ls)[2], const int (&lsd)[2],
                                                 const int jj, const bool col_ok, const int gg,
                                                 const int tok_base, const int start_k, const int kv_len,
                                                 const h16x8 (&qB)[4], const float qs, const float sc_l2,
                                                 h16* stage, float& m_run, float& l_part, float& pb,
                                                 f32x4 (&acc)[8]) {
  using C = DecodeCfg<BITS, GS, HG>;
  constexpr int G = C::G, TPL = C::TPL, NT = C::NT, NA = C::NA, KW = C::KW, NWS = C::NWS, W = C::W;
  constexpr int SPIECES = G * NT / 2;  // dwords of one staged array per iteration

  // ---- issue the iteration's loads: K sub-tiles, V dim rows, staged scale/bias dwords
  uint32_t kw[NA][KW];
#pragma unroll
  for (int at = 0; at < NA; ++at) {
#pragma unroll
    for (int v = 0; v < KW / 4; ++v) {
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rs.k, lk + (4 * at * W + 4 * v) * 4, it * NT * W * 4,
                                                            kLoadAux);
      kw[at][4 * v + 0] = x[0];
      kw[at][4 * v + 1] = x[1];
      kw[at][4 * v + 2] = x[2];
      kw[at][4 * v + 3] = x[3];
    }
  }
  uint32_t vw[8][2];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(rs.v, lv, dt * 16 * RW * 4 + it * NT * BITS / 8, kLoadAux);
    vw[dt][0] = x[0];
    vw[dt][1] = x[1];
  }
  uint32_t sw[4][2];
#pragma unroll
  for (int arr = 0; arr < 4; ++arr) {
#pragma unroll
    for (int k = 0; k < (SPIECES + 63) / 64; ++k) {
      if (SPIECES % 64 == 0 || lsd[k] >= 0)
        sw[arr][k] = __builtin_amdgcn_raw_buffer_load_b32(rs.s[arr], ls[k], it * NT * 2, kLoadAux);
    }
  }
  if (!full) {
    // scale/bias of tokens outside [start_k, kv_len) may be garbage: stage zeros instead
#pragma unroll
    for (int k = 0; k < (SPIECES + 63) / 64; ++k) {
      const int t = lsd[k] % NT;  // token of the dword's low half
      const int pos = tok_base + t;
      const uint32_t keep = (pos >= start_k && pos < kv_len ? 0x0000FFFFu : 0u) |
                            (pos + 1 >= start_k && pos + 1 < kv_len ? 0xFFFF0000u : 0u);
#pragma unroll
      for (int arr = 0; arr < 4; ++arr) sw[arr][k] &= keep;
    }
  }
#pragma unroll
  for (int arr = 0; arr < 4; ++arr) {
#pragma unroll
    for (int k = 0; k < (SPIECES + 63) / 64; ++k) {
      if (SPIECES % 64 == 0 || lsd[k] >= 0)
        *reinterpret_cast<uint32_t*>(stage + arr * G * NT + lsd[k]) = sw[arr][k];
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
      const h16x8 A = BITS == 4 ? unpack4(kw[at][w]) : unpack8(kw[at][2 * w], kw[at][2 * w + 1]);
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

  // ---- online softmax in base 2 (scores scaled by sc_l2 = softmax_scale*log2(e)*2^24)
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
  tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
  tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
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

  // ---- O += P V: B = p * v_scale (fp16), bias term accumulated on the side
  const h16* svs = stage + (2 * G + gg) * NT + TPL * jj;
  const h16* svb = stage + (3 * G + gg) * NT + TPL * jj;
#pragma unroll
  for (int w = 0; w < NWS; ++w) {
    const h16x8 vs8 = *reinterpret_cast<const h16x8*>(svs + 8 * w);
    const h16x8 vb8 = *reinterpret_cast<const h16x8*>(svb + 8 * w);
    h16x8 pB;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = 8 * w + slot_perm<BITS>(i);
      const float p = sc[j >> 2][j & 3];
      pB[i] = col_ok ? (h16)(p * (float)vs8[slot_perm<BITS>(i)]) : (h16)0.0f;
      pb = fmaf(p, (float)vb8[slot_perm<BITS>(i)], pb);
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const h16x8 A = BITS == 4 ? unpack4(vw[dt][w]) : unpack8(vw[dt][0], vw[dt][1]);
      acc[dt] = mfma16x16x32(A, pB, acc[dt]);
    }
  }
}

template <int BITS, int GS, int HG>
__global__ __launch_bounds__(256, 4) void decode_affine_d128(DecodeArgs a) {
  using C = DecodeCfg<BITS, GS, HG>;
  constexpr int D = C::D, G = C::G, GSTRIDE = C::GSTRIDE, NT = C::NT;
  static_assert(G * NT / 2 <= 128, "staging assumes <= 2 dwords per lane per array");

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int jj = lane >> 4;
  const int hh = col % GSTRIDE;
  const int gg = col / GSTRIDE;
  const bool col_ok = hh < HG;

  int bid = blockIdx.x;
  const int kvh = bid % a.Hkv;
  bid /= a.Hkv;
  const int s = bid % a.S;
  const int split = bid / a.S;

  __shared__ float so[4][HG * D];
  __shared__ float sm[4][HG];
  __shared__ float sl[4][HG];
  __shared__ __attribute__((aligned(16))) h16 stage_all[4][C::SHALVES];

  h16* out = a.out + ((size_t)s * a.Hq + (size_t)kvh * HG) * D;
  int kv_len = a.kv_lens[s];
  kv_len = min(kv_len, a.max_blocks * a.bs);
  if (kv_len <= 0) {
    if (split == 0)
      for (int i = threadIdx.x; i < HG * D; i += 256) out[i] = (h16)0.0f;
    return;
  }
  const int start_k = a.window > 0 ? max(0, kv_len - a.window) : 0;
  const int tile_first = start_k >> 7;
  const int tile_last = (kv_len - 1) >> 7;
  const int n_splits = (tile_last - tile_first + a.tiles_per_split) / a.tiles_per_split;
  if (split >= n_splits) return;
  const int t_begin = tile_first + split * a.tiles_per_split;
  const int t_end = min(t_begin + a.tiles_per_split, tile_last + 1);

  // ---- query operand: lane holds dims 32*jj .. 32*jj+31 of head hh, zero outside group gg
  h16x8 qB[4];
  float qsum = 0.f;
  {
    const u32x4* qp = reinterpret_cast<const u32x4*>(
        a.q + ((size_t)s * a.Hq + (size_t)kvh * HG + (col_ok ? hh : 0)) * D + 32 * jj);
    u32x4 raw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) raw[i] = qp[i];
    const h16* qv = reinterpret_cast<const h16*>(raw);
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
  }
  const float qs = qsum * (1.0f / kTwo24);   // bias term in the 2^-24 units of the MFMA output
  const float sc_l2 = a.scale_log2 * kTwo24;

  float m_run = -INFINITY;
  float l_part = 0.f;
  float pb = 0.f;
  f32x4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  h16* stage = stage_all[wv];

  // per-lane byte offsets inside a tile (constant for the whole kernel)
  const int RW = a.bs * BITS / 32;  // code words per V dim row
  const int lk = ((C::TPL * (col >> 2) + (col & 3)) * C::W + C::KW * jj) * 4;
  const int lv = (col * RW + C::TPL * jj * BITS / 32) * 4;
  int ls[2], lsd[2];  // staged scale/bias dword: global byte offset, LDS half index (-1 = none)
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int pc = lane + 64 * k;
    const int g = pc / (NT / 2), c2 = pc % (NT / 2);
    const bool ok = pc < G * NT / 2;
    ls[k] = ok ? (g * a.bs + 2 * c2) * 2 : 0;
    lsd[k] = ok ? g * NT + 2 * c2 : -1;
  }

  for (int tile = t_begin + wv; tile < t_end; tile += 4) {
    const int tok0 = tile << 7;
    const int page = tok0 / a.bs;
    const int off = tok0 - page * a.bs;
    const int blk = __builtin_amdgcn_readfirstlane(a.block_tables[(size_t)s * a.max_blocks + page]);
    if (blk < 0 || blk >= a.nb) continue;
    const size_t ph = (size_t)blk * a.Hkv + kvh;
    TileRsrc rs;
    rs.k = __builtin_amdgcn_make_buffer_rsrc((void*)(a.kc + (ph * a.bs + off) * C::W), (short)0, 128 * C::W * 4,
                                             kRsrcFlags);
    rs.v = __builtin_amdgcn_make_buffer_rsrc((void*)(a.vc + ph * D * RW + off * BITS / 32), (short)0,
                                             (D * RW - off * BITS / 32) * 4, kRsrcFlags);
    const h16* sp[4] = {a.ks, a.kb, a.vs, a.vb};
#pragma unroll
    for (int arr = 0; arr < 4; ++arr)
      rs.s[arr] = __builtin_amdgcn_make_buffer_rsrc((void*)(sp[arr] + ph * G * a.bs + off), (short)0,
                                                    (G * a.bs - off) * 2, kRsrcFlags);
#pragma unroll 1
    for (int it = 0; it < 128 / NT; ++it) {
      const int tb = tok0 + it * NT;
      if (tb >= kv_len) break;
      if (tb + NT <= start_k) continue;
      const bool full = tb >= start_k && tb + NT <= kv_len;
      decode_iteration<BITS, GS, HG>(full, rs, RW, it, lk, lv, ls, lsd, jj, col_ok, gg, tb, start_k, kv_len, qB, qs,
                                     sc_l2, stage, m_run, l_part, pb, acc);
    }
  }

  // ---- per-wave epilogue -> LDS (acc is in 2^-24 units)
  l_part += __shfl_xor(l_part, 16, 64);
  l_part += __shfl_xor(l_part, 32, 64);
  pb += __shfl_xor(pb, 16, 64);
  pb += __shfl_xor(pb, 32, 64);
  if (col_ok && gg == 0 && jj == 0) {
    sm[wv][hh] = m_run;
    sl[wv][hh] = l_part;
  }
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int d = 16 * dt + 4 * jj + r;
      if (col_ok && d / GS == gg) so[wv][hh * D + d] = acc[dt][r] * kTwo24 + pb;
    }
  }
  __syncthreads();

  // ---- merge the 4 waves
  const size_t unit = (size_t)s * a.Hkv + kvh;
  if (n_splits == 1) {
    for (int i = threadIdx.x; i < HG * D; i += 256) {
      const int h = i / D;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < 4; ++w) M = fmaxf(M, sm[w][h]);
      float L = 0.f, o = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        if (sm[w][h] != -INFINITY) {
          const float f = exp2f(sm[w][h] - M);
          L += sl[w][h] * f;
          o += so[w][i] * f;
        }
      }
      out[i] = (h16)(L > 0.f ? o / L : 0.f);
    }
    return;
  }

  float* wo = a.ws_o + (unit * a.max_splits + split) * (HG * D);
  float* wml = a.ws_ml + (unit * a.max_splits + split) * (HG * 2);
  for (int i = threadIdx.x; i < HG * D; i += 256) {
    const int h = i / D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sm[w][h]);
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if (sm[w][h] != -INFINITY) {
        const float f = exp2f(sm[w][h] - M);
        L += sl[w][h] * f;
        o += so[w][i] * f;
      }
    }
    wo[i] = o;
    if ((i % D) == 0) {
      wml[2 * h] = M;
      wml[2 * h + 1] = L;
    }
  }
}

// Merge the split-K partials of every (seq, kv_head) that was split (the
// reduce pass of page_attention.py:2006-2059): out = sum_p 2^(m_p - M) o_p /
// sum_p 2^(m_p - M) l_p.  Launched after decode_affine_d128 on the same stream.
template <int HG>
__global__ __launch_bounds__(256) void decode_merge_d128(DecodeArgs a) {
  constexpr int D = 128;
  const int unit = blockIdx.x;
  const int kvh = unit % a.Hkv;
  const int s = unit / a.Hkv;
  int kv_len = min(a.kv_lens[s], a.max_blocks * a.bs);
  if (kv_len <= 0) return;
  const int start_k = a.window > 0 ? max(0, kv_len - a.window) : 0;
  const int n_tiles = ((kv_len - 1) >> 7) - (start_k >> 7) + 1;
  const int n_splits = (n_tiles + a.tiles_per_split - 1) / a.tiles_per_split;
  if (n_splits <= 1) return;

  __shared__ float wts[512 * HG];  // n_splits <= 512
  __shared__ float sL[HG];
  const float* po = a.ws_o + (size_t)unit * a.max_splits * (HG * D);
  const float* pml = a.ws_ml + (size_t)unit * a.max_splits * (HG * 2);
  if (threadIdx.x < HG) {
    const int h = threadIdx.x;
    float M = -INFINITY;
    for (int sp = 0; sp < n_splits; ++sp) M = fmaxf(M, pml[sp * HG * 2 + 2 * h]);
    float L = 0.f;
    for (int sp = 0; sp < n_splits; ++sp) {
      const float m = pml[sp * HG * 2 + 2 * h];
      const float f = m != -INFINITY ? exp2f(m - M) : 0.f;
      L += f * pml[sp * HG * 2 + 2 * h + 1];
      wts[sp * HG + h] = f;
    }
    sL[h] = L;
  }
  __syncthreads();
  h16* out = a.out + ((size_t)s * a.Hq + (size_t)kvh * HG) * D;
  for (int i = threadIdx.x; i < HG * D; i += 256) {
    const int h = i / D;
    float o = 0.f;
    for (int sp = 0; sp < n_splits; ++sp) {
      const float f = wts[sp * HG + h];
      if (f != 0.f) o += f * po[(size_t)sp * HG * D + i];
    }
    const float L = sL[h];
    out[i] = (h16)(L > 0.f ? o / L : 0.f);
  }
}

}  // namespace emx
