// Multi-token (prefill) paged attention over affine-quantized pages, head_dim 128, MFMA.
//
// Replaces the ragged / causal Metal kernel of the reference for the query rows
// of sequences with more than one query token
// (lib/python/easymlx/operations/kernels/unified_attention.py:290-465, causal
// limit :357-361, sliding window :369-376) and the single-sequence causal path
// (page_attention.py:84-133).  Decode rows (one query token) of the same batch
// go to the decode kernels (decode_q4_d128 / decode_affine_d128).
//
// Work: one workgroup (4 waves) per (sequence, kv_head, tile of 128/HG query
// tokens); a wave owns 32 query columns = (token, head) pairs, head fastest.
// Keys are walked in NT-token steps (64 at 4-bit, 32 at 8-bit) up to the tile's
// causal limit; each step's K/V codes and scales are loaded once per workgroup
// into LDS (double-buffered) and shared by the four waves.
//
// Arithmetic is exact in the codes, like the decode kernel: codes enter
// v_mfma_f32_16x16x32_f16 as fp16 subnormals (code * 2^-24) and the affine
// scale / bias are applied in fp32 afterwards.
//   S^T: A = K codes (rows = keys; row rho of sub-tile a is key
//        TPL*(rho/4) + 4a + rho%4), B = queries; MFMA w spans dims
//        [32w, 32w+32), so each quantization group accumulates separately:
//          s = 2^24 * sum_g ks[t,g] C_g[t,c] + sum_g kb[t,g] * sum_{d in g} q[c,d]
//   PV : A = V codes (rows = dims), B = p * vs[t, g] in fp16 for the dims of
//        group g; sum_t p * vb[t, g] is accumulated in fp32.
#pragma once

#include "common.hpp"
#include "decode_affine.hpp"

namespace emx {

struct PrefillArgs {
  const h16* q;                 // [T, Hq, 128]
  const uint32_t* kc;           // [nb, Hkv, bs, 128*BITS/32]
  const h16 *ks, *kb;           // [nb, Hkv, G, bs]
  const uint32_t* vc;           // [nb, Hkv, bs/NT, 128, 8]
  const h16 *vs, *vb;           // [nb, Hkv, G, bs]
  const int32_t* block_tables;  // [S, max_blocks]
  const int32_t* kv_lens;       // [S]
  const int32_t* qsl;           // [S + 1]
  h16* out;                     // [T, Hq, 128]
  int S, Hq, Hkv, bs, nb, max_blocks;
  float scale_log2;             // softmax_scale * log2(e)
  int window;                   // sliding window, 0 = off
};

template <int BITS, int GS, int HG>
struct PrefillCfg {
  using C = DecodeCfg<BITS, GS, 1>;
  static constexpr int D = 128, G = C::G, NT = C::NT, TPL = C::TPL, NA = C::NA, NWS = C::NWS, W = C::W;
  static constexpr int COLS = 32;                  // query columns per wave
  static constexpr int TOKW = COLS / HG;           // query tokens per wave
  static constexpr int TOKB = 4 * TOKW;            // query tokens per workgroup
  static constexpr int KROW = W + 4;               // LDS words per key row (padded)
  static constexpr int KBYTES = NT * KROW * 4;     // K codes of one step
  static constexpr int VBYTES = 4096;              // V tile of one step
  static constexpr int SBYTES = 4 * G * NT * 2;    // ks, kb, vs, vb of one step
  static constexpr int BUF = KBYTES + VBYTES + SBYTES;
  static constexpr int SEGS = 4 * G;               // contiguous scale segments per step
  static constexpr int SEGB = NT * 2;              // bytes per segment
  static_assert(COLS % HG == 0, "query columns per wave must hold whole tokens");
};

// Number of query-token tiles of sequence s (0 for decode rows and empty rows).
__device__ __forceinline__ int prefill_tiles(const PrefillArgs& a, const int s, const int tokb) {
  const int ql = a.qsl[s + 1] - a.qsl[s];
  return ql > 1 ? (ql + tokb - 1) / tokb : 0;
}

template <int BITS, int GS, int HG>
__global__ __launch_bounds__(256, 2) void prefill_affine_d128(PrefillArgs a) {
  using P = PrefillCfg<BITS, GS, HG>;
  constexpr int D = P::D, G = P::G, NT = P::NT, TPL = P::TPL, NA = P::NA, NWS = P::NWS, W = P::W;
  constexpr int KW = BITS;  // K words a lane reads per sub-tile (4 MFMAs x 32 dims)

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;
  const int jj = lane >> 4;

  // ---- work item: blockIdx -> (sequence, tile, kv_head); later tiles (more keys) first
  __shared__ int tcum[kMaxSeqs + 1];
  if (tid == 0) {
    int c = 0;
    for (int s = 0; s < a.S; ++s) {
      tcum[s] = c;
      c += prefill_tiles(a, s, P::TOKB);
    }
    tcum[a.S] = c;
  }
  __syncthreads();
  const int ntiles = tcum[a.S];
  const int item = blockIdx.x / a.Hkv;
  if (item >= ntiles) return;
  const int kvh = blockIdx.x % a.Hkv;
  int s = 0;
  while (tcum[s + 1] <= item) ++s;
  const int nt_s = tcum[s + 1] - tcum[s];
  const int tile = nt_s - 1 - (item - tcum[s]);  // last tile first
  const int q0 = a.qsl[s];
  const int qlen = a.qsl[s + 1] - q0;
  const int kv_len = min(max(a.kv_lens[s], 0), a.max_blocks * a.bs);
  const int past = kv_len - qlen;  // query i sees keys [.., past + i]
  const int tok_lo = tile * P::TOKB;

  // ---- this lane's query columns: c = 16*ct + col of the wave's 32, token = c / HG, head = c % HG
  int ctok[2], chead[2], limit[2], start[2];
  bool cvalid[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int c = wv * P::COLS + 16 * ct + col;
    ctok[ct] = tok_lo + c / HG;
    chead[ct] = c % HG;
    cvalid[ct] = ctok[ct] < qlen;
    limit[ct] = min(past + ctok[ct], kv_len - 1);
    start[ct] = a.window > 0 ? max(0, past + ctok[ct] - a.window + 1) : 0;
    if (!cvalid[ct]) limit[ct] = -1;
  }
  // key range of the whole workgroup
  const int t_first = tok_lo, t_last = min(tok_lo + P::TOKB, qlen) - 1;
  const int k_hi = min(past + t_last, kv_len - 1);
  const int k_lo = a.window > 0 ? max(0, past + t_first - a.window + 1) : 0;
  const int step_lo = k_lo / NT, step_hi = k_hi >= 0 ? k_hi / NT : -1;

  // ---- query operands: MFMA w spans dims [32w, 32w + 32); lane group jj holds dims 32w + 8jj + slot(i)
  h16x8 qB[2][4];
  float qs[2][G];  // per-group sum of the query, in the 2^-24 units of the MFMA output
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const h16* qp = a.q + ((size_t)(q0 + (cvalid[ct] ? ctok[ct] : 0)) * a.Hq + (size_t)kvh * HG + chead[ct]) * D;
    float gs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const h16x8 raw = *reinterpret_cast<const h16x8*>(qp + 32 * w + 8 * jj);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const h16 v = cvalid[ct] ? raw[slot_perm<BITS>(i)] : (h16)0.0f;
        qB[ct][w][i] = v;
        gs[(32 * w) / GS] += (float)v;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float x = gs[g];
      x += __shfl_xor(x, 16, 64);
      x += __shfl_xor(x, 32, 64);
      qs[ct][g] = x * (1.0f / kTwo24);
    }
  }

  // ---- LDS: two step buffers [K rows (padded, MFMA order) | V tile | scales]
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][P::BUF];

  // Cooperative load of one step into registers: thread owns one 16-byte piece of K and of V,
  // and (threads < 8*G*... ) one piece of the scales.
  u32x4 rk, rv, rsc;
  auto load_step = [&](const int st) {
    const int pos0 = st * NT;
    const int blk_i = a.block_tables[(size_t)s * a.max_blocks + pos0 / a.bs];
    const int blk = (unsigned)blk_i < (unsigned)a.nb ? blk_i : 0;
    const int off = pos0 % a.bs;
    const size_t ph = (size_t)blk * a.Hkv + kvh;
    // K: NT rows x W words = 4 KiB; piece tid -> row tid / (W/4), words 4*(tid % (W/4)) ..
    const int krow = tid / (W / 4), kq = tid % (W / 4);
    rk = *reinterpret_cast<const u32x4*>(a.kc + (ph * a.bs + off + krow) * W + 4 * kq);
    // V: the step's 4 KiB tile, in HBM order
    const int RW = a.bs * BITS / 32;
    rv = *reinterpret_cast<const u32x4*>(a.vc + ph * D * RW + (off / NT) * D * 8 + 4 * tid);
    // scales: segment (arr, g) of NT halves; 16 bytes per thread
    constexpr int PER = P::SEGB / 16;
    if (tid < P::SEGS * PER) {
      const int seg = tid / PER, piece = tid % PER;
      const int arr = seg / G, g = seg % G;
      const h16* base = arr == 0 ? a.ks : arr == 1 ? a.kb : arr == 2 ? a.vs : a.vb;
      rsc = *reinterpret_cast<const u32x4*>(base + (ph * G + g) * a.bs + off + 8 * piece);
      // positions past kv_len may hold anything: zero their scales so that p = 0 contributes 0
      const int live = kv_len - (pos0 + 8 * piece);
      if (live < 8) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t keep = (2 * e < live ? 0x0000FFFFu : 0u) | (2 * e + 1 < live ? 0xFFFF0000u : 0u);
          rsc[e] &= keep;
        }
      }
    }
  };
  auto store_step = [&](const int buf) {
    uint8_t* L = lds[buf];
    // K: word w' of the row goes to position 4*jj + w for w' = 4w + jj (4-bit), so a lane's
    // four MFMA words are contiguous; 8-bit keeps word pairs: w' = 8w + 2jj + e -> 8jj + 2w + e
    const int krow = tid / (W / 4), kq = tid % (W / 4);
    uint32_t* kr = reinterpret_cast<uint32_t*>(L) + krow * P::KROW;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int wp = 4 * kq + e;
      int pos;
      if constexpr (BITS == 4) {
        pos = 4 * (wp % 4) + wp / 4;
      } else {
        pos = 8 * ((wp % 8) / 2) + 2 * (wp / 8) + wp % 2;
      }
      kr[pos] = rk[e];
    }
    reinterpret_cast<u32x4*>(L + P::KBYTES)[tid] = rv;
    constexpr int PER = P::SEGB / 16;
    if (tid < P::SEGS * PER) reinterpret_cast<u32x4*>(L + P::KBYTES + P::VBYTES)[tid] = rsc;
  };

  float m_run[2] = {-INFINITY, -INFINITY}, l_part[2] = {0.f, 0.f};
  float pb[2][G];
  f32x4 acc[2][8];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
#pragma unroll
    for (int g = 0; g < G; ++g) pb[ct][g] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[ct][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float sc_l2 = a.scale_log2 * kTwo24;

  if (step_lo <= step_hi) load_step(step_lo);
  for (int st = step_lo; st <= step_hi; ++st) {
    const int buf = (st - step_lo) & 1;
    __syncthreads();  // buffer `buf` is no longer read (step st - 2)
    store_step(buf);
    __syncthreads();
    if (st + 1 <= step_hi) load_step(st + 1);
    const int pos0 = st * NT;
    const int blk_i = a.block_tables[(size_t)s * a.max_blocks + pos0 / a.bs];
    if ((unsigned)blk_i >= (unsigned)a.nb) continue;  // an invalid page is skipped
    const uint8_t* L = lds[buf];
    const uint32_t* Kl = reinterpret_cast<const uint32_t*>(L);
    const uint32_t* Vl = reinterpret_cast<const uint32_t*>(L + P::KBYTES);
    const h16* Sl = reinterpret_cast<const h16*>(L + P::KBYTES + P::VBYTES);  // [arr][g][NT]

    // ---- S^T per sub-tile a and query tile ct, per quantization group
    float sc[2][NA][4];
#pragma unroll
    for (int at = 0; at < NA; ++at) {
      const int row = TPL * (col >> 2) + 4 * at + (col & 3);
      uint32_t kw[KW];
#pragma unroll
      for (int v = 0; v < KW / 4; ++v) {
        const u32x4 x = *reinterpret_cast<const u32x4*>(Kl + row * P::KROW + KW * jj + 4 * v);
#pragma unroll
        for (int e = 0; e < 4; ++e) kw[4 * v + e] = x[e];
      }
      f32x4 cg[2][G];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int g = 0; g < G; ++g) cg[ct][g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const h16x8 A = BITS == 4 ? unpack4(kw[w]) : unpack8(kw[2 * w], kw[2 * w + 1]);
        const int g = (32 * w) / GS;
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) cg[ct][g] = mfma16x16x32(A, qB[ct][w], cg[ct][g]);
      }
      // lane holds keys TPL*jj + 4*at + r (r = 0..3) of the step
      typedef h16 h16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[ct][at][r] = 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const h16x4 ks4 = *reinterpret_cast<const h16x4*>(Sl + (0 * G + g) * NT + TPL * jj + 4 * at);
        const h16x4 kb4 = *reinterpret_cast<const h16x4*>(Sl + (1 * G + g) * NT + TPL * jj + 4 * at);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            sc[ct][at][r] = fmaf(cg[ct][g][r], (float)ks4[r], fmaf((float)kb4[r], qs[ct][g], sc[ct][at][r]));
      }
    }

    // ---- mask (causal / window / kv_len) where the step is not fully visible to every column
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const bool full = pos0 >= start[ct] && pos0 + NT - 1 <= limit[ct];
      if (!full) {
#pragma unroll
        for (int at = 0; at < NA; ++at)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int p = pos0 + TPL * jj + 4 * at + r;
            if (p < start[ct] || p > limit[ct]) sc[ct][at][r] = -INFINITY;
          }
      }
    }

    // ---- online softmax per column (base 2), then O += P V per quantization group of dims
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      float tmax = -INFINITY;
#pragma unroll
      for (int at = 0; at < NA; ++at)
#pragma unroll
        for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, sc[ct][at][r]);
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float m_new = fmaxf(m_run[ct], tmax * sc_l2);
      if (m_new == -INFINITY) {  // nothing visible yet for this column
#pragma unroll
        for (int at = 0; at < NA; ++at)
#pragma unroll
          for (int r = 0; r < 4; ++r) sc[ct][at][r] = 0.f;
      } else {
        if (__any(m_new != m_run[ct])) {
          const float alpha = __builtin_amdgcn_exp2f(m_run[ct] - m_new);
          l_part[ct] *= alpha;
#pragma unroll
          for (int g = 0; g < G; ++g) pb[ct][g] *= alpha;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) acc[ct][dt] *= alpha;
          m_run[ct] = m_new;
        }
#pragma unroll
        for (int at = 0; at < NA; ++at)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float p = __builtin_amdgcn_exp2f(fmaf(sc[ct][at][r], sc_l2, -m_run[ct]));
            sc[ct][at][r] = p;
            l_part[ct] += p;
          }
      }
    }
#pragma unroll
    for (int w = 0; w < NWS; ++w) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        // V codes of this lane's 8 keys (TPL*jj + 8w ..) for the dim tiles of group g
        constexpr int DTG = 8 / G;  // dim tiles per quantization group
        h16x8 Av[DTG];
#pragma unroll
        for (int e = 0; e < DTG; ++e) {
          const int dt = g * DTG + e;
          typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
          const u32x2v x = *reinterpret_cast<const u32x2v*>(Vl + (16 * dt + col) * 8 + TPL * jj * BITS / 32);
          Av[e] = BITS == 4 ? unpack4(w == 0 ? x[0] : x[1]) : unpack8(x[0], x[1]);
        }
        const h16x8 vs8 = *reinterpret_cast<const h16x8*>(Sl + (2 * G + g) * NT + TPL * jj + 8 * w);
        const h16x8 vb8 = *reinterpret_cast<const h16x8*>(Sl + (3 * G + g) * NT + TPL * jj + 8 * w);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          h16x8 pB;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int j = 8 * w + i;  // unpacked value element i is token i of the word
            const float p = sc[ct][j >> 2][j & 3];
            pB[i] = (h16)(p * (float)vs8[i]);
            pb[ct][g] = fmaf(p, (float)vb8[i], pb[ct][g]);
          }
#pragma unroll
          for (int e = 0; e < DTG; ++e) acc[ct][g * DTG + e] = mfma16x16x32(Av[e], pB, acc[ct][g * DTG + e]);
        }
      }
    }
  }

  // ---- normalise and write: lane (col, jj) holds dims 16*dt + 4*jj + r of its column
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    float l = l_part[ct] + __shfl_xor(l_part[ct], 16, 64);
    l += __shfl_xor(l, 32, 64);
    float pbs[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float x = pb[ct][g] + __shfl_xor(pb[ct][g], 16, 64);
      pbs[g] = x + __shfl_xor(x, 32, 64);
    }
    if (!cvalid[ct]) continue;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    h16* op = a.out + ((size_t)(q0 + ctok[ct]) * a.Hq + (size_t)kvh * HG + chead[ct]) * D;
    typedef h16 h16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int d = 16 * dt + 4 * jj;
      const float b = pbs[d / GS];
      *reinterpret_cast<h16x4*>(op + d) = h16x4{(h16)((acc[ct][dt][0] * kTwo24 + b) * inv),
                                                (h16)((acc[ct][dt][1] * kTwo24 + b) * inv),
                                                (h16)((acc[ct][dt][2] * kTwo24 + b) * inv),
                                                (h16)((acc[ct][dt][3] * kTwo24 + b) * inv)};
    }
  }
}

}  // namespace emx
