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
//   K/V byte.  Splits of one (seq, kv_head) are merged by the last workgroup
//   to finish (atomic ticket), so there is a single launch.
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
  int* ws_cnt;                // [S, Hkv]  (zero between launches)
  int S, Hq, Hkv, bs, nb, max_blocks;
  float scale_log2;           // softmax_scale * log2(e)
  int window;                 // sliding window, 0 = off
  int tiles_per_split;
  int max_splits;
};

template <int BITS, int GS, int HG>
__global__ __launch_bounds__(256) void decode_affine_d128(DecodeArgs a) {
  constexpr int D = 128;
  constexpr int G = D / GS;
  constexpr int NCOL = HG * G;
  constexpr int W = D * BITS / 32;        // code words per token
  constexpr int KW = BITS == 4 ? 4 : 8;   // code words a lane holds per (token | dim row)
  static_assert(NCOL <= 16, "GQA group x quant groups must fit 16 MFMA columns");

  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int col = lane & 15;
  const int jj = lane >> 4;
  const bool col_ok = col < NCOL;
  const int hh = col_ok ? col % HG : 0;
  const int gg = col_ok ? col / HG : 0;

  int bid = blockIdx.x;
  const int kvh = bid % a.Hkv;
  bid /= a.Hkv;
  const int s = bid % a.S;
  const int split = bid / a.S;

  __shared__ float so[4][HG * D];
  __shared__ float sm[4][HG];
  __shared__ float sl[4][HG];
  __shared__ int s_last;

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

  // ---- query operand: lane holds dims 32*jj .. 32*jj+31 of head hh, group gg only.
  h16x8 qB[4];
  float qsum = 0.f;
  {
    const u32x4* qp = reinterpret_cast<const u32x4*>(a.q + ((size_t)s * a.Hq + (size_t)kvh * HG + hh) * D + 32 * jj);
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

  float m_run = -INFINITY;
  float l_part = 0.f;
  float pb = 0.f;
  f32x4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int rtok = 32 * (col >> 2) + (col & 3);  // token of MFMA row `col` in sub-tile 0
  const int RW = a.bs * BITS / 32;               // code words per V dim row

  for (int tile = t_begin + wv; tile < t_end; tile += 4) {
    const int tok0 = tile << 7;
    const int page = tok0 / a.bs;
    const int off = tok0 - page * a.bs;
    const int blk = a.block_tables[(size_t)s * a.max_blocks + page];
    if (blk < 0 || blk >= a.nb) continue;
    const size_t ph = (size_t)blk * a.Hkv + kvh;

    // ---- issue every load of the tile up front
    uint32_t kw[8][KW];
    {
      const uint32_t* kp = a.kc + (ph * a.bs + off) * W;
#pragma unroll
      for (int at = 0; at < 8; ++at) {
        const u32x4* p = reinterpret_cast<const u32x4*>(kp + (size_t)(rtok + 4 * at) * W + KW * jj);
#pragma unroll
        for (int v = 0; v < KW / 4; ++v) {
          u32x4 x = p[v];
          kw[at][4 * v + 0] = x[0];
          kw[at][4 * v + 1] = x[1];
          kw[at][4 * v + 2] = x[2];
          kw[at][4 * v + 3] = x[3];
        }
      }
    }
    uint32_t vw[8][KW];
    {
      const uint32_t* vp = a.vc + ph * D * RW + off * BITS / 32 + KW * jj;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const u32x4* p = reinterpret_cast<const u32x4*>(vp + (size_t)(16 * dt + col) * RW);
#pragma unroll
        for (int v = 0; v < KW / 4; ++v) {
          u32x4 x = p[v];
          vw[dt][4 * v + 0] = x[0];
          vw[dt][4 * v + 1] = x[1];
          vw[dt][4 * v + 2] = x[2];
          vw[dt][4 * v + 3] = x[3];
        }
      }
    }
    u32x4 ksr[4], kbr[4], vsr[4], vbr[4];
    {
      const size_t so_ = (ph * G + gg) * a.bs + off + 32 * jj;
      const u32x4* p0 = reinterpret_cast<const u32x4*>(a.ks + so_);
      const u32x4* p1 = reinterpret_cast<const u32x4*>(a.kb + so_);
      const u32x4* p2 = reinterpret_cast<const u32x4*>(a.vs + so_);
      const u32x4* p3 = reinterpret_cast<const u32x4*>(a.vb + so_);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ksr[i] = p0[i];
        kbr[i] = p1[i];
        vsr[i] = p2[i];
        vbr[i] = p3[i];
      }
    }
    const h16* ksv = reinterpret_cast<const h16*>(ksr);
    const h16* kbv = reinterpret_cast<const h16*>(kbr);
    const h16* vsv = reinterpret_cast<const h16*>(vsr);
    const h16* vbv = reinterpret_cast<const h16*>(vbr);

    // ---- S = Q K^T  (lane holds tokens 32*jj + 4*at + r)
    float sc[8][4];
#pragma unroll
    for (int at = 0; at < 8; ++at) {
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const h16x8 A = BITS == 4 ? unpack4(kw[at][w]) : unpack8(kw[at][2 * w], kw[at][2 * w + 1]);
        c = mfma16x16x32(A, qB[w], c);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 4 * at + r;
        float v = c[r] * ((float)ksv[t] * kTwo24) + (float)kbv[t] * qsum;
        if constexpr (G == 2) {
          v += __shfl_xor(v, HG, 64);
        } else if constexpr (G == 4) {
          v += __shfl_xor(v, HG, 64);
          v += __shfl_xor(v, 2 * HG, 64);
        }
        sc[at][r] = v;
      }
    }

    // ---- online softmax (base 2)
    float tmax = -INFINITY;
#pragma unroll
    for (int at = 0; at < 8; ++at) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int pos = tok0 + 32 * jj + 4 * at + r;
        const bool ok = pos >= start_k && pos < kv_len;
        const float x = ok ? sc[at][r] * a.scale_log2 : -INFINITY;
        sc[at][r] = x;
        tmax = fmaxf(tmax, x);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = exp2f(m_run - m_new);
    float psum = 0.f;
#pragma unroll
    for (int at = 0; at < 8; ++at) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = exp2f(sc[at][r] - m_new);
        sc[at][r] = p;
        psum += p;
      }
    }
    l_part = l_part * alpha + psum;
    pb *= alpha;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;
    m_run = m_new;

    // ---- PV
    h16x8 pB[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int j = 8 * w + slot_perm<BITS>(i);
        const float p = sc[j >> 2][j & 3];
        const bool live = col_ok && p != 0.f;
        pB[w][i] = live ? (h16)(p * (float)vsv[j]) : (h16)0.0f;
        pb += live ? p * (float)vbv[j] : 0.f;
      }
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const h16x8 A = BITS == 4 ? unpack4(vw[dt][w]) : unpack8(vw[dt][2 * w], vw[dt][2 * w + 1]);
        acc[dt] = mfma16x16x32(A, pB[w], acc[dt]);
      }
    }
  }

  // ---- per-wave epilogue -> LDS
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
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int old = atomicAdd(a.ws_cnt + unit, 1);
    s_last = (old == n_splits - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  // ---- last workgroup: merge all splits of this (seq, kv_head)
  const float* po = a.ws_o + unit * a.max_splits * (HG * D);
  const float* pml = a.ws_ml + unit * a.max_splits * (HG * 2);
  // weights per (split, head) staged in LDS (reuses `so`)
  float* wts = &so[0][0];  // [max_splits][HG], max_splits*HG <= 4*HG*D
  __shared__ float sL[HG];
  if (threadIdx.x < HG) {
    const int h = threadIdx.x;
    float M = -INFINITY;
    for (int sp = 0; sp < n_splits; ++sp) M = fmaxf(M, __builtin_nontemporal_load(pml + sp * HG * 2 + 2 * h));
    float L = 0.f;
    for (int sp = 0; sp < n_splits; ++sp) {
      const float m = __builtin_nontemporal_load(pml + sp * HG * 2 + 2 * h);
      const float f = m != -INFINITY ? exp2f(m - M) : 0.f;
      L += f * __builtin_nontemporal_load(pml + sp * HG * 2 + 2 * h + 1);
      wts[sp * HG + h] = f;
    }
    sL[h] = L;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < HG * D; i += 256) {
    const int h = i / D;
    float o = 0.f;
    for (int sp = 0; sp < n_splits; ++sp) {
      const float f = wts[sp * HG + h];
      if (f != 0.f) o += f * __builtin_nontemporal_load(po + (size_t)sp * HG * D + i);
    }
    const float L = sL[h];
    out[i] = (h16)(L > 0.f ? o / L : 0.f);
  }
  if (threadIdx.x == 0) a.ws_cnt[unit] = 0;
}

}  // namespace emx
