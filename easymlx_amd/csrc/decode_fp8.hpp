// Single-token paged decode over an FP8 (E4M3) page cache with one fp32 scale
// per page, head_dim 128, MFMA, split-K.
//
// Replaces the reference's FP8 decode loop (lib/python/easymlx/operations/
// kernels/unified_attention.py:892-939 dequantization inside the per-query key
// loop :467-609) for caches laid out as the reference keeps them:
// key/value [nb, bs, Hkv, 128] uint8, k_scale/v_scale [nb] fp32.
//
// Work decomposition: as the affine split-K decode (decode_affine.hpp): work
// items of 32 tokens of one (sequence, kv head) unit, contiguous item ranges per
// wave, partials of cut units merged in-kernel by the last arrival.  An item
// never crosses a page (page_size % 32 == 0), so one key scale and one value
// scale cover it.
//
// Exact fp16 operands: an E4M3 byte b placed as a 16-bit value
// (b + (b & 0x80)) << 7 is the fp16 whose sign is b's sign and whose exponent /
// mantissa fields are b's shifted up by seven bits, i.e. dec(b) * 2^-8 for every
// code (normals: exponent bias 15 vs 7; sub-normals: mantissa * 2^-24 * 2^7
// = m * 2^-17 = m * 2^-9 * 2^-8), and 0x7F gives 1.875 = 480 * 2^-8, the
// reference decoder's value for that code.  The 2^8 and the page scale are
// applied in fp32 after each MFMA.
//
// Per item (lane l: i = l % 16, jj = l / 16)
//   QK^T : 2 token sub-tiles x 4 dim slices of v_mfma_f32_16x16x32_f16.
//          A row i of sub-tile at = token 16 at + i; lane jj holds that token's
//          dims 16 jj .. 16 jj + 15 and 64 + 16 jj .. 64 + 16 jj + 15 (two
//          16-byte loads; a load instruction reads 64 contiguous bytes of each
//          row), slices 0-1 the first half, 2-3 the second.  B column h = query
//          head h of the GQA group (zero beyond HG).  Output rows 4 jj + r:
//          lane (h, jj) holds the scores of tokens 16 at + 4 jj + r.
//   softmax: online, base 2, fp32.
//   PV   : O = V^T P on 8 dim sub-tiles.  The k slot 8 jj + e is token
//          16 (e / 4) + 4 jj + e % 4 -- exactly the eight scores lane (h, jj)
//          already holds, so P needs no lane exchange.  A lane (i, jj) loads
//          dims 8 i .. 8 i + 7 of those eight tokens (8-byte loads; a load
//          instruction covers four whole 128-byte rows) and sub-tile b takes
//          byte b: row i of sub-tile b is dim 8 i + b.  The output rows 4 jj + r
//          of sub-tile b are dims 32 jj + 8 r + b: lane (h, jj) ends with head
//          h's dims 32 jj .. 32 jj + 31.
#pragma once

#include "decode_affine.hpp"

namespace emx {

constexpr int kFp8DecodeNT = 32;  // tokens per work item


struct Fp8Loads {
  uint32_t k[2][8];  // [sub-tile][dword]: 32 bytes of one token
  uint32_t v[8][2];  // [token slot e][dword]: 8 bytes of one token
};

struct Fp8Rsrc {
  __amdgpu_buffer_rsrc_t k, v;
};

// Rows of tokens off .. off + 31 of (page blk, kv head kvh); live = false gives
// empty descriptors (loads return zeros and touch nothing).
__device__ __forceinline__ Fp8Rsrc fp8_rsrc(const DecodeArgs& a, const int blk, const int kvh, const int off,
                                            const bool live) {
  const int RS = a.Hkv * 128;
  const size_t base = ((size_t)blk * a.bs + off) * RS + (size_t)kvh * 128;
  const int bytes = live ? 31 * RS + 128 : 0;
  Fp8Rsrc r;
  r.k = uniform_rsrc(reinterpret_cast<const uint8_t*>(a.kc) + base, bytes);
  r.v = uniform_rsrc(reinterpret_cast<const uint8_t*>(a.vc) + base, bytes);
  return r;
}

__device__ __forceinline__ void fp8_issue(Fp8Loads& L, const Fp8Rsrc& rs, const int RS, const int lk,
                                          const int lv) {
  const int rs_ = __builtin_amdgcn_readfirstlane(RS);
#pragma unroll
  for (int at = 0; at < 2; ++at) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rs.k, lk + 64 * h, at * 16 * rs_, kLoadAux);
#pragma unroll
      for (int c = 0; c < 4; ++c) L.k[at][4 * h + c] = x[c];
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(rs.v, lv, (16 * (e >> 2) + (e & 3)) * rs_, kLoadAux);
    L.v[e][0] = x[0];
    L.v[e][1] = x[1];
  }
}

// One 32-token item.  kf = softmax_scale * log2(e) * 2^8 * key page scale,
// vf = 2^8 * value page scale.
template <int HG>
__device__ __forceinline__ void fp8_compute(const Fp8Loads& L, const bool full, const int jj, const int tok_base,
                                            const int start_k, const int kv_len, const h16x8 (&qB)[4],
                                            const float kf, const float vf, float& m_run, float& l_part,
                                            f32x4 (&acc)[8]) {
  float sc[2][4];
#pragma unroll
  for (int at = 0; at < 2; ++at) {
    f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t d0 = L.k[at][2 * w], d1 = L.k[at][2 * w + 1];
      const h16x8 A = as_h8(e4m3x2_to_h16x2(__builtin_amdgcn_perm(0u, d0, 0x0C010C00u)),
                            e4m3x2_to_h16x2(__builtin_amdgcn_perm(0u, d0, 0x0C030C02u)),
                            e4m3x2_to_h16x2(__builtin_amdgcn_perm(0u, d1, 0x0C010C00u)),
                            e4m3x2_to_h16x2(__builtin_amdgcn_perm(0u, d1, 0x0C030C02u)));
      c = mfma16x16x32(A, qB[w], c);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[at][r] = c[r] * kf;
  }
  if (!full) {
#pragma unroll
    for (int at = 0; at < 2; ++at) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int pos = tok_base + 16 * at + 4 * jj + r;
        if (pos < start_k || pos >= kv_len) sc[at][r] = -INFINITY;
      }
    }
  }
  float tmax = -INFINITY;
#pragma unroll
  for (int at = 0; at < 2; ++at) {
#pragma unroll
    for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, sc[at][r]);
  }
  tmax = rows4_max(tmax);
  const float m_new = fmaxf(m_run, tmax);
  if (__any(m_new != m_run)) {
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    l_part *= alpha;
#pragma unroll
    for (int b = 0; b < 8; ++b) acc[b] *= alpha;
    m_run = m_new;
  }
  h16x8 pB;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float p = __builtin_amdgcn_exp2f(sc[e >> 2][e & 3] - m_run);
    l_part += p;
    pB[e] = (h16)p;
  }
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    constexpr uint32_t kSel = 0x0C000C00u;
    const uint32_t sel = kSel | (uint32_t)(b & 3) | ((uint32_t)(4 + (b & 3)) << 16);
    h16x8 A;
    uint32_t wv[4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
      wv[m] = e4m3x2_to_h16x2(__builtin_amdgcn_perm(L.v[2 * m + 1][b >> 2], L.v[2 * m][b >> 2], sel));
    A = as_h8(wv[0], wv[1], wv[2], wv[3]);
    const f32x4 t = mfma16x16x32(A, pB, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[b][r] = fmaf(t[r], vf, acc[b][r]);
  }
}

// The kernel body as workgroup `bid` of `nblocks` (a grid of its own, or the
// decode part of a mixed batch's single launch, unified_fp8); a.num_waves is the
// number of waves the ranges are split over.
template <int HG>
__device__ __forceinline__ void decode_fp8_body(const DecodeArgs& a, const int bid, const int nblocks) {
  constexpr int D = 128, NT = kFp8DecodeNT;
  static_assert(HG >= 1 && HG <= 16, "GQA group must fit 16 MFMA columns");

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int jj = lane >> 4;
  const bool col_ok = col < HG;

  // LDS, carved from the shared arena
  constexpr int oCum = 0, oKvl = lds_next(oCum, 4 * (kMaxSeqs + 1)), oQrw = lds_next(oKvl, 4 * kMaxSeqs);
  constexpr int oXst = lds_next(oQrw, 4 * kMaxSeqs), oEnd = lds_next(oXst, 4 * 4 * HG * D);
  static_assert(oEnd <= kArenaBytes, "LDS arena too small");
  int(&cum)[kMaxSeqs + 1] = lds_at<int[kMaxSeqs + 1]>(oCum);
  int(&kvl)[kMaxSeqs] = lds_at<int[kMaxSeqs]>(oKvl);
  int(&qrw)[kMaxSeqs] = lds_at<int[kMaxSeqs]>(oQrw);
  float(&xst)[4][HG * D] = lds_at<float[4][HG * D]>(oXst);  // per wave: a partial, head-major
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
  auto uru = [](int v) { return __builtin_amdgcn_readfirstlane(v); };
  const long long I = (long long)Hkv * uru(cum[S]);
  const int NW = (int)min((long long)a.num_waves, I);
  const int W = bid * 4 + wv;
  if (W >= NW) return;
  const long long g0 = ((long long)W * I) / NW;
  const long long g1 = ((long long)(W + 1) * I) / NW;

  auto seq_of = [&](long long g, int s_from) {
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

  // page id of every item of the range, one item per lane (64 items per chunk)
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

  // query operand: lane (h, jj) holds dims 16 jj .. 16 jj + 15 and 64 + 16 jj .. of head h
  u32x4 qraw[4];
  auto issue_q = [&](int seq, int kh) {
    const u32x4* qp = reinterpret_cast<const u32x4*>(
        a.q + ((size_t)qrw[seq] * a.Hq + (size_t)kh * HG + (col_ok ? col : 0)) * D + 16 * jj);
#pragma unroll
    for (int i = 0; i < 4; ++i) qraw[i] = qp[(i & 1) + 8 * (i >> 1)];
  };
  h16x8 qB[4];
  auto build_q = [&]() {
#pragma unroll
    for (int w = 0; w < 4; ++w) qB[w] = col_ok ? __builtin_bit_cast(h16x8, qraw[w]) : h16x8{};
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

  const int RS = Hkv * D;
  const int lk = col * RS + 16 * jj;
  const int lv = 4 * jj * RS + 8 * col;
  const float kl2 = a.scale_log2 * 256.0f;

  int tb = (it_lo + j) * NT;
  int blk = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(blkv, 0));
  bool bok = (unsigned)blk < (unsigned)a.nb;
  Fp8Loads bufA, bufB;
  fp8_issue(bufA, fp8_rsrc(a, bok ? blk : 0, kvh, tb % a.bs, true), RS, lk, lv);
  float ksc = bok ? a.kps[blk] : 0.f, vsc = bok ? a.vps[blk] : 0.f;
  build_q();

  float m_run = -INFINITY, l_part = 0.f;
  f32x4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  long long unit_first = (long long)Hkv * cum[s] + (long long)kvh * n_s;

  auto step = [&](Fp8Loads& cur, Fp8Loads& nxt, const long long g) {
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
    const bool bok1 = (unsigned)blk1 < (unsigned)a.nb;
    // issued on every path (an empty descriptor reads nothing), so the wait
    // before this item's compute leaves them in flight
    fp8_issue(nxt, fp8_rsrc(a, bok1 ? blk1 : 0, kvh1, tb1 % a.bs, has_next), RS, lk, lv);
    const float ksc1 = has_next && bok1 ? a.kps[blk1] : 0.f;
    const float vsc1 = has_next && bok1 ? a.vps[blk1] : 0.f;
    if (has_next && unit_end) issue_q(s1, kvh1);

    // an invalid page is skipped like the reference's Metal kernel
    if (bok) {
      const bool full = tb >= start_k && tb + NT <= kv_len;
      // the page scales enter their products here, at the item that uses them: a product hoisted
      // to where the scale was loaded (the previous item) would wait there for every load in
      // flight, the next item's pages included
      float ks_ = ksc, vs_ = vsc;
      asm volatile("" : "+v"(ks_), "+v"(vs_));
      fp8_compute<HG>(cur, full, jj, tb, start_k, kv_len, qB, kl2 * ks_, 256.0f * vs_, m_run, l_part, acc);
    }

    if (unit_end) {
      float l = l_part + __shfl_xor(l_part, 16, 64);
      l += __shfl_xor(l, 32, 64);
      const bool whole = unit_first >= g0 && unit_first + n_s <= g1;
      if (whole) {
        if (col_ok) {
          h16* out = a.out + ((size_t)qrw[s] * a.Hq + (size_t)kvh * HG + col) * D + 32 * jj;
          const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            h16x8 o;
#pragma unroll
            for (int b = 0; b < 8; ++b) o[b] = (h16)(acc[b][r] * inv);
            *reinterpret_cast<h16x8*>(out + 8 * r) = o;
          }
        }
      } else {
        const PieceInfo pi = piece_info<HG>(a, W, s * Hkv + kvh, unit_first, n_s, I, NW);
        // the partial goes through the wave's LDS slot so that every store
        // instruction writes 512 contiguous bytes (whole lines, not scattered pieces)
        float* xw = xst[wv];
        if (col_ok) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int c = 0; c < 2; ++c)
              *reinterpret_cast<f32x4*>(xw + col * D + 32 * jj + 8 * r + 4 * c) =
                  f32x4{acc[4 * c][r], acc[4 * c + 1][r], acc[4 * c + 2][r], acc[4 * c + 3][r]};
          if (jj == 0)
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f32x2{m_run, l}), pi.rm, col * 8,
                                                  pi.me * HG * 8, kCoherent);
        }
        store_partial_lds<HG>(xw, pi.ro, pi.me, lane);
        merge_pieces<HG>(a, pi, s * Hkv + kvh, qrw[s], kvh, lane);
      }
      m_run = -INFINITY;
      l_part = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (has_next) {
        unit_first = g + 1;
        build_q();
      }
    }

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
    bok = bok1;
    ksc = ksc1;
    vsc = vsc1;
  };
  for (long long g = g0; g < g1; g += 2) {
    step(bufA, bufB, g);
    if (g + 1 >= g1) break;
    step(bufB, bufA, g + 1);
  }
}

template <int HG>
__global__ __launch_bounds__(256, 2) void decode_fp8_d128(DecodeArgs a) {
  decode_fp8_body<HG>(a, blockIdx.x, gridDim.x);
}

}  // namespace emx
