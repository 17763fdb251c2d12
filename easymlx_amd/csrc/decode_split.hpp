// Split-K single-token decode for the shapes outside the MFMA decode kernels:
// any head_dim that is a multiple of 32 up to 256, pages of a multiple of 8
// tokens, affine pages with group sizes that are multiples of 32, dense
// fp16/bf16/fp32 caches and FP8 pages, fp16/bf16/fp32 queries.
//
// Replaces the reference's per-(seq, q_head) serial key loop
// (lib/python/easymlx/operations/kernels/unified_attention.py:467-609, and the
// head-256 variants :611-775, :1103-1268) with its split-K form
// (page_attention.py:1718-2059: partitions, then a reduce).
//
//   decode_split: one wave per (sequence, kv head, <= 16 query heads, chunk of
//     kSplitChunk keys).  The query rows sit in LDS; per 64-key step lane L
//     takes key L: its K row 32 dims at a time through the cache's loader
//     (vector loads of the packed codes, the group's scale and bias; on affine
//     pages every piece of the row is loaded before the first is decoded) against
//     every query head of the GQA group, an online softmax in base 2 over the
//     wave, then lane L takes dims L, L + 64, .. and walks the 64 keys in
//     groups of 8 (one value word of 4-bit pages) with the probabilities from
//     LDS.  The chunk's (acc, m, l) go to the workspace.
//   decode_split_merge: one workgroup per (sequence, kv head, head chunk)
//     combines the chunks: O = sum 2^(m_c - M) acc_c, L = sum 2^(m_c - M) l_c,
//     out = O / L (page_attention.py:2006-2059); zero rows for empty sequences.
//     Every chunk's (m, l) goes to LDS in one round of loads and the weights
//     2^(m_c - M) are formed there, so each output value is one pass of
//     independent loads over the chunks.
//
// Chunks start on 64-key boundaries (the first one at the window start rounded
// down); keys outside [start_k, kv_len) or on pages with an invalid id are
// masked, as the reference skips block < 0.
#pragma once

#include "paged_generic.hpp"

namespace emx {

constexpr int kSplitChunk = 256;  // keys per wave

struct SplitArgs {
  const void* q;               // [S, Hq, D]
  void* out;                   // [S, Hq, D]
  const int32_t* block_tables; // [S, max_blocks]
  const int32_t* kv_lens;      // [S]
  float* part;                 // [S, Hkv * nhc, nchunk, hc, D + 2]: acc, then (m, l)
  int S, Hq, Hkv, D, bs, nb, max_blocks;
  int hc;                      // query heads per wave (<= 16)
  int nchunk;                  // chunk slots per (sequence, kv head): ceil(max_blocks * bs / kSplitChunk) + 1
  float scale_log2;
  int window;
};

__device__ __forceinline__ size_t split_part_index(const SplitArgs& a, int s, int y, int c) {
  return (((size_t)s * gridDim.y + y) * a.nchunk + c) * (size_t)a.hc * (a.D + 2);
}

// --- row loaders: 32 K dims of one key, 8 keys' values of one dim

template <typename Tag>
__device__ __forceinline__ void key32(const DenseKV<Tag>& kv, int blk, int off, int h, int d0, float (&x)[32]) {
  const typename Tag::T* p = kv.k + (((size_t)blk * kv.bs + off) * kv.Hkv + h) * kv.D + d0;
#pragma unroll
  for (int j = 0; j < 32; ++j) x[j] = to_f32(p[j]);
}
template <typename Tag>
__device__ __forceinline__ void val8(const DenseKV<Tag>& kv, int blk, int off8, int h, int d, float (&v)[8]) {
  const typename Tag::T* p = kv.v + (((size_t)blk * kv.bs + off8) * kv.Hkv + h) * kv.D + d;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = to_f32(p[(size_t)j * kv.Hkv * kv.D]);
}

template <int BITS>
__device__ __forceinline__ void key32(const AffineKV<BITS>& kv, int blk, int off, int h, int d0, float (&x)[32]) {
  constexpr int PW = 32 / BITS;
  const size_t ph = (size_t)blk * kv.Hkv + h;
  const uint32_t* w = kv.kc + (ph * kv.bs + off) * (kv.D / PW) + d0 / PW;
  const size_t si = (ph * (kv.D / kv.gs) + d0 / kv.gs) * kv.bs + off;  // 32 dims lie in one group
  const float sc = (float)kv.ks[si], bi = (float)kv.kb[si];
#pragma unroll
  for (int i = 0; i < BITS; ++i) {
    const uint32_t x4 = w[i];
#pragma unroll
    for (int j = 0; j < PW; ++j) x[PW * i + j] = fmaf(sc, (float)((x4 >> (j * BITS)) & ((1u << BITS) - 1u)), bi);
  }
}
template <int BITS>
__device__ __forceinline__ void val8(const AffineKV<BITS>& kv, int blk, int off8, int h, int d, float (&v)[8]) {
  constexpr int PW = 32 / BITS;
  const size_t ph = (size_t)blk * kv.Hkv + h;
  const size_t si = (ph * (kv.D / kv.gs) + d / kv.gs) * kv.bs + off8;
  const u32x4 s4 = *reinterpret_cast<const u32x4*>(kv.vs + si);  // 8 fp16 scales (off8 % 8 == 0)
  const u32x4 b4 = *reinterpret_cast<const u32x4*>(kv.vb + si);
#pragma unroll
  for (int k = 0; k < 8 / PW; ++k) {
    const uint32_t w = kv.vc[v_word_index<BITS>(ph, off8 + PW * k, d, kv.D, kv.bs)];
#pragma unroll
    for (int j = 0; j < PW; ++j) {
      const int t = PW * k + j;
      const float sc = (float)__builtin_bit_cast(h16, (uint16_t)(s4[t >> 1] >> (16 * (t & 1))));
      const float bi = (float)__builtin_bit_cast(h16, (uint16_t)(b4[t >> 1] >> (16 * (t & 1))));
      v[t] = fmaf(sc, (float)((w >> v_shift<BITS>(t)) & ((1u << BITS) - 1u)), bi);
    }
  }
}

// Affine pages, loads apart from their use: the raw words, scale and bias of one 32-dim K
// piece (key32 split in two, so that every piece's loads can leave before the first is
// decoded).
template <int BITS>
struct KPieceRaw {
  uint32_t w[BITS];
  h16 sc, bi;
};
template <int BITS>
__device__ __forceinline__ void key32_load(const AffineKV<BITS>& kv, int blk, int off, int h, int d0,
                                           KPieceRaw<BITS>& r) {
  constexpr int PW = 32 / BITS;
  const size_t ph = (size_t)blk * kv.Hkv + h;
  const uint32_t* w = kv.kc + (ph * kv.bs + off) * (kv.D / PW) + d0 / PW;
  const size_t si = (ph * (kv.D / kv.gs) + d0 / kv.gs) * kv.bs + off;
#pragma unroll
  for (int i = 0; i < BITS; ++i) r.w[i] = w[i];
  r.sc = kv.ks[si];
  r.bi = kv.kb[si];
}
template <int BITS>
__device__ __forceinline__ void key32_decode(const KPieceRaw<BITS>& r, float (&x)[32]) {
  constexpr int PW = 32 / BITS;
  const float sc = (float)r.sc, bi = (float)r.bi;
#pragma unroll
  for (int i = 0; i < BITS; ++i)
#pragma unroll
    for (int j = 0; j < PW; ++j) x[PW * i + j] = fmaf(sc, (float)((r.w[i] >> (j * BITS)) & ((1u << BITS) - 1u)), bi);
}
template <typename KV>
struct AffineBits {
  static constexpr int value = 0;
};
template <int BITS>
struct AffineBits<AffineKV<BITS>> {
  static constexpr int value = BITS;
};

__device__ __forceinline__ void key32(const Fp8KV& kv, int blk, int off, int h, int d0, float (&x)[32]) {
  const uint32_t* p = reinterpret_cast<const uint32_t*>(kv.k + (((size_t)blk * kv.bs + off) * kv.Hkv + h) * kv.D + d0);
  const float sc = kv.ks[blk];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t w = p[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) x[4 * i + j] = e4m3_to_f32((w >> (8 * j)) & 0xFFu) * sc;
  }
}
__device__ __forceinline__ void val8(const Fp8KV& kv, int blk, int off8, int h, int d, float (&v)[8]) {
  const uint8_t* p = kv.v + (((size_t)blk * kv.bs + off8) * kv.Hkv + h) * kv.D + d;
  const float sc = kv.vs[blk];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = e4m3_to_f32(p[(size_t)j * kv.Hkv * kv.D]) * sc;
}

// Loaders this kernel can use: 32 K dims must lie in one quantization group.
template <typename Tag>
__host__ __device__ inline bool split_kv_ok(const DenseKV<Tag>&) { return true; }
template <int BITS>
__host__ __device__ inline bool split_kv_ok(const AffineKV<BITS>& kv) { return kv.gs % 32 == 0; }
__host__ __device__ inline bool split_kv_ok(const Fp8KV&) { return true; }

// grid (nchunk, Hkv * head chunks, S), 64 threads; dynamic LDS: q rows [hc][D], p [hc][64].
// MAXH >= hc: the per-head registers (scores, maxima, sums, 4 accumulators per head) are
// sized by it, so a GQA group of 4 holds a quarter of what 16 heads need (more waves in flight).
template <typename QT, typename KV, int MAXH>
__global__ __launch_bounds__(64) void decode_split(SplitArgs a, KV kv) {
  constexpr int MAXD = 256;
  extern __shared__ float dyn_lds[];
  const int lane = threadIdx.x;
  const int c = blockIdx.x, s = blockIdx.z;
  const int HG = a.Hq / a.Hkv, nhc = (HG + a.hc - 1) / a.hc;
  const int kvh = blockIdx.y / nhc, h0 = (blockIdx.y % nhc) * a.hc;
  const int nh = min(a.hc, HG - h0), D = a.D;
  const int kl = max(min(a.kv_lens[s], a.max_blocks * a.bs), 0);
  const int start_k = a.window > 0 ? max(0, kl - a.window) : 0;
  const int c0 = (start_k & ~63) + c * kSplitChunk;
  const int c1 = min(kl, c0 + kSplitChunk);
  float* part = a.part + split_part_index(a, s, blockIdx.y, c);
  if (c0 >= kl) return;  // no chunk here (the merge reads only the chunks that exist)

  float* qs = dyn_lds;          // [hc][D]
  float* ps = dyn_lds + a.hc * D;  // [hc][64]
  const QT* q = reinterpret_cast<const QT*>(a.q) + ((size_t)s * a.Hq + (size_t)kvh * HG + h0) * D;
  for (int i = lane; i < nh * D; i += 64) qs[i] = to_f32(q[i]);
  __syncthreads();

  float m[MAXH], l[MAXH], acc[MAXH][MAXD / 64];
#pragma unroll
  for (int h = 0; h < MAXH; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int i = 0; i < MAXD / 64; ++i) acc[h][i] = 0.f;
  }
  const int32_t* bt = a.block_tables + (size_t)s * a.max_blocks;

  for (int base = c0; base < c1; base += 64) {
    // ---- scores: lane L takes key base + L
    const int pos = base + lane;
    const bool in = pos >= start_k && pos < c1;
    const int blk = pos < kl ? bt[pos / a.bs] : -1;
    const bool ok = in && blk >= 0 && blk < a.nb;
    float sc[MAXH];
#pragma unroll
    for (int h = 0; h < MAXH; ++h) sc[h] = 0.f;
    auto dot32 = [&](const float (&x)[32], const int d0) {
#pragma unroll
      for (int h = 0; h < MAXH; ++h) {
        if (h < nh) {
          const float4* qv = reinterpret_cast<const float4*>(qs + h * D + d0);
          float t = sc[h];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float4 q4 = qv[j];
            t = fmaf(q4.x, x[4 * j], t);
            t = fmaf(q4.y, x[4 * j + 1], t);
            t = fmaf(q4.z, x[4 * j + 2], t);
            t = fmaf(q4.w, x[4 * j + 3], t);
          }
          sc[h] = t;
        }
      }
    };
    if constexpr (AffineBits<KV>::value > 0) {
      // every piece's loads first (one round trip for the key), then decode and dot
      constexpr int BITS = AffineBits<KV>::value;
      const int off = pos % a.bs;
      KPieceRaw<BITS> raw[MAXD / 32];
      if (ok) {
#pragma unroll
        for (int pc = 0; pc < MAXD / 32; ++pc)
          if (32 * pc < D) key32_load(kv, blk, off, kvh, 32 * pc, raw[pc]);
#pragma unroll
        for (int pc = 0; pc < MAXD / 32; ++pc) {
          if (32 * pc < D) {
            float x[32];
            key32_decode(raw[pc], x);
            dot32(x, 32 * pc);
          }
        }
      }
    } else if (ok) {
      const int off = pos % a.bs;
      for (int d0 = 0; d0 < D; d0 += 32) {
        float x[32];
        key32(kv, blk, off, kvh, d0, x);
        dot32(x, d0);
      }
    }
    // ---- online softmax (base 2) over the wave, one head at a time
#pragma unroll
    for (int h = 0; h < MAXH; ++h) {
      if (h < nh) {
        const float x = ok ? sc[h] * a.scale_log2 : -INFINITY;
        const float m_new = fmaxf(m[h], wave_max(x));
        float p = 0.f, alpha = 1.f;
        if (m_new != -INFINITY) {
          p = ok ? exp2f(x - m_new) : 0.f;
          alpha = exp2f(m[h] - m_new);
        }
        l[h] = l[h] * alpha + wave_sum(p);
        m[h] = m_new;
        ps[h * 64 + lane] = p;
#pragma unroll
        for (int i = 0; i < MAXD / 64; ++i) acc[h][i] *= alpha;
      }
    }
    __syncthreads();
    // ---- values: lane takes dims lane + 64 i; keys in groups of 8 (one page each)
    // (the page of key group t8 is lane t8's page from the score pass, not a second table read)
    const int nk = min(64, c1 - base);
    auto pv8 = [&](const float (&v)[8], const int t8, const int i) {
#pragma unroll
      for (int h = 0; h < MAXH; ++h) {
        if (h < nh) {
          float t = acc[h][i];
#pragma unroll
          for (int j = 0; j < 8; ++j) t = fmaf(ps[h * 64 + t8 + j], v[j], t);
          acc[h][i] = t;
        }
      }
    };
    auto group_page = [&](const int t8) {  // -1: no live page (its probabilities are zero)
      const int b = __builtin_amdgcn_readlane(pos < kl ? blk : -1, t8);
      return b >= 0 && b < a.nb ? b : -1;
    };
    for (int t8 = 0; t8 < nk; t8 += 8) {
      const int b = group_page(t8);
      if (b < 0) continue;
      const int off8 = (base + t8) % a.bs;
#pragma unroll
      for (int i = 0; i < MAXD / 64; ++i) {
        const int d = lane + 64 * i;
        if (d < D) {
          float v[8];
          val8(kv, b, off8, kvh, d, v);
          pv8(v, t8, i);
        }
      }
    }
    __syncthreads();
  }

  // ---- this chunk's partial state
#pragma unroll
  for (int h = 0; h < MAXH; ++h) {
    if (h < nh) {
      float* ph = part + (size_t)h * (D + 2);
#pragma unroll
      for (int i = 0; i < MAXD / 64; ++i) {
        const int d = lane + 64 * i;
        if (d < D) ph[d] = acc[h][i];
      }
      if (lane == 0) {
        ph[D] = m[h];
        ph[D + 1] = l[h];
      }
    }
  }
}

// grid (Hkv * head chunks, S), 256 threads
template <typename QT>
__global__ __launch_bounds__(256) void decode_split_merge(SplitArgs a) {
  const int s = blockIdx.y;
  const int HG = a.Hq / a.Hkv, nhc = (HG + a.hc - 1) / a.hc;
  const int kvh = blockIdx.x / nhc, h0 = (blockIdx.x % nhc) * a.hc;
  const int nh = min(a.hc, HG - h0), D = a.D;
  const int kl = max(min(a.kv_lens[s], a.max_blocks * a.bs), 0);
  const int start_k = a.window > 0 ? max(0, kl - a.window) : 0;
  const int first = start_k & ~63;
  const int nc = kl > first ? (kl - first + kSplitChunk - 1) / kSplitChunk : 0;
  QT* out = reinterpret_cast<QT*>(a.out) + ((size_t)s * a.Hq + (size_t)kvh * HG + h0) * D;
  const float* part = a.part + (((size_t)s * gridDim.x + blockIdx.x) * a.nchunk) * (size_t)a.hc * (D + 2);
  const size_t stride = (size_t)a.hc * (D + 2);
  // every chunk's (m, l) into LDS at once (one round of loads), then each head's maximum and
  // the chunk weights 2^(m_c - M) there; the per-dim sums below are independent loads
  extern __shared__ float mlw[];  // [hc][nchunk]: m, then the weight; [hc][nchunk]: l; [hc]: L
  float* wt = mlw;
  float* lt = mlw + a.hc * a.nchunk;
  float* Lh = lt + a.hc * a.nchunk;
  for (int e = threadIdx.x; e < nh * nc; e += 256) {
    const int h = e / nc, c = e % nc;
    const float* ph = part + c * stride + (size_t)h * (D + 2);
    wt[h * a.nchunk + c] = ph[D];
    lt[h * a.nchunk + c] = ph[D + 1];
  }
  __syncthreads();
  if (threadIdx.x < nh) {
    const int h = threadIdx.x;
    float M = -INFINITY;
    for (int c = 0; c < nc; ++c) M = fmaxf(M, wt[h * a.nchunk + c]);
    float L = 0.f;
    for (int c = 0; c < nc; ++c) {
      const float mc = wt[h * a.nchunk + c];
      const float f = M == -INFINITY || mc == -INFINITY ? 0.f : exp2f(mc - M);  // a chunk without a live key: 0
      wt[h * a.nchunk + c] = f;
      L = fmaf(f, lt[h * a.nchunk + c], L);
    }
    Lh[h] = L;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < nh * D; e += 256) {
    const int h = e / D, d = e % D;
    const float* ph = part + (size_t)h * (D + 2) + d;
    const float* w = wt + h * a.nchunk;
    float O = 0.f;
    int c = 0;
    for (; c + 4 <= nc; c += 4) {
      const float x0 = ph[c * stride], x1 = ph[(c + 1) * stride], x2 = ph[(c + 2) * stride], x3 = ph[(c + 3) * stride];
      O = fmaf(w[c], x0, O);
      O = fmaf(w[c + 1], x1, O);
      O = fmaf(w[c + 2], x2, O);
      O = fmaf(w[c + 3], x3, O);
    }
    for (; c < nc; ++c) O = fmaf(w[c], ph[c * stride], O);
    const float L = Lh[h];
    from_f32(L > 0.f ? O / L : 0.f, out + (size_t)h * D + d);
  }
}

}  // namespace emx
