// Ragged / causal paged attention for any head_dim <= 256 and any page size.
//
// Semantics follow the reference's generic Metal kernel
// (lib/python/easymlx/operations/kernels/unified_attention.py:290-465):
// sequence lookup by query_start_loc, causal limit
// max_k = min(kv_len-1, (kv_len - q_len) + q_pos), optional sliding window,
// pages with an invalid block id skipped, zero rows for empty sequences.
//
// One wavefront per (token, kv_head, chunk of <=16 query heads): every K/V
// element read is shared by the whole GQA group.  Keys are processed 64 at a
// time (one per lane for QK^T, then one dim per lane for PV with the
// probabilities staged in LDS).  This is the path for prefill rows, odd
// shapes and unquantized caches; single-token decode over affine pages with
// head_dim 128 uses decode_affine_d128.
#pragma once

#include "common.hpp"

namespace emx {

struct GenericArgs {
  const void* q;                 // [T, Hq, D] (q dtype)
  void* out;                     // [T, Hq, D]
  const int32_t* block_tables;   // [S, max_blocks]
  const int32_t* kv_lens;        // [S]
  const int32_t* qsl;            // [S+1]
  int T, S, Hq, Hkv, D, bs, nb, max_blocks;
  float scale_log2;
  int window;
  int decode;                    // 1: token i is sequence i (query_start_loc ignored)
};

// Dense cache in the reference layout [nb, bs, Hkv, D].
template <typename Tag>
struct DenseKV {
  typedef typename Tag::T T;
  const T* k;
  const T* v;
  int Hkv, D, bs;
  __device__ __forceinline__ float key(int blk, int off, int h, int d) const {
    return to_f32(k[(((size_t)blk * bs + off) * Hkv + h) * D + d]);
  }
  __device__ __forceinline__ float val(int blk, int off, int h, int d) const {
    return to_f32(v[(((size_t)blk * bs + off) * Hkv + h) * D + d]);
  }
};

// Affine pages: K codes [nb, Hkv, bs, D*b/32], V codes [nb, Hkv, D, bs*b/32],
// scales/biases [nb, Hkv, D/gs, bs] fp16.
template <int BITS>
struct AffineKV {
  const uint32_t* kc;
  const h16 *ks, *kb;
  const uint32_t* vc;
  const h16 *vs, *vb;
  int Hkv, D, bs, gs;
  __device__ __forceinline__ float key(int blk, int off, int h, int d) const {
    constexpr int PW = 32 / BITS;
    const size_t ph = (size_t)blk * Hkv + h;
    const uint32_t w = kc[(ph * bs + off) * (D / PW) + d / PW];
    const float q = (float)((w >> ((d % PW) * BITS)) & ((1u << BITS) - 1u));
    const size_t si = (ph * (D / gs) + d / gs) * bs + off;
    return (float)ks[si] * q + (float)kb[si];
  }
  __device__ __forceinline__ float val(int blk, int off, int h, int d) const {
    constexpr int PW = 32 / BITS;
    const size_t ph = (size_t)blk * Hkv + h;
    const uint32_t w = vc[v_word_index<BITS>(ph, off, d, D, bs)];
    const float q = (float)((w >> v_shift<BITS>(off % PW)) & ((1u << BITS) - 1u));
    const size_t si = (ph * (D / gs) + d / gs) * bs + off;
    return (float)vs[si] * q + (float)vb[si];
  }
};

// FP8 E4M3 cache in the reference layout [nb, bs, Hkv, D] uint8 with one fp32
// scale per page for K and V (unified_attention.py:892-939: dec(code) * scale[block]).
struct Fp8KV {
  const uint8_t* k;
  const uint8_t* v;
  const float* ks;
  const float* vs;
  int Hkv, D, bs;
  __device__ __forceinline__ float key(int blk, int off, int h, int d) const {
    return e4m3_to_f32(k[(((size_t)blk * bs + off) * Hkv + h) * D + d]) * ks[blk];
  }
  __device__ __forceinline__ float val(int blk, int off, int h, int d) const {
    return e4m3_to_f32(v[(((size_t)blk * bs + off) * Hkv + h) * D + d]) * vs[blk];
  }
};

template <typename QT, typename KV>
__global__ __launch_bounds__(64) void paged_generic(GenericArgs a, KV kv) {
  constexpr int MAXH = 16;
  constexpr int MAXD = 256;
  const int lane = threadIdx.x;
  const int token = blockIdx.x;
  const int kvh = blockIdx.y;
  const int HG = a.Hq / a.Hkv;
  const int h0 = blockIdx.z * MAXH;
  const int nh = min(MAXH, HG - h0);
  const int D = a.D;
  const QT* q = reinterpret_cast<const QT*>(a.q);
  QT* out = reinterpret_cast<QT*>(a.out) + ((size_t)token * a.Hq + (size_t)kvh * HG + h0) * D;

  __shared__ float qs[MAXH][MAXD];
  __shared__ float ps[MAXH][64];

  // ---- locate the sequence and the causal key range
  int s = -1;
  if (a.decode) {
    s = token < a.S ? token : -1;
  } else {
    int lo = 0, hi = a.S;  // largest s in [0, S) with qsl[s] <= token
    if (a.S > 0 && a.qsl[0] <= token) {
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (a.qsl[mid] <= token) lo = mid; else hi = mid;
      }
      if (token < a.qsl[lo + 1]) s = lo;
    }
  }
  int q_len = 0, seq_len = 0, q_pos = 0;
  if (s >= 0) {
    q_len = a.decode ? 1 : a.qsl[s + 1] - a.qsl[s];
    q_pos = a.decode ? 0 : token - a.qsl[s];
    seq_len = min(a.kv_lens[s], a.max_blocks * a.bs);
  }
  const int max_k = min(seq_len - 1, (seq_len - q_len) + q_pos);
  if (s < 0 || q_len <= 0 || seq_len <= 0 || max_k < 0) {
    for (int i = lane; i < nh * D; i += 64) from_f32(0.f, out + (size_t)(i / D) * D + (i % D));
    return;
  }
  const int start_k = a.window > 0 ? max(0, max_k - a.window + 1) : 0;

  for (int i = lane; i < nh * D; i += 64) {
    const int h = i / D, d = i % D;
    qs[h][d] = to_f32(q[((size_t)token * a.Hq + (size_t)kvh * HG + h0 + h) * D + d]);
  }
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

  for (int base = start_k; base <= max_k; base += 64) {
    const int pos = base + lane;
    int blk = -1;
    if (pos <= max_k) blk = bt[pos / a.bs];
    const bool ok = blk >= 0 && blk < a.nb;
    float sc[MAXH];
#pragma unroll
    for (int h = 0; h < MAXH; ++h) sc[h] = 0.f;
    if (ok) {
      const int off = pos % a.bs;
      for (int d = 0; d < D; ++d) {
        const float kd = kv.key(blk, off, kvh, d);
#pragma unroll
        for (int h = 0; h < MAXH; ++h)
          if (h < nh) sc[h] += qs[h][d] * kd;
      }
    }
#pragma unroll
    for (int h = 0; h < MAXH; ++h) {
      if (h < nh) {
        const float x = ok ? sc[h] * a.scale_log2 : -INFINITY;
        const float mx = wave_max(x);
        const float m_new = fmaxf(m[h], mx);
        float p = 0.f, alpha = 1.f;
        if (m_new != -INFINITY) {
          p = exp2f(x - m_new);
          alpha = exp2f(m[h] - m_new);
        }
        l[h] = l[h] * alpha + wave_sum(p);
        m[h] = m_new;
        ps[h][lane] = p;
#pragma unroll
        for (int i = 0; i < MAXD / 64; ++i) acc[h][i] *= alpha;
      }
    }
    __syncthreads();
    const int nk = min(64, max_k - base + 1);
    for (int t = 0; t < nk; ++t) {
      const int pt = base + t;
      const int b = bt[pt / a.bs];
      if (b < 0 || b >= a.nb) continue;
      const int off = pt % a.bs;
#pragma unroll
      for (int i = 0; i < MAXD / 64; ++i) {
        const int d = lane + 64 * i;
        if (d < D) {
          const float vd = kv.val(b, off, kvh, d);
#pragma unroll
          for (int h = 0; h < MAXH; ++h)
            if (h < nh) acc[h][i] += ps[h][t] * vd;
        }
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int h = 0; h < MAXH; ++h) {
    if (h < nh) {
      const float inv = l[h] > 0.f ? 1.f / l[h] : 0.f;
#pragma unroll
      for (int i = 0; i < MAXD / 64; ++i) {
        const int d = lane + 64 * i;
        if (d < D) from_f32(acc[h][i] * inv, out + (size_t)h * D + d);
      }
    }
  }
}

}  // namespace emx

namespace emx {

// Dense K/V of a ragged batch from pages (PageCacheView.gather_kv_cache,
// lib/python/easymlx/caching/paged/cache.py:974-1027; Metal kernel :138-193):
// token t of sequence b (cu[b] <= t < cu[b+1]) at offset j = t - cu[b] is
// entry j % bs of page block_table[b, j / bs]; out [T, Hkv, D] in the output
// dtype, through the cache's loader (affine / FP8 dequantized in fp32, dense
// cast).  A page id outside [0, nb) or a column beyond the table yields zeros.
// One workgroup per token.
template <typename OutTag, typename KV>
__global__ __launch_bounds__(256) void gather_kv(KV kv, const int32_t* block_table, const int32_t* cu, int S,
                                                 int max_blocks, int T, int nb, void* k_out, void* v_out) {
  typedef typename OutTag::T OT;
  const int t = blockIdx.x;
  if (t >= T) return;
  int lo = 0, hi = S;  // the b with cu[b] <= t < cu[b + 1]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (cu[mid] <= t) lo = mid; else hi = mid;
  }
  const int j = t - cu[lo];
  const int col = j / kv.bs;
  const int blk = col < max_blocks ? block_table[(size_t)lo * max_blocks + col] : -1;
  const bool ok = blk >= 0 && blk < nb;
  const int n = kv.Hkv * kv.D;
  OT* ko = reinterpret_cast<OT*>(k_out) + (size_t)t * n;
  OT* vo = reinterpret_cast<OT*>(v_out) + (size_t)t * n;
  for (int e = threadIdx.x; e < n; e += 256) {
    const int h = e / kv.D, d = e % kv.D;
    from_f32(ok ? kv.key(blk, j % kv.bs, h, d) : 0.f, ko + e);
    from_f32(ok ? kv.val(blk, j % kv.bs, h, d) : 0.f, vo + e);
  }
}

}  // namespace emx
