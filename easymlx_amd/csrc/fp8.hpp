// FP8 (E4M3) quantize-on-write into a page cache [nb, bs, Hkv, D] uint8 with one
// fp32 scale per page, as the reference's PageCacheView.concatenate_to_cache
// writes an FP8 cache (lib/python/easymlx/caching/paged/cache.py:1171-1184):
//   * one scale per call for K and one for V: max|x| / 240 over the written
//     tokens (_KV_SCALE_UPDATE_SOURCE :195-239, compute_kv_scales :430-463);
//   * codes enc(x / max(scale, 1e-12)) with the reference's E4M3 encoder
//     (_fp8_quantize :466-478; encoder _metal_header.py:339-419);
//   * each written page's scale raised to max(page_scale, scale); the page's
//     earlier codes are not requantized (the reference's rule);
//   * a slot of -1, or one whose page lies outside the pool, is skipped: it is
//     neither written nor counted in the call's maxima.
// Two launches: per-workgroup maxima into a small workspace, then every
// workgroup reduces them and quantizes its share (4 values per thread).  Writes
// of up to kFp8SelfMax values per tensor (decode appends) take one launch in
// which every workgroup computes the maxima itself.
#pragma once

#include "common.hpp"
#include "quantize.hpp"  // turn_rows

namespace emx {

constexpr int kFp8Parts = 256;      // workgroups of the max pass (partials in the workspace)
constexpr int kFp8SelfMax = 65536;  // values per tensor of the one-launch write

struct Fp8WriteArgs {
  const void* k;         // [T, Hkv, D] in the input dtype
  const void* v;
  const int32_t* slot;   // [T] block * bs + offset, -1 skips the token
  int T, Hkv, D, bs, nb;
  uint8_t* kc;           // [nb, bs, Hkv, D]
  uint8_t* vc;
  float* ks;             // [nb]
  float* vs;
  float* part;           // [2][kFp8Parts] per-workgroup maxima
  RopeArgs rope;         // K turned before the scale and the codes (inv_freq null: none)
  h16* q;                // [T, Hq, D] fp16 turned queries, written by the one-launch write (null: none)
  const h16* q_in;       // the queries to turn (== q: in place)
  int Hq;
  int nwg;               // workgroups of the write proper; later ones turn the queries
  // Decode append (the one-launch write; slot null): token t is the next token of
  // sequence slot_ids[t] (emx_affine_cache_append_rope's rule), kv_lens advances by one.
  const int32_t* slot_ids;  // [T], T <= kFp8AppendMax
  int32_t* kv_lens;         // [S]
  const int32_t* bt;        // [S, max_blocks]
  int S, max_blocks;
  int* counter;             // workgroups that have read kv_lens: zero before and after every launch
};

constexpr int kFp8AppendMax = 1024;  // tokens of a one-launch decode append
constexpr int kFp8RopeTab = 4096;    // (token, pair) angles of the one-launch write's LDS table

__device__ __forceinline__ float round_to(float x, h16*) { return (float)(h16)x; }
__device__ __forceinline__ float round_to(float x, uint16_t*) { return bf16_to_f32(f32_to_bf16(x)); }
__device__ __forceinline__ float round_to(float x, float*) { return x; }

// The word whose values pair with word e's in the rotation (non-traditional: the
// other half of the rotated dims); e itself when word e is not turned in pairs
// across words.
__device__ __forceinline__ uint32_t k_partner(const Fp8WriteArgs& a, const uint32_t e) {
  const RopeArgs& r = a.rope;
  if (r.inv_freq == nullptr || r.traditional) return e;
  const uint32_t wpr = a.D / 4;
  const int d0 = 4 * (int)(e % wpr);
  if (d0 >= r.rot) return e;
  const int half = r.rot / 2;
  return d0 < half ? e + half / 4 : e - half / 4;
}

// Word e's 4 values x turned, given its partner word's values p (k_partner).
template <typename T>
__device__ __forceinline__ void k_turn(const Fp8WriteArgs& a, const uint32_t e, float (&x)[4], const float (&p)[4],
                                       const float2* tab) {
  const RopeArgs& r = a.rope;
  if (r.inv_freq == nullptr) return;
  const uint32_t wpr = a.D / 4;  // words per head row
  const int d0 = 4 * (int)(e % wpr);
  if (d0 >= r.rot) return;
  const uint32_t t = e / ((uint32_t)a.Hkv * wpr);
  const float pos = tab ? 0.f : (float)r.positions[t];
  const float2* tt = tab ? tab + (size_t)t * (r.rot / 2) : nullptr;
  float y[4];
  if (r.traditional) {
#pragma unroll
    for (int j = 0; j < 4; j += 2) {
      const int i = (d0 + j) >> 1;
      if (tab)
        rope_rotate_sc(x[j], x[j + 1], tt[i], y[j], y[j + 1]);
      else
        rope_rotate(x[j], x[j + 1], pos * r.inv_freq[i], y[j], y[j + 1]);
    }
  } else {
    const int half = r.rot / 2;
    const bool lo = d0 < half;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float y0, y1;
      const int i = (lo ? d0 : d0 - half) + j;
      if (tab) {
        if (lo)
          rope_rotate_sc(x[j], p[j], tt[i], y0, y1);
        else
          rope_rotate_sc(p[j], x[j], tt[i], y1, y0);
      } else {
        if (lo)
          rope_rotate(x[j], p[j], pos * r.inv_freq[i], y0, y1);
        else
          rope_rotate(p[j], x[j], pos * r.inv_freq[i], y1, y0);
      }
      y[j] = y0;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) x[j] = round_to(y[j], (T*)nullptr);
}

// The 4 K values of word e (dims 4w .. 4w+3 of one token and head), turned by
// the call's RoPE and rounded to the input dtype when a.rope is set (the
// reference writes the rotated keys of the model's dtype).  Needs rot % 8 == 0
// (non-traditional): a word and its partner word lie in one half each.
// tab: null, or (sin, cos) of positions[t] * inv_freq[i] at t * (rot / 2) + i (the
// one-launch write builds it once per workgroup instead of a sincosf per value).
template <typename T>
__device__ __forceinline__ void k_word(const Fp8WriteArgs& a, const T* k, const uint32_t e, float (&x)[4],
                                       const float2* tab = nullptr) {
#pragma unroll
  for (int j = 0; j < 4; ++j) x[j] = to_f32(k[4 * (size_t)e + j]);
  if (a.rope.inv_freq == nullptr) return;  // unturned keys
  const uint32_t pe = k_partner(a, e);
  float p[4] = {x[0], x[1], x[2], x[3]};
  if (pe != e) {  // the partner word is loaded only where the rotation pairs two words
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = to_f32(k[4 * (size_t)pe + j]);
  }
  k_turn<T>(a, e, x, p, tab);
}

template <typename Tag>
__global__ __launch_bounds__(256) void fp8_amax(Fp8WriteArgs a) {
  typedef typename Tag::T T;
  const T* k = reinterpret_cast<const T*>(a.k);
  const T* v = reinterpret_cast<const T*>(a.v);
  const uint32_t row4 = (uint32_t)a.Hkv * a.D / 4, n4 = (uint32_t)a.T * row4;  // n4 < 2^31 (host check)
  float mk = 0.f, mv = 0.f;
  for (uint32_t e = blockIdx.x * 256u + threadIdx.x; e < n4; e += gridDim.x * 256u) {
    const int sl = a.slot[e / row4];
    if (sl < 0 || sl / a.bs >= a.nb) continue;  // skipped slots (-1 or page outside the pool) do not count
    float x[4];
    k_word(a, k, e, x);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      mk = fmaxf(mk, fabsf(x[j]));
      mv = fmaxf(mv, fabsf(to_f32(v[4 * (size_t)e + j])));
    }
  }
  mk = wave_max(mk);
  mv = wave_max(mv);
  __shared__ float sm[2][4];
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sm[0][w] = mk;
    sm[1][w] = mv;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    const float* x = sm[threadIdx.x];
    a.part[threadIdx.x * kFp8Parts + blockIdx.x] = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
  }
}

template <typename Tag, bool SELF = false>
__global__ __launch_bounds__(SELF ? 1024 : 256) void fp8_write(Fp8WriteArgs a, int nparts) {
  typedef typename Tag::T T;
  constexpr int NTH = SELF ? 1024 : 256;  // threads per workgroup
  __shared__ float sc[2];
  // Decode append (one-launch write with a.slot_ids): every workgroup derives the
  // tokens' slots and positions into LDS (the arithmetic of cache_slots), counts
  // itself once they are there, and the workgroup counted last advances kv_lens at
  // its end, so no workgroup reads an advanced length.
  const bool app = SELF && a.slot_ids != nullptr;
  int arrived = 0;
  if constexpr (SELF) {
    __shared__ int fslot[kFp8AppendMax], fpos[kFp8AppendMax], fseq[kFp8AppendMax];
    if (app) {
      for (int t = threadIdx.x; t < a.T; t += NTH) {
        int s = a.slot_ids[t], pos = 0, m = -1;
        if (s >= 0 && s < a.S) {
          pos = a.kv_lens[s];
          const int col = pos / a.bs;
          if (pos >= 0 && col < a.max_blocks) {
            const int b = a.bt[(size_t)s * a.max_blocks + col];
            if (b >= 0) m = b * a.bs + pos % a.bs;
          }
        } else {
          s = -1;
        }
        fslot[t] = m;
        fpos[t] = pos;
        fseq[t] = s;
      }
      a.slot = fslot;
      a.rope.positions = fpos;
      __syncthreads();  // every kv_lens read of the workgroup has returned
      if (threadIdx.x == 0)
        arrived = __hip_atomic_fetch_add(a.counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  auto finish = [&]() {  // the end of the workgroup: the last one counted advances kv_lens
    if constexpr (SELF) {
      if (!app) return;
      __shared__ int slast;
      if (threadIdx.x == 0) {
        slast = arrived == (int)gridDim.x - 1;
        if (arrived == (int)gridDim.x - 1)
          __hip_atomic_store(a.counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (slast)
        for (int t = threadIdx.x; t < a.T; t += NTH)
          if (a.rope.positions != nullptr && a.slot_ids[t] >= 0 && a.slot_ids[t] < a.S)
            a.kv_lens[a.slot_ids[t]] = a.rope.positions[t] + 1;
    }
  };
  // (sin, cos) of every (token, pair) angle, once per workgroup, for the K rotations
  // of the maxima and of the codes (a sincosf per value made every workgroup of a
  // 32-token append spend ~20 us turning all the keys for the maxima)
  const float2* rtab = nullptr;
  if constexpr (SELF) {
    __shared__ float2 rsc[kFp8RopeTab];
    const int half = a.rope.rot / 2;
    if (a.rope.inv_freq != nullptr && (int)blockIdx.x < a.nwg && a.T * half <= kFp8RopeTab) {
      for (int i = threadIdx.x; i < a.T * half; i += NTH) {
        float sn, cs;
        sincosf((float)a.rope.positions[i / half] * a.rope.inv_freq[i % half], &sn, &cs);
        rsc[i] = float2{sn, cs};
      }
      __syncthreads();
      rtab = rsc;
    }
  }
  if constexpr (SELF) {
    if ((int)blockIdx.x >= a.nwg) {  // the query rotation rides in the same launch
      turn_rows(a.q, a.q_in, a.T, a.Hq, a.D, a.rope, (long)(blockIdx.x - a.nwg) * NTH + threadIdx.x,
                (long)(gridDim.x - a.nwg) * NTH);
      finish();
      return;
    }
    // a small write in one launch: every workgroup takes the maxima over all the
    // written values itself (exact and order-free, so each gets the same
    // scales); four words per thread in flight together
    const T* k = reinterpret_cast<const T*>(a.k);
    const T* v = reinterpret_cast<const T*>(a.v);
    const uint32_t row4 = (uint32_t)a.Hkv * a.D / 4, n4 = (uint32_t)a.T * row4;
    float mk = 0.f, mv = 0.f;
    for (uint32_t e0 = threadIdx.x; e0 < n4; e0 += 4 * NTH) {
      float x[4][4], y[4][4];
      bool live[4];
      float p[4][4];
      uint32_t ee[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {  // every load of the four words first, then the turns
        const uint32_t e = e0 + (uint32_t)u * NTH;
        const int sl = e < n4 ? a.slot[e / row4] : -1;
        live[u] = sl >= 0 && sl / a.bs < a.nb;  // as the write loop: a page outside the pool is skipped
        ee[u] = e < n4 ? e : e0;
        const uint32_t pe = k_partner(a, ee[u]);  // ee[u] itself without a pairing rotation
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[u][j] = to_f32(k[4 * (size_t)ee[u] + j]);
          y[u][j] = to_f32(v[4 * (size_t)ee[u] + j]);
        }
        if (pe != ee[u]) {  // the partner word only where the rotation pairs two words
#pragma unroll
          for (int j = 0; j < 4; ++j) p[u][j] = to_f32(k[4 * (size_t)pe + j]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) p[u][j] = x[u][j];
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) k_turn<T>(a, ee[u], x[u], p[u], rtab);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (!live[u]) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          mk = fmaxf(mk, fabsf(x[u][j]));
          mv = fmaxf(mv, fabsf(y[u][j]));
        }
      }
    }
    mk = wave_max(mk);
    mv = wave_max(mv);
    __shared__ float sm[2][NTH / 64];
    if ((threadIdx.x & 63) == 0) {
      sm[0][threadIdx.x >> 6] = mk;
      sm[1][threadIdx.x >> 6] = mv;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int i = 0; i < NTH / 64; ++i) {
        a0 = fmaxf(a0, sm[0][i]);
        a1 = fmaxf(a1, sm[1][i]);
      }
      sc[0] = a0 / 240.0f;
      sc[1] = a1 / 240.0f;
    }
  } else if (threadIdx.x < 64) {
    float mk = 0.f, mv = 0.f;
    for (int i = threadIdx.x; i < nparts; i += 64) {
      mk = fmaxf(mk, a.part[i]);
      mv = fmaxf(mv, a.part[kFp8Parts + i]);
    }
    mk = wave_max(mk);
    mv = wave_max(mv);
    if (threadIdx.x == 0) {
      sc[0] = mk / 240.0f;
      sc[1] = mv / 240.0f;
    }
  }
  __syncthreads();
  const float ksc = sc[0], vsc = sc[1];
  const float kq = fmaxf(ksc, 1e-12f), vq = fmaxf(vsc, 1e-12f);
  const T* k = reinterpret_cast<const T*>(a.k);
  const T* v = reinterpret_cast<const T*>(a.v);
  const uint32_t row4 = (uint32_t)a.Hkv * a.D / 4;
  const uint32_t n4 = (uint32_t)a.T * row4;
  const uint32_t nwg = SELF ? a.nwg : gridDim.x;
  for (uint32_t e = blockIdx.x * (uint32_t)NTH + threadIdx.x; e < n4; e += nwg * NTH) {
    const int t = (int)(e / row4), r = (int)(e % row4);
    const int slot = a.slot[t];
    if (slot < 0) continue;
    const int blk = slot / a.bs, off = slot % a.bs;
    if (blk >= a.nb) continue;
    float x[4];
    k_word(a, k, e, x, rtab);
    uint32_t ck = 0, cv = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ck |= f32_to_e4m3(x[j] / kq) << (8 * j);
      cv |= f32_to_e4m3(to_f32(v[4 * (size_t)e + j]) / vq) << (8 * j);
    }
    const size_t dst = ((size_t)blk * a.bs + off) * (size_t)row4 + r;  // [nb, bs, Hkv*D/4] words
    reinterpret_cast<uint32_t*>(a.kc)[dst] = ck;
    reinterpret_cast<uint32_t*>(a.vc)[dst] = cv;
    if (r == 0) {  // once per written token: the page keeps the larger scale (scales are >= 0)
      atomicMax(reinterpret_cast<unsigned int*>(a.ks) + blk, __float_as_uint(ksc));
      atomicMax(reinterpret_cast<unsigned int*>(a.vs) + blk, __float_as_uint(vsc));
    }
  }
  finish();
}

}  // namespace emx
