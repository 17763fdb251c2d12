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
// of up to kFp8SelfMax values per tensor take one launch in which every
// workgroup computes the maxima itself; the decode append (fp8_append_grid)
// spreads the call over small workgroups that exchange their maxima once.
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
  // workgroups past a.nwg turn the queries: 16-byte pieces, loads sent before the
  // positions are derived
  constexpr int QU = 2;
  const bool qwg = SELF && (int)blockIdx.x >= a.nwg;
  const bool qvec = qwg && turn_rows_vec_ok(a.D, a.rope.rot, a.rope.traditional);
  TurnRowsVec<QU> tv(a.T, a.Hq, a.D, a.rope);
  const int qstride = (int)(gridDim.x - a.nwg) * NTH;
  const int qfirst = (int)(blockIdx.x - a.nwg) * NTH + threadIdx.x;
  if (qvec) tv.issue(a.q_in, a.D, a.rope, qfirst, qstride);
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
        rope_sincos((float)a.rope.positions[i / half] * a.rope.inv_freq[i % half], &sn, &cs);
        rsc[i] = float2{sn, cs};
      }
      __syncthreads();
      rtab = rsc;
    }
  }
  if constexpr (SELF) {
    if (qwg) {  // the query rotation rides in the same launch
      if (qvec) {
        tv.finish(a.q, a.Hq, a.D, a.rope);
        for (int i0 = qfirst + QU * qstride; i0 < tv.n; i0 += QU * qstride) {
          tv.issue(a.q_in, a.D, a.rope, i0, qstride);
          tv.finish(a.q, a.Hq, a.D, a.rope);
        }
      } else {
        turn_rows(a.q, a.q_in, a.T, a.Hq, a.D, a.rope, (long)qfirst, (long)qstride);
      }
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


// 8 values of T, raw (16-byte loads; 32 bytes for fp32).
template <typename T>
struct Fp8Piece {
  u32x4 w[sizeof(T) / 2];
  __device__ __forceinline__ void load(const T* p) {
#pragma unroll
    for (int i = 0; i < (int)(sizeof(T) / 2); ++i) w[i] = reinterpret_cast<const u32x4*>(p)[i];
  }
  __device__ __forceinline__ float at(const int j) const {
    if constexpr (sizeof(T) == 4) {
      return __uint_as_float(w[j / 4][j % 4]);
    } else {
      const uint16_t b = (uint16_t)(w[0][j / 2] >> (16 * (j & 1)));
      if constexpr (__is_same(T, h16))
        return (float)__builtin_bit_cast(h16, b);
      else
        return bf16_to_f32(b);
    }
  }
};

// ---- Decode append by a grid that waits on itself once (fp8_append_grid).
// The call's single scale pair needs the maxima of every value before any code
// is written.  Workgroups of 256 threads each take 256 pieces of 8 values of the
// call (K pieces, then V pieces; a rotated K piece also loads the piece it pairs
// with), load them with the slots and
// positions of every token, turn their K from a (sin, cos) table of their own
// tokens, and reduce their maxima; thread 0 folds them into the call's maxima
// (atomicMax on the bits of non-negative floats, counter[2] and [3]), counts the
// workgroup on counter[1], and waits until all a.nwg write workgroups have
// counted.  Then every workgroup encodes its own tasks with the call's scales.
// The workgroups (at most kFp8GridMaxWG, each small) are all resident at once on
// an otherwise busy GPU, so the wait ends; it is bounded all the same.  Workgroups
// a.nwg.. turn the queries, one token each.  counter[0] counts every workgroup
// at its end; the last one clears counter[0..3] and advances kv_lens, so the
// four ints are zero between calls.  Same bits as fp8_write: the same turned
// values, the same maxima (a maximum is exact in any order) and encoder.
constexpr int kFp8GridMaxWG = 128;
constexpr int kFp8GridTab = 4096;

__host__ __device__ inline bool fp8_grid_fits(const int T, const int Hkv, const int D, const int rot,
                                              const int trad) {
  if (T <= 0 || T > kFp8AppendMax || D % 8 != 0 || D > 256 || rot <= 0 || !turn_rows_vec_ok(D, rot, trad))
    return false;
  const long tasks = 2L * T * Hkv * (D / 8);  // K pieces, then V pieces
  return (tasks + 255) / 256 <= kFp8GridMaxWG;
}

template <typename Tag>
__global__ __launch_bounds__(256) void fp8_append_grid(Fp8WriteArgs a) {
  typedef typename Tag::T T;
  constexpr int NTH = 256, KT = kFp8AppendMax / NTH;
  const int tid = threadIdx.x;
  const int nwg = a.nwg;
  const bool qwg = (int)blockIdx.x >= nwg;
  const RopeArgs& r = a.rope;
  const int rot = r.rot, half = rot / 2, trad = r.traditional;
  const int pr = a.D / 8, nrp = rot / 8;  // pieces per (token, head) row, of them rotated
  const int nk = a.T * a.Hkv * pr, nv = nk;
  const T* k = reinterpret_cast<const T*>(a.k);
  const T* v = reinterpret_cast<const T*>(a.v);
  int* const cnt = a.counter;

  // ---- loads that depend on nothing: this thread's task, or a query token's rows
  const int j0 = (int)blockIdx.x * NTH, j = j0 + tid;
  Fp8Piece<T> lo, hi;
  const int tq = (int)blockIdx.x - nwg;  // query workgroup: its token
  TurnRowsVec<2> tv(1, a.Hq, a.D, r);
  if (qwg) {
    tv.issue(a.q_in + (size_t)tq * a.Hq * a.D, a.D, r, tid, NTH);
  } else if (j < nk) {
    const int c = j % pr;
    const T* row = k + (size_t)(j / pr) * a.D;
    lo.load(row + 8 * c);
    if (c < nrp && !trad) hi.load(row + 8 * (c < nrp / 2 ? c + nrp / 2 : c - nrp / 2));
  } else if (j < nk + nv) {
    lo.load(v + 8 * (size_t)(j - nk));
  }
  const float inv_in = tid < half ? r.inv_freq[tid] : 0.f;  // half <= 128
  // slots and positions of every token (as cache_slots derives them)
  int sl[KT], pos[KT], sq[KT];
#pragma unroll
  for (int u = 0; u < KT; ++u) {
    const int t = tid + u * NTH;
    sl[u] = -1;
    pos[u] = 0;
    sq[u] = -1;
    if (t < a.T) {
      const int s = a.slot_ids[t];
      if (s >= 0 && s < a.S) {
        sq[u] = s;
        pos[u] = a.kv_lens[s];
        const int col = pos[u] / a.bs;
        if (pos[u] >= 0 && col < a.max_blocks) {
          const int b = a.bt[(size_t)s * a.max_blocks + col];
          if (b >= 0) sl[u] = b * a.bs + pos[u] % a.bs;
        }
      }
    }
  }
  __shared__ int fslot[kFp8AppendMax], fpos[kFp8AppendMax], fseq[kFp8AppendMax];
  __shared__ float sinv[128];
  __shared__ float2 stab[kFp8GridTab];
  __shared__ unsigned int sred[2][NTH / 64];
  __shared__ int sflag;
#pragma unroll
  for (int u = 0; u < KT; ++u) {
    const int t = tid + u * NTH;
    if (t < a.T) {
      fslot[t] = sl[u] >= 0 && sl[u] / a.bs < a.nb ? sl[u] : -1;  // a page outside the pool: skipped
      fpos[t] = pos[u];
      fseq[t] = sq[u];
    }
  }
  if (tid < half) sinv[tid] = inv_in;
  __syncthreads();

  // ---- the (sin, cos) table of this workgroup's tokens [t_lo, t_hi]
  int t_lo = tq, t_hi = tq;
  if (!qwg) {
    const int k_end = min(j0 + NTH, nk);
    t_lo = j0 < nk ? (j0 / pr) / a.Hkv : 0;
    t_hi = j0 < nk ? ((k_end - 1) / pr) / a.Hkv : -1;
  }
  const int ntab = (t_hi - t_lo + 1) * half;  // <= kFp8GridTab (fp8_grid_fits)
  for (int i = tid; i < ntab; i += NTH) {
    float sn, cs;
    rope_sincos((float)fpos[t_lo + i / half] * sinv[i % half], &sn, &cs);
    stab[i] = float2{sn, cs};
  }
  __syncthreads();

  auto count_and_finish = [&]() {  // every workgroup at its end, once
    if (tid == 0) {
      const int arrived = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sflag = arrived == (int)gridDim.x - 1;
      if (sflag) {  // every workgroup has read the maxima and kv_lens: clear for the next call
        __hip_atomic_store(cnt + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(cnt + 2, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(cnt + 3, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();
    if (sflag)
      for (int t = tid; t < a.T; t += NTH)
        if (fseq[t] >= 0) a.kv_lens[fseq[t]] = fpos[t] + 1;
  };
  if (qwg) {
    h16* qo = a.q + (size_t)tq * a.Hq * a.D;
    const h16* qi = a.q_in + (size_t)tq * a.Hq * a.D;
    tv.finish(qo, a.Hq, a.D, r, stab);
    for (int i0 = tid + 2 * NTH; i0 < tv.n; i0 += 2 * NTH) {
      tv.issue(qi, a.D, r, i0, NTH);
      tv.finish(qo, a.Hq, a.D, r, stab);
    }
    count_and_finish();
    return;
  }

  // ---- this piece's values (K turned and rounded to T), the workgroup's maxima
  float x[8];
  int kind = 0, rr = 0, c = 0, t = 0;  // kind 1: K piece, 2: V piece
  if (j < nk + nv) {
    kind = j < nk ? 1 : 2;
    const int i = kind == 1 ? j : j - nk;
    rr = i / pr;
    c = i % pr;
    t = rr / a.Hkv;
#pragma unroll
    for (int q = 0; q < 8; ++q) x[q] = lo.at(q);
  }
  if (kind == 1 && c < nrp) {
    const float2* tt = stab + (t - t_lo) * half;
    if (trad) {
#pragma unroll
      for (int q = 0; q < 8; q += 2) {
        float y0, y1;
        rope_rotate_sc(x[q], x[q + 1], tt[4 * c + q / 2], y0, y1);
        x[q] = round_to(y0, (T*)nullptr);
        x[q + 1] = round_to(y1, (T*)nullptr);
      }
    } else if (c < nrp / 2) {  // the first elements of their pairs
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        float y0, y1;
        rope_rotate_sc(x[q], hi.at(q), tt[8 * c + q], y0, y1);
        x[q] = round_to(y0, (T*)nullptr);
      }
    } else {  // the second elements
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        float y0, y1;
        rope_rotate_sc(hi.at(q), x[q], tt[8 * (c - nrp / 2) + q], y0, y1);
        x[q] = round_to(y1, (T*)nullptr);
      }
    }
  }
  const int slot = kind ? fslot[t] : -1;
  float m = 0.f;
  if (slot >= 0) {
#pragma unroll
    for (int q = 0; q < 8; ++q) m = fmaxf(m, fabsf(x[q]));
  }
  float mk = wave_max(kind == 1 ? m : 0.f), mv = wave_max(kind == 2 ? m : 0.f);
  if ((tid & 63) == 0) {
    sred[0][tid >> 6] = __float_as_uint(mk);
    sred[1][tid >> 6] = __float_as_uint(mv);
  }
  __syncthreads();
  // ---- the call's maxima: fold, count, wait for every write workgroup (bounded)
  if (tid == 0) {
    unsigned int bk = 0u, bv = 0u;
#pragma unroll
    for (int w = 0; w < NTH / 64; ++w) {
      bk = max(bk, sred[0][w]);
      bv = max(bv, sred[1][w]);
    }
    // Only atomics touch counter[1..3], and an agent-scope atomic is performed where
    // every XCD sees it, so relaxed order suffices once the two maxima have returned
    // before the count goes out (the empty asm makes the count wait for them); release
    // and acquire fences would write back and invalidate whole L2s for nothing.
    const unsigned int ok = __hip_atomic_fetch_max(reinterpret_cast<unsigned int*>(cnt + 2), bk, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
    const unsigned int ov = __hip_atomic_fetch_max(reinterpret_cast<unsigned int*>(cnt + 3), bv, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("" ::"v"(ok), "v"(ov));
    __hip_atomic_fetch_add(cnt + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int it = 0; it < (1 << 22); ++it) {
      if (__hip_atomic_load(cnt + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= nwg) break;
      __builtin_amdgcn_s_sleep(1);
    }
    sred[0][0] = __hip_atomic_load(reinterpret_cast<unsigned int*>(cnt + 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sred[1][0] = __hip_atomic_load(reinterpret_cast<unsigned int*>(cnt + 3), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  const float ksc = __uint_as_float(sred[0][0]) / 240.0f, vsc = __uint_as_float(sred[1][0]) / 240.0f;
  const float kq = fmaxf(ksc, 1e-12f), vq = fmaxf(vsc, 1e-12f);

  // ---- codes: 8 bytes per piece, [nb, bs, Hkv, D]
  if (slot >= 0) {
    auto enc8 = [](const float (&z)[8], const float qd) {
      uint32_t w0 = 0, w1 = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        w0 |= f32_to_e4m3(z[q] / qd) << (8 * q);
        w1 |= f32_to_e4m3(z[q + 4] / qd) << (8 * q);
      }
      return uint2{w0, w1};
    };
    const size_t rowb = ((size_t)slot * a.Hkv + rr % a.Hkv) * (size_t)a.D;
    if (kind == 1) {
      *reinterpret_cast<uint2*>(a.kc + rowb + 8 * c) = enc8(x, kq);
      if (c == 0 && rr % a.Hkv == 0) {  // once per written token: the page keeps the larger scale
        atomicMax(reinterpret_cast<unsigned int*>(a.ks) + slot / a.bs, __float_as_uint(ksc));
        atomicMax(reinterpret_cast<unsigned int*>(a.vs) + slot / a.bs, __float_as_uint(vsc));
      }
    } else {
      *reinterpret_cast<uint2*>(a.vc + rowb + 8 * c) = enc8(x, vq);
    }
  }
  count_and_finish();
}

}  // namespace emx
