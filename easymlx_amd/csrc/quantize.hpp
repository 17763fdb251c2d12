// Affine quantize (MLX "affine" mode) and fused quantize-on-write into pages.
//
// Per group of `gs` contiguous elements (fp32 arithmetic, IEEE division,
// round-half-to-even), as mlx.core.quantize(w, group_size, bits) -- called by
// the reference at lib/python/easymlx/infra/mixins/bridge.py:304,361:
//   mask  = |min| > |max|;  scale = max((max-min)/(2^b-1), 1e-7), negated if !mask
//   edge  = mask ? min : max;  q0 = rint(edge/scale)
//   q0 != 0 -> scale = edge/q0, bias = edge;  else bias = 0
//   code  = clamp(rint((w-bias)/scale), 0, 2^b-1);  scale/bias stored as fp16.
// Fused write replaces the write step of PageCacheView.concatenate_to_cache
// (lib/python/easymlx/caching/paged/cache.py:1155-1190, 1254-1290): token t goes
// to page slot_mapping[t] / bs, offset slot_mapping[t] % bs (-1 = not written).
#pragma once

#include "common.hpp"

namespace emx {

#pragma clang fp contract(off)

__device__ __forceinline__ void affine_params(float wmin, float wmax, float n_bins, float& scale, float& bias) {
  const bool mask = fabsf(wmin) > fabsf(wmax);
  float sc = fmaxf((wmax - wmin) / n_bins, 1e-7f);
  sc = mask ? sc : -sc;
  const float edge = mask ? wmin : wmax;
  const float q0 = rintf(edge / sc);
  bias = 0.f;
  if (q0 != 0.f) {
    sc = edge / q0;
    bias = edge;
  }
  scale = sc;
}

__device__ __forceinline__ uint32_t affine_code(float w, float scale, float bias, float n_bins) {
  float q = rintf((w - bias) / scale);
  q = fminf(fmaxf(q, 0.f), n_bins);
  return (uint32_t)q;
}

// Reads one group of fp16 values, returns fp32 scale/bias.
__device__ __forceinline__ void group_minmax(const h16* src, int gs, float& wmin, float& wmax) {
  wmin = INFINITY;
  wmax = -INFINITY;
  const u32x4* p = reinterpret_cast<const u32x4*>(src);
  for (int i = 0; i < gs / 8; ++i) {
    const u32x4 x = p[i];
    const h16* h = reinterpret_cast<const h16*>(&x);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float v = (float)h[k];
      wmin = fminf(wmin, v);
      wmax = fmaxf(wmax, v);
    }
  }
}

// min / max of gs contiguous fp16 values held in LDS.
__device__ __forceinline__ void lds_minmax(const h16* src, int gs, float& wmin, float& wmax) {
  wmin = INFINITY;
  wmax = -INFINITY;
  for (int i = 0; i < gs; i += 8) {
    const h16x8 x = *reinterpret_cast<const h16x8*>(src + i);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float v = (float)x[k];
      wmin = fminf(wmin, v);
      wmax = fmaxf(wmax, v);
    }
  }
}

// x [rows, D] fp16 -> codes [rows, D*b/32] u32, scales/biases [rows, D/gs] fp16 (MLX layout).
// One thread per (row, group).
template <int BITS>
__global__ __launch_bounds__(256) void affine_quantize_rows(const h16* x, long rows, int D, int gs, uint32_t* codes,
                                                           h16* scales, h16* biases) {
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int G = D / gs;
  if (gid >= rows * G) return;
  const long row = gid / G;
  const int g = (int)(gid % G);
  const float n_bins = (float)((1 << BITS) - 1);
  const h16* src = x + row * D + (long)g * gs;
  float wmin, wmax, scale, bias;
  group_minmax(src, gs, wmin, wmax);
  affine_params(wmin, wmax, n_bins, scale, bias);
  constexpr int PW = 32 / BITS;
  uint32_t* dst = codes + row * (D / PW) + (long)g * (gs / PW);
  for (int w = 0; w < gs / PW; ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int k = 0; k < PW; ++k) word |= affine_code((float)src[w * PW + k], scale, bias, n_bins) << (k * BITS);
    dst[w] = word;
  }
  scales[gid] = (h16)scale;
  biases[gid] = (h16)bias;
}

// K rows turn (RopeArgs, common.hpp) inside a fused write and rows of Q in
// rope_rows; the result is rounded to fp16, the dtype the reference's rotated
// keys have when written.
__device__ __forceinline__ void rope_pair(h16& a0, h16& a1, const float theta) {
  float y0, y1;
  rope_rotate((float)a0, (float)a1, theta, y0, y1);
  a0 = (h16)y0;
  a1 = (h16)y1;
}

// Rows [rows, heads, D] fp16: x = src turned; row r is at positions[r].  src ==
// x turns in place; otherwise the dims past r.rot are copied as they are.  Pair
// slot i of a thread range [i_first, n) with stride `stride`.
__device__ __forceinline__ void turn_rows(h16* x, const h16* src, const int rows, const int heads, const int D,
                                          const RopeArgs& r, const long i_first, const long stride) {
  const int half = r.rot / 2;
  const int per_row = src == x ? half : D / 2;  // out of place: every dim pair of the row
  const long n = (long)rows * heads * per_row;
  for (long i = i_first; i < n; i += stride) {
    const int p = (int)(i % per_row);
    const long rh = i / per_row;
    const h16* u = src + rh * D;
    h16* v = x + rh * D;
    if (p < half) {
      const int i0 = r.traditional ? 2 * p : p, i1 = r.traditional ? 2 * p + 1 : p + half;
      h16 a0 = u[i0], a1 = u[i1];
      rope_pair(a0, a1, (float)r.positions[rh / heads] * r.inv_freq[p]);
      v[i0] = a0;
      v[i1] = a1;
    } else {
      const int j = r.rot + 2 * (p - half);
      v[j] = u[j];
      v[j + 1] = u[j + 1];
    }
  }
}

// turn_rows in 16-byte pieces, out of place (every dim of a row written): a task
// is one piece of 4 adjacent pairs (traditional), 8 pairs of a piece and its
// partner piece half a rotation on (neox order), or a piece past r.rot that is
// copied.  rope_pair on each pair, so the bits are turn_rows'.  Applies when
// D % 8 == 0 and r.rot is a multiple of 8 (traditional) or 16 (neox); the
// caller checks (turn_rows_vec_ok).  The loads of a pass of U tasks per thread
// go out together: issue() then finish(), with the positions needed only in
// finish() (a caller may wait for them in between).
__host__ __device__ inline bool turn_rows_vec_ok(const int D, const int rot, const int traditional) {
  return D % 8 == 0 && rot % (traditional ? 8 : 16) == 0;
}

template <int U>
struct TurnRowsVec {
  h16x8 lo[U], hi[U];
  int rh[U], c[U];
  int nrot, per, n;

  __device__ __forceinline__ TurnRowsVec(const int rows, const int heads, const int D, const RopeArgs& r) {
    nrot = r.traditional ? r.rot / 8 : r.rot / 16;
    per = nrot + (D - r.rot) / 8;
    n = rows * heads * per;
  }
  __device__ __forceinline__ void issue(const h16* src, const int D, const RopeArgs& r, const int i0, const int stride) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * stride;
      rh[u] = i < n ? i / per : -1;
      c[u] = i < n ? i % per : 0;
      if (rh[u] >= 0) {
        const h16* row = src + (size_t)rh[u] * D;
        const int off = c[u] < nrot ? 8 * c[u] : r.rot + 8 * (c[u] - nrot);
        lo[u] = *reinterpret_cast<const h16x8*>(row + off);
        if (c[u] < nrot && !r.traditional) hi[u] = *reinterpret_cast<const h16x8*>(row + r.rot / 2 + off);
      }
    }
  }
  // tab: null, or (sin, cos) of positions[t] * inv_freq[p] at t * (r.rot / 2) + p
  // (rope_rotate_sc on it gives rope_pair's bits)
  __device__ __forceinline__ void finish(h16* x, const int heads, const int D, const RopeArgs& r,
                                         const float2* tab = nullptr) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (rh[u] < 0) continue;
      h16* row = x + (size_t)rh[u] * D;
      if (c[u] >= nrot) {
        *reinterpret_cast<h16x8*>(row + r.rot + 8 * (c[u] - nrot)) = lo[u];
        continue;
      }
      const int t = rh[u] / heads;
      const float pos = tab ? 0.f : (float)r.positions[t];
      const float2* tt = tab ? tab + (size_t)t * (r.rot / 2) : nullptr;
      auto turn = [&](h16& a0, h16& a1, const int p) {
        if (tab) {
          float y0, y1;
          rope_rotate_sc((float)a0, (float)a1, tt[p], y0, y1);
          a0 = (h16)y0;
          a1 = (h16)y1;
        } else {
          rope_pair(a0, a1, pos * r.inv_freq[p]);
        }
      };
      if (r.traditional) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          h16 a0 = lo[u][2 * k], a1 = lo[u][2 * k + 1];
          turn(a0, a1, 4 * c[u] + k);
          lo[u][2 * k] = a0;
          lo[u][2 * k + 1] = a1;
        }
        *reinterpret_cast<h16x8*>(row + 8 * c[u]) = lo[u];
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          h16 a0 = lo[u][k], a1 = hi[u][k];
          turn(a0, a1, 8 * c[u] + k);
          lo[u][k] = a0;
          hi[u][k] = a1;
        }
        *reinterpret_cast<h16x8*>(row + 8 * c[u]) = lo[u];
        *reinterpret_cast<h16x8*>(row + r.rot / 2 + 8 * c[u]) = hi[u];
      }
    }
  }
};


__global__ __launch_bounds__(256) void rope_rows(h16* x, const h16* src, int rows, int heads, int D, RopeArgs r) {
  turn_rows(x, src, rows, heads, D, r, (long)blockIdx.x * 256 + threadIdx.x, (long)gridDim.x * 256);
}

struct WriteArgs {
  const h16* keys;             // [T, Hkv, D]
  const h16* values;           // [T, Hkv, D]
  const int32_t* slot_mapping; // [T]
  uint32_t* kc;                // [nb, Hkv, bs, D*b/32]
  h16 *ks, *kb;                // [nb, Hkv, D/gs, bs]
  uint32_t* vc;                // [nb, Hkv, bs/T, D, T*b/32], T = min(bs, 256/b) (v_word_index)
  h16 *vs, *vb;                // [nb, Hkv, D/gs, bs]
  int T, Hkv, D, gs, bs, nb;
  RopeArgs rope;               // K rotation before quantizing (inv_freq null: none)
  h16* q;                      // [T, Hq, D] turned queries, written by the same launch (null: none)
  const h16* q_in;             // the queries to turn (== q: in place)
  int Hq;
  // Decode append (slot_mapping null): token t is the next token of sequence
  // slot_ids[t]; its position is kv_lens[slot] and its slot comes from the block
  // table (the arithmetic of cache_slots), and kv_lens advances by one.
  const int32_t* slot_ids;     // [T]
  int32_t* kv_lens;            // [S]
  const int32_t* bt;           // [S, max_blocks]
  int S, max_blocks;
  int* counter;                // workgroups that have read kv_lens: zero before and after every launch
};

constexpr int kQRopeBlocks = 4;     // extra workgroup rows of the small write that turn the queries
constexpr int kSmallRopeTab = 2048;  // (token, pair) angles the query workgroups tabulate

// One workgroup per (32 consecutive tokens, kv head):
//   1. per (token, group, K|V): min/max -> scale/bias (kept in LDS, stored as fp16);
//   2. K codes: one 32-bit word per (token, 32/BITS dims), plain stores;
//   3. V codes: 4-bit words hold 8 tokens of one dim.  When the 8 tokens of an
//      aligned octet have consecutive slots starting at a word boundary (a
//      prefill chunk), the word is written whole; otherwise (decode appends,
//      chunk edges) each token updates its nibble atomically.  8-bit codes are
//      single bytes and are stored directly.
constexpr int kWriteTokens = 32;
constexpr int kWriteMaxGroups = 32;
constexpr int kWriteMaxDim = 256;

template <int BITS>
__global__ __launch_bounds__(256) void affine_cache_write(WriteArgs a) {
  constexpr int TW = kWriteTokens;
  constexpr int PW = 32 / BITS;
  const int tid = threadIdx.x;
  const int t0 = blockIdx.x * TW;
  const int h = blockIdx.y;
  const int nt = min(TW, a.T - t0);
  const int G = a.D / a.gs;
  const float n_bins = (float)((1 << BITS) - 1);

  __shared__ float sp[2][TW][kWriteMaxGroups][2];  // [K|V][token][group] -> (scale, bias)
  __shared__ int sslot[TW];
  __shared__ __attribute__((aligned(16))) h16 sval[2][TW][kWriteMaxDim];  // this head's K / V rows
  if (tid < TW) {
    int sl = tid < nt ? a.slot_mapping[t0 + tid] : -1;
    if (sl >= 0 && sl / a.bs >= a.nb) sl = -1;  // page out of range: not written
    sslot[tid] = sl;
  }
  {  // one cooperative load of every value the block quantizes (16 bytes per piece)
    const int per_row = a.D / 8;
    for (int i = tid; i < 2 * nt * per_row; i += 256) {
      const int kv = i / (nt * per_row), r = i % (nt * per_row);
      const int t = r / per_row, c = r % per_row;
      const h16* src = (kv ? a.values : a.keys) + ((size_t)(t0 + t) * a.Hkv + h) * a.D + 8 * c;
      *reinterpret_cast<u32x4*>(&sval[kv][t][8 * c]) = *reinterpret_cast<const u32x4*>(src);
    }
  }
  __syncthreads();
  if (a.rope.inv_freq != nullptr) {  // fused RoPE: the K rows turn in LDS before quantizing
    const RopeArgs& r = a.rope;
    const int half = r.rot / 2;
    for (int task = tid; task < nt * half; task += 256) {
      const int t = task / half, p = task % half;
      const int i0 = r.traditional ? 2 * p : p, i1 = r.traditional ? 2 * p + 1 : p + half;
      rope_pair(sval[0][t][i0], sval[0][t][i1], (float)r.positions[t0 + t] * r.inv_freq[p]);
    }
    __syncthreads();
  }

  // ---- 1. scale / bias of every (K|V, token, group)
  for (int task = tid; task < 2 * TW * G; task += 256) {
    const int kv = task / (TW * G), rem = task % (TW * G);
    const int t = rem / G, g = rem % G;
    const int sl = t < nt ? sslot[t] : -1;
    if (sl < 0) continue;
    float wmin, wmax, scale, bias;
    lds_minmax(&sval[kv][t][g * a.gs], a.gs, wmin, wmax);
    affine_params(wmin, wmax, n_bins, scale, bias);
    sp[kv][t][g][0] = scale;
    sp[kv][t][g][1] = bias;
    const size_t ph = (size_t)(sl / a.bs) * a.Hkv + h;
    const size_t si = (ph * G + g) * a.bs + sl % a.bs;
    (kv ? a.vs : a.ks)[si] = (h16)scale;
    (kv ? a.vb : a.kb)[si] = (h16)bias;
  }
  __syncthreads();

  // ---- 2. K codes: token-major words
  const int KW = a.D / PW;
  for (int task = tid; task < TW * KW; task += 256) {
    const int t = task / KW, w = task % KW;
    const int sl = t < nt ? sslot[t] : -1;
    if (sl < 0) continue;
    const int g = (w * PW) / a.gs;
    const float sc = sp[0][t][g][0], bi = sp[0][t][g][1];
    const h16* src = &sval[0][t][w * PW];
    uint32_t word = 0;
#pragma unroll
    for (int k = 0; k < PW; ++k) word |= affine_code((float)src[k], sc, bi, n_bins) << (k * BITS);
    const size_t ph = (size_t)(sl / a.bs) * a.Hkv + h;
    a.kc[(ph * a.bs + sl % a.bs) * KW + w] = word;
  }

  // ---- 3. V codes
  if constexpr (BITS == 4) {
    for (int task = tid; task < (TW / 8) * a.D; task += 256) {
      const int o = task / a.D, d = task % a.D;
      const int g = d / a.gs;
      const int tb = 8 * o;
      const int s0 = tb < nt ? sslot[tb] : -1;
      bool whole = s0 >= 0 && s0 % 8 == 0 && tb + 8 <= nt;
#pragma unroll
      for (int k = 1; k < 8; ++k) whole = whole && sslot[tb + k] == s0 + k;
      if (whole) {
        uint32_t word = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float v = (float)sval[1][tb + k][d];
          word |= affine_code(v, sp[1][tb + k][g][0], sp[1][tb + k][g][1], n_bins) << v_shift<4>(k);
        }
        const size_t ph = (size_t)(s0 / a.bs) * a.Hkv + h;
        a.vc[v_word_index<4>(ph, s0 % a.bs, d, a.D, a.bs)] = word;
      } else {
        for (int k = 0; k < 8; ++k) {
          const int t = tb + k;
          const int sl = t < nt ? sslot[t] : -1;
          if (sl < 0) continue;
          const float v = (float)sval[1][t][d];
          const uint32_t code = affine_code(v, sp[1][t][g][0], sp[1][t][g][1], n_bins);
          const size_t ph = (size_t)(sl / a.bs) * a.Hkv + h;
          uint32_t* wp = a.vc + v_word_index<4>(ph, sl % a.bs, d, a.D, a.bs);
          const int sh = v_shift<4>(sl % 8);
          atomicAnd(wp, ~(0xFu << sh));
          atomicOr(wp, code << sh);
        }
      }
    }
  } else {
    for (int task = tid; task < TW * a.D; task += 256) {
      const int t = task / a.D, d = task % a.D;
      const int sl = t < nt ? sslot[t] : -1;
      if (sl < 0) continue;
      const int g = d / a.gs;
      const float v = (float)sval[1][t][d];
      const uint32_t code = affine_code(v, sp[1][t][g][0], sp[1][t][g][1], n_bins);
      const size_t ph = (size_t)(sl / a.bs) * a.Hkv + h;
      uint32_t* wp = a.vc + v_word_index<8>(ph, sl % a.bs, d, a.D, a.bs);
      reinterpret_cast<uint8_t*>(wp)[sl % 4] = (uint8_t)code;
    }
  }
}

// Small writes (decode appends, T <= kSmallWrite tokens): one workgroup per
// (kv head, 16-dim block) sees every token, so each value word has a single
// writing workgroup.  A token's 4-bit value code goes into its 8-token word by
// an atomic AND and OR that return nothing (tokens of the call sharing a word
// touch disjoint bits); a plain read-modify-write of the word (where no other
// token of the call shares it) measured 0.85 us slower per append, its read
// being one more round trip.  Scales, biases
// and K codes of the head are written by the workgroup of dim block 0 / by the
// owner of each K word.
constexpr int kSmallWrite = 128;
constexpr int kSmallMaxGroup = 64;

// ROPE: the K rows of every token are loaded whole, turned in LDS (pairs span
// quantization groups), and the block's group is taken from the turned rows.
template <int BITS, bool ROPE = false>
__global__ __launch_bounds__(256) void affine_cache_write_small(WriteArgs a) {
  constexpr int PW = 32 / BITS;
  constexpr int DB = 16;  // dims per workgroup
  const int tid = threadIdx.x;
  const int h = blockIdx.x;
  const int d0 = blockIdx.y * DB;
  // Decode append (a.slot_ids set): every workgroup derives the tokens' positions
  // and slots itself (cache_slots folded in; slots.hpp: position kv_lens[s], page
  // block_tables[s, position / bs], -1 for a slot id outside [0, S), a column past
  // the table or a negative page id), issuing those reads before its page data
  // loads so both are in flight together.  Once its kv_lens values are in LDS it
  // counts itself (the atomic's answer is only needed at its end); the workgroup
  // counted last advances kv_lens at its end, so no workgroup reads an advanced
  // length.
  const bool app = a.slot_ids != nullptr;
  __shared__ int spos[kSmallWrite];
  __shared__ int sseq[kSmallWrite];
  int sl_dev = -1, app_s = -1, app_pos = 0;
  RopeArgs rope = a.rope;
  // with ROPE, the positions (when given) and inv_freq go to LDS with the first
  // barrier: the rotation loops then read no global memory
  __shared__ float sinv[kWriteMaxDim / 2];
  const int half = ROPE ? rope.rot / 2 : 0;
  const float inv_in = ROPE && tid < half ? rope.inv_freq[tid] : 0.f;
  if (ROPE && !app && tid < a.T) app_pos = rope.positions[tid];
  if (app) {
    if (tid < a.T) {
      const int s = a.slot_ids[tid];
      if (s >= 0 && s < a.S) {
        app_s = s;
        app_pos = a.kv_lens[s];
        const int col = app_pos / a.bs;
        if (app_pos >= 0 && col < a.max_blocks) {
          const int b = a.bt[(size_t)s * a.max_blocks + col];
          if (b >= 0) sl_dev = b * a.bs + app_pos % a.bs;
        }
      }
    }
  }
  if (ROPE) {
    rope.positions = spos;
    rope.inv_freq = sinv;
  }
  int arrived = 0;
  auto publish = [&]() {  // before a barrier: this workgroup's positions and sequences to LDS
    if ((app || ROPE) && tid < a.T) {
      spos[tid] = app_pos;
      sseq[tid] = app_s;
    }
    if (ROPE && tid < half) sinv[tid] = inv_in;
  };
  auto count = [&]() {  // after that barrier: every kv_lens read of the workgroup has returned
    if (app && tid == 0) arrived = __hip_atomic_fetch_add(a.counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  auto finish = [&]() {  // the end of the workgroup: the last one counted advances kv_lens
    if (!app) return;
    __shared__ int slast;
    if (tid == 0) {
      const int nwg = (int)(gridDim.x * gridDim.y);
      slast = arrived == nwg - 1;
      if (arrived == nwg - 1) __hip_atomic_store(a.counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (slast && tid < a.T && sseq[tid] >= 0) a.kv_lens[sseq[tid]] = spos[tid] + 1;
  };
  const int T = a.T;
  if constexpr (ROPE) {
    // the extra rows of workgroups turn the queries (rows of gridDim.x * kQRopeBlocks workgroups)
    if (d0 >= a.D) {
      const int nwg = gridDim.x * kQRopeBlocks;
      const int wg = (blockIdx.y - a.D / DB) * gridDim.x + blockIdx.x;
      // 16-byte pieces, the first pass's loads in flight while the positions arrive
      const bool vec = a.q != nullptr && turn_rows_vec_ok(a.D, rope.rot, rope.traditional);
      constexpr int U = 2;
      TurnRowsVec<U> tv(a.T, a.Hq, a.D, rope);
      const int stride = nwg * 256;
      if (vec) tv.issue(a.q_in, a.D, rope, wg * 256 + tid, stride);
      publish();
      __syncthreads();
      count();
      // (sin, cos) of the call's (token, pair) angles once per workgroup, when they fit
      __shared__ float2 stab[kSmallRopeTab];
      const bool tab = vec && T * half <= kSmallRopeTab;
      if (tab) {
        for (int i = tid; i < T * half; i += 256) {
          float sn, cs;
          rope_sincos((float)spos[i / half] * sinv[i % half], &sn, &cs);
          stab[i] = float2{sn, cs};
        }
        __syncthreads();
      }
      if (vec) {
        tv.finish(a.q, a.Hq, a.D, rope, tab ? stab : nullptr);
        for (int i0 = wg * 256 + tid + U * stride; i0 < tv.n; i0 += U * stride) {
          tv.issue(a.q_in, a.D, rope, i0, stride);
          tv.finish(a.q, a.Hq, a.D, rope, tab ? stab : nullptr);
        }
      } else if (a.q != nullptr) {
        turn_rows(a.q, a.q_in, a.T, a.Hq, a.D, rope, (long)wg * 256 + tid, (long)stride);
      }
      finish();
      return;
    }
  }
  const int G = a.D / a.gs;
  const float n_bins = (float)((1 << BITS) - 1);
  __shared__ float sp[2][kSmallWrite][2];  // [K|V][token] -> (scale, bias) of this block's group
  __shared__ __attribute__((aligned(16))) h16 sgrp[2][kSmallWrite][kSmallMaxGroup];  // group values
  __shared__ __attribute__((aligned(16))) int sslot[kSmallWrite];
  // One round trip for what the workgroup reads: the tokens' slots and the
  // quantization group holding this dim block (neither depends on the other).
  // Every load is issued unconditionally (buffer loads: an offset past the end
  // returns zeros), so none waits behind a branch for the one before it.
  const int g = d0 / a.gs;
  constexpr int kOob = 0x7FFFFFF0;  // past the end of every descriptor below
  const int sl_raw = (int)__builtin_amdgcn_raw_buffer_load_b32(
      uniform_rsrc(a.slot_mapping, a.slot_mapping ? T * 4 : 0), tid < T ? tid * 4 : kOob, 0, kLoadAux);
  const int sl_in = tid < T ? (a.slot_ids != nullptr ? sl_dev : sl_raw) : -1;
  constexpr int kPieces = 2 * kSmallWrite * (kSmallMaxGroup / 8) / 256;  // 16-byte pieces per thread
  const int per_tok = a.gs / 8;
  const int row_bytes = T * a.Hkv * a.D * 2;
  const __amdgpu_buffer_rsrc_t rkey = uniform_rsrc(a.keys, row_bytes), rval = uniform_rsrc(a.values, row_bytes);
  // byte offset of piece c of token t's group (this head)
  auto goff = [&](int t, int c) { return ((t * a.Hkv + h) * a.D + g * a.gs + 8 * c) * 2; };
  u32x4 piece[kPieces];
  if constexpr (ROPE) {
    __shared__ __attribute__((aligned(16))) h16 krow[kSmallWrite][kWriteMaxDim];
#pragma unroll
    for (int k = 0; k < kPieces / 2; ++k) {  // V only: K comes from the turned rows
      const int i = tid + 256 * k;
      piece[k] = __builtin_amdgcn_raw_buffer_load_b128(rval, i < T * per_tok ? goff(i / per_tok, i % per_tok) : kOob,
                                                       0, kLoadAux);
    }
    // the head's K rows, four 16-byte pieces per thread in flight at a time
    for (int i0 = tid; i0 < T * (a.D / 8); i0 += 4 * 256) {
      u32x4 kp[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + 256 * u;
        const int t = i / (a.D / 8), c = i % (a.D / 8);
        kp[u] = __builtin_amdgcn_raw_buffer_load_b128(rkey, i < T * (a.D / 8) ? ((t * a.Hkv + h) * a.D + 8 * c) * 2 : kOob,
                                                      0, kLoadAux);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + 256 * u;
        if (i < T * (a.D / 8)) *reinterpret_cast<u32x4*>(&krow[i / (a.D / 8)][8 * (i % (a.D / 8))]) = kp[u];
      }
    }
    publish();
    __syncthreads();
    count();
    const RopeArgs& r = rope;  // positions and inv_freq in LDS
    for (int task = tid; task < T * half; task += 256) {
      const int t = task / half, p = task % half;
      const int i0 = r.traditional ? 2 * p : p, i1 = r.traditional ? 2 * p + 1 : p + half;
      rope_pair(krow[t][i0], krow[t][i1], (float)spos[t] * sinv[p]);
    }
    __syncthreads();
    for (int i = tid; i < T * per_tok; i += 256) {
      const int t = i / per_tok, c = i % per_tok;
      *reinterpret_cast<u32x4*>(&sgrp[0][t][8 * c]) = *reinterpret_cast<const u32x4*>(&krow[t][g * a.gs + 8 * c]);
    }
#pragma unroll
    for (int k = 0; k < kPieces / 2; ++k) {
      const int i = tid + 256 * k;
      if (i < T * per_tok) *reinterpret_cast<u32x4*>(&sgrp[1][i / per_tok][8 * (i % per_tok)]) = piece[k];
    }
  } else {
#pragma unroll
    for (int k = 0; k < kPieces; ++k) {  // pieces of K first, then of V (a piece index is uniform in kv per k
      const int i = tid + 256 * k;      // only when T * per_tok is a multiple of 256, so both are issued)
      const int r = i % (T * per_tok);
      const int off = i < 2 * T * per_tok ? goff(r / per_tok, r % per_tok) : kOob;
      const u32x4 pk = __builtin_amdgcn_raw_buffer_load_b128(rkey, i < T * per_tok ? off : kOob, 0, kLoadAux);
      const u32x4 pv = __builtin_amdgcn_raw_buffer_load_b128(rval, i >= T * per_tok ? off : kOob, 0, kLoadAux);
      piece[k] = pk | pv;  // one of the two is zeros
    }
#pragma unroll
    for (int k = 0; k < kPieces; ++k) {
      const int i = tid + 256 * k;
      if (i < 2 * T * per_tok) {
        const int kv = i / (T * per_tok), r = i % (T * per_tok);
        *reinterpret_cast<u32x4*>(&sgrp[kv][r / per_tok][8 * (r % per_tok)]) = piece[k];
      }
    }
  }
  if (tid < T) sslot[tid] = sl_in >= 0 && sl_in / a.bs >= a.nb ? -1 : sl_in;  // page out of range: not written
  if constexpr (!ROPE) publish();  // (with ROPE: published at the K rows' barrier above)
  __syncthreads();
  if constexpr (!ROPE) count();
  constexpr int kVTasks = kSmallWrite * DB / 256;
  // scale / bias of each (K|V, token) of this block's group, into LDS
  for (int task = tid; task < 2 * T; task += 256) {
    const int kv = task / T, t = task % T;
    const int sl = sslot[t];
    if (sl < 0) continue;
    float wmin, wmax, scale, bias;
    lds_minmax(&sgrp[kv][t][0], a.gs, wmin, wmax);
    affine_params(wmin, wmax, n_bins, scale, bias);
    sp[kv][t][0] = scale;
    sp[kv][t][1] = bias;
  }
  __syncthreads();
  // (stored after the barrier: a barrier waits for the stores issued before it)
  if (d0 % a.gs == 0) {  // the first dim block of each group stores them
    for (int task = tid; task < 2 * T; task += 256) {
      const int kv = task / T, t = task % T;
      const int sl = sslot[t];
      if (sl < 0) continue;
      const size_t ph = (size_t)(sl / a.bs) * a.Hkv + h;
      const size_t si = (ph * G + g) * a.bs + sl % a.bs;
      (kv ? a.vs : a.ks)[si] = (h16)sp[kv][t][0];
      (kv ? a.vb : a.kb)[si] = (h16)sp[kv][t][1];
    }
  }
  // K words of this block: DB / PW per token
  for (int task = tid; task < T * (DB / PW); task += 256) {
    const int t = task / (DB / PW), w = d0 / PW + task % (DB / PW);
    const int sl = sslot[t];
    if (sl < 0) continue;
    const h16* src = &sgrp[0][t][w * PW - g * a.gs];
    uint32_t word = 0;
#pragma unroll
    for (int k = 0; k < PW; ++k) word |= affine_code((float)src[k], sp[0][t][0], sp[0][t][1], n_bins) << (k * BITS);
    const size_t ph = (size_t)(sl / a.bs) * a.Hkv + h;
    a.kc[(ph * a.bs + sl % a.bs) * (a.D / PW) + w] = word;
  }
  // V codes: one value per (token, dim)
#pragma unroll
  for (int k = 0; k < kVTasks; ++k) {
    const int task = tid + 256 * k;
    if (task >= T * DB) continue;
    const int t = task / DB, d = d0 + task % DB;
    const int sl = sslot[t];
    if (sl < 0) continue;
    const float v = (float)sgrp[1][t][d - g * a.gs];
    const uint32_t code = affine_code(v, sp[1][t][0], sp[1][t][1], n_bins);
    const size_t ph = (size_t)(sl / a.bs) * a.Hkv + h;
    uint32_t* wp = a.vc + v_word_index<BITS>(ph, sl % a.bs, d, a.D, a.bs);
    const int sh = v_shift<BITS>(sl % PW);
    constexpr uint32_t M = (1u << BITS) - 1u;
    if (BITS == 8) {
      reinterpret_cast<uint8_t*>(wp)[sl % 4] = (uint8_t)code;
    } else {  // the nibble by two atomics that return nothing: no read of the word to wait for
      atomicAnd(wp, ~(M << sh));
      atomicOr(wp, code << sh);
    }
  }
  finish();
}

#pragma clang fp contract(on)


}  // namespace emx
