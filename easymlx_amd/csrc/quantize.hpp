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

struct WriteArgs {
  const h16* keys;             // [T, Hkv, D]
  const h16* values;           // [T, Hkv, D]
  const int32_t* slot_mapping; // [T]
  uint32_t* kc;                // [nb, Hkv, bs, D*b/32]
  h16 *ks, *kb;                // [nb, Hkv, D/gs, bs]
  uint32_t* vc;                // [nb, Hkv, bs/T, D, T*b/32], T = min(bs, 256/b) (v_word_index)
  h16 *vs, *vb;                // [nb, Hkv, D/gs, bs]
  int T, Hkv, D, gs, bs, nb;
};

// One thread per (token, kv_head, group, {K, V}).
template <int BITS>
__global__ __launch_bounds__(256) void affine_cache_write(WriteArgs a) {
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int G = a.D / a.gs;
  const long per_tok = (long)a.Hkv * G * 2;
  if (gid >= (long)a.T * per_tok) return;
  const int t = (int)(gid / per_tok);
  int rem = (int)(gid % per_tok);
  const int is_v = rem & 1;
  rem >>= 1;
  const int h = rem / G;
  const int g = rem % G;
  const int slot = a.slot_mapping[t];
  if (slot < 0) return;
  const int blk = slot / a.bs;
  const int off = slot % a.bs;
  if (blk >= a.nb) return;

  const float n_bins = (float)((1 << BITS) - 1);
  const h16* src = (is_v ? a.values : a.keys) + ((size_t)t * a.Hkv + h) * a.D + (size_t)g * a.gs;
  float wmin, wmax, scale, bias;
  group_minmax(src, a.gs, wmin, wmax);
  affine_params(wmin, wmax, n_bins, scale, bias);
  const size_t ph = (size_t)blk * a.Hkv + h;
  const size_t si = (ph * G + g) * a.bs + off;
  constexpr int PW = 32 / BITS;
  if (!is_v) {
    uint32_t* dst = a.kc + (ph * a.bs + off) * (a.D / PW) + (size_t)g * (a.gs / PW);
    for (int w = 0; w < a.gs / PW; ++w) {
      uint32_t word = 0;
#pragma unroll
      for (int k = 0; k < PW; ++k) word |= affine_code((float)src[w * PW + k], scale, bias, n_bins) << (k * BITS);
      dst[w] = word;
    }
    a.ks[si] = (h16)scale;
    a.kb[si] = (h16)bias;
  } else {
    for (int i = 0; i < a.gs; ++i) {
      const uint32_t code = affine_code((float)src[i], scale, bias, n_bins);
      uint32_t* wp = a.vc + v_word_index<BITS>(ph, off, g * a.gs + i, a.D, a.bs);
      if constexpr (BITS == 8) {
        reinterpret_cast<uint8_t*>(wp)[off % PW] = (uint8_t)code;
      } else {
        const int sh = (off % PW) * BITS;
        atomicAnd(wp, ~(0xFu << sh));
        atomicOr(wp, code << sh);
      }
    }
    a.vs[si] = (h16)scale;
    a.vb[si] = (h16)bias;
  }
}

#pragma clang fp contract(on)

}  // namespace emx
