// Page lifecycle kernels: copy-on-write block copies and page zeroing over
// every array of a cache (codes, scales, biases: each [num_blocks, ...]).
//
// copy_blocks follows PageCacheView.copy_blocks
// (lib/python/easymlx/caching/paged/cache.py:944-972; Metal kernel :95-136):
// for each pair (src, dst) of block_mapping [num_pairs, 2], block dst of every
// array becomes a copy of block src as it was before the call (the reference
// kernel reads its input arrays and writes separate outputs), so swapped and
// chained pairs are well defined; of several pairs with one destination the
// last one counts.  Two launches through a staging buffer: every pair's source
// blocks are gathered, then scattered to the destinations.  zero_blocks
// follows the runner's _zero_pages (lib/python/easymlx/inference/esurge/
// runners/model_runner.py:1058-1094) and PageCacheView.reset (cache.py:874-906,
// pages addressed by id): the listed blocks of every array become zero.  Block
// ids outside [0, num_blocks) are skipped.  One workgroup per (pair or page,
// array); 16-byte words when a block's bytes allow it, else 4-byte words.
#pragma once

#include "common.hpp"

namespace emx {

constexpr int kMaxPageArrays = 8;

struct PageArrays {
  void* base[kMaxPageArrays];
  long long block_bytes[kMaxPageArrays];  // bytes of one block of the array (a multiple of 4)
  long long stage_off[kMaxPageArrays];    // copy_blocks: byte offset of the array's staged blocks
  char* stage;                            // copy_blocks: staging buffer (16-byte aligned)
  int n;
  int nb;
};

template <typename W>
__device__ __forceinline__ void copy_words(const char* src, char* dst, long long bytes) {
  const W* s = reinterpret_cast<const W*>(src);
  W* d = reinterpret_cast<W*>(dst);
  const long long n = bytes / (long long)sizeof(W);
  for (long long i = threadIdx.x; i < n; i += blockDim.x) d[i] = s[i];
}

template <typename W>
__device__ __forceinline__ void zero_words(char* dst, long long bytes) {
  W* d = reinterpret_cast<W*>(dst);
  const long long n = bytes / (long long)sizeof(W);
  for (long long i = threadIdx.x; i < n; i += blockDim.x) d[i] = W{};
}

template <typename W>
__device__ __forceinline__ void copy_block(const char* s, char* d, const long long bb, const bool w16) {
  if (w16)
    copy_words<u32x4>(s, d, bb);
  else
    copy_words<uint32_t>(s, d, bb);
}

// grid (num_pairs, n arrays): staged block p of array k <- block src of pair p
__global__ __launch_bounds__(256) void copy_blocks_gather(PageArrays a, const int32_t* mapping) {
  const int p = blockIdx.x, k = blockIdx.y;
  const int src = mapping[2 * p], dst = mapping[2 * p + 1];
  if (src < 0 || src >= a.nb || dst < 0 || dst >= a.nb || src == dst) return;
  const long long bb = a.block_bytes[k];
  const bool w16 = bb % 16 == 0 && (reinterpret_cast<uintptr_t>(a.base[k]) & 15) == 0;
  copy_block<int>(static_cast<const char*>(a.base[k]) + (long long)src * bb, a.stage + a.stage_off[k] + p * bb, bb,
                  w16);
}

// grid (num_pairs, n arrays): block dst of pair p <- staged block p, unless a later
// pair has the same destination
__global__ __launch_bounds__(256) void copy_blocks_scatter(PageArrays a, const int32_t* mapping, const int num_pairs) {
  const int p = blockIdx.x, k = blockIdx.y;
  const int src = mapping[2 * p], dst = mapping[2 * p + 1];
  if (src < 0 || src >= a.nb || dst < 0 || dst >= a.nb || src == dst) return;
  int later = 0;
  for (int q = p + 1 + (int)threadIdx.x; q < num_pairs; q += blockDim.x) {
    const int s2 = mapping[2 * q], d2 = mapping[2 * q + 1];
    later |= d2 == dst && s2 >= 0 && s2 < a.nb && s2 != d2;
  }
  if (__syncthreads_or(later)) return;
  const long long bb = a.block_bytes[k];
  const bool w16 = bb % 16 == 0 && (reinterpret_cast<uintptr_t>(a.base[k]) & 15) == 0;
  copy_block<int>(a.stage + a.stage_off[k] + p * bb, static_cast<char*>(a.base[k]) + (long long)dst * bb, bb, w16);
}

// grid (num_pages, n arrays)
__global__ __launch_bounds__(256) void zero_blocks(PageArrays a, const int32_t* pages) {
  const int p = blockIdx.x, k = blockIdx.y;
  const int b = pages[p];
  if (b < 0 || b >= a.nb) return;
  const long long bb = a.block_bytes[k];
  char* d = static_cast<char*>(a.base[k]) + (long long)b * bb;
  if (bb % 16 == 0 && (reinterpret_cast<uintptr_t>(a.base[k]) & 15) == 0)
    zero_words<u32x4>(d, bb);
  else
    zero_words<uint32_t>(d, bb);
}


// Conversions between the logical affine layout (what mlx.core.quantize of the
// reference's dense cache [nb, bs, Hkv, D] gives; cache.py:790-791):
//   codes uint32 [nb, bs, Hkv, D*b/32] (dims packed along a word, dim d at bits
//   (d % (32/b)) * b), scales / biases fp16 [nb, bs, Hkv, D/gs]
// and the page layout the kernels read (k codes [nb, Hkv, bs, W], v codes
// tiled dim-major with v_word_index / v_shift, scales [nb, Hkv, G, bs]).
// One thread per destination element (grid-stride), so each is written once.
struct LayoutArgs {
  const uint32_t* sk;  // source K codes
  const uint32_t* sv;  // source V codes
  const h16* ss[4];    // source k_scales, k_biases, v_scales, v_biases
  uint32_t* dk;
  uint32_t* dv;
  h16* ds[4];
  int nb, bs, Hkv, D, gs;
};

// code of (block b, token t, head h, dim d) in the logical layout
template <int BITS>
__device__ __forceinline__ uint32_t logical_code(const uint32_t* c, const LayoutArgs& a, int b, int t, int h, int d) {
  constexpr int PW = 32 / BITS;
  const uint32_t w = c[(((size_t)b * a.bs + t) * a.Hkv + h) * (a.D / PW) + d / PW];
  return (w >> ((d % PW) * BITS)) & ((1u << BITS) - 1u);
}

template <int BITS>
__global__ __launch_bounds__(256) void pages_from_logical(LayoutArgs a) {
  constexpr int PW = 32 / BITS;
  const int W = a.D / PW, G = a.D / a.gs;
  const long nk = (long)a.nb * a.Hkv * a.bs * W;  // K words (and V words: the same count)
  const long ns = (long)a.nb * a.Hkv * G * a.bs;  // scale elements per array
  const long stride = (long)gridDim.x * 256;
  for (long e = (long)blockIdx.x * 256 + threadIdx.x; e < nk; e += stride) {
    // K: page order (b, h, t, w)
    const int w = (int)(e % W), t = (int)((e / W) % a.bs), h = (int)((e / W / a.bs) % a.Hkv);
    const int b = (int)(e / W / a.bs / a.Hkv);
    a.dk[e] = a.sk[(((size_t)b * a.bs + t) * a.Hkv + h) * W + w];
  }
  // V: one destination word = PW consecutive tokens of one dim (tiles of T tokens)
  constexpr int TMAX = 256 / BITS;
  const int T = a.bs < TMAX ? a.bs : TMAX;
  const int WPD = T / PW;  // words per dim inside a tile
  for (long e = (long)blockIdx.x * 256 + threadIdx.x; e < nk; e += stride) {
    const int u = (int)(e % WPD);
    const int d = (int)((e / WPD) % a.D);
    const long tile = e / WPD / a.D;  // (ph, j)
    const int j = (int)(tile % (a.bs / T));
    const long ph = tile / (a.bs / T);
    const int h = (int)(ph % a.Hkv), b = (int)(ph / a.Hkv);
    uint32_t word = 0;
    for (int k = 0; k < PW; ++k) {
      const int off = j * T + u * PW + k;
      word |= logical_code<BITS>(a.sv, a, b, off, h, d) << v_shift<BITS>(off % PW);
    }
    a.dv[e] = word;
  }
  for (long e = (long)blockIdx.x * 256 + threadIdx.x; e < ns; e += stride) {
    const int t = (int)(e % a.bs), g = (int)((e / a.bs) % G), h = (int)((e / a.bs / G) % a.Hkv);
    const int b = (int)(e / a.bs / G / a.Hkv);
    const size_t src = (((size_t)b * a.bs + t) * a.Hkv + h) * G + g;
#pragma unroll
    for (int i = 0; i < 4; ++i) a.ds[i][e] = a.ss[i][src];
  }
}

template <int BITS>
__global__ __launch_bounds__(256) void logical_from_pages(LayoutArgs a) {
  constexpr int PW = 32 / BITS;
  const int W = a.D / PW, G = a.D / a.gs;
  const long nk = (long)a.nb * a.bs * a.Hkv * W;
  const long ns = (long)a.nb * a.bs * a.Hkv * G;
  const long stride = (long)gridDim.x * 256;
  for (long e = (long)blockIdx.x * 256 + threadIdx.x; e < nk; e += stride) {
    // logical order (b, t, h, w)
    const int w = (int)(e % W), h = (int)((e / W) % a.Hkv), t = (int)((e / W / a.Hkv) % a.bs);
    const int b = (int)(e / W / a.Hkv / a.bs);
    const size_t ph = (size_t)b * a.Hkv + h;
    a.dk[e] = a.sk[(ph * a.bs + t) * W + w];
    uint32_t word = 0;
    for (int k = 0; k < PW; ++k) {  // dims w*PW .. + PW - 1 of token t
      const int d = w * PW + k;
      const uint32_t pw = a.sv[v_word_index<BITS>(ph, t, d, a.D, a.bs)];
      word |= ((pw >> v_shift<BITS>(t % PW)) & ((1u << BITS) - 1u)) << (k * BITS);
    }
    a.dv[e] = word;
  }
  for (long e = (long)blockIdx.x * 256 + threadIdx.x; e < ns; e += stride) {
    const int g = (int)(e % G), h = (int)((e / G) % a.Hkv), t = (int)((e / G / a.Hkv) % a.bs);
    const int b = (int)(e / G / a.Hkv / a.bs);
    const size_t src = (((size_t)b * a.Hkv + h) * G + g) * a.bs + t;
#pragma unroll
    for (int i = 0; i < 4; ++i) a.ds[i][e] = a.ss[i][src];
  }
}

}  // namespace emx
