// Page lifecycle kernels: copy-on-write block copies and page zeroing over
// every array of a cache (codes, scales, biases: each [num_blocks, ...]).
//
// copy_blocks follows PageCacheView.copy_blocks
// (lib/python/easymlx/caching/paged/cache.py:944-972; Metal kernel :95-136):
// for each pair (src, dst) of block_mapping [num_pairs, 2], block dst of every
// array becomes a copy of block src.  zero_blocks follows the runner's
// _zero_pages (lib/python/easymlx/inference/esurge/runners/model_runner.py:
// 1058-1094) and PageCacheView.reset (cache.py:874-906, pages addressed by id):
// the listed blocks of every array become zero.  Block ids outside
// [0, num_blocks) are skipped.  One workgroup per (pair or page, array);
// 16-byte words when a block's bytes allow it, else 4-byte words.
#pragma once

#include "common.hpp"

namespace emx {

constexpr int kMaxPageArrays = 8;

struct PageArrays {
  void* base[kMaxPageArrays];
  long long block_bytes[kMaxPageArrays];  // bytes of one block of the array (a multiple of 4)
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

// grid (num_pairs, n arrays)
__global__ __launch_bounds__(256) void copy_blocks(PageArrays a, const int32_t* mapping) {
  const int p = blockIdx.x, k = blockIdx.y;
  const int src = mapping[2 * p], dst = mapping[2 * p + 1];
  if (src < 0 || src >= a.nb || dst < 0 || dst >= a.nb || src == dst) return;
  const long long bb = a.block_bytes[k];
  const char* s = static_cast<const char*>(a.base[k]) + (long long)src * bb;
  char* d = static_cast<char*>(a.base[k]) + (long long)dst * bb;
  if (bb % 16 == 0 && (reinterpret_cast<uintptr_t>(a.base[k]) & 15) == 0)
    copy_words<u32x4>(s, d, bb);
  else
    copy_words<uint32_t>(s, d, bb);
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

}  // namespace emx
