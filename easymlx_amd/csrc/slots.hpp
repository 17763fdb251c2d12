// Device-side write-position arithmetic of a cache write and the unquantized
// cache write, so that a write needs no host round trip (and can be captured
// in a HIP graph).
//
// cache_slots follows PageCacheView.concatenate_to_cache
// (lib/python/easymlx/caching/paged/cache.py:1126-1170 decode, :1211-1261
// multi-token) and the compiled decode proxy
// (lib/python/easymlx/inference/esurge/runners/model_runner.py:164-184):
//   token t of sequence i (query_start_loc[i] <= t < query_start_loc[i+1]) of
//   slot s = slot_ids[i] sits at position p = kv_lens[s] + (t - query_start_loc[i]),
//   in page block_tables[s, p / bs] at offset p % bs;
//   afterwards kv_lens[s] = old kv_lens[s] + query length of i.
// A token whose slot is outside [0, num_seqs), whose page column is beyond the
// table or whose block id is negative gets slot -1 (the write kernels skip it).
//
// dense_cache_write is reshape_and_cache for an unquantized cache
// [nb, bs, Hkv, D] (cache.py:36-93, the cast-and-scatter of :1186-1190).
#pragma once

#include "common.hpp"

namespace emx {

constexpr int kMaxSlots = 4096;  // sequences of one write (LDS tables of cache_slots)

struct SlotArgs {
  const int32_t* slot_ids;  // [n]
  const int32_t* qsl;       // [n + 1] token offsets of the write's sequences
  int n, T;                 // sequences written, tokens written (= qsl[n])
  const int32_t* bt;        // [S, max_blocks]
  int S, max_blocks, bs;
  int32_t* kv_lens;         // [S], advanced in place
  int32_t* mapping;         // [T] out: block * bs + offset, or -1
  int32_t* positions;       // [T] out: position of the token in its sequence
};

// One workgroup: every kv_lens entry is read before any is advanced.
__global__ __launch_bounds__(1024) void cache_slots(SlotArgs a) {
  __shared__ int sq[kMaxSlots + 1];
  __shared__ int sbase[kMaxSlots];
  __shared__ int sslot[kMaxSlots];
  for (int i = threadIdx.x; i <= a.n; i += 1024) sq[i] = a.qsl[i];
  for (int i = threadIdx.x; i < a.n; i += 1024) {
    const int s = a.slot_ids[i];
    const bool ok = s >= 0 && s < a.S;
    sslot[i] = ok ? s : -1;
    sbase[i] = ok ? a.kv_lens[s] : 0;
  }
  __syncthreads();
  for (int t = threadIdx.x; t < a.T; t += 1024) {
    int lo = 0, hi = a.n;  // the i with sq[i] <= t < sq[i + 1]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (sq[mid] <= t)
        lo = mid;
      else
        hi = mid;
    }
    const int s = sslot[lo];
    const int pos = sbase[lo] + (t - sq[lo]);
    const int col = pos / a.bs;
    int m = -1;
    if (s >= 0 && pos >= 0 && col < a.max_blocks) {
      const int b = a.bt[(size_t)s * a.max_blocks + col];
      if (b >= 0) m = b * a.bs + pos % a.bs;
    }
    a.mapping[t] = m;
    a.positions[t] = pos;
  }
  for (int i = threadIdx.x; i < a.n; i += 1024) {
    const int s = sslot[i];
    if (s >= 0) a.kv_lens[s] = sbase[i] + max(0, sq[i + 1] - sq[i]);
  }
}

// Token t's rows [Hkv, D] of keys/values to slot mapping[t] of an unquantized
// cache in the same dtype (4-byte words; -1 or a page outside the pool skips).
__global__ __launch_bounds__(256) void dense_cache_write(const uint32_t* k, const uint32_t* v, const int32_t* mapping,
                                                         int T, int row_words, int bs, int nb, uint32_t* kc,
                                                         uint32_t* vc) {
  const long n = (long)T * row_words;
  for (long e = (long)blockIdx.x * 256 + threadIdx.x; e < n; e += (long)gridDim.x * 256) {
    const int t = (int)(e / row_words), w = (int)(e % row_words);
    const int m = mapping[t];
    if (m < 0 || m / bs >= nb) continue;
    kc[(size_t)m * row_words + w] = k[e];
    vc[(size_t)m * row_words + w] = v[e];
  }
}

}  // namespace emx
