// Page-read probe: reads exactly the page bytes a 4-bit / 8-bit affine decode
// call over head_dim 128 reads (K codes, V codes and the four scale / bias
// runs of every 64-token slice of a page-head that holds a live token), with
// nothing else to do, so its rate is the read bandwidth the memory system
// gives this call's scattered access pattern.  Measurement only: it has no
// counterpart in the reference and computes no attention.
//
// Each wave takes slices round-robin (slice i, i + waves, ...) with two slices
// in flight (the next one's loads issued before the current one is consumed).
// Loads are unconditional buffer loads through per-slice descriptors (an empty
// descriptor for a slice without a live token reads nothing), so the compiler
// counts them exactly and never drains the slice in flight.  Every lane XORs
// the 16-byte pieces it read and each workgroup stores one word, so a test can
// check that exactly these bytes were read.
#pragma once

#include "common.hpp"

namespace emx {

struct ProbeArgs {
  const uint32_t* kc;  // [nb, Hkv, bs, 128*BITS/32]
  const h16 *ks, *kb, *vs, *vb;  // [nb, Hkv, G, bs]
  const uint32_t* vc;  // [nb, Hkv, bs/NT, 128, 8]
  const int32_t* block_tables;  // [S, max_blocks]
  const int32_t* kv_lens;       // [S]
  uint32_t* sink;               // [gridDim.x]
  int S, Hkv, bs, nb, max_blocks, G;
  int nsl;                      // slices: S * max_blocks * (bs / 64) * Hkv (< 2^31, checked on the host)
};

// Slice i = ((s * max_blocks + page) * (bs / 64) + half) * Hkv + kvh.
template <int BITS>
__global__ __launch_bounds__(256) void probe_page_read(ProbeArgs a) {
  constexpr int D = 128, NT = BITS == 4 ? 64 : 32;
  constexpr int CH = 64 * D * BITS / 8 / 16 / 64;  // 16-byte pieces per lane of K (and of V) per slice
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6)), nwaves = gridDim.x * 4;
  const int halves = a.bs / 64, nsl = a.nsl;
  struct Buf {
    u32x4 k[CH], v[CH], s[4];
  };
  // page id of slice i, -1 when it holds no live token or its page id is invalid
  auto page_of = [&](int i) {
    const int r = i / a.Hkv;
    const int half = r % halves, pg = (r / halves) % a.max_blocks, s = r / halves / a.max_blocks;
    int kl = a.kv_lens[s];
    kl = kl < 0 ? 0 : kl;
    if (pg * a.bs + half * 64 >= kl) return -1;
    const int b = a.block_tables[(size_t)s * a.max_blocks + pg];
    return (unsigned)b < (unsigned)a.nb ? b : -1;
  };
  // The page ids of the wave's next 64 slices are looked up together (lane k: slice
  // i + k * nwaves), so no slice's page loads wait behind a table lookup.
  int chunk0 = -64, pids = -1;
  const int soff = lane < 8 * a.G ? ((lane >> 3) * a.bs + 8 * (lane & 7)) * 2 : 0x40000000;  // scale piece offset
  auto issue = [&](int i, Buf& x) {
    const int k = (i - wave) / nwaves;  // this wave's k-th slice
    if (k - chunk0 >= 64) {
      chunk0 = k;
      const long long il = wave + (long long)(k + lane) * nwaves;
      pids = il < nsl ? page_of((int)il) : -1;
    }
    const int b = i < nsl ? __builtin_amdgcn_readlane(pids, k - chunk0) : -1;
    const bool ok = b >= 0;
    const int kvh = i % a.Hkv, t0 = ((i / a.Hkv) % halves) * 64;
    const size_t ph = (size_t)(ok ? b : 0) * a.Hkv + kvh;
    const __amdgpu_buffer_rsrc_t rk =
        uniform_rsrc(a.kc + (ph * a.bs + t0) * (D * BITS / 32), ok ? 64 * D * BITS / 8 : 0);
    const __amdgpu_buffer_rsrc_t rv =
        uniform_rsrc(a.vc + ph * D * (a.bs * BITS / 32) + (t0 / NT) * D * 8, ok ? 64 * D * BITS / 8 : 0);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      x.k[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, (64 * c + lane) * 16, 0, 0));
      x.v[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, (64 * c + lane) * 16, 0, 0));
    }
    // scales: per array, lanes 8g .. 8g+7 read group g's 64 halves (128 bytes)
    const h16* sp[4] = {a.ks, a.kb, a.vs, a.vb};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const __amdgpu_buffer_rsrc_t rs = uniform_rsrc(sp[r] + ph * a.G * a.bs + t0, ok ? (a.G * a.bs - t0) * 2 : 0);
      x.s[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, soff, 0, 0));
    }
  };
  u32x4 acc = {0u, 0u, 0u, 0u};
  auto fold = [&](const Buf& x) {
#pragma unroll
    for (int c = 0; c < CH; ++c) acc ^= x.k[c] ^ x.v[c];
#pragma unroll
    for (int r = 0; r < 4; ++r) acc ^= x.s[r];
  };
  Buf A, B;
  int i = wave;
  if (i < nsl) {
    issue(i, A);
    for (; i < nsl; i += 2 * nwaves) {
      issue(i + nwaves, B);
      __builtin_amdgcn_sched_barrier(0);  // the next slice's loads go out before this one is waited for
      fold(A);
      if (i + nwaves >= nsl) break;
      issue(i + 2 * nwaves, A);
      __builtin_amdgcn_sched_barrier(0);
      fold(B);
    }
  }
  uint32_t w = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  for (int o = 1; o < 64; o <<= 1) w ^= __shfl_xor(w, o, 64);
  __shared__ uint32_t part[4];
  if (lane == 0) part[threadIdx.x >> 6] = w;
  __syncthreads();
  if (threadIdx.x == 0) a.sink[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

// The same over an FP8 (E4M3) cache in the reference layout [nb, bs, Hkv, 128]
// uint8 with one fp32 scale per page (k_scale / v_scale [nb]): slices of 32
// tokens of one kv head (the FP8 decode's work item: 32 rows of 128 bytes,
// Hkv * 128 bytes apart, for K and for V, and the page's two scales).
// Slice i = ((s * max_blocks + page) * (bs / 32) + part) * Hkv + kvh.  The XOR
// covers the scales' bits too (once per slice).
struct ProbeFp8Args {
  const uint8_t *k8, *v8;       // [nb, bs, Hkv, 128]
  const float *kps, *vps;       // [nb]
  const int32_t* block_tables;  // [S, max_blocks]
  const int32_t* kv_lens;       // [S]
  uint32_t* sink;               // [gridDim.x]
  int S, Hkv, bs, nb, max_blocks;
  int nsl;                      // slices: S * max_blocks * (bs / 32) * Hkv (< 2^31, checked on the host)
};

__global__ __launch_bounds__(256) void probe_page_read_fp8(ProbeFp8Args a) {
  constexpr int D = 128, NT = 32;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6)), nwaves = gridDim.x * 4;
  const int parts = a.bs / NT, nsl = a.nsl;
  struct Buf {
    u32x4 k[4], v[4];
    uint32_t sk, sv;
  };
  auto page_of = [&](int i) {
    const int r = i / a.Hkv;
    const int part = r % parts, pg = (r / parts) % a.max_blocks, s = r / parts / a.max_blocks;
    int kl = a.kv_lens[s];
    kl = kl < 0 ? 0 : kl;
    if (pg * a.bs + part * NT >= kl) return -1;
    const int b = a.block_tables[(size_t)s * a.max_blocks + pg];
    return (unsigned)b < (unsigned)a.nb ? b : -1;
  };
  int chunk0 = -64, pids = -1;
  const int rowb = a.Hkv * D;  // bytes between the rows of consecutive tokens
  auto issue = [&](int i, Buf& x) {
    const int k = (i - wave) / nwaves;
    if (k - chunk0 >= 64) {
      chunk0 = k;
      const long long il = wave + (long long)(k + lane) * nwaves;
      pids = il < nsl ? page_of((int)il) : -1;
    }
    const int b = i < nsl ? __builtin_amdgcn_readlane(pids, k - chunk0) : -1;
    const bool ok = b >= 0;
    const int kvh = i % a.Hkv, t0 = ((i / a.Hkv) % parts) * NT;
    const size_t base = ((size_t)(ok ? b : 0) * a.bs + t0) * rowb + (size_t)kvh * D;
    const __amdgpu_buffer_rsrc_t rk = uniform_rsrc(a.k8 + base, ok ? (NT - 1) * rowb + D : 0);
    const __amdgpu_buffer_rsrc_t rv = uniform_rsrc(a.v8 + base, ok ? (NT - 1) * rowb + D : 0);
#pragma unroll
    for (int c = 0; c < 4; ++c) {  // piece 64c + lane: row (64c + lane) / 8, bytes 16 * (lane % 8) ..
      const int off = ((64 * c + lane) >> 3) * rowb + 16 * (lane & 7);
      x.k[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
      x.v[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
    }
    const __amdgpu_buffer_rsrc_t rks = uniform_rsrc(a.kps + (ok ? b : 0), ok ? 4 : 0);
    const __amdgpu_buffer_rsrc_t rvs = uniform_rsrc(a.vps + (ok ? b : 0), ok ? 4 : 0);
    const int soff = lane == 0 ? 0 : 0x40000000;
    x.sk = __builtin_amdgcn_raw_buffer_load_b32(rks, soff, 0, 0);  // lane 0 reads the page's scales
    x.sv = __builtin_amdgcn_raw_buffer_load_b32(rvs, soff, 0, 0);
  };
  u32x4 acc = {0u, 0u, 0u, 0u};
  auto fold = [&](const Buf& x) {
#pragma unroll
    for (int c = 0; c < 4; ++c) acc ^= x.k[c] ^ x.v[c];
    acc[0] ^= x.sk ^ x.sv;
  };
  Buf A, B;
  int i = wave;
  if (i < nsl) {
    issue(i, A);
    for (; i < nsl; i += 2 * nwaves) {
      issue(i + nwaves, B);
      __builtin_amdgcn_sched_barrier(0);
      fold(A);
      if (i + nwaves >= nsl) break;
      issue(i + 2 * nwaves, A);
      __builtin_amdgcn_sched_barrier(0);
      fold(B);
    }
  }
  uint32_t w = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  for (int o = 1; o < 64; o <<= 1) w ^= __shfl_xor(w, o, 64);
  __shared__ uint32_t part[4];
  if (lane == 0) part[threadIdx.x >> 6] = w;
  __syncthreads();
  if (threadIdx.x == 0) a.sink[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

}  // namespace emx
