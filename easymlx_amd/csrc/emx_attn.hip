// C-ABI entry points of libemx_attn.so (declared in include/emx_attn.h).
// Host-side validation happens here so that no kernel is launched with shapes
// it does not assume.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/emx_attn.h"
#include "decode_affine.hpp"
#include "paged_generic.hpp"
#include "decode_split.hpp"
#include "prefill_affine.hpp"
#include "decode_q4.hpp"
#include "unified.hpp"
#include "quantize.hpp"
#include "fp8.hpp"
#include "decode_fp8.hpp"
#include "slots.hpp"
#include "probe.hpp"
#include "pages.hpp"

constexpr int kNoallocScratchFloats = 2 * emx::kFp8Parts;  // 2 KiB per stream slot
constexpr int kNoallocSlots = 8;                            // streams with a slot of their own

// Scratch of emx_fp8_cache_write_noalloc: the two-launch FP8 write's
// per-workgroup maxima (written by fp8_amax before fp8_write reads them, so it
// needs no clearing), one 2 KiB slot per stream that calls it (up to
// kNoallocSlots streams per GPU), so calls on different streams never share
// one.  Each GPU holds its own copy until the process ends.  In host code
// `scratch` is only a symbol: kernels get the device address that
// hipGetSymbolAddress returns for the current device (noalloc_scratch()).
static __device__ __align__(256) float scratch[kNoallocSlots][kNoallocScratchFloats];


namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(EMX_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return EMX_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Compute units of the current device (256 on MI355X).
int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess || cus <= 0)
    return 256;
  return cus;
}

// The 16x16 / FP8 decode grid: one four-wave workgroup per CU (measured faster than
// two: these kernels are latency-bound, and more waves add split-K pieces rather
// than bandwidth).
int decode_num_waves() { return device_cus() * 4; }
// The 4-bit kernel runs two four-wave workgroups per CU.
int decode_q4_num_waves() { return device_cus() * 8; }
// Partial slots are sized for the larger of the two persistent grids.
int decode_max_waves() { return std::max(decode_num_waves(), decode_q4_num_waves()); }

// Unit counters, then per-group counters indexed by partial slot (< kMaxWaves + kMaxUnits).
// Then the prefill key-split counters.
constexpr size_t kCounterInts = 2 * (size_t)emx::kMaxUnits + emx::kMaxWaves + emx::kPrefillCounters;
// The 4-bit decode's plan cache follows the counters; the split-K partials follow it.
constexpr size_t kPartialsInt = kCounterInts + emx::kPlanInts;
constexpr size_t kPrefillCounterOff = 2 * (size_t)emx::kMaxUnits + emx::kMaxWaves;

// Prefill tiles per kv head a call with num_tokens query rows can have: a
// sequence with q >= 2 query tokens has ceil(q / tokb) <= q / tokb + 1 tiles.
long prefill_max_items(int num_tokens, int num_seqs, int tokb) {
  return (long)(num_tokens + tokb - 1) / tokb + std::min(num_seqs, num_tokens / 2);
}

// Wires the key split of the prefill kernel when the workspace holds the
// partial states after the decode region (`need` bytes).
void prefill_split(emx::PrefillArgs& p, int num_tokens, int num_q_heads, int num_kv_heads, void* workspace,
                   size_t workspace_bytes, size_t need) {
  p.nparts = 1;
  p.max_items = 0;
  p.ws_cnt = nullptr;
  p.ws_part = nullptr;
  const size_t extra = emx_paged_prefill_workspace_bytes(num_tokens, p.S, num_q_heads, num_kv_heads, 128);
  if (extra == 0 || workspace == nullptr || workspace_bytes < need + extra) return;
  const size_t base = (need + 255) & ~(size_t)255;
  p.nparts = emx::kPrefillParts;
  p.max_items = (int)prefill_max_items(num_tokens, p.S, 128 / (num_q_heads / num_kv_heads));
  p.ws_cnt = reinterpret_cast<int*>(workspace) + kPrefillCounterOff;
  p.ws_part = reinterpret_cast<float*>(static_cast<char*>(workspace) + base);
}

// Pages of 16, 32 or 64 tokens (the reference's PageCacheConfig default is 16): pure
// decode calls over 4-bit pages with group 64 and GQA 1, 2, 4 or 16 (decode_q4_d128's
// small-page variant).
bool small_page_q4(int page_size, int bits, int group_size, int hg, int single_token_decode) {
  return (page_size == 16 || page_size == 32 || page_size == 64) && bits == 4 && group_size == 64 &&
         (hg == 1 || hg == 2 || hg == 4 || hg == 16) && single_token_decode;
}

bool decode_fast_path(int head_dim, int page_size, int bits, int group_size, int hg, int num_seqs,
                      int single_token_decode) {
  if (head_dim != 128 || num_seqs > emx::kMaxSeqs) return false;
  if (page_size % 128 != 0) return small_page_q4(page_size, bits, group_size, hg, single_token_decode);
  if (bits != 4 && bits != 8) return false;
  if (group_size != 32 && group_size != 64 && group_size != 128) return false;
  if (hg < 1 || hg > 16 || (hg & (hg - 1)) != 0) return false;
  return hg * (head_dim / group_size) <= 16;
}

typedef void (*DecodeFn)(emx::DecodeArgs);

template <int BITS, int GS>
DecodeFn pick_decode_hg(int hg) {
  constexpr int G = 128 / GS;
  switch (hg) {
    case 1: return emx::decode_affine_d128<BITS, GS, 1>;
    case 2: return emx::decode_affine_d128<BITS, GS, 2>;
    case 4: return emx::decode_affine_d128<BITS, GS, 4>;
    case 8: if constexpr (8 * G <= 16) return emx::decode_affine_d128<BITS, GS, 8>; else return nullptr;
    case 16: if constexpr (16 * G <= 16) return emx::decode_affine_d128<BITS, GS, 16>; else return nullptr;
  }
  return nullptr;
}

// 4-bit pages, group 64 / 128, GQA ratio 1, 2, 4 or 16: the 4x4x4 MFMA decode kernel.
// GQA 8 with groups of 64 fills all 16 columns of the 16x16x32 kernel, which serves it.
typedef void (*Q4Fn)(int*, const int32_t*, const int32_t*, int, int, emx::DecodeArgs);

template <int GS, int PS = 0>
Q4Fn pick_decode_q4_hg(int hg) {
  switch (hg) {
    case 1: return emx::decode_q4_d128<GS, 1, PS>;
    case 2: return emx::decode_q4_d128<GS, 2, PS>;
    case 4: return emx::decode_q4_d128<GS, 4, PS>;
    case 16: return emx::decode_q4_d128<GS, 16, PS>;
  }
  return nullptr;
}

// page_size a multiple of 128, or 16 / 32 / 64 (group 64 only)
Q4Fn pick_decode_q4(int gs, int hg, int page_size) {
  if (page_size < 128) {
    if (gs != 64) return nullptr;
    if (page_size == 16) return pick_decode_q4_hg<64, 16>(hg);
    if (page_size == 32) return pick_decode_q4_hg<64, 32>(hg);
    if (page_size == 64) return pick_decode_q4_hg<64, 64>(hg);
    return nullptr;
  }
  if (gs == 64) return pick_decode_q4_hg<64>(hg);
  if (gs == 128) return pick_decode_q4_hg<128>(hg);
  return nullptr;
}

// A mixed batch over 4-bit pages in one launch (prefill and 4-bit decode bodies).
typedef void (*UnifiedFn)(emx::PrefillArgs, emx::DecodeArgs, int);

template <int GS>
UnifiedFn pick_unified_q4_hg(int hg) {
  switch (hg) {
    case 1: return emx::unified_q4<GS, 1>;
    case 2: return emx::unified_q4<GS, 2>;
    case 4: return emx::unified_q4<GS, 4>;
    case 16: return emx::unified_q4<GS, 16>;
  }
  return nullptr;
}

template <int BITS, int GS>
UnifiedFn pick_unified_affine_hg(int hg) {
  constexpr int G = 128 / GS;
  switch (hg) {
    case 1: return emx::unified_affine<BITS, GS, 1>;
    case 2: return emx::unified_affine<BITS, GS, 2>;
    case 4: return emx::unified_affine<BITS, GS, 4>;
    case 8: if constexpr (8 * G <= 16) return emx::unified_affine<BITS, GS, 8>; else return nullptr;
    case 16: if constexpr (16 * G <= 16) return emx::unified_affine<BITS, GS, 16>; else return nullptr;
  }
  return nullptr;
}

template <int BITS>
UnifiedFn pick_unified_affine(int gs, int hg) {
  switch (gs) {
    case 32: return pick_unified_affine_hg<BITS, 32>(hg);
    case 64: return pick_unified_affine_hg<BITS, 64>(hg);
    case 128: return pick_unified_affine_hg<BITS, 128>(hg);
  }
  return nullptr;
}

UnifiedFn pick_unified_fp8(int hg) {
  switch (hg) {
    case 1: return emx::unified_fp8<1>;
    case 2: return emx::unified_fp8<2>;
    case 4: return emx::unified_fp8<4>;
    case 8: return emx::unified_fp8<8>;
    case 16: return emx::unified_fp8<16>;
  }
  return nullptr;
}

UnifiedFn pick_unified_q4(int gs, int hg) {
  if (gs == 64) return pick_unified_q4_hg<64>(hg);
  if (gs == 128) return pick_unified_q4_hg<128>(hg);
  return nullptr;
}

template <int BITS>
DecodeFn pick_decode_gs(int gs, int hg) {
  switch (gs) {
    case 32: return pick_decode_hg<BITS, 32>(hg);
    case 64: return pick_decode_hg<BITS, 64>(hg);
    case 128: return pick_decode_hg<BITS, 128>(hg);
  }
  return nullptr;
}

bool prefill_fast_path(int hg) { return hg == 1 || hg == 2 || hg == 4 || hg == 8 || hg == 16; }

typedef void (*PrefillFn)(emx::PrefillArgs);

template <int BITS, int GS>
PrefillFn pick_prefill_hg(int hg) {
  switch (hg) {
    case 1: return emx::prefill_affine_d128<BITS, GS, 1>;
    case 2: return emx::prefill_affine_d128<BITS, GS, 2>;
    case 4: return emx::prefill_affine_d128<BITS, GS, 4>;
    case 8: return emx::prefill_affine_d128<BITS, GS, 8>;
    case 16: return emx::prefill_affine_d128<BITS, GS, 16>;
  }
  return nullptr;
}

PrefillFn pick_prefill_fp8(int hg) {
  switch (hg) {
    case 1: return emx::prefill_affine_d128<4, 128, 1, true>;
    case 2: return emx::prefill_affine_d128<4, 128, 2, true>;
    case 4: return emx::prefill_affine_d128<4, 128, 4, true>;
    case 8: return emx::prefill_affine_d128<4, 128, 8, true>;
    case 16: return emx::prefill_affine_d128<4, 128, 16, true>;
  }
  return nullptr;
}

DecodeFn pick_decode_fp8(int hg) {
  switch (hg) {
    case 1: return emx::decode_fp8_d128<1>;
    case 2: return emx::decode_fp8_d128<2>;
    case 4: return emx::decode_fp8_d128<4>;
    case 8: return emx::decode_fp8_d128<8>;
    case 16: return emx::decode_fp8_d128<16>;
  }
  return nullptr;
}

template <int BITS>
PrefillFn pick_prefill_gs(int gs, int hg) {
  switch (gs) {
    case 32: return pick_prefill_hg<BITS, 32>(hg);
    case 64: return pick_prefill_hg<BITS, 64>(hg);
    case 128: return pick_prefill_hg<BITS, 128>(hg);
  }
  return nullptr;
}

int validate_common(const void* q, int num_tokens, int hq, int d, int hkv, int nb, int bs, const int32_t* bt, int S,
                    int max_blocks, const int32_t* kv_lens, const int32_t* qsl, int decode, const void* out) {
  if (num_tokens < 0 || S < 0) return fail(EMX_ERR_INVALID, "num_tokens/num_seqs must be >= 0");
  if (hq <= 0 || hkv <= 0 || d <= 0) return fail(EMX_ERR_INVALID, "head counts and head_dim must be positive");
  if (hq % hkv != 0) return fail(EMX_ERR_INVALID, "num_q_heads must be divisible by num_kv_heads (GQA)");
  if (d > 256) return fail(EMX_ERR_UNSUPPORTED, "head_dim %d > 256 is not supported", d);
  if (bs <= 0 || nb <= 0) return fail(EMX_ERR_INVALID, "page_size and num_blocks must be positive");
  if (max_blocks <= 0 && S > 0) return fail(EMX_ERR_INVALID, "max_blocks_per_seq must be positive");
  if (num_tokens > 0 && (!q || !out)) return fail(EMX_ERR_INVALID, "queries/out must not be null");
  if (S > 0 && (!bt || !kv_lens)) return fail(EMX_ERR_INVALID, "block_tables/kv_lens must not be null");
  if (decode) {
    if (num_tokens != S) return fail(EMX_ERR_INVALID, "single_token_decode requires num_tokens == num_seqs");
  } else if (S > 0 && !qsl) {
    return fail(EMX_ERR_INVALID, "query_start_loc must not be null");
  }
  return EMX_OK;
}

// Single-token decode outside the MFMA kernels: the split-K kernel (decode_split.hpp)
// when the shape allows it (head_dim a multiple of 32 up to 256, pages of a multiple
// of 8 tokens) and the workspace holds its partials.
bool split_shape_ok(int head_dim, int page_size) {
  return head_dim % 32 == 0 && head_dim <= 256 && page_size % 8 == 0;
}

void split_geometry(int num_q_heads, int num_kv_heads, int max_blocks, int page_size, int& hc, int& nhc,
                    int& nchunk) {
  const int hg = num_q_heads / num_kv_heads;
  hc = std::min(hg, 16);
  nhc = (hg + hc - 1) / hc;
  nchunk = (int)(((long long)max_blocks * page_size + emx::kSplitChunk - 1) / emx::kSplitChunk) + 1;
}

size_t split_workspace_bytes(int num_seqs, int num_q_heads, int num_kv_heads, int head_dim, int max_blocks,
                             int page_size) {
  if (!split_shape_ok(head_dim, page_size) || num_seqs <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 ||
      max_blocks <= 0 || num_q_heads % num_kv_heads)
    return 0;
  int hc, nhc, nchunk;
  split_geometry(num_q_heads, num_kv_heads, max_blocks, page_size, hc, nhc, nchunk);
  return (size_t)num_seqs * num_kv_heads * nhc * nchunk * hc * (head_dim + 2) * sizeof(float);
}

// The merge keeps every chunk's weight and sum of a workgroup's heads in LDS: at most
// 64 KiB (contexts up to ~500k tokens at 16 heads a workgroup); longer ones take the
// generic kernel.
bool split_merge_lds_ok(const emx::GenericArgs& ga) {
  int hc, nhc, nchunk;
  split_geometry(ga.Hq, ga.Hkv, ga.max_blocks, ga.bs, hc, nhc, nchunk);
  return (2 * (size_t)hc * nchunk + hc) * sizeof(float) <= 65536;
}

template <typename QT, typename KV>
int launch_split(const emx::GenericArgs& ga, const KV& kv, float* part, hipStream_t st) {
  emx::SplitArgs sa;
  sa.q = ga.q;
  sa.out = ga.out;
  sa.block_tables = ga.block_tables;
  sa.kv_lens = ga.kv_lens;
  sa.part = part;
  sa.S = ga.S;
  sa.Hq = ga.Hq;
  sa.Hkv = ga.Hkv;
  sa.D = ga.D;
  sa.bs = ga.bs;
  sa.nb = ga.nb;
  sa.max_blocks = ga.max_blocks;
  sa.scale_log2 = ga.scale_log2;
  sa.window = ga.window;
  int nhc;
  split_geometry(ga.Hq, ga.Hkv, ga.max_blocks, ga.bs, sa.hc, nhc, sa.nchunk);
  const size_t lds = (size_t)sa.hc * (ga.D + 64) * sizeof(float);
  const dim3 grid((unsigned)sa.nchunk, (unsigned)(ga.Hkv * nhc), (unsigned)ga.S);
  if (sa.hc <= 4)
    hipLaunchKernelGGL((emx::decode_split<QT, KV, 4>), grid, dim3(64), lds, st, sa, kv);
  else
    hipLaunchKernelGGL((emx::decode_split<QT, KV, 16>), grid, dim3(64), lds, st, sa, kv);
  if (int r = check_launch("decode_split")) return r;
  const size_t merge_lds = (2 * (size_t)sa.hc * sa.nchunk + sa.hc) * sizeof(float);  // chunk weights and sums
  hipLaunchKernelGGL((emx::decode_split_merge<QT>), dim3((unsigned)(ga.Hkv * nhc), (unsigned)ga.S), dim3(256),
                     merge_lds, st, sa);
  return check_launch("decode_split_merge");
}

template <typename QT, typename KV>
int launch_generic_only(const emx::GenericArgs& ga, const KV& kv, hipStream_t st);

// The generic kernel, or the split-K decode for single-token calls it covers
// (ws: the caller's workspace, or null).
template <typename QT, typename KV>
int launch_generic(const emx::GenericArgs& ga, const KV& kv, hipStream_t st, void* ws = nullptr,
                   size_t ws_bytes = 0) {
  if (ga.decode && ws && ga.S == ga.T && emx::split_kv_ok(kv) && split_merge_lds_ok(ga) &&
      ws_bytes >= (size_t)kPartialsInt * sizeof(int) +
                      split_workspace_bytes(ga.S, ga.Hq, ga.Hkv, ga.D, ga.max_blocks, ga.bs) &&
      split_workspace_bytes(ga.S, ga.Hq, ga.Hkv, ga.D, ga.max_blocks, ga.bs) > 0)
    return launch_split<QT>(ga, kv, reinterpret_cast<float*>(static_cast<int*>(ws) + kPartialsInt), st);
  return launch_generic_only<QT>(ga, kv, st);
}

template <typename QT, typename KV>
int launch_generic_only(const emx::GenericArgs& ga, const KV& kv, hipStream_t st) {
  const int hg = ga.Hq / ga.Hkv;
  dim3 grid(ga.T, ga.Hkv, (hg + 15) / 16);
  hipLaunchKernelGGL((emx::paged_generic<QT, KV>), grid, dim3(64), 0, st, ga, kv);
  return check_launch("paged_generic");
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
void* g_scratch_stream[kMaxDevices][kNoallocSlots] = {};  // the stream holding each slot
int g_scratch_used[kMaxDevices] = {};

// Device address of the scratch slot of `stream` on the current device: the
// symbol's address is looked up once per device (with that device current), a
// slot is given to each new stream, up to kNoallocSlots per device.  Null, with
// the last error set, on failure (*rc: the status to return).
void* noalloc_scratch(void* stream, int* rc) {
  int dev = 0;
  *rc = EMX_ERR_HIP;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(EMX_ERR_HIP, "emx_fp8_cache_write_noalloc: no current device (or device id >= %d)", kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      fail(EMX_ERR_HIP, "emx_fp8_cache_write_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  int slot = -1;
  for (int i = 0; i < g_scratch_used[dev]; ++i)
    if (g_scratch_stream[dev][i] == stream) slot = i;
  if (slot < 0) {
    if (g_scratch_used[dev] == kNoallocSlots) {
      *rc = EMX_ERR_UNSUPPORTED;
      fail(EMX_ERR_UNSUPPORTED,
           "emx_fp8_cache_write_noalloc: more than %d streams on this device (each holds a scratch slot); "
           "use emx_fp8_cache_write with a workspace",
           kNoallocSlots);
      return nullptr;
    }
    slot = g_scratch_used[dev]++;
    g_scratch_stream[dev][slot] = stream;
  }
  *rc = EMX_OK;
  return static_cast<char*>(g_scratch_ptr[dev]) + (size_t)slot * sizeof(float) * kNoallocScratchFloats;
}

template <typename KV>
int launch_gather(const KV& kv, const int32_t* block_table, int num_seqs, int max_blocks,
                         const int32_t* cu_seq_lens, int total_tokens, int num_blocks, int out_dtype, void* k_out,
                         void* v_out, void* stream) {
  if (num_seqs <= 0 || max_blocks <= 0 || total_tokens < 0 || num_blocks <= 0)
    return fail(EMX_ERR_INVALID, "num_seqs, max_blocks and num_blocks must be positive, total_tokens >= 0");
  if (total_tokens == 0) return EMX_OK;
  if (!block_table || !cu_seq_lens || !k_out || !v_out) return fail(EMX_ERR_INVALID, "null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)total_tokens);
  switch (out_dtype) {
    case EMX_DTYPE_F16:
      hipLaunchKernelGGL((emx::gather_kv<emx::F16, KV>), grid, dim3(256), 0, st, kv, block_table, cu_seq_lens,
                         num_seqs, max_blocks, total_tokens, num_blocks, k_out, v_out);
      break;
    case EMX_DTYPE_BF16:
      hipLaunchKernelGGL((emx::gather_kv<emx::BF16, KV>), grid, dim3(256), 0, st, kv, block_table, cu_seq_lens,
                         num_seqs, max_blocks, total_tokens, num_blocks, k_out, v_out);
      break;
    case EMX_DTYPE_F32:
      hipLaunchKernelGGL((emx::gather_kv<emx::F32, KV>), grid, dim3(256), 0, st, kv, block_table, cu_seq_lens,
                         num_seqs, max_blocks, total_tokens, num_blocks, k_out, v_out);
      break;
    default: return fail(EMX_ERR_INVALID, "unknown out_dtype %d", out_dtype);
  }
  return check_launch("gather_kv");
}

}  // namespace

extern "C" {

int emx_version(void) { return 100; }

const char* emx_last_error(void) { return g_last_error.c_str(); }

int emx_affine_quantize(const void* x, long rows, int head_dim, int group_size, int bits, uint32_t* codes,
                        void* scales, void* biases, void* stream) {
  if (rows < 0) return fail(EMX_ERR_INVALID, "rows must be >= 0");
  if (bits != 4 && bits != 8) return fail(EMX_ERR_UNSUPPORTED, "bits must be 4 or 8, got %d", bits);
  if (group_size <= 0 || group_size % 8 != 0 || head_dim % group_size != 0)
    return fail(EMX_ERR_INVALID, "head_dim %d must be a multiple of group_size %d (a multiple of 8)", head_dim,
                group_size);
  if (rows == 0) return EMX_OK;
  if (!x || !codes || !scales || !biases) return fail(EMX_ERR_INVALID, "null pointer");
  if (!aligned16(x)) return fail(EMX_ERR_INVALID, "x must be 16-byte aligned");
  const long n = rows * (head_dim / group_size);
  const int blocks = (int)((n + 255) / 256);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const emx::h16* xp = reinterpret_cast<const emx::h16*>(x);
  emx::h16* sp = reinterpret_cast<emx::h16*>(scales);
  emx::h16* bp = reinterpret_cast<emx::h16*>(biases);
  if (bits == 4)
    hipLaunchKernelGGL(emx::affine_quantize_rows<4>, dim3(blocks), dim3(256), 0, st, xp, rows, head_dim, group_size,
                       codes, sp, bp);
  else
    hipLaunchKernelGGL(emx::affine_quantize_rows<8>, dim3(blocks), dim3(256), 0, st, xp, rows, head_dim, group_size,
                       codes, sp, bp);
  return check_launch("affine_quantize");
}

static int affine_write_impl(const void* keys, const void* values, const int32_t* slot_mapping, int num_tokens,
                      int num_kv_heads, int head_dim, int group_size, int bits, int page_size, int num_blocks,
                      uint32_t* k_codes, void* k_scales, void* k_biases, uint32_t* v_codes, void* v_scales,
                      void* v_biases, const emx::RopeArgs& rope, const void* queries_in, void* queries,
                      int num_q_heads, void* stream) {
  if (num_tokens < 0) return fail(EMX_ERR_INVALID, "num_tokens must be >= 0");
  if (bits != 4 && bits != 8) return fail(EMX_ERR_UNSUPPORTED, "bits must be 4 or 8, got %d", bits);
  if (num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0 || num_blocks <= 0)
    return fail(EMX_ERR_INVALID, "num_kv_heads, head_dim, page_size, num_blocks must be positive");
  if (group_size <= 0 || group_size % 8 != 0 || head_dim % group_size != 0)
    return fail(EMX_ERR_INVALID, "head_dim %d must be a multiple of group_size %d (a multiple of 8)", head_dim,
                group_size);
  if ((page_size * bits) % 32 != 0 || (page_size > 256 / bits && page_size % (256 / bits) != 0))
    return fail(EMX_ERR_INVALID, "page_size %d must be a multiple of 32/bits, and of 256/bits when larger", page_size);
  if (num_tokens == 0) return EMX_OK;
  if (!keys || !values || !slot_mapping || !k_codes || !k_scales || !k_biases || !v_codes || !v_scales || !v_biases)
    return fail(EMX_ERR_INVALID, "null pointer");
  if (!aligned16(keys) || !aligned16(values)) return fail(EMX_ERR_INVALID, "keys/values must be 16-byte aligned");
  emx::WriteArgs a;
  a.keys = reinterpret_cast<const emx::h16*>(keys);
  a.values = reinterpret_cast<const emx::h16*>(values);
  a.slot_mapping = slot_mapping;
  a.kc = k_codes;
  a.ks = reinterpret_cast<emx::h16*>(k_scales);
  a.kb = reinterpret_cast<emx::h16*>(k_biases);
  a.vc = v_codes;
  a.vs = reinterpret_cast<emx::h16*>(v_scales);
  a.vb = reinterpret_cast<emx::h16*>(v_biases);
  a.T = num_tokens;
  a.Hkv = num_kv_heads;
  a.D = head_dim;
  a.gs = group_size;
  a.bs = page_size;
  a.nb = num_blocks;
  if (head_dim / group_size > emx::kWriteMaxGroups || head_dim > emx::kWriteMaxDim)
    return fail(EMX_ERR_UNSUPPORTED, "head_dim %d above %d or more than %d quantization groups per head", head_dim,
                emx::kWriteMaxDim, emx::kWriteMaxGroups);
  a.rope = rope;
  a.q = reinterpret_cast<emx::h16*>(queries);
  a.q_in = queries_in ? reinterpret_cast<const emx::h16*>(queries_in) : a.q;
  a.Hq = num_q_heads;
  a.slot_ids = nullptr;  // slot_mapping given (the decode append sets these: emx_affine_cache_append_rope)
  a.kv_lens = nullptr;
  a.bt = nullptr;
  a.S = a.max_blocks = 0;
  a.counter = nullptr;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (num_tokens <= emx::kSmallWrite && head_dim % 16 == 0 && group_size % 16 == 0 &&
      group_size <= emx::kSmallMaxGroup) {
    const bool r = rope.inv_freq != nullptr;
    // with RoPE and queries: kQRopeBlocks more rows of workgroups turn the queries in the same launch
    const dim3 sgrid((unsigned)num_kv_heads,
                     (unsigned)(head_dim / 16 + (r && queries ? emx::kQRopeBlocks : 0)));
    typedef void (*SmallFn)(emx::WriteArgs);
    SmallFn fn = bits == 4 ? (r ? emx::affine_cache_write_small<4, true> : emx::affine_cache_write_small<4, false>)
                           : (r ? emx::affine_cache_write_small<8, true> : emx::affine_cache_write_small<8, false>);
    hipLaunchKernelGGL(fn, sgrid, dim3(256), 0, st, a);
    return check_launch("affine_cache_write_small");
  }
  const dim3 grid((unsigned)((num_tokens + emx::kWriteTokens - 1) / emx::kWriteTokens), (unsigned)num_kv_heads);
  if (bits == 4)
    hipLaunchKernelGGL(emx::affine_cache_write<4>, grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(emx::affine_cache_write<8>, grid, dim3(256), 0, st, a);
  if (int rc = check_launch("affine_cache_write")) return rc;
  if (rope.inv_freq != nullptr && queries != nullptr) {  // larger writes: the queries in their own launch
    const long n = (long)num_tokens * num_q_heads * (head_dim / 2);
    const unsigned qgrid = (unsigned)std::min<long>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(emx::rope_rows, dim3(qgrid), dim3(256), 0, st, a.q, a.q_in, num_tokens, num_q_heads, head_dim,
                       rope);
    return check_launch("rope_rows");
  }
  return EMX_OK;
}

int emx_affine_cache_write(const void* keys, const void* values, const int32_t* slot_mapping, int num_tokens,
                           int num_kv_heads, int head_dim, int group_size, int bits, int page_size, int num_blocks,
                           uint32_t* k_codes, void* k_scales, void* k_biases, uint32_t* v_codes, void* v_scales,
                           void* v_biases, void* stream) {
  return affine_write_impl(keys, values, slot_mapping, num_tokens, num_kv_heads, head_dim, group_size, bits,
                           page_size, num_blocks, k_codes, k_scales, k_biases, v_codes, v_scales, v_biases,
                           emx::RopeArgs{nullptr, nullptr, 0, 0}, nullptr, nullptr, 0, stream);
}

static bool rope_ok(const int32_t* positions, const float* inv_freq, int rot_dims, int head_dim) {
  return positions && inv_freq && rot_dims > 0 && rot_dims % 2 == 0 && rot_dims <= head_dim;
}

int emx_affine_cache_write_rope(const void* keys, const void* values, const int32_t* slot_mapping, int num_tokens,
                                int num_kv_heads, int head_dim, int group_size, int bits, int page_size,
                                int num_blocks, uint32_t* k_codes, void* k_scales, void* k_biases, uint32_t* v_codes,
                                void* v_scales, void* v_biases, const int32_t* positions, const float* inv_freq,
                                int rot_dims, int traditional, const void* queries_in, void* queries,
                                int num_q_heads, void* stream) {
  if (num_tokens > 0 && !rope_ok(positions, inv_freq, rot_dims, head_dim))
    return fail(EMX_ERR_INVALID, "rope: positions and inv_freq needed, rot_dims even and in (0, head_dim]");
  if (queries != nullptr && (num_q_heads <= 0 || !aligned16(queries)))
    return fail(EMX_ERR_INVALID, "queries need num_q_heads > 0 and 16-byte alignment");
  if (queries_in != nullptr && queries == nullptr) return fail(EMX_ERR_INVALID, "queries_in needs queries");
  return affine_write_impl(keys, values, slot_mapping, num_tokens, num_kv_heads, head_dim, group_size, bits,
                           page_size, num_blocks, k_codes, k_scales, k_biases, v_codes, v_scales, v_biases,
                           emx::RopeArgs{inv_freq, positions, rot_dims, traditional ? 1 : 0}, queries_in, queries,
                           num_q_heads, stream);
}

int emx_affine_cache_append_rope(const void* keys, const void* values, const int32_t* slot_ids, int num_tokens,
                                 const int32_t* block_tables, int num_seqs, int max_blocks_per_seq, int32_t* kv_lens,
                                 int* counter, int num_kv_heads, int head_dim, int group_size, int bits,
                                 int page_size, int num_blocks, uint32_t* k_codes, void* k_scales, void* k_biases,
                                 uint32_t* v_codes, void* v_scales, void* v_biases, const float* inv_freq,
                                 int rot_dims, int traditional, const void* queries_in, void* queries,
                                 int num_q_heads, void* stream) {
  if (num_tokens < 0 || num_seqs <= 0 || max_blocks_per_seq <= 0)
    return fail(EMX_ERR_INVALID, "num_tokens >= 0, num_seqs and max_blocks_per_seq > 0 needed");
  if (num_tokens > emx::kSmallWrite || head_dim % 16 != 0 || group_size % 16 != 0 ||
      group_size > emx::kSmallMaxGroup || head_dim > emx::kWriteMaxDim)
    return fail(EMX_ERR_UNSUPPORTED, "decode append: at most %d tokens, head_dim and group_size multiples of 16, "
                "group_size <= %d", emx::kSmallWrite, emx::kSmallMaxGroup);
  if (num_tokens == 0) return EMX_OK;
  if (!slot_ids || !block_tables || !kv_lens || !counter) return fail(EMX_ERR_INVALID, "null pointer");
  if (!inv_freq || rot_dims <= 0 || rot_dims % 2 != 0 || rot_dims > head_dim)
    return fail(EMX_ERR_INVALID, "rope: inv_freq needed, rot_dims even and in (0, head_dim]");
  if (queries != nullptr && (num_q_heads <= 0 || !aligned16(queries)))
    return fail(EMX_ERR_INVALID, "queries need num_q_heads > 0 and 16-byte alignment");
  if (queries_in != nullptr && queries == nullptr) return fail(EMX_ERR_INVALID, "queries_in needs queries");
  if (bits != 4 && bits != 8) return fail(EMX_ERR_UNSUPPORTED, "bits must be 4 or 8, got %d", bits);
  if (num_kv_heads <= 0 || page_size <= 0 || num_blocks <= 0 || group_size <= 0 || head_dim % group_size != 0)
    return fail(EMX_ERR_INVALID, "num_kv_heads, page_size, num_blocks positive; head_dim a multiple of group_size");
  if ((page_size * bits) % 32 != 0 || (page_size > 256 / bits && page_size % (256 / bits) != 0))
    return fail(EMX_ERR_INVALID, "page_size %d must be a multiple of 32/bits, and of 256/bits when larger", page_size);
  if (!keys || !values || !k_codes || !k_scales || !k_biases || !v_codes || !v_scales || !v_biases)
    return fail(EMX_ERR_INVALID, "null pointer");
  if (!aligned16(keys) || !aligned16(values)) return fail(EMX_ERR_INVALID, "keys/values must be 16-byte aligned");
  emx::WriteArgs a;
  a.keys = reinterpret_cast<const emx::h16*>(keys);
  a.values = reinterpret_cast<const emx::h16*>(values);
  a.slot_mapping = nullptr;
  a.kc = k_codes;
  a.ks = reinterpret_cast<emx::h16*>(k_scales);
  a.kb = reinterpret_cast<emx::h16*>(k_biases);
  a.vc = v_codes;
  a.vs = reinterpret_cast<emx::h16*>(v_scales);
  a.vb = reinterpret_cast<emx::h16*>(v_biases);
  a.T = num_tokens;
  a.Hkv = num_kv_heads;
  a.D = head_dim;
  a.gs = group_size;
  a.bs = page_size;
  a.nb = num_blocks;
  a.rope = emx::RopeArgs{inv_freq, nullptr, rot_dims, traditional ? 1 : 0};
  a.q = reinterpret_cast<emx::h16*>(queries);
  a.q_in = queries_in ? reinterpret_cast<const emx::h16*>(queries_in) : a.q;
  a.Hq = num_q_heads;
  a.slot_ids = slot_ids;
  a.kv_lens = kv_lens;
  a.bt = block_tables;
  a.S = num_seqs;
  a.max_blocks = max_blocks_per_seq;
  a.counter = counter;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 sgrid((unsigned)num_kv_heads, (unsigned)(head_dim / 16 + (queries ? emx::kQRopeBlocks : 0)));
  typedef void (*SmallFn)(emx::WriteArgs);
  SmallFn fn = bits == 4 ? emx::affine_cache_write_small<4, true> : emx::affine_cache_write_small<8, true>;
  hipLaunchKernelGGL(fn, sgrid, dim3(256), 0, st, a);
  return check_launch("affine_cache_write_small (append)");
}

int emx_cache_slots(const int32_t* slot_ids, const int32_t* query_start_loc, int num_slots, int num_tokens,
                    const int32_t* block_tables, int num_seqs, int max_blocks_per_seq, int page_size,
                    int32_t* kv_lens, int32_t* slot_mapping, int32_t* positions, void* stream) {
  if (num_slots < 0 || num_tokens < 0) return fail(EMX_ERR_INVALID, "num_slots and num_tokens must be >= 0");
  if (num_slots > emx::kMaxSlots)
    return fail(EMX_ERR_UNSUPPORTED, "%d sequences in one write exceed %d", num_slots, emx::kMaxSlots);
  if (num_seqs <= 0 || max_blocks_per_seq <= 0 || page_size <= 0)
    return fail(EMX_ERR_INVALID, "num_seqs, max_blocks_per_seq and page_size must be positive");
  if (num_slots == 0) return num_tokens == 0 ? EMX_OK : fail(EMX_ERR_INVALID, "tokens without sequences");
  if (!slot_ids || !query_start_loc || !block_tables || !kv_lens || (num_tokens > 0 && (!slot_mapping || !positions)))
    return fail(EMX_ERR_INVALID, "null pointer");
  emx::SlotArgs a{slot_ids, query_start_loc, num_slots, num_tokens, block_tables, num_seqs, max_blocks_per_seq,
                  page_size, kv_lens, slot_mapping, positions};
  hipLaunchKernelGGL(emx::cache_slots, dim3(1), dim3(1024), 0, reinterpret_cast<hipStream_t>(stream), a);
  return check_launch("cache_slots");
}

int emx_dense_cache_write(const void* keys, const void* values, int dtype, const int32_t* slot_mapping,
                          int num_tokens, int num_kv_heads, int head_dim, int page_size, int num_blocks,
                          void* key_cache, void* value_cache, void* stream) {
  if (num_tokens < 0) return fail(EMX_ERR_INVALID, "num_tokens must be >= 0");
  if (num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0 || num_blocks <= 0)
    return fail(EMX_ERR_INVALID, "num_kv_heads, head_dim, page_size, num_blocks must be positive");
  const int elem = dtype == EMX_DTYPE_F32 ? 4 : dtype == EMX_DTYPE_F16 || dtype == EMX_DTYPE_BF16 ? 2 : 0;
  if (elem == 0) return fail(EMX_ERR_INVALID, "unknown dtype %d", dtype);
  const long row_bytes = (long)num_kv_heads * head_dim * elem;
  if (row_bytes % 4) return fail(EMX_ERR_UNSUPPORTED, "a token's row of %ld bytes is not whole words", row_bytes);
  if (num_tokens == 0) return EMX_OK;
  if (!keys || !values || !slot_mapping || !key_cache || !value_cache) return fail(EMX_ERR_INVALID, "null pointer");
  const long n = (long)num_tokens * (row_bytes / 4);
  const unsigned grid = (unsigned)std::min<long>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(emx::dense_cache_write, dim3(grid), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<const uint32_t*>(keys), reinterpret_cast<const uint32_t*>(values), slot_mapping,
                     num_tokens, (int)(row_bytes / 4), page_size, num_blocks, reinterpret_cast<uint32_t*>(key_cache),
                     reinterpret_cast<uint32_t*>(value_cache));
  return check_launch("dense_cache_write");
}

static int page_arrays(int num_arrays, void* const* arrays, const int64_t* block_bytes, int num_blocks,
                       emx::PageArrays& pa) {
  if (num_arrays <= 0 || num_arrays > emx::kMaxPageArrays)
    return fail(EMX_ERR_INVALID, "num_arrays must be in [1, %d]", emx::kMaxPageArrays);
  if (num_blocks <= 0) return fail(EMX_ERR_INVALID, "num_blocks must be positive");
  if (!arrays || !block_bytes) return fail(EMX_ERR_INVALID, "null pointer");
  pa.n = num_arrays;
  pa.nb = num_blocks;
  for (int k = 0; k < num_arrays; ++k) {
    if (!arrays[k] || block_bytes[k] <= 0 || block_bytes[k] % 4 || (reinterpret_cast<uintptr_t>(arrays[k]) & 3))
      return fail(EMX_ERR_INVALID, "array %d: null, unaligned or a block of %lld bytes (need a positive multiple of 4)",
                  k, (long long)block_bytes[k]);
    pa.base[k] = arrays[k];
    pa.block_bytes[k] = block_bytes[k];
  }
  return EMX_OK;
}

size_t emx_copy_blocks_workspace_bytes(int num_arrays, const int64_t* block_bytes, int num_pairs) {
  if (num_arrays <= 0 || num_arrays > emx::kMaxPageArrays || !block_bytes || num_pairs <= 0) return 0;
  size_t total = 0;
  for (int k = 0; k < num_arrays; ++k) {
    if (block_bytes[k] <= 0) return 0;
    total += (((size_t)block_bytes[k] * (size_t)num_pairs) + 255) & ~(size_t)255;
  }
  return total;
}

int emx_copy_blocks(int num_arrays, void* const* arrays, const int64_t* block_bytes, int num_blocks,
                    const int32_t* block_mapping, int num_pairs, void* workspace, size_t workspace_bytes,
                    void* stream) {
  if (num_pairs < 0) return fail(EMX_ERR_INVALID, "num_pairs must be >= 0");
  emx::PageArrays pa{};
  if (int rc = page_arrays(num_arrays, arrays, block_bytes, num_blocks, pa)) return rc;
  if (num_pairs == 0) return EMX_OK;
  if (!block_mapping) return fail(EMX_ERR_INVALID, "null block_mapping");
  const size_t need = emx_copy_blocks_workspace_bytes(num_arrays, block_bytes, num_pairs);
  if (!workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 15))
    return fail(EMX_ERR_INVALID, "copy_blocks staging workspace: need %zu bytes (16-byte aligned), got %zu", need,
                workspace_bytes);
  pa.stage = static_cast<char*>(workspace);
  size_t off = 0;
  for (int k = 0; k < num_arrays; ++k) {
    pa.stage_off[k] = (long long)off;
    off += (((size_t)block_bytes[k] * (size_t)num_pairs) + 255) & ~(size_t)255;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(emx::copy_blocks_gather, dim3((unsigned)num_pairs, (unsigned)num_arrays), dim3(256), 0, st, pa,
                     block_mapping);
  if (int rc = check_launch("copy_blocks_gather")) return rc;
  hipLaunchKernelGGL(emx::copy_blocks_scatter, dim3((unsigned)num_pairs, (unsigned)num_arrays), dim3(256), 0, st, pa,
                     block_mapping, num_pairs);
  return check_launch("copy_blocks_scatter");
}

int emx_zero_blocks(int num_arrays, void* const* arrays, const int64_t* block_bytes, int num_blocks,
                    const int32_t* page_ids, int num_pages, void* stream) {
  if (num_pages < 0) return fail(EMX_ERR_INVALID, "num_pages must be >= 0");
  emx::PageArrays pa{};
  if (int rc = page_arrays(num_arrays, arrays, block_bytes, num_blocks, pa)) return rc;
  if (num_pages == 0) return EMX_OK;
  if (!page_ids) return fail(EMX_ERR_INVALID, "null page_ids");
  hipLaunchKernelGGL(emx::zero_blocks, dim3((unsigned)num_pages, (unsigned)num_arrays), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), pa, page_ids);
  return check_launch("zero_blocks");
}

namespace {

int convert_layout(bool to_pages, const uint32_t* kc, const uint32_t* vc, const void* const (&sc)[4], int num_blocks,
                   int page_size, int num_kv_heads, int head_dim, int bits, int group_size, uint32_t* kd,
                   uint32_t* vd, void* const (&sd)[4], void* stream) {
  if (bits != 4 && bits != 8) return fail(EMX_ERR_UNSUPPORTED, "bits must be 4 or 8, got %d", bits);
  if (num_blocks < 0 || num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0 || group_size <= 0 ||
      head_dim % group_size || (head_dim * bits) % 32 || (page_size * bits) % 32 ||
      (page_size > 256 / bits && page_size % (256 / bits)))
    return fail(EMX_ERR_INVALID, "affine page geometry (head_dim %d, group_size %d, page_size %d, bits %d)", head_dim,
                group_size, page_size, bits);
  if (num_blocks == 0) return EMX_OK;
  if (!kc || !vc || !kd || !vd) return fail(EMX_ERR_INVALID, "null codes pointer");
  emx::LayoutArgs a;
  a.sk = kc;
  a.sv = vc;
  a.dk = kd;
  a.dv = vd;
  for (int i = 0; i < 4; ++i) {
    if (!sc[i] || !sd[i]) return fail(EMX_ERR_INVALID, "null scale / bias pointer");
    a.ss[i] = static_cast<const emx::h16*>(sc[i]);
    a.ds[i] = static_cast<emx::h16*>(sd[i]);
  }
  a.nb = num_blocks;
  a.bs = page_size;
  a.Hkv = num_kv_heads;
  a.D = head_dim;
  a.gs = group_size;
  const long words = (long)num_blocks * num_kv_heads * page_size * head_dim * bits / 32;
  const unsigned grid = (unsigned)std::min<long>((words + 255) / 256, 8192);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (to_pages)
    hipLaunchKernelGGL(bits == 4 ? emx::pages_from_logical<4> : emx::pages_from_logical<8>, dim3(grid), dim3(256), 0,
                       st, a);
  else
    hipLaunchKernelGGL(bits == 4 ? emx::logical_from_pages<4> : emx::logical_from_pages<8>, dim3(grid), dim3(256), 0,
                       st, a);
  return check_launch(to_pages ? "pages_from_logical" : "logical_from_pages");
}

}  // namespace

int emx_affine_pages_from_logical(const uint32_t* k_codes_in, const uint32_t* v_codes_in, const void* k_scales_in,
                                  const void* k_biases_in, const void* v_scales_in, const void* v_biases_in,
                                  int num_blocks, int page_size, int num_kv_heads, int head_dim, int bits,
                                  int group_size, uint32_t* k_codes, uint32_t* v_codes, void* k_scales,
                                  void* k_biases, void* v_scales, void* v_biases, void* stream) {
  const void* const src[4] = {k_scales_in, k_biases_in, v_scales_in, v_biases_in};
  void* const dst[4] = {k_scales, k_biases, v_scales, v_biases};
  return convert_layout(true, k_codes_in, v_codes_in, src, num_blocks, page_size, num_kv_heads, head_dim, bits,
                        group_size, k_codes, v_codes, dst, stream);
}

int emx_affine_logical_from_pages(const uint32_t* k_codes, const uint32_t* v_codes, const void* k_scales,
                                  const void* k_biases, const void* v_scales, const void* v_biases, int num_blocks,
                                  int page_size, int num_kv_heads, int head_dim, int bits, int group_size,
                                  uint32_t* k_codes_out, uint32_t* v_codes_out, void* k_scales_out,
                                  void* k_biases_out, void* v_scales_out, void* v_biases_out, void* stream) {
  const void* const src[4] = {k_scales, k_biases, v_scales, v_biases};
  void* const dst[4] = {k_scales_out, k_biases_out, v_scales_out, v_biases_out};
  return convert_layout(false, k_codes, v_codes, src, num_blocks, page_size, num_kv_heads, head_dim, bits,
                        group_size, k_codes_out, v_codes_out, dst, stream);
}

int emx_gather_kv_affine(const uint32_t* k_codes, const void* k_scales, const void* k_biases, const uint32_t* v_codes,
                         const void* v_scales, const void* v_biases, int num_blocks, int page_size, int num_kv_heads,
                         int head_dim, int bits, int group_size, const int32_t* block_table, int num_seqs,
                         int max_blocks_per_seq, const int32_t* cu_seq_lens, int total_tokens, int out_dtype,
                         void* k_out, void* v_out, void* stream) {
  if (bits != 4 && bits != 8) return fail(EMX_ERR_UNSUPPORTED, "bits must be 4 or 8, got %d", bits);
  if (num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0 || group_size <= 0 || head_dim % group_size ||
      (head_dim * bits) % 32 || (page_size * bits) % 32 || (page_size > 256 / bits && page_size % (256 / bits)))
    return fail(EMX_ERR_INVALID, "affine page geometry (head_dim %d, group_size %d, page_size %d, bits %d)", head_dim,
                group_size, page_size, bits);
  if (total_tokens > 0 && (!k_codes || !k_scales || !k_biases || !v_codes || !v_scales || !v_biases))
    return fail(EMX_ERR_INVALID, "null cache pointer");
  const emx::h16 *ks = reinterpret_cast<const emx::h16*>(k_scales), *kb = reinterpret_cast<const emx::h16*>(k_biases);
  const emx::h16 *vs = reinterpret_cast<const emx::h16*>(v_scales), *vb = reinterpret_cast<const emx::h16*>(v_biases);
  if (bits == 4)
    return launch_gather(emx::AffineKV<4>{k_codes, ks, kb, v_codes, vs, vb, num_kv_heads, head_dim, page_size,
                                          group_size},
                         block_table, num_seqs, max_blocks_per_seq, cu_seq_lens, total_tokens, num_blocks, out_dtype,
                         k_out, v_out, stream);
  return launch_gather(emx::AffineKV<8>{k_codes, ks, kb, v_codes, vs, vb, num_kv_heads, head_dim, page_size,
                                        group_size},
                       block_table, num_seqs, max_blocks_per_seq, cu_seq_lens, total_tokens, num_blocks, out_dtype,
                       k_out, v_out, stream);
}

int emx_probe_page_read(const uint32_t* k_codes, const void* k_scales, const void* k_biases, const uint32_t* v_codes,
                        const void* v_scales, const void* v_biases, int num_blocks, int page_size, int num_kv_heads,
                        int head_dim, int bits, int group_size, const int32_t* block_tables, int num_seqs,
                        int max_blocks_per_seq, const int32_t* kv_lens, uint32_t* sink, int sink_words,
                        void* stream) {
  if (bits != 4 && bits != 8) return fail(EMX_ERR_UNSUPPORTED, "bits must be 4 or 8, got %d", bits);
  if (head_dim != 128 || page_size <= 0 || page_size % 64 || num_kv_heads <= 0 || num_blocks <= 0 ||
      (group_size != 32 && group_size != 64 && group_size != 128))
    return fail(EMX_ERR_UNSUPPORTED, "probe geometry: head_dim 128, page_size a multiple of 64, group 32/64/128");
  if (num_seqs <= 0 || max_blocks_per_seq <= 0 || sink_words <= 0)
    return fail(EMX_ERR_INVALID, "num_seqs, max_blocks_per_seq and sink_words must be > 0");
  if (!k_codes || !k_scales || !k_biases || !v_codes || !v_scales || !v_biases || !block_tables || !kv_lens || !sink)
    return fail(EMX_ERR_INVALID, "null pointer");
  if (!aligned16(k_codes) || !aligned16(v_codes) || !aligned16(k_scales) || !aligned16(k_biases) ||
      !aligned16(v_scales) || !aligned16(v_biases))
    return fail(EMX_ERR_INVALID, "cache tensors must be 16-byte aligned");
  emx::ProbeArgs a;
  a.kc = k_codes;
  a.ks = reinterpret_cast<const emx::h16*>(k_scales);
  a.kb = reinterpret_cast<const emx::h16*>(k_biases);
  a.vs = reinterpret_cast<const emx::h16*>(v_scales);
  a.vb = reinterpret_cast<const emx::h16*>(v_biases);
  a.vc = v_codes;
  a.block_tables = block_tables;
  a.kv_lens = kv_lens;
  a.sink = sink;
  a.S = num_seqs;
  a.Hkv = num_kv_heads;
  a.bs = page_size;
  a.nb = num_blocks;
  a.max_blocks = max_blocks_per_seq;
  a.G = head_dim / group_size;
  const long long nsl = (long long)num_seqs * max_blocks_per_seq * (page_size / 64) * num_kv_heads;
  if (nsl >= (1LL << 31) - (1LL << 24)) return fail(EMX_ERR_UNSUPPORTED, "too many page slices (%lld)", nsl);
  a.nsl = (int)nsl;
  const int grid = std::min(sink_words, 8 * device_cus());
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (bits == 4)
    hipLaunchKernelGGL(emx::probe_page_read<4>, dim3(grid), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(emx::probe_page_read<8>, dim3(grid), dim3(256), 0, st, a);
  return check_launch("probe_page_read");
}

int emx_probe_page_read_fp8(const uint8_t* key_cache, const uint8_t* value_cache, const float* k_scale,
                            const float* v_scale, int num_blocks, int page_size, int num_kv_heads, int head_dim,
                            const int32_t* block_tables, int num_seqs, int max_blocks_per_seq, const int32_t* kv_lens,
                            uint32_t* sink, int sink_words, void* stream) {
  if (head_dim != 128 || page_size <= 0 || page_size % 32 || num_kv_heads <= 0 || num_blocks <= 0)
    return fail(EMX_ERR_UNSUPPORTED, "probe geometry: head_dim 128, page_size a multiple of 32");
  if (num_seqs <= 0 || max_blocks_per_seq <= 0 || sink_words <= 0)
    return fail(EMX_ERR_INVALID, "num_seqs, max_blocks_per_seq and sink_words must be > 0");
  if (!key_cache || !value_cache || !k_scale || !v_scale || !block_tables || !kv_lens || !sink)
    return fail(EMX_ERR_INVALID, "null pointer");
  const long long nsl = (long long)num_seqs * max_blocks_per_seq * (page_size / 32) * num_kv_heads;
  if (nsl >= (1LL << 31) - (1LL << 24)) return fail(EMX_ERR_UNSUPPORTED, "too many page slices (%lld)", nsl);
  emx::ProbeFp8Args a;
  a.k8 = key_cache;
  a.v8 = value_cache;
  a.kps = k_scale;
  a.vps = v_scale;
  a.block_tables = block_tables;
  a.kv_lens = kv_lens;
  a.sink = sink;
  a.S = num_seqs;
  a.Hkv = num_kv_heads;
  a.bs = page_size;
  a.nb = num_blocks;
  a.max_blocks = max_blocks_per_seq;
  a.nsl = (int)nsl;
  const int grid = std::min(sink_words, 8 * device_cus());
  hipLaunchKernelGGL(emx::probe_page_read_fp8, dim3(grid), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), a);
  return check_launch("probe_page_read_fp8");
}

int emx_gather_kv_fp8(const uint8_t* key_cache, const uint8_t* value_cache, const float* k_scale,
                      const float* v_scale, int num_blocks, int page_size, int num_kv_heads, int head_dim,
                      const int32_t* block_table, int num_seqs, int max_blocks_per_seq, const int32_t* cu_seq_lens,
                      int total_tokens, int out_dtype, void* k_out, void* v_out, void* stream) {
  if (num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0) return fail(EMX_ERR_INVALID, "bad cache geometry");
  if (total_tokens > 0 && (!key_cache || !value_cache || !k_scale || !v_scale))
    return fail(EMX_ERR_INVALID, "null cache pointer");
  return launch_gather(emx::Fp8KV{key_cache, value_cache, k_scale, v_scale, num_kv_heads, head_dim, page_size},
                       block_table, num_seqs, max_blocks_per_seq, cu_seq_lens, total_tokens, num_blocks, out_dtype,
                       k_out, v_out, stream);
}

int emx_gather_kv_dense(const void* key_cache, const void* value_cache, int dtype, int num_blocks, int page_size,
                        int num_kv_heads, int head_dim, const int32_t* block_table, int num_seqs,
                        int max_blocks_per_seq, const int32_t* cu_seq_lens, int total_tokens, int out_dtype,
                        void* k_out, void* v_out, void* stream) {
  if (num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0) return fail(EMX_ERR_INVALID, "bad cache geometry");
  if (total_tokens > 0 && (!key_cache || !value_cache)) return fail(EMX_ERR_INVALID, "null cache pointer");
  switch (dtype) {
    case EMX_DTYPE_F16:
      return launch_gather(emx::DenseKV<emx::F16>{reinterpret_cast<const emx::h16*>(key_cache),
                                                  reinterpret_cast<const emx::h16*>(value_cache), num_kv_heads,
                                                  head_dim, page_size},
                           block_table, num_seqs, max_blocks_per_seq, cu_seq_lens, total_tokens, num_blocks,
                           out_dtype, k_out, v_out, stream);
    case EMX_DTYPE_BF16:
      return launch_gather(emx::DenseKV<emx::BF16>{reinterpret_cast<const uint16_t*>(key_cache),
                                                   reinterpret_cast<const uint16_t*>(value_cache), num_kv_heads,
                                                   head_dim, page_size},
                           block_table, num_seqs, max_blocks_per_seq, cu_seq_lens, total_tokens, num_blocks,
                           out_dtype, k_out, v_out, stream);
    case EMX_DTYPE_F32:
      return launch_gather(emx::DenseKV<emx::F32>{reinterpret_cast<const float*>(key_cache),
                                                  reinterpret_cast<const float*>(value_cache), num_kv_heads,
                                                  head_dim, page_size},
                           block_table, num_seqs, max_blocks_per_seq, cu_seq_lens, total_tokens, num_blocks,
                           out_dtype, k_out, v_out, stream);
  }
  return fail(EMX_ERR_INVALID, "unknown dtype %d", dtype);
}

int emx_rope_rows(void* x, int rows, int heads, int head_dim, const int32_t* positions, const float* inv_freq,
                  int rot_dims, int traditional, void* stream) {
  if (rows < 0 || heads <= 0 || head_dim <= 0) return fail(EMX_ERR_INVALID, "rows >= 0, heads and head_dim > 0");
  if (rows == 0) return EMX_OK;
  if (!x || !rope_ok(positions, inv_freq, rot_dims, head_dim))
    return fail(EMX_ERR_INVALID, "rope: x, positions and inv_freq needed, rot_dims even and in (0, head_dim]");
  const long n = (long)rows * heads * (rot_dims / 2);
  const unsigned grid = (unsigned)std::min<long>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(emx::rope_rows, dim3(grid), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<emx::h16*>(x), reinterpret_cast<const emx::h16*>(x), rows, heads, head_dim,
                     emx::RopeArgs{inv_freq, positions, rot_dims, traditional ? 1 : 0});
  return check_launch("rope_rows");
}

size_t emx_paged_prefill_workspace_bytes(int num_tokens, int num_seqs, int num_q_heads, int num_kv_heads,
                                         int head_dim) {
  if (num_tokens <= 0 || num_seqs <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || head_dim != 128 ||
      num_q_heads % num_kv_heads != 0)
    return 0;
  const int hg = num_q_heads / num_kv_heads;
  if (hg > 16 || (hg & (hg - 1)) != 0) return 0;
  const long items = prefill_max_items(num_tokens, num_seqs, 128 / hg);
  if (items * num_kv_heads * 4 > emx::kPrefillCounters) return 0;
  return 256 + (size_t)items * num_kv_heads * emx::kPrefillParts * emx::kPrefillPartBytes;
}

size_t emx_paged_workspace_bytes(int num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                                 int max_blocks_per_seq, int page_size) {
  if (num_seqs <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || max_blocks_per_seq <= 0 || page_size <= 0 ||
      num_seqs > emx::kMaxSeqs || (long)num_seqs * num_kv_heads > emx::kMaxUnits || num_q_heads % num_kv_heads)
    return 0;
  size_t fast = 0;
  const int hg = num_q_heads / num_kv_heads;
  if (head_dim == 128 && page_size % 16 == 0 && decode_max_waves() <= emx::kMaxWaves) {
    // arrival counters and the plan cache at fixed offsets (so every call finds them as
    // the last call left them), then the split-K partials
    const size_t slots = (size_t)decode_max_waves() + (size_t)num_seqs * num_kv_heads;
    fast = kPartialsInt * sizeof(int) + slots * hg * (head_dim + 2) * sizeof(float);
  }
  // the split-K decode of the other shapes keeps its chunks' partials after the same offset
  const size_t split = split_workspace_bytes(num_seqs, num_q_heads, num_kv_heads, head_dim, max_blocks_per_seq,
                                             page_size);
  return std::max(fast, split ? kPartialsInt * sizeof(int) + split : 0);
}

int emx_paged_attention_affine(const void* queries, int num_tokens, int num_q_heads, int head_dim,
                               const uint32_t* k_codes, const void* k_scales, const void* k_biases,
                               const uint32_t* v_codes, const void* v_scales, const void* v_biases, int num_blocks,
                               int page_size, int num_kv_heads, int bits, int group_size,
                               const int32_t* block_tables, int num_seqs, int max_blocks_per_seq,
                               const int32_t* kv_lens, const int32_t* query_start_loc, float softmax_scale,
                               int sliding_window, int single_token_decode, void* workspace, size_t workspace_bytes,
                               void* out, void* stream) {
  int rc = validate_common(queries, num_tokens, num_q_heads, head_dim, num_kv_heads, num_blocks, page_size,
                           block_tables, num_seqs, max_blocks_per_seq, kv_lens, query_start_loc, single_token_decode,
                           out);
  if (rc) return rc;
  if (bits != 4 && bits != 8) return fail(EMX_ERR_UNSUPPORTED, "bits must be 4 or 8, got %d", bits);
  if (group_size <= 0 || head_dim % group_size != 0)
    return fail(EMX_ERR_INVALID, "head_dim %d must be a multiple of group_size %d", head_dim, group_size);
  if ((head_dim * bits) % 32 != 0 || (page_size * bits) % 32 != 0)
    return fail(EMX_ERR_INVALID, "head_dim * bits and page_size * bits must be multiples of 32");
  if (page_size > 256 / bits && page_size % (256 / bits) != 0)
    return fail(EMX_ERR_INVALID, "page_size %d above 256/bits must be a multiple of 256/bits", page_size);
  if (!std::isfinite(softmax_scale)) return fail(EMX_ERR_INVALID, "softmax_scale must be finite");
  if (num_tokens == 0) return EMX_OK;
  if (!k_codes || !k_scales || !k_biases || !v_codes || !v_scales || !v_biases)
    return fail(EMX_ERR_INVALID, "null cache pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int hg = num_q_heads / num_kv_heads;
  const float scale_log2 = softmax_scale * emx::kLog2e;
  const int window = sliding_window > 0 ? sliding_window : 0;

  const size_t need =
      emx_paged_workspace_bytes(num_seqs, num_q_heads, num_kv_heads, head_dim, max_blocks_per_seq, page_size);
  // MFMA paths: decode rows (one query token) on the split-K decode kernel, rows of
  // longer queries on the prefill kernel; anything else on the generic kernel.
  if (need > 0 && decode_fast_path(head_dim, page_size, bits, group_size, hg, num_seqs, single_token_decode) &&
      (single_token_decode || prefill_fast_path(hg))) {
    if (!aligned16(queries) || !aligned16(k_codes) || !aligned16(v_codes) || !aligned16(k_scales) ||
        !aligned16(k_biases) || !aligned16(v_scales) || !aligned16(v_biases))
      return fail(EMX_ERR_INVALID, "queries and cache tensors must be 16-byte aligned");
    if (workspace == nullptr || workspace_bytes < need)
      return fail(EMX_ERR_INVALID, "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    emx::PrefillArgs p;
    long pgrid = 0;          // prefill workgroups (mixed batch)
    UnifiedFn uf = nullptr;  // the mixed batch's single launch
    if (!single_token_decode) {
      p.q = reinterpret_cast<const emx::h16*>(queries);
      p.kc = k_codes;
      p.ks = reinterpret_cast<const emx::h16*>(k_scales);
      p.kb = reinterpret_cast<const emx::h16*>(k_biases);
      p.vc = v_codes;
      p.vs = reinterpret_cast<const emx::h16*>(v_scales);
      p.vb = reinterpret_cast<const emx::h16*>(v_biases);
      p.block_tables = block_tables;
      p.kv_lens = kv_lens;
      p.qsl = query_start_loc;
      p.out = reinterpret_cast<emx::h16*>(out);
      p.S = num_seqs;
      p.Hq = num_q_heads;
      p.Hkv = num_kv_heads;
      p.bs = page_size;
      p.nb = num_blocks;
      p.max_blocks = max_blocks_per_seq;
      p.scale_log2 = scale_log2;
      p.window = window;
      p.min_q = 2;
      prefill_split(p, num_tokens, num_q_heads, num_kv_heads, workspace, workspace_bytes, need);
      PrefillFn pf = bits == 4 ? pick_prefill_gs<4>(group_size, hg) : pick_prefill_gs<8>(group_size, hg);
      if (!pf)
        return fail(EMX_ERR_UNSUPPORTED, "no prefill kernel for bits=%d group_size=%d gqa=%d", bits, group_size, hg);
      // tiles of 128/hg query tokens: at most num_tokens/tile + num_seqs of them per kv head
      const int tokb = 128 / hg;
      pgrid = (long)((num_tokens + tokb - 1) / tokb + num_seqs) * num_kv_heads * p.nparts;
      // prefill and decode rows go out as one launch (below) when a unified kernel
      // pairs this prefill with the decode kernel picked for the rows
      const bool q4u = bits == 4 && (page_size & (page_size - 1)) == 0 && pick_decode_q4(group_size, hg, page_size);
      uf = q4u ? pick_unified_q4(group_size, hg)
               : bits == 4 ? pick_unified_affine<4>(group_size, hg) : pick_unified_affine<8>(group_size, hg);
      if (!uf) {
        hipLaunchKernelGGL(pf, dim3((unsigned)pgrid), dim3(256), 0, st, p);
        if (int r = check_launch("prefill_affine_d128")) return r;
        pgrid = 0;
      }
    }
    // the 4-bit kernel addresses pages with shifts: power-of-two page sizes
    const Q4Fn q4fn =
        bits == 4 && (page_size & (page_size - 1)) == 0 ? pick_decode_q4(group_size, hg, page_size) : nullptr;
    const bool q4 = q4fn != nullptr;
    const int nw = q4 ? decode_q4_num_waves() : decode_num_waves();
    const DecodeFn fn = q4 ? nullptr : bits == 4 ? pick_decode_gs<4>(group_size, hg) : pick_decode_gs<8>(group_size, hg);
    if (!q4 && !fn)
      return fail(EMX_ERR_UNSUPPORTED, "no decode kernel for bits=%d group_size=%d gqa=%d", bits, group_size, hg);
    emx::DecodeArgs a;
    a.q = reinterpret_cast<const emx::h16*>(queries);
    a.kc = k_codes;
    a.ks = reinterpret_cast<const emx::h16*>(k_scales);
    a.kb = reinterpret_cast<const emx::h16*>(k_biases);
    a.vc = v_codes;
    a.vs = reinterpret_cast<const emx::h16*>(v_scales);
    a.vb = reinterpret_cast<const emx::h16*>(v_biases);
    a.block_tables = block_tables;
    a.kv_lens = kv_lens;
    a.qsl = single_token_decode ? nullptr : query_start_loc;
    a.out = reinterpret_cast<emx::h16*>(out);
    const size_t slots = (size_t)decode_max_waves() + (size_t)num_seqs * num_kv_heads;
    a.ws_cnt = reinterpret_cast<int*>(workspace);
    a.ws_cnt_grp = a.ws_cnt + emx::kMaxUnits;
    a.ws_o = reinterpret_cast<float*>(a.ws_cnt + kPartialsInt);
    a.ws_ml = a.ws_o + slots * hg * head_dim;
    a.S = num_seqs;
    a.Hq = num_q_heads;
    a.Hkv = num_kv_heads;
    a.bs = page_size;
    a.nb = num_blocks;
    a.max_blocks = max_blocks_per_seq;
    a.scale_log2 = scale_log2;
    a.window = window;
    a.num_waves = nw;
    // tokens per work item: per wave (16x16 kernel) or per workgroup (4-bit kernel)
    // tokens per work item: per workgroup (4-bit kernel) or per wave (16x16 kernel)
    a.nt = q4 ? 64 * (4 / ((hg + 3) / 4)) : bits == 4 ? 64 : 32;
    if (pgrid > 0) {
      // Decode workgroups sized to the decode rows' share of the step: prefill time
      // ~ prefill tokens * Hq (matrix work), decode time ~ decode rows * Hkv * page
      // bytes per token; 28 is their ratio at 144 bytes (4-bit, group 64) at the
      // rates measured on MI355X.  Enough workgroups that the decode, beside the
      // prefill, ends with it (c3: 112; 64 .. 128 all gave 96 us against 105 us for
      // two launches, 32 gave 123 us).
      const double tok_bytes = 2.0 * head_dim * bits / 8 + 8.0 * head_dim / group_size;
      const double share = 28.0 * tok_bytes / 144.0 * num_seqs / std::max(1, num_tokens - num_seqs) * num_kv_heads /
                           num_q_heads;
      const int ndec = std::clamp((int)std::ceil(1024.0 * share), device_cus() / 4, nw / 4);
      a.num_waves = 4 * ndec;  // the 16x16 body splits its ranges over these waves
      hipLaunchKernelGGL(uf, dim3((unsigned)(pgrid + ndec)), dim3(256), 0, st, p, a, ndec);
      return check_launch(q4 ? "unified_q4" : "unified_affine");
    }
    // two workgroups per compute unit: the second of each starts later (4-bit kernel's range balance)
    a.first_slot = q4 ? nw / 8 : 0;
    // pure decode on the 4-bit kernel: the plan cache in the workspace
    a.plan = q4 && single_token_decode && nw / 4 <= emx::kPlanMaxWG ? a.ws_cnt + kCounterInts : nullptr;
    if (q4) {
      hipLaunchKernelGGL(q4fn, dim3((unsigned)(nw / 4)), dim3(256), 0, st, a.plan, a.kv_lens, a.block_tables, a.S,
                         a.max_blocks, a);
      return check_launch("decode_q4_d128");
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)(nw / 4)), dim3(256), 0, st, a);
    return check_launch("decode_affine_d128");
  }

  if (queries && !aligned16(queries)) return fail(EMX_ERR_INVALID, "queries must be 16-byte aligned");
  emx::GenericArgs ga;
  ga.q = queries;
  ga.out = out;
  ga.block_tables = block_tables;
  ga.kv_lens = kv_lens;
  ga.qsl = query_start_loc;
  ga.T = num_tokens;
  ga.S = num_seqs;
  ga.Hq = num_q_heads;
  ga.Hkv = num_kv_heads;
  ga.D = head_dim;
  ga.bs = page_size;
  ga.nb = num_blocks;
  ga.max_blocks = max_blocks_per_seq;
  ga.scale_log2 = scale_log2;
  ga.window = window;
  ga.decode = single_token_decode ? 1 : 0;
  if (bits == 4) {
    emx::AffineKV<4> kv{k_codes,
                        reinterpret_cast<const emx::h16*>(k_scales),
                        reinterpret_cast<const emx::h16*>(k_biases),
                        v_codes,
                        reinterpret_cast<const emx::h16*>(v_scales),
                        reinterpret_cast<const emx::h16*>(v_biases),
                        num_kv_heads,
                        head_dim,
                        page_size,
                        group_size};
    return launch_generic<emx::h16>(ga, kv, st, workspace, workspace_bytes);
  }
  emx::AffineKV<8> kv{k_codes,
                      reinterpret_cast<const emx::h16*>(k_scales),
                      reinterpret_cast<const emx::h16*>(k_biases),
                      v_codes,
                      reinterpret_cast<const emx::h16*>(v_scales),
                      reinterpret_cast<const emx::h16*>(v_biases),
                      num_kv_heads,
                      head_dim,
                      page_size,
                      group_size};
  return launch_generic<emx::h16>(ga, kv, st, workspace, workspace_bytes);
}

int emx_paged_attention_dense(const void* queries, int num_tokens, int num_q_heads, int head_dim, int dtype,
                              const void* key_cache, const void* value_cache, int num_blocks, int page_size,
                              int num_kv_heads, const int32_t* block_tables, int num_seqs, int max_blocks_per_seq,
                              const int32_t* kv_lens, const int32_t* query_start_loc, float softmax_scale,
                              int sliding_window, int single_token_decode, void* workspace, size_t workspace_bytes,
                              void* out, void* stream) {
  int rc = validate_common(queries, num_tokens, num_q_heads, head_dim, num_kv_heads, num_blocks, page_size,
                           block_tables, num_seqs, max_blocks_per_seq, kv_lens, query_start_loc, single_token_decode,
                           out);
  if (rc) return rc;
  if (!std::isfinite(softmax_scale)) return fail(EMX_ERR_INVALID, "softmax_scale must be finite");
  if (num_tokens == 0) return EMX_OK;
  if (!key_cache || !value_cache) return fail(EMX_ERR_INVALID, "null cache pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  emx::GenericArgs ga;
  ga.q = queries;
  ga.out = out;
  ga.block_tables = block_tables;
  ga.kv_lens = kv_lens;
  ga.qsl = query_start_loc;
  ga.T = num_tokens;
  ga.S = num_seqs;
  ga.Hq = num_q_heads;
  ga.Hkv = num_kv_heads;
  ga.D = head_dim;
  ga.bs = page_size;
  ga.nb = num_blocks;
  ga.max_blocks = max_blocks_per_seq;
  ga.scale_log2 = softmax_scale * emx::kLog2e;
  ga.window = sliding_window > 0 ? sliding_window : 0;
  ga.decode = single_token_decode ? 1 : 0;
  switch (dtype) {
    case EMX_DTYPE_F16: {
      emx::DenseKV<emx::F16> kv{reinterpret_cast<const emx::h16*>(key_cache),
                                reinterpret_cast<const emx::h16*>(value_cache), num_kv_heads, head_dim, page_size};
      return launch_generic<emx::h16>(ga, kv, st, workspace, workspace_bytes);
    }
    case EMX_DTYPE_BF16: {
      emx::DenseKV<emx::BF16> kv{reinterpret_cast<const uint16_t*>(key_cache),
                                 reinterpret_cast<const uint16_t*>(value_cache), num_kv_heads, head_dim, page_size};
      return launch_generic<uint16_t>(ga, kv, st, workspace, workspace_bytes);
    }
    case EMX_DTYPE_F32: {
      emx::DenseKV<emx::F32> kv{reinterpret_cast<const float*>(key_cache),
                                reinterpret_cast<const float*>(value_cache), num_kv_heads, head_dim, page_size};
      return launch_generic<float>(ga, kv, st, workspace, workspace_bytes);
    }
  }
  return fail(EMX_ERR_UNSUPPORTED, "unknown dtype code %d", dtype);
}

size_t emx_fp8_write_workspace_bytes(void) { return sizeof(float) * 2 * emx::kFp8Parts; }

static int fp8_write_impl(const void* keys, const void* values, int dtype, const int32_t* slot_mapping, int num_tokens,
                          int num_kv_heads, int head_dim, int page_size, int num_blocks, uint8_t* key_cache,
                          uint8_t* value_cache, float* k_scales, float* v_scales, void* workspace,
                          size_t workspace_bytes, const emx::RopeArgs& rope, const void* queries_in,
                          void* queries, int num_q_heads, void* stream) {
  if (num_tokens < 0) return fail(EMX_ERR_INVALID, "num_tokens must be >= 0");
  if (num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0 || num_blocks <= 0)
    return fail(EMX_ERR_INVALID, "num_kv_heads, head_dim, page_size, num_blocks must be positive");
  if (head_dim % 4 != 0) return fail(EMX_ERR_UNSUPPORTED, "head_dim %d must be a multiple of 4", head_dim);
  if (dtype != EMX_DTYPE_F16 && dtype != EMX_DTYPE_BF16 && dtype != EMX_DTYPE_F32)
    return fail(EMX_ERR_INVALID, "unknown dtype %d", dtype);
  if (num_tokens == 0) return EMX_OK;
  if (!keys || !values || !slot_mapping || !key_cache || !value_cache || !k_scales || !v_scales || !workspace)
    return fail(EMX_ERR_INVALID, "null pointer");
  if (workspace_bytes < emx_fp8_write_workspace_bytes())
    return fail(EMX_ERR_INVALID, "workspace of %zu bytes, %zu needed", workspace_bytes, emx_fp8_write_workspace_bytes());
  if ((reinterpret_cast<uintptr_t>(key_cache) | reinterpret_cast<uintptr_t>(value_cache)) & 3)
    return fail(EMX_ERR_INVALID, "key/value cache must be 4-byte aligned");
  emx::Fp8WriteArgs a;
  a.k = keys;
  a.v = values;
  a.slot = slot_mapping;
  a.T = num_tokens;
  a.Hkv = num_kv_heads;
  a.D = head_dim;
  a.bs = page_size;
  a.nb = num_blocks;
  a.kc = key_cache;
  a.vc = value_cache;
  a.ks = k_scales;
  a.vs = v_scales;
  a.part = reinterpret_cast<float*>(workspace);
  a.rope = rope;
  a.q = reinterpret_cast<emx::h16*>(queries);
  a.q_in = queries_in ? reinterpret_cast<const emx::h16*>(queries_in) : a.q;
  a.Hq = num_q_heads;
  a.slot_ids = nullptr;  // slot_mapping given (emx_fp8_cache_append_rope sets these)
  a.kv_lens = nullptr;
  a.bt = nullptr;
  a.S = a.max_blocks = 0;
  a.counter = nullptr;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const size_t n = (size_t)num_tokens * num_kv_heads * head_dim;
  if (n / 4 >= ((size_t)1 << 31)) return fail(EMX_ERR_UNSUPPORTED, "%zu values per tensor exceed the 2^33 limit", n);
  const int nparts = (int)std::min<size_t>(emx::kFp8Parts, (n / 4 + 255) / 256);
  const int nwrite = (int)std::min<size_t>(1024, (n / 4 + 255) / 256);
  const bool turn_q = rope.inv_freq != nullptr && queries != nullptr;
  if (n <= (size_t)emx::kFp8SelfMax) {  // one launch: each workgroup takes the maxima itself
    a.nwg = (int)((n / 4 + 1023) / 1024);
    const dim3 g1((unsigned)(a.nwg + (turn_q ? 4 : 0)));  // + workgroups that turn the queries
    switch (dtype) {
      case EMX_DTYPE_F16: hipLaunchKernelGGL((emx::fp8_write<emx::F16, true>), g1, dim3(1024), 0, st, a, 0); break;
      case EMX_DTYPE_BF16: hipLaunchKernelGGL((emx::fp8_write<emx::BF16, true>), g1, dim3(1024), 0, st, a, 0); break;
      default: hipLaunchKernelGGL((emx::fp8_write<emx::F32, true>), g1, dim3(1024), 0, st, a, 0); break;
    }
    return check_launch("fp8_cache_write");
  }
  switch (dtype) {
    case EMX_DTYPE_F16:
      hipLaunchKernelGGL(emx::fp8_amax<emx::F16>, dim3(nparts), dim3(256), 0, st, a);
      hipLaunchKernelGGL(emx::fp8_write<emx::F16>, dim3(nwrite), dim3(256), 0, st, a, nparts);
      break;
    case EMX_DTYPE_BF16:
      hipLaunchKernelGGL(emx::fp8_amax<emx::BF16>, dim3(nparts), dim3(256), 0, st, a);
      hipLaunchKernelGGL(emx::fp8_write<emx::BF16>, dim3(nwrite), dim3(256), 0, st, a, nparts);
      break;
    default:
      hipLaunchKernelGGL(emx::fp8_amax<emx::F32>, dim3(nparts), dim3(256), 0, st, a);
      hipLaunchKernelGGL(emx::fp8_write<emx::F32>, dim3(nwrite), dim3(256), 0, st, a, nparts);
      break;
  }
  if (int rc = check_launch("fp8_cache_write")) return rc;
  if (turn_q) {  // larger writes: the queries in their own launch
    const long nq = (long)num_tokens * num_q_heads * (head_dim / 2);
    hipLaunchKernelGGL(emx::rope_rows, dim3((unsigned)std::min<long>((nq + 255) / 256, 4096)), dim3(256), 0, st,
                       a.q, a.q_in, num_tokens, num_q_heads, head_dim, rope);
    return check_launch("rope_rows");
  }
  return EMX_OK;
}

int emx_fp8_cache_write(const void* keys, const void* values, int dtype, const int32_t* slot_mapping, int num_tokens,
                        int num_kv_heads, int head_dim, int page_size, int num_blocks, uint8_t* key_cache,
                        uint8_t* value_cache, float* k_scales, float* v_scales, void* workspace,
                        size_t workspace_bytes, void* stream) {
  return fp8_write_impl(keys, values, dtype, slot_mapping, num_tokens, num_kv_heads, head_dim, page_size, num_blocks,
                        key_cache, value_cache, k_scales, v_scales, workspace, workspace_bytes,
                        emx::RopeArgs{nullptr, nullptr, 0, 0}, nullptr, nullptr, 0, stream);
}

int emx_fp8_cache_write_noalloc(const void* keys, const void* values, int dtype, const int32_t* slot_mapping,
                                int num_tokens, int num_kv_heads, int head_dim, int page_size, int num_blocks,
                                uint8_t* key_cache, uint8_t* value_cache, float* k_scales, float* v_scales,
                                void* stream) {
  static_assert(sizeof(float) * kNoallocScratchFloats >= sizeof(float) * 2 * emx::kFp8Parts,
                "scratch holds the FP8 write's per-workgroup maxima");
  // the scratch is a fixed 2 KiB whatever the call's size; the size limit is the
  // FP8 write's own (fewer than 2^33 values per tensor, checked by fp8_write_impl)
  int rc = EMX_OK;
  void* ws = num_tokens > 0 ? noalloc_scratch(stream, &rc) : nullptr;
  if (num_tokens > 0 && ws == nullptr) return rc;
  return fp8_write_impl(keys, values, dtype, slot_mapping, num_tokens, num_kv_heads, head_dim, page_size, num_blocks,
                        key_cache, value_cache, k_scales, v_scales, ws, sizeof(float) * kNoallocScratchFloats,
                        emx::RopeArgs{nullptr, nullptr, 0, 0}, nullptr, nullptr, 0, stream);
}

int emx_fp8_cache_write_rope(const void* keys, const void* values, int dtype, const int32_t* slot_mapping,
                             int num_tokens, int num_kv_heads, int head_dim, int page_size, int num_blocks,
                             uint8_t* key_cache, uint8_t* value_cache, float* k_scales, float* v_scales,
                             void* workspace, size_t workspace_bytes, const int32_t* positions, const float* inv_freq,
                             int rot_dims, int traditional, const void* queries_in, void* queries,
                             int num_q_heads, void* stream) {
  if (num_tokens > 0 && (!rope_ok(positions, inv_freq, rot_dims, head_dim) || rot_dims % (traditional ? 4 : 8) != 0))
    return fail(EMX_ERR_INVALID,
                "rope: positions and inv_freq needed, rot_dims in (0, head_dim] and a multiple of 8 (4 if traditional)");
  if (queries != nullptr && num_q_heads <= 0) return fail(EMX_ERR_INVALID, "queries need num_q_heads > 0");
  if (queries_in != nullptr && queries == nullptr) return fail(EMX_ERR_INVALID, "queries_in needs queries");
  return fp8_write_impl(keys, values, dtype, slot_mapping, num_tokens, num_kv_heads, head_dim, page_size, num_blocks,
                        key_cache, value_cache, k_scales, v_scales, workspace, workspace_bytes,
                        emx::RopeArgs{inv_freq, positions, rot_dims, traditional ? 1 : 0}, queries_in, queries,
                        num_q_heads, stream);
}

int emx_fp8_cache_append_rope(const void* keys, const void* values, int dtype, const int32_t* slot_ids,
                              int num_tokens, const int32_t* block_tables, int num_seqs, int max_blocks_per_seq,
                              int32_t* kv_lens, int* counter, int num_kv_heads, int head_dim, int page_size,
                              int num_blocks, uint8_t* key_cache, uint8_t* value_cache, float* k_scales,
                              float* v_scales, const float* inv_freq, int rot_dims, int traditional,
                              const void* queries_in, void* queries, int num_q_heads, void* stream) {
  if (num_tokens < 0 || num_seqs <= 0 || max_blocks_per_seq <= 0)
    return fail(EMX_ERR_INVALID, "num_tokens >= 0, num_seqs and max_blocks_per_seq > 0 needed");
  if (num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0 || num_blocks <= 0)
    return fail(EMX_ERR_INVALID, "num_kv_heads, head_dim, page_size, num_blocks must be positive");
  if (head_dim % 4 != 0) return fail(EMX_ERR_UNSUPPORTED, "head_dim %d must be a multiple of 4", head_dim);
  if (dtype != EMX_DTYPE_F16 && dtype != EMX_DTYPE_BF16 && dtype != EMX_DTYPE_F32)
    return fail(EMX_ERR_INVALID, "unknown dtype %d", dtype);
  const size_t n = (size_t)num_tokens * num_kv_heads * head_dim;
  if (num_tokens > emx::kFp8AppendMax || n > (size_t)emx::kFp8SelfMax)
    return fail(EMX_ERR_UNSUPPORTED, "decode append: at most %d tokens and %d values per tensor", emx::kFp8AppendMax,
                emx::kFp8SelfMax);
  if (num_tokens == 0) return EMX_OK;
  if (!inv_freq || rot_dims <= 0 || rot_dims > head_dim || rot_dims % (traditional ? 4 : 8) != 0)
    return fail(EMX_ERR_INVALID, "rope: inv_freq needed, rot_dims in (0, head_dim] and a multiple of 8 (4 if traditional)");
  if (queries != nullptr && num_q_heads <= 0) return fail(EMX_ERR_INVALID, "queries need num_q_heads > 0");
  if (queries_in != nullptr && queries == nullptr) return fail(EMX_ERR_INVALID, "queries_in needs queries");
  if (!keys || !values || !slot_ids || !block_tables || !kv_lens || !counter || !key_cache || !value_cache ||
      !k_scales || !v_scales)
    return fail(EMX_ERR_INVALID, "null pointer");
  if ((reinterpret_cast<uintptr_t>(key_cache) | reinterpret_cast<uintptr_t>(value_cache)) & 3)
    return fail(EMX_ERR_INVALID, "key/value cache must be 4-byte aligned");
  emx::Fp8WriteArgs a;
  a.k = keys;
  a.v = values;
  a.slot = nullptr;
  a.T = num_tokens;
  a.Hkv = num_kv_heads;
  a.D = head_dim;
  a.bs = page_size;
  a.nb = num_blocks;
  a.kc = key_cache;
  a.vc = value_cache;
  a.ks = k_scales;
  a.vs = v_scales;
  a.part = nullptr;
  a.rope = emx::RopeArgs{inv_freq, nullptr, rot_dims, traditional ? 1 : 0};
  a.q = reinterpret_cast<emx::h16*>(queries);
  a.q_in = queries_in ? reinterpret_cast<const emx::h16*>(queries_in) : a.q;
  a.Hq = num_q_heads;
  a.slot_ids = slot_ids;
  a.kv_lens = kv_lens;
  a.bt = block_tables;
  a.S = num_seqs;
  a.max_blocks = max_blocks_per_seq;
  a.counter = counter;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const uintptr_t in16 = reinterpret_cast<uintptr_t>(keys) | reinterpret_cast<uintptr_t>(values) |
                         reinterpret_cast<uintptr_t>(queries) | reinterpret_cast<uintptr_t>(a.q_in);
  const uintptr_t out8 = reinterpret_cast<uintptr_t>(key_cache) | reinterpret_cast<uintptr_t>(value_cache);
  if (emx::fp8_grid_fits(num_tokens, num_kv_heads, head_dim, rot_dims, traditional ? 1 : 0) && !(in16 & 15) &&
      !(out8 & 7)) {
    const long tasks = 2L * num_tokens * num_kv_heads * (head_dim / 8);  // K pieces, then V pieces
    a.nwg = (int)((tasks + 255) / 256);
    const dim3 g((unsigned)(a.nwg + (queries ? num_tokens : 0)));  // + one workgroup per query token
    switch (dtype) {
      case EMX_DTYPE_F16: hipLaunchKernelGGL(emx::fp8_append_grid<emx::F16>, g, dim3(256), 0, st, a); break;
      case EMX_DTYPE_BF16: hipLaunchKernelGGL(emx::fp8_append_grid<emx::BF16>, g, dim3(256), 0, st, a); break;
      default: hipLaunchKernelGGL(emx::fp8_append_grid<emx::F32>, g, dim3(256), 0, st, a); break;
    }
    return check_launch("fp8_append_grid");
  }
  a.nwg = (int)((n / 4 + 1023) / 1024);
  const dim3 g1((unsigned)(a.nwg + (queries ? 4 : 0)));  // + workgroups that turn the queries
  switch (dtype) {
    case EMX_DTYPE_F16: hipLaunchKernelGGL((emx::fp8_write<emx::F16, true>), g1, dim3(1024), 0, st, a, 0); break;
    case EMX_DTYPE_BF16: hipLaunchKernelGGL((emx::fp8_write<emx::BF16, true>), g1, dim3(1024), 0, st, a, 0); break;
    default: hipLaunchKernelGGL((emx::fp8_write<emx::F32, true>), g1, dim3(1024), 0, st, a, 0); break;
  }
  return check_launch("fp8_cache_write (append)");
}

int emx_paged_attention_fp8(const void* queries, int num_tokens, int num_q_heads, int head_dim, int dtype,
                            const uint8_t* key_cache, const uint8_t* value_cache, const float* k_scale,
                            const float* v_scale, int num_blocks, int page_size, int num_kv_heads,
                            const int32_t* block_tables, int num_seqs, int max_blocks_per_seq, const int32_t* kv_lens,
                            const int32_t* query_start_loc, float softmax_scale, int sliding_window,
                            int single_token_decode, void* workspace, size_t workspace_bytes, void* out,
                            void* stream) {
  int rc = validate_common(queries, num_tokens, num_q_heads, head_dim, num_kv_heads, num_blocks, page_size,
                           block_tables, num_seqs, max_blocks_per_seq, kv_lens, query_start_loc, single_token_decode,
                           out);
  if (rc) return rc;
  if (!std::isfinite(softmax_scale)) return fail(EMX_ERR_INVALID, "softmax_scale must be finite");
  if (num_tokens == 0) return EMX_OK;
  if (!key_cache || !value_cache || !k_scale || !v_scale) return fail(EMX_ERR_INVALID, "null cache or scale pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  emx::GenericArgs ga;
  ga.q = queries;
  ga.out = out;
  ga.block_tables = block_tables;
  ga.kv_lens = kv_lens;
  ga.qsl = query_start_loc;
  ga.T = num_tokens;
  ga.S = num_seqs;
  ga.Hq = num_q_heads;
  ga.Hkv = num_kv_heads;
  ga.D = head_dim;
  ga.bs = page_size;
  ga.nb = num_blocks;
  ga.max_blocks = max_blocks_per_seq;
  ga.scale_log2 = softmax_scale * emx::kLog2e;
  ga.window = sliding_window > 0 ? sliding_window : 0;
  ga.decode = single_token_decode ? 1 : 0;
  const int hg = num_q_heads / num_kv_heads;
  const bool mfma_ok = dtype == EMX_DTYPE_F16 && head_dim == 128 && page_size % 32 == 0 &&
                       num_seqs <= emx::kMaxSeqs && aligned16(queries) && aligned16(key_cache) &&
                       aligned16(value_cache);
  const size_t need =
      emx_paged_workspace_bytes(num_seqs, num_q_heads, num_kv_heads, head_dim, max_blocks_per_seq, page_size);
  const DecodeFn dfn = mfma_ok && need > 0 ? pick_decode_fp8(hg) : nullptr;
  // the FP8 prefill kernel walks 64-key steps inside one page
  const PrefillFn pf = mfma_ok && page_size % 64 == 0 ? pick_prefill_fp8(hg) : nullptr;
  auto prefill_args = [&](int min_q) {
    emx::PrefillArgs p{};
    p.q = reinterpret_cast<const emx::h16*>(queries);
    p.block_tables = block_tables;
    p.kv_lens = kv_lens;
    p.qsl = query_start_loc;
    p.out = reinterpret_cast<emx::h16*>(out);
    p.S = num_seqs;
    p.Hq = num_q_heads;
    p.Hkv = num_kv_heads;
    p.bs = page_size;
    p.nb = num_blocks;
    p.max_blocks = max_blocks_per_seq;
    p.scale_log2 = ga.scale_log2;
    p.window = ga.window;
    p.min_q = min_q;
    p.k8 = key_cache;
    p.v8 = value_cache;
    p.kps = k_scale;
    p.vps = v_scale;
    prefill_split(p, num_tokens, num_q_heads, num_kv_heads, workspace, workspace_bytes, need);
    return p;
  };
  auto prefill_grid = [&](const emx::PrefillArgs& p) {
    const int tokb = 128 / hg;
    return (long)((num_tokens + tokb - 1) / tokb + num_seqs) * num_kv_heads * p.nparts;
  };
  auto launch_prefill = [&](int min_q) {
    const emx::PrefillArgs p = prefill_args(min_q);
    hipLaunchKernelGGL(pf, dim3((unsigned)prefill_grid(p)), dim3(256), 0, st, p);
    return check_launch("prefill_affine_d128 (fp8)");
  };
  // head_dim 128, fp16 queries: decode rows (one query token) on the split-K FP8
  // decode kernel, rows of longer queries on the MFMA prefill kernel
  if (dfn && (single_token_decode || (pf && query_start_loc))) {
    if (workspace == nullptr || workspace_bytes < need)
      return fail(EMX_ERR_INVALID, "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    const int nw = decode_num_waves();
    emx::DecodeArgs a{};
    a.q = reinterpret_cast<const emx::h16*>(queries);
    a.kc = reinterpret_cast<const uint32_t*>(key_cache);
    a.vc = reinterpret_cast<const uint32_t*>(value_cache);
    a.kps = k_scale;
    a.vps = v_scale;
    a.block_tables = block_tables;
    a.kv_lens = kv_lens;
    a.qsl = single_token_decode ? nullptr : query_start_loc;
    a.out = reinterpret_cast<emx::h16*>(out);
    const size_t slots = (size_t)decode_max_waves() + (size_t)num_seqs * num_kv_heads;
    a.ws_cnt = reinterpret_cast<int*>(workspace);
    a.ws_cnt_grp = a.ws_cnt + emx::kMaxUnits;
    a.ws_o = reinterpret_cast<float*>(a.ws_cnt + kPartialsInt);
    a.ws_ml = a.ws_o + slots * hg * head_dim;
    a.S = num_seqs;
    a.Hq = num_q_heads;
    a.Hkv = num_kv_heads;
    a.bs = page_size;
    a.nb = num_blocks;
    a.max_blocks = max_blocks_per_seq;
    a.scale_log2 = ga.scale_log2;
    a.window = ga.window;
    a.num_waves = nw;
    a.nt = emx::kFp8DecodeNT;
    if (!single_token_decode) {
      // a mixed batch in one launch: the decode workgroups first, sized to the decode
      // rows' share of the step as for affine pages (ratio 50: 256 page bytes per
      // token and kv head against 144)
      const emx::PrefillArgs p = prefill_args(2);
      const double share = 50.0 * num_seqs / std::max(1, num_tokens - num_seqs) * num_kv_heads / num_q_heads;
      const int ndec = std::clamp((int)std::ceil(1024.0 * share), device_cus() / 4, nw / 4);
      a.num_waves = 4 * ndec;
      hipLaunchKernelGGL(pick_unified_fp8(hg), dim3((unsigned)(prefill_grid(p) + ndec)), dim3(256), 0, st, p, a,
                         ndec);
      return check_launch("unified_fp8");
    }
    hipLaunchKernelGGL(dfn, dim3((unsigned)(nw / 4)), dim3(256), 0, st, a);
    return check_launch("decode_fp8_d128");
  }
  // other GQA ratios: the MFMA prefill kernel over every row (a decode row is a
  // tile of one query token)
  if (pf && query_start_loc) return launch_prefill(1);
  const emx::Fp8KV kv{key_cache, value_cache, k_scale, v_scale, num_kv_heads, head_dim, page_size};
  switch (dtype) {
    case EMX_DTYPE_F16: return launch_generic<emx::h16>(ga, kv, st, workspace, workspace_bytes);
    case EMX_DTYPE_BF16: return launch_generic<uint16_t>(ga, kv, st, workspace, workspace_bytes);
    case EMX_DTYPE_F32: return launch_generic<float>(ga, kv, st, workspace, workspace_bytes);
  }
  return fail(EMX_ERR_INVALID, "unknown dtype %d", dtype);
}

}  // extern "C"
