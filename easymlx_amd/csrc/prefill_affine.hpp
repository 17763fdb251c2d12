// Multi-token (prefill) paged attention over affine-quantized pages, head_dim 128, MFMA.
//
// Replaces the ragged / causal Metal kernel of the reference for the query rows
// of sequences with more than one query token
// (lib/python/easymlx/operations/kernels/unified_attention.py:290-465, causal
// limit :357-361, sliding window :369-376) and the single-sequence causal path
// (page_attention.py:84-133).  Decode rows (one query token) of the same batch
// go to the decode kernels (decode_q4_d128 / decode_affine_d128).
//
// Work: one workgroup (4 waves) per (sequence, kv_head, tile of 128/HG query
// tokens); a wave owns 32 query columns = (token, head) pairs, head fastest.
// Keys are walked in NT-token steps (64 at 4-bit, 32 at 8-bit) up to the
// tile's causal limit.  Per step, once per workgroup:
//   * K/V codes and scales arrive in LDS (the next step's loads are in flight
//     in registers meanwhile);
//   * K codes are expanded into LDS as exact fp16 subnormals (code * 2^-24),
//     K scales / biases converted to fp32;
//   * V is dequantized into LDS as fp16 (v_scale * code + v_bias), dim-major,
//     with the keys of each 32-key block in the order the PV B operand holds
//     them.
// Then each wave, on v_mfma_f32_16x16x32_f16:
//   S^T: A = expanded K (rows = keys), B = queries; MFMA w spans dims
//        [32w, 32w+32), so each quantization group accumulates separately and
//        the scores stay exact in the codes:
//          s = 2^24 * sum_g ks[t,g] C_g[t,c] + sum_g kb[t,g] * sum_{d in g} q[c,d]
//   online softmax per column (base 2, fp32);
//   O^T += V^T P^T with P in fp16.
// Only V is rounded to fp16 before use; its error is relative to |v| and
// stays inside the relative tolerance, while a rounded K would move scores.
#pragma once

#include "common.hpp"
#include "decode_affine.hpp"

namespace emx {

struct PrefillArgs {
  const h16* q;                 // [T, Hq, 128]
  const uint32_t* kc;           // [nb, Hkv, bs, 128*BITS/32]
  const h16 *ks, *kb;           // [nb, Hkv, G, bs]
  const uint32_t* vc;           // [nb, Hkv, bs/NT, 128, 8]
  const h16 *vs, *vb;           // [nb, Hkv, G, bs]
  const int32_t* block_tables;  // [S, max_blocks]
  const int32_t* kv_lens;       // [S]
  const int32_t* qsl;           // [S + 1]
  h16* out;                     // [T, Hq, 128]
  int S, Hq, Hkv, bs, nb, max_blocks;
  float scale_log2;             // softmax_scale * log2(e)
  int window;                   // sliding window, 0 = off
  int min_q;                    // rows with fewer query tokens go to the decode kernels (2), or none (1)
  // FP8 (E4M3) cache instead of affine pages: key/value [nb, bs, Hkv, 128]
  // uint8 with one fp32 scale per page (unified_attention.py:892-939)
  const uint8_t* k8;
  const uint8_t* v8;
  const float* kps;             // [nb]
  const float* vps;             // [nb]
  // Key split: a tile with many key steps is cut into up to nparts parts (one
  // workgroup each); every wave stores its part's state and the last of a
  // wave's parts merges them.  nparts = 1: no split (ws_* unused).
  int nparts;
  int max_items;                // tiles the workspace holds per kv head
  int* ws_cnt;                  // [max_items * Hkv * 4] arrival counters: zero before and after every launch
  float* ws_part;               // [max_items * Hkv][kPrefillParts][kPrefillPartFloats]
};

constexpr int kPrefillParts = 3;          // most parts a tile is split into
constexpr float kLazyMax = 8.f;           // growth of a column's maximum (log2 units) that triggers a rescale
constexpr int kPrefillSplitKeys = 512;    // keys per part the split aims at (c3: 768 -> 121.5, 512 -> 111.7, 384 -> 117.6 us)
constexpr int kPrefillPartVec = 17;       // f32x4 per lane of a stored state: acc[2][8], (m0, m1, l0, l1)
constexpr int kPrefillPartBytes = 4 * kPrefillPartVec * 64 * 16;  // one part of one workgroup
constexpr int kPrefillCounters = 65536;   // arrival counters (max_items * Hkv * 4 must fit)

template <int BITS, int GS, int HG>
struct PrefillCfg {
  static constexpr int D = 128, G = D / GS;
  static constexpr int NT = 256 / BITS;            // keys per step (64 at 4-bit, 32 at 8-bit)
  static constexpr int NA = NT / 16;               // 16-key S^T sub-tiles per step
  static constexpr int NKS = NT / 32;              // 32-key PV k-steps per step
  static constexpr int W = D * BITS / 32;          // code words per key
  static constexpr int COLS = 32;                  // query columns per wave
  static constexpr int TOKW = COLS / HG;           // query tokens per wave
  static constexpr int TOKB = 4 * TOKW;            // query tokens per workgroup
  static constexpr int KSTR = D + 8;               // halves per expanded key row (padded)
  static constexpr int VSTR = NT + 16;             // halves per dequantized value dim (padded; c3: +8 95.1, +16 93.1, +24 95.6 us)
  static constexpr int RAWV = 4096;                // bytes of the step's V tile
  static constexpr int RAWS = 4 * G * NT * 2;      // bytes of the step's ks, kb, vs, vb
  static constexpr int SEGS = 4 * G;               // contiguous scale segments per step
  static constexpr int SEGB = NT * 2;              // bytes per segment
  static_assert(COLS % HG == 0, "query columns per wave must hold whole tokens");
  static_assert(W * NT == 1024, "a step's K codes are 4 KiB: one 16-byte piece per thread");
};

// Number of query-token tiles of sequence s (0 for decode rows and empty rows).
__device__ __forceinline__ int prefill_tiles(const PrefillArgs& a, const int s, const int tokb) {
  const int ql = a.qsl[s + 1] - a.qsl[s];
  return ql >= a.min_q ? (ql + tokb - 1) / tokb : 0;
}

// Position, inside its 32-key block, at which the dequantized value of key k
// (0..31 within the block) is stored: the PV B operand of lane (col, kg) holds
// keys kg*4 + {0..3} and 16 + kg*4 + {0..3} of the block, in that order.
__device__ __forceinline__ constexpr int pv_slot(int k) { return 8 * ((k & 15) >> 2) + 4 * (k >> 4) + (k & 3); }

// FP8: the same kernel over an FP8 cache, on the 64-key step geometry of BITS 4
// with one group (two 16-byte pieces of K and of V per thread and step; pages
// of a multiple of 64 tokens): K expands to dec(code) * 2^-8 exactly with the
// page scale * 2^8 * 2^-24 as the key scale (so the scores keep the affine
// formula with zero biases), V dequantizes to dec(code) * scale.
// The kernel body as workgroup `bid` (a grid of its own, or the prefill part of
// a mixed batch's single launch, unified_q4).
template <int BITS, int GS, int HG, bool FP8 = false>
__device__ __forceinline__ void prefill_body(const PrefillArgs& a, const int bid) {
  static_assert(!FP8 || (BITS == 4 && GS == 128), "the FP8 cache runs on the 64-key geometry, one group");
  constexpr int RAWV = FP8 ? 2 * PrefillCfg<BITS, GS, HG>::RAWV : PrefillCfg<BITS, GS, HG>::RAWV;
  using P = PrefillCfg<BITS, GS, HG>;
  constexpr int D = P::D, G = P::G, NT = P::NT, NA = P::NA, NKS = P::NKS, W = P::W;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;
  const int jj = lane >> 4;

  // ---- work item: blockIdx -> (sequence, tile, kv_head); later tiles (more keys) first
  // ---- per-sequence tile counts, scanned by the whole workgroup (one pass of
  // global loads in parallel, not a serial walk by one thread)
  // LDS, carved from the shared arena
  constexpr int oTcum = 0, oWred = lds_next(oTcum, 4 * (kMaxSeqs + 1)), oRawv = lds_next(oWred, 16);
  constexpr int oRaws = lds_next(oRawv, RAWV), oKe = lds_next(oRaws, 2 * 4 * G * NT);
  constexpr int oVe = lds_next(oKe, 2 * NT * P::KSTR), oKsf = lds_next(oVe, 2 * D * P::VSTR);
  constexpr int oKbe = lds_next(oKsf, 4 * G * NT), oEnd = lds_next(oKbe, 16 * NT);
  static_assert(oEnd <= kArenaBytes, "LDS arena too small");
  int(&tcum)[kMaxSeqs + 1] = lds_at<int[kMaxSeqs + 1]>(oTcum);
  int(&wred)[4] = lds_at<int[4]>(oWred);
  {
    const int ch = (a.S + 255) / 256, s0 = tid * ch;
    int tsum = 0;
    for (int i = 0; i < ch; ++i) {
      const int si = s0 + i;
      if (si >= a.S) break;
      const int nt = prefill_tiles(a, si, P::TOKB);
      tcum[si] = nt;  // the count for now
      tsum += nt;
    }
    int x = tsum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) wred[tid >> 6] = x;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < (tid >> 6); ++w) base += wred[w];
    int run = base + x - tsum;
    for (int i = 0; i < ch; ++i) {
      const int si = s0 + i;
      if (si >= a.S) break;
      const int n = tcum[si];
      tcum[si] = run;
      run += n;
    }
    if (tid == 255) tcum[a.S] = base + x;
  }
  __syncthreads();
  const int ntiles = tcum[a.S];
  const int kvh = bid % a.Hkv;
  const int part = (bid / a.Hkv) % a.nparts;
  const int item = bid / a.Hkv / a.nparts;
  if (item >= ntiles) return;
  int s = 0;
  while (tcum[s + 1] <= item) ++s;
  s = __builtin_amdgcn_readfirstlane(s);
  const int nt_s = tcum[s + 1] - tcum[s];
  const int tile = __builtin_amdgcn_readfirstlane(nt_s - 1 - (item - tcum[s]));  // last tile first
  const int q0 = a.qsl[s];
  const int qlen = a.qsl[s + 1] - q0;
  const int kv_len = min(max(a.kv_lens[s], 0), a.max_blocks * a.bs);
  const int past = kv_len - qlen;  // query i sees keys [.., past + i]
  const int tok_lo = tile * P::TOKB;

  // ---- this lane's query columns: c = 16*ct + col of the wave's 32, token = c / HG, head = c % HG
  int ctok[2], chead[2], limit[2], start[2];
  bool cvalid[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int c = wv * P::COLS + 16 * ct + col;
    ctok[ct] = tok_lo + c / HG;
    chead[ct] = c % HG;
    cvalid[ct] = ctok[ct] < qlen;
    limit[ct] = min(past + ctok[ct], kv_len - 1);
    start[ct] = a.window > 0 ? max(0, past + ctok[ct] - a.window + 1) : 0;
    if (!cvalid[ct]) limit[ct] = -1;
  }
  // key range of the whole workgroup
  const int t_first = tok_lo, t_last = min(tok_lo + P::TOKB, qlen) - 1;
  const int k_hi = min(past + t_last, kv_len - 1);
  const int k_lo = a.window > 0 ? max(0, past + t_first - a.window + 1) : 0;
  const int steps_all = k_hi >= 0 ? max(k_hi / NT - k_lo / NT + 1, 0) : 0;
  // parts of this tile: the steps split evenly, at most nparts, about kPrefillSplitKeys keys each
  const int nparts = a.nparts > 1 && item < a.max_items
                         ? max(1, min(a.nparts, (steps_all * NT + kPrefillSplitKeys - 1) / kPrefillSplitKeys))
                         : 1;
  if (part >= nparts) return;
  const int step_lo = k_lo / NT + part * steps_all / nparts;
  const int step_hi = k_lo / NT + (part + 1) * steps_all / nparts - 1;

  // ---- query operands: MFMA w spans dims [32w, 32w + 32); lane group jj holds dims
  // 32w + 8jj + i in the element order of the expanded keys (unpack4 / unpack8 order)
  h16x8 qB[2][4];
  // B operand of the bias MFMA: lane group 0 holds the query's per-group sums, each
  // as fp16 hi + lo (x = hi + lo to ~22 bits), k-elements 2g, 2g + 1; the other lanes 0
  h16x8 qbias[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const h16* qp = a.q + ((size_t)(q0 + (cvalid[ct] ? ctok[ct] : 0)) * a.Hq + (size_t)kvh * HG + chead[ct]) * D;
    float gs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const h16x8 raw = *reinterpret_cast<const h16x8*>(qp + 32 * w + 8 * jj);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const h16 v = cvalid[ct] ? raw[slot_perm<FP8 ? 8 : BITS>(i)] : (h16)0.0f;
        qB[ct][w][i] = v;
        gs[(32 * w) / GS] += (float)v;
      }
    }
    qbias[ct] = h16x8{(h16)0.f, (h16)0.f, (h16)0.f, (h16)0.f, (h16)0.f, (h16)0.f, (h16)0.f, (h16)0.f};
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float x = gs[g];
      x += __shfl_xor(x, 16, 64);
      x += __shfl_xor(x, 32, 64);
      const h16 hi = (h16)x;
      const h16 lo = (h16)(x - (float)hi);
      if (jj == 0) {
        qbias[ct][2 * g] = hi;
        qbias[ct][2 * g + 1] = lo;
      }
    }
  }

  // ---- LDS: the step's raw V tile and scales, then the expanded K, dequantized V and fp32 K scales
  uint8_t(&raw_v)[RAWV] = lds_at<uint8_t[RAWV]>(oRawv);
  h16(&raw_s)[4 * G * NT] = lds_at<h16[4 * G * NT]>(oRaws);  // [arr][g][NT]
  h16(&ke)[NT * P::KSTR] = lds_at<h16[NT * P::KSTR]>(oKe);    // [key][dims, unpack order]
  h16(&ve)[D * P::VSTR] = lds_at<h16[D * P::VSTR]>(oVe);      // [dim][keys, pv_slot order]
  float(&ksf)[G][NT] = lds_at<float[G][NT]>(oKsf);            // k_scale * 2^24 in fp32
  h16x8(&kbe)[NT] = lds_at<h16x8[NT]>(oKbe);                  // A operand of the bias MFMA: kb_g at 2g, 2g + 1

  // Cooperative load of one step into registers: thread owns one 16-byte piece of K and of V,
  // and (threads < SEGS * SEGB / 16) one piece of the scales.
  u32x4 rk, rv, rsc, rk2, rv2;  // rk2 / rv2: FP8's second pieces (key rows 32 .. 63 of the step)
  float psk = 0.f, psv = 0.f;  // FP8: the loaded step's page scales
  float vsc = 0.f;             // FP8: the expanded step's value scale
  auto load_step = [&](const int st) {
    const int pos0 = st * NT;
    const int blk_i = a.block_tables[(size_t)s * a.max_blocks + pos0 / a.bs];
    const int blk = (unsigned)blk_i < (unsigned)a.nb ? blk_i : 0;
    const int off = pos0 % a.bs;
    if constexpr (FP8) {
      // 64 key rows of 128 bytes, Hkv * 128 bytes apart: thread -> rows tid / 8 and 32 + tid / 8,
      // bytes 16 * (tid % 8) ..
      const size_t rowb = (size_t)a.Hkv * D;
      const size_t base = ((size_t)blk * a.bs + off + (tid >> 3)) * rowb + (size_t)kvh * D + 16 * (tid & 7);
      rk = *reinterpret_cast<const u32x4*>(a.k8 + base);
      rv = *reinterpret_cast<const u32x4*>(a.v8 + base);
      rk2 = *reinterpret_cast<const u32x4*>(a.k8 + base + 32 * rowb);
      rv2 = *reinterpret_cast<const u32x4*>(a.v8 + base + 32 * rowb);
      psk = a.kps[blk];
      psv = a.vps[blk];
      return;
    }
    const size_t ph = (size_t)blk * a.Hkv + kvh;
    // K: NT rows x W words = 4 KiB; piece tid -> row tid / (W/4), words 4*(tid % (W/4)) ..
    const int krow = tid / (W / 4), kq = tid % (W / 4);
    rk = *reinterpret_cast<const u32x4*>(a.kc + (ph * a.bs + off + krow) * W + 4 * kq);
    // V: the step's 4 KiB tile, in HBM order
    const int RW = a.bs * BITS / 32;
    rv = *reinterpret_cast<const u32x4*>(a.vc + ph * D * RW + (off / NT) * D * 8 + 4 * tid);
    // scales: segment (arr, g) of NT halves; 16 bytes per thread
    constexpr int PER = P::SEGB / 16;
    if (tid < P::SEGS * PER) {
      const int seg = tid / PER, piece = tid % PER;
      const int arr = seg / G, g = seg % G;
      // the four bases as scalar values: a per-lane pick among the struct's fields would
      // be a vector load of the chosen pointer, and its wait would also wait for the
      // page loads issued just above
      const h16 *b_ks = a.ks, *b_kb = a.kb, *b_vs = a.vs, *b_vb = a.vb;
      asm("" : "+s"(b_ks), "+s"(b_kb), "+s"(b_vs), "+s"(b_vb));
      const h16* base = arr == 0 ? b_ks : arr == 1 ? b_kb : arr == 2 ? b_vs : b_vb;
      typedef const __attribute__((address_space(1))) u32x4* gu32x4;  // a global load, not a flat one
      rsc = *(gu32x4)(base + (ph * G + g) * a.bs + off + 8 * piece);
      // positions past kv_len may hold anything: zero their scales so that p = 0 contributes 0
      const int live = kv_len - (pos0 + 8 * piece);
      if (live < 8) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t keep = (2 * e < live ? 0x0000FFFFu : 0u) | (2 * e + 1 < live ? 0xFFFF0000u : 0u);
          rsc[e] &= keep;
        }
      }
    }
  };

  // Expansion, part 1 (from registers): K codes -> exact fp16 subnormals; raw V and scales -> LDS.
  auto expand_k = [&]() {
    if constexpr (FP8) {
      // rows tid / 8 and 32 + tid / 8: the 16 codes of dims 16kq .. 16kq+15 as the exact fp16
      // values dec(code) * 2^-8
      const int kq = tid & 7;
#pragma unroll
      for (int pc = 0; pc < 2; ++pc) {
        const u32x4 w = pc ? rk2 : rk;
        h16* kr = ke + ((tid >> 3) + 32 * pc) * P::KSTR;
#pragma unroll
        for (int e = 0; e < 2; ++e)
          *reinterpret_cast<h16x8*>(kr + 16 * kq + 8 * e) =
              as_h8(e4m3x2_to_h16x2(__builtin_amdgcn_perm(0u, w[2 * e], 0x0C010C00u)),
                    e4m3x2_to_h16x2(__builtin_amdgcn_perm(0u, w[2 * e], 0x0C030C02u)),
                    e4m3x2_to_h16x2(__builtin_amdgcn_perm(0u, w[2 * e + 1], 0x0C010C00u)),
                    e4m3x2_to_h16x2(__builtin_amdgcn_perm(0u, w[2 * e + 1], 0x0C030C02u)));
      }
      // scores keep the affine formula: key scale = page scale * 2^8 (codes are value * 2^-8), biases 0
      if (tid < NT) ksf[0][tid] = psk * 256.0f;
      vsc = psv;
      reinterpret_cast<u32x4*>(raw_v)[tid] = rv;  // [64 keys][128 bytes]
      reinterpret_cast<u32x4*>(raw_v)[256 + tid] = rv2;
      return;
    }
    const int krow = tid / (W / 4), kq = tid % (W / 4);
    h16* kr = ke + krow * P::KSTR;
    if constexpr (BITS == 4) {
      // words 4kq .. 4kq+3 hold dims 32kq .. 32kq+31: one MFMA k-step, lane group e of it
#pragma unroll
      for (int e = 0; e < 4; ++e)
        *reinterpret_cast<h16x8*>(kr + 32 * kq + 8 * e) = unpack4(rk[e]);
    } else {
      // words 4kq .. 4kq+3 hold dims 16kq .. 16kq+15: half of k-step kq/2, lane groups 2(kq%2), +1
#pragma unroll
      for (int e = 0; e < 2; ++e)
        *reinterpret_cast<h16x8*>(kr + 16 * kq + 8 * e) = unpack8(rk[2 * e], rk[2 * e + 1]);
    }
    reinterpret_cast<u32x4*>(raw_v)[tid] = rv;
    constexpr int PER = P::SEGB / 16;
    if (tid < P::SEGS * PER) reinterpret_cast<u32x4*>(raw_s)[tid] = rsc;
  };

  // Expansion, part 2 (from LDS): V -> fp16 v_scale * code + v_bias; K scales -> fp32.
  // Thread -> dim, TPT consecutive keys of the step (a whole 32-key block at 4-bit,
  // half of one at 8-bit); keys go to their pv_slot positions in runs of 4.
  auto expand_v = [&]() {
    constexpr int TPT = NT * D / 256;  // values per thread (32 at 4-bit, 16 at 8-bit)
    constexpr int PW = 32 / BITS;      // keys per word
    const int dim = tid * TPT / NT;
    const int k0 = (tid * TPT) % NT;   // first key (multiple of 16)
    const int g = dim / GS;
    typedef h16 h16x4 __attribute__((ext_vector_type(4)));
    if constexpr (FP8) {  // token-major raw tile: key k's code of dim d at byte 128k + d
      h16* vd = ve + dim * P::VSTR + 32 * (k0 >> 5);
#pragma unroll
      for (int q4 = 0; q4 < TPT / 4; ++q4) {
        const int kk = (k0 & 31) + 4 * q4;
        h16x4 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) {  // (dec * 2^-8) * (scale * 2^8): the same product as dec * scale
          const uint32_t h = e4m3x2_to_h16x2(raw_v[(k0 + 4 * q4 + r) * D + dim]);
          o[r] = (h16)((float)__builtin_bit_cast(h16, (uint16_t)h) * (vsc * 256.0f));
        }
        *reinterpret_cast<h16x4*>(vd + pv_slot(kk)) = o;
      }
      return;
    }
    // Two keys at a time in packed fp16: a pair of codes placed as 0x6400 | code is
    // 1024 + code exactly; minus 1024, then one fused multiply-add with the keys'
    // (scale, bias) pairs (single rounding to fp16, as the fp32 path rounds once).
    typedef h16 h16x2 __attribute__((ext_vector_type(2)));
    const uint32_t* vw = reinterpret_cast<const uint32_t*>(raw_v) + dim * 8 + k0 / PW;
    const uint32_t* vsp = reinterpret_cast<const uint32_t*>(raw_s + (2 * G + g) * NT + k0);
    const uint32_t* vbp = reinterpret_cast<const uint32_t*>(raw_s + (3 * G + g) * NT + k0);
    h16* vd = ve + dim * P::VSTR + 32 * (k0 >> 5);
    const h16x2 k1024 = {(h16)1024.0f, (h16)1024.0f};
#pragma unroll
    for (int q4 = 0; q4 < TPT / 4; ++q4) {  // keys k0 + 4q4 .. +3 (consecutive slots)
      const int kk = (k0 & 31) + 4 * q4;     // key within its 32-key block
      uint32_t o[2];
#pragma unroll
      for (int hp = 0; hp < 2; ++hp) {
        const int e = 4 * q4 + 2 * hp;  // first value index of the pair (keys e, e + 1 of the thread)
        const uint32_t x = vw[e / PW];
        uint32_t pair;  // the two codes at bits 0 and 16
        if constexpr (BITS == 4)
          pair = (x >> (4 * ((e % PW) >> 1))) & 0x000F000Fu;  // keys 2m, 2m + 1 sit at nibbles m, m + 4
        else
          pair = __builtin_amdgcn_perm(0u, x, (e % PW) == 0 ? 0x0C010C00u : 0x0C030C02u);
        const h16x2 c = __builtin_bit_cast(h16x2, pair | 0x64006400u) - k1024;
        const h16x2 v = __builtin_elementwise_fma(c, __builtin_bit_cast(h16x2, vsp[e / 2]),
                                                  __builtin_bit_cast(h16x2, vbp[e / 2]));
        o[hp] = __builtin_bit_cast(uint32_t, v);
      }
      *reinterpret_cast<u32x2*>(vd + pv_slot(kk)) = u32x2{o[0], o[1]};
    }
    // K scales of the step in fp32, times 2^24 (the codes enter the MFMA as code * 2^-24), and
    // the K biases as the bias MFMA's A rows
    // (by waves 1 .. 3: wave 0 also loads the scales)
    for (int i = tid - 64; i >= 0 && i < G * NT; i += 192) ksf[i / NT][i % NT] = (float)raw_s[i] * kTwo24;
    if (tid >= 256 - NT) {
      const int k = tid - (256 - NT);
      h16x8 b = {(h16)0.f, (h16)0.f, (h16)0.f, (h16)0.f, (h16)0.f, (h16)0.f, (h16)0.f, (h16)0.f};
#pragma unroll
      for (int g = 0; g < G; ++g) b[2 * g] = b[2 * g + 1] = raw_s[(G + g) * NT + k];
      kbe[k] = b;
    }
  };

  float m_run[2] = {-INFINITY, -INFINITY}, l_part[2] = {0.f, 0.f};
  f32x4 acc[2][8];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[ct][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float sc_l2 = a.scale_log2;  // the scores come out in natural units

  if (step_lo <= step_hi) load_step(step_lo);
  for (int st = step_lo; st <= step_hi; ++st) {
    __syncthreads();  // the previous step's expanded tiles are no longer read
    expand_k();
    __syncthreads();
    if (st + 1 <= step_hi) load_step(st + 1);
    expand_v();
    __syncthreads();
    const int pos0 = st * NT;
    const int blk_i = a.block_tables[(size_t)s * a.max_blocks + pos0 / a.bs];
    if ((unsigned)blk_i >= (unsigned)a.nb) continue;  // an invalid page is skipped

    // The step in halves of 32 keys (sub-tiles 2h, 2h + 1): scores, softmax, then PV,
    // which keeps one half's scores and operand reads live at a time.
#pragma unroll
    for (int h = 0; h < NKS; ++h) {
      // ---- S^T per query tile ct and key sub-tile, per quantization group
      float sc[2][2][4];  // [ct][sub-tile 2h + t][r]: key 32h + 16t + 4jj + r of the step
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int at = 2 * h + t;
          const h16* kr = ke + (16 * at + col) * P::KSTR + 8 * jj;
          f32x4 cg[G];
#pragma unroll
          for (int g = 0; g < G; ++g) cg[g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const h16x8 A = *reinterpret_cast<const h16x8*>(kr + 32 * w);
            cg[(32 * w) / GS] = mfma16x16x32(A, qB[ct][w], cg[(32 * w) / GS]);
          }
          // bias term sum_g kb[t,g] * sum_{d in g} q_d on the matrix core (FP8: no biases)
          // (every lane reads the key's biases: the B operand is zero outside lane group 0, and
          // the biases are finite, so the other lane groups add exact zeros)
          f32x4 cb = {0.f, 0.f, 0.f, 0.f};
          if constexpr (!FP8) cb = mfma16x16x32(kbe[16 * at + col], qbias[ct], cb);
          float v[4] = {cb[0], cb[1], cb[2], cb[3]};
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const f32x4 ks4 = *reinterpret_cast<const f32x4*>(&ksf[g][16 * at + 4 * jj]);
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = fmaf(cg[g][r], ks4[r], v[r]);
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) sc[ct][t][r] = v[r];
        }
      }

      // ---- mask (causal / window / kv_len) where the half is not fully visible to every
      // column (one branch for both query tiles)
      const int kpos0 = pos0 + 32 * h;
      const bool full = kpos0 >= start[0] && kpos0 + 31 <= limit[0] && kpos0 >= start[1] && kpos0 + 31 <= limit[1];
      if (!full) {
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int p = kpos0 + 16 * t + 4 * jj + r;
              if (p < start[ct] || p > limit[ct]) sc[ct][t][r] = -INFINITY;
            }
      }

      // ---- online softmax per column (base 2).  The reference maximum m_run moves only when
      // a score passes it by more than kLazyMax (log2 units), so the accumulator is rescaled
      // rarely (one branch for both query tiles); p <= 2^kLazyMax otherwise, well inside
      // fp16.  The result does not depend on the reference.
      float m_new[2];
      bool grow[2];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        float tmax = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, sc[ct][t][r]);
        tmax = rows4_max(tmax);
        m_new[ct] = fmaxf(m_run[ct], tmax * sc_l2);
        grow[ct] = m_new[ct] > m_run[ct] + kLazyMax;  // also the first finite maximum
      }
      if (__any(grow[0] || grow[1])) {
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          const float m_ref = grow[ct] ? m_new[ct] : m_run[ct];
          const float alpha = grow[ct] ? __builtin_amdgcn_exp2f(m_run[ct] - m_ref) : 1.f;
          l_part[ct] *= alpha;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) acc[ct][dt] *= alpha;
          m_run[ct] = m_ref;
        }
      }
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        // nothing visible yet (m_run = -inf): every score is -inf and p = 0
        const float m_sub = fmaxf(m_run[ct], -3.0e38f);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float p = __builtin_amdgcn_exp2f(fmaf(sc[ct][t][r], sc_l2, -m_sub));
            sc[ct][t][r] = p;
            l_part[ct] += p;
          }
      }

      // ---- O^T += V^T P^T over the half's 32 keys: lane (col, jj) holds keys
      // 32h + 4jj + r (sub-tile 2h) and 32h + 16 + 4jj + r (sub-tile 2h + 1)
      h16x8 pB[2];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        typedef float f32x2v __attribute__((ext_vector_type(2)));
        typedef h16 h16x2v __attribute__((ext_vector_type(2)));
        uint32_t pw[4];  // pairs converted together (v_cvt_pk_f16_f32)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 4; r += 2)
            pw[2 * t + r / 2] = __builtin_bit_cast(
                uint32_t, __builtin_convertvector(f32x2v{sc[ct][t][r], sc[ct][t][r + 1]}, h16x2v));
        pB[ct] = __builtin_bit_cast(h16x8, u32x4{pw[0], pw[1], pw[2], pw[3]});
      }
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const h16x8 Av = *reinterpret_cast<const h16x8*>(ve + (16 * dt + col) * P::VSTR + 32 * h + 8 * jj);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) acc[ct][dt] = mfma16x16x32(Av, pB[ct], acc[ct][dt]);
      }
    }
  }

  // ---- split tile: store this wave's state; the wave arriving last among the parts merges
  if (nparts > 1) {
    const int u = item * a.Hkv + kvh;
    const __amdgpu_buffer_rsrc_t rp =
        uniform_rsrc(reinterpret_cast<uint8_t*>(a.ws_part) + (size_t)u * kPrefillParts * kPrefillPartBytes,
                     kPrefillParts * kPrefillPartBytes);
    auto vo = [&](int k) { return ((wv * kPrefillPartVec + k) * 64 + lane) * 16; };
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) store_f32x4(acc[ct][dt], rp, vo(8 * ct + dt), part * kPrefillPartBytes);
    store_f32x4(f32x4{m_run[0], m_run[1], l_part[0], l_part[1]}, rp, vo(16), part * kPrefillPartBytes);
    if (!arrive_last(a.ws_cnt + u * 4 + wv, nparts, lane)) return;
    // every part (this one's too) read back in part order: the result does not
    // depend on which part arrived last
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      m_run[ct] = -INFINITY;
      l_part[ct] = 0.f;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[ct][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int q = 0; q < nparts; ++q) {
      f32x4 o[16];
#pragma unroll
      for (int k = 0; k < 16; ++k)
        o[k] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, vo(k), q * kPrefillPartBytes,
                                                                               kCoherent));
      const f32x4 ml =
          __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, vo(16), q * kPrefillPartBytes, kCoherent));
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const float m1 = ml[ct], l1 = ml[2 + ct];
        const float mn = fmaxf(m_run[ct], m1);
        const float f0 = m_run[ct] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run[ct] - mn);
        const float f1 = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - mn);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[ct][dt] = acc[ct][dt] * f0 + o[8 * ct + dt] * f1;
        l_part[ct] = l_part[ct] * f0 + l1 * f1;
        m_run[ct] = mn;
      }
    }
  }

  // ---- normalise and write: lane (col, jj) holds dims 16*dt + 4*jj + r of its column
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    float l = l_part[ct] + __shfl_xor(l_part[ct], 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (!cvalid[ct]) continue;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    h16* op = a.out + ((size_t)(q0 + ctok[ct]) * a.Hq + (size_t)kvh * HG + chead[ct]) * D;
    typedef h16 h16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int d = 16 * dt + 4 * jj;
      *reinterpret_cast<h16x4*>(op + d) = h16x4{(h16)(acc[ct][dt][0] * inv), (h16)(acc[ct][dt][1] * inv),
                                                (h16)(acc[ct][dt][2] * inv), (h16)(acc[ct][dt][3] * inv)};
    }
  }
}

template <int BITS, int GS, int HG, bool FP8 = false>
__global__ __launch_bounds__(256, 2) void prefill_affine_d128(PrefillArgs a) {
  prefill_body<BITS, GS, HG, FP8>(a, blockIdx.x);
}

}  // namespace emx
