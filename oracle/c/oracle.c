/*
 * Independent scalar C restatement of MLX 0.31.1's affine quantizer and of the
 * reference's paged decode attention over affine pages.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/ to cross-check oracle/affine.py bit
 * for bit, and by bench.py's cpu_baseline leg.  Never linked into the product.
 *
 *   oracle_affine_quantize  -- mlx.core.quantize(mode="affine") as used at
 *       lib/python/easymlx/infra/mixins/bridge.py:304,361 (algorithm restated
 *       in oracle/affine.py's module docstring); fp16<->fp32 conversions are
 *       written out here (not taken from a library) so the two restatements
 *       share no code.
 *   oracle_decode_affine    -- single-token paged decode
 *       (lib/python/easymlx/operations/kernels/unified_attention.py:467-609
 *       semantics, reference math :187-281) reading the logical MLX layout
 *       codes [nb, bs, Hkv, D*bits/32], scales/biases [nb, bs, Hkv, D/g],
 *       dequantised per element as fp16(scale*q + bias), fp32 softmax.
 *       Parallelised over (seq, kv_head) with OpenMP.
 *   oracle_attention_affine -- ragged / causal / sliding-window paged attention
 *       (unified_attention.py:187-281 with the kernels' edge semantics
 *       :290-465: causal limit max_k = kv_len - q_len + i, window start
 *       max_k - window + 1, pages with a block id outside [0, nb) skipped,
 *       empty rows zero) over the same logical affine layout, in double
 *       precision, dequantising either exactly (scale*q + bias in fp32, the
 *       fp32 parity target) or rounded to fp16.  Each (sequence, kv_head)
 *       dequantises its keys once; rows run in parallel.  Used by tests/ as
 *       the checker at the benchmark's full sizes, where the numpy oracle
 *       takes minutes.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

static float h2f(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: value = man * 2^-24 */
      float v = (float)man * (1.0f / 16777216.0f);
      memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* fp32 -> fp16, round to nearest even, subnormals kept, overflow -> inf. */
static uint16_t f2h(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) /* inf / nan */
    return sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0);
  float a;
  memcpy(&a, &ax, 4);
  if (a >= 65520.0f) return sign | 0x7c00u;
  if (a < 6.103515625e-05f) { /* result is subnormal (or zero): quantum 2^-24 */
    float q = a * 16777216.0f;   /* exact scaling by a power of two */
    float r = rintf(q);          /* half-to-even */
    return sign | (uint16_t)r;   /* r may reach 1024 = smallest normal */
  }
  uint32_t e = (ax >> 23) - 112u;  /* biased fp16 exponent, 1..30 */
  uint32_t man = ax & 0x7fffffu;
  uint32_t keep = man >> 13;
  uint32_t rest = man & 0x1fffu;
  uint32_t h = (e << 10) | keep;
  if (rest > 0x1000u || (rest == 0x1000u && (keep & 1u))) h += 1; /* carry may bump exponent */
  return sign | (uint16_t)h;
}

void oracle_affine_quantize(const uint16_t* w, long rows, int d, int group_size, int bits,
                            uint32_t* codes, uint16_t* scales, uint16_t* biases) {
  const float n_bins = (float)((1 << bits) - 1);
  const float eps = 1e-7f;
  const int per_word = 32 / bits;
  const int groups = d / group_size;
  const int words = d * bits / 32;
  for (long r = 0; r < rows; ++r) {
    const uint16_t* wr = w + r * d;
    uint32_t* cr = codes + r * words;
    memset(cr, 0, sizeof(uint32_t) * words);
    for (int g = 0; g < groups; ++g) {
      float w_max = -INFINITY, w_min = INFINITY;
      for (int i = 0; i < group_size; ++i) {
        float v = h2f(wr[g * group_size + i]);
        if (v > w_max) w_max = v;
        if (v < w_min) w_min = v;
      }
      int mask = fabsf(w_min) > fabsf(w_max);
      float scale = (w_max - w_min) / n_bins;
      if (scale < eps) scale = eps;
      if (!mask) scale = -scale;
      float edge = mask ? w_min : w_max;
      float q0 = rintf(edge / scale);
      float bias = 0.0f;
      if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
      }
      for (int i = 0; i < group_size; ++i) {
        int e = g * group_size + i;
        float q = rintf((h2f(wr[e]) - bias) / scale);
        if (q < 0.0f) q = 0.0f;
        if (q > n_bins) q = n_bins;
        cr[e / per_word] |= ((uint32_t)q) << ((e % per_word) * bits);
      }
      scales[r * groups + g] = f2h(scale);
      biases[r * groups + g] = f2h(bias);
    }
  }
}

uint16_t oracle_f2h(float f) { return f2h(f); }
float oracle_h2f(uint16_t h) { return h2f(h); }

static inline float deq(const uint32_t* codes_tok, const uint16_t* s_tok, const uint16_t* b_tok,
                        int dim, int group_size, int bits) {
  int per_word = 32 / bits;
  uint32_t q = (codes_tok[dim / per_word] >> ((dim % per_word) * bits)) & ((1u << bits) - 1u);
  float v = h2f(s_tok[dim / group_size]) * (float)q + h2f(b_tok[dim / group_size]);
  return h2f(f2h(v));
}

/* q fp16 [S, Hq, D]; out fp32 [S, Hq, D]. */
void oracle_decode_affine(const uint16_t* q, const uint32_t* k_codes, const uint16_t* k_scales,
                          const uint16_t* k_biases, const uint32_t* v_codes, const uint16_t* v_scales,
                          const uint16_t* v_biases, const int32_t* block_tables, const int32_t* kv_lens,
                          int num_seqs, int hq, int hkv, int d, int bs, int num_blocks, int max_blocks,
                          int bits, int group_size, float softmax_scale, float* out) {
  const int words = d * bits / 32;
  const int groups = d / group_size;
  const int rep = hq / hkv;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int s = 0; s < num_seqs; ++s) {
    for (int kh = 0; kh < hkv; ++kh) {
      int len = kv_lens[s];
      if (len > max_blocks * bs) len = max_blocks * bs;
      float* kf = (float*)malloc(sizeof(float) * (size_t)d);
      float* vf = (float*)malloc(sizeof(float) * (size_t)d);
      float* qf = (float*)malloc(sizeof(float) * (size_t)rep * d);
      float* acc = (float*)calloc((size_t)rep * d, sizeof(float));
      float* m = (float*)malloc(sizeof(float) * rep);
      float* l = (float*)calloc(rep, sizeof(float));
      for (int h = 0; h < rep; ++h) {
        m[h] = -INFINITY;
        for (int i = 0; i < d; ++i) qf[h * d + i] = h2f(q[((size_t)s * hq + kh * rep + h) * d + i]) * softmax_scale;
      }
      for (int pos = 0; pos < len; ++pos) {
        int blk = block_tables[(size_t)s * max_blocks + pos / bs];
        if (blk < 0 || blk >= num_blocks) continue;
        size_t tok = ((size_t)blk * bs + pos % bs) * hkv + kh;
        for (int i = 0; i < d; ++i) {
          kf[i] = deq(k_codes + tok * words, k_scales + tok * groups, k_biases + tok * groups, i, group_size, bits);
          vf[i] = deq(v_codes + tok * words, v_scales + tok * groups, v_biases + tok * groups, i, group_size, bits);
        }
        for (int h = 0; h < rep; ++h) {
          float sc = 0.0f;
          for (int i = 0; i < d; ++i) sc += qf[h * d + i] * kf[i];
          float mn = sc > m[h] ? sc : m[h];
          float alpha = expf(m[h] - mn), p = expf(sc - mn);
          l[h] = l[h] * alpha + p;
          m[h] = mn;
          for (int i = 0; i < d; ++i) acc[h * d + i] = acc[h * d + i] * alpha + p * vf[i];
        }
      }
      for (int h = 0; h < rep; ++h)
        for (int i = 0; i < d; ++i)
          out[((size_t)s * hq + kh * rep + h) * d + i] = l[h] > 0.0f ? acc[h * d + i] / l[h] : 0.0f;
      free(kf); free(vf); free(qf); free(acc); free(m); free(l);
    }
  }
}

/* Dequantised sequence of one kv head: out[pos * d + i], valid[pos]. */
static void deq_sequence(const uint32_t* codes, const uint16_t* sc, const uint16_t* bi, const int32_t* table,
                         int len, int kh, int hkv, int d, int bs, int num_blocks, int bits, int group_size,
                         int round_fp16, double* out, unsigned char* valid) {
  const int words = d * bits / 32, groups = d / group_size, per_word = 32 / bits;
  for (int pos = 0; pos < len; ++pos) {
    const int blk = table[pos / bs];
    valid[pos] = blk >= 0 && blk < num_blocks;
    if (!valid[pos]) {
      for (int i = 0; i < d; ++i) out[(size_t)pos * d + i] = 0.0;
      continue;
    }
    const size_t tok = ((size_t)blk * bs + pos % bs) * hkv + kh;
    for (int i = 0; i < d; ++i) {
      const uint32_t q = (codes[tok * words + i / per_word] >> ((i % per_word) * bits)) & ((1u << bits) - 1u);
      float v = h2f(sc[tok * groups + i / group_size]) * (float)q + h2f(bi[tok * groups + i / group_size]);
      if (round_fp16) v = h2f(f2h(v));
      out[(size_t)pos * d + i] = (double)v;
    }
  }
}

/* q fp16 [T, Hq, D] (rows of sequence s at query_start_loc[s] ..); out double [T, Hq, D]. */
void oracle_attention_affine(const uint16_t* q, const uint32_t* k_codes, const uint16_t* k_scales,
                             const uint16_t* k_biases, const uint32_t* v_codes, const uint16_t* v_scales,
                             const uint16_t* v_biases, const int32_t* block_tables, const int32_t* kv_lens,
                             const int32_t* query_start_loc, int num_seqs, int hq, int hkv, int d, int bs,
                             int num_blocks, int max_blocks, int bits, int group_size, double softmax_scale,
                             int sliding_window, int round_fp16, double* out) {
  const int rep = hq / hkv;
  const int total = query_start_loc[num_seqs];
  memset(out, 0, sizeof(double) * (size_t)total * hq * d);
  for (int s = 0; s < num_seqs; ++s) {
    const int q0 = query_start_loc[s], q_len = query_start_loc[s + 1] - q0;
    int len = kv_lens[s];
    if (len > max_blocks * bs) len = max_blocks * bs;
    if (q_len <= 0 || len <= 0) continue;
    double* kf = (double*)malloc(sizeof(double) * (size_t)len * d);
    double* vf = (double*)malloc(sizeof(double) * (size_t)len * d);
    unsigned char* valid = (unsigned char*)malloc((size_t)len);
    for (int kh = 0; kh < hkv; ++kh) {
      const int32_t* table = block_tables + (size_t)s * max_blocks;
      deq_sequence(k_codes, k_scales, k_biases, table, len, kh, hkv, d, bs, num_blocks, bits, group_size,
                   round_fp16, kf, valid);
      deq_sequence(v_codes, v_scales, v_biases, table, len, kh, hkv, d, bs, num_blocks, bits, group_size,
                   round_fp16, vf, valid);
#pragma omp parallel for collapse(2) schedule(dynamic)
      for (int i = 0; i < q_len; ++i) {
        for (int h = 0; h < rep; ++h) {
          const int head = kh * rep + h;
          const int max_k = (len - q_len) + i < len - 1 ? (len - q_len) + i : len - 1;
          if (max_k < 0) continue;
          int start_k = 0;
          if (sliding_window > 0 && max_k - sliding_window + 1 > 0) start_k = max_k - sliding_window + 1;
          double qd[256];
          const uint16_t* qp = q + ((size_t)(q0 + i) * hq + head) * d;
          /* q scaled in fp32 before the dot product, as the reference does */
          for (int c = 0; c < d; ++c) qd[c] = (double)(h2f(qp[c]) * (float)softmax_scale);
          double* sc = (double*)malloc(sizeof(double) * (size_t)(max_k + 1));
          double mx = -INFINITY;
          for (int k = start_k; k <= max_k; ++k) {
            if (!valid[k]) continue;
            double acc = 0.0;
            const double* kr = kf + (size_t)k * d;
            for (int c = 0; c < d; ++c) acc += qd[c] * kr[c];
            sc[k] = acc;
            if (acc > mx) mx = acc;
          }
          double* o = out + ((size_t)(q0 + i) * hq + head) * d;
          if (mx == -INFINITY) { free(sc); continue; }
          double l = 0.0;
          for (int k = start_k; k <= max_k; ++k) {
            if (!valid[k]) continue;
            const double p = exp(sc[k] - mx);
            l += p;
            const double* vr = vf + (size_t)k * d;
            for (int c = 0; c < d; ++c) o[c] += p * vr[c];
          }
          for (int c = 0; c < d; ++c) o[c] /= l;
          free(sc);
        }
      }
    }
    free(kf); free(vf); free(valid);
  }
}
