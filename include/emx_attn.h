/*
 * emx_attn -- MI355X (gfx950) paged attention over affine-quantized KV pages.
 *
 * C ABI: plain device pointers, sizes and a hipStream_t passed as void*.
 * The library never allocates on these paths; the caller owns every buffer.
 * Every entry point returns EMX_OK (0) or a negative status; the message of the
 * last failure on the calling thread is available from emx_last_error().
 *
 * Page layout (per block `b`, kv head `h`; G = head_dim / group_size):
 *   key codes    uint32 [num_blocks, Hkv, page_size, head_dim*bits/32]  token-major
 *   value codes  uint32 [num_blocks, Hkv, page_size/T, head_dim, T*bits/32]
 *                with T = min(page_size, 256/bits) tokens per tile, dim-major inside
 *                a tile (a word packs 32/bits consecutive tokens of one dim: 8-bit in
 *                byte order, 4-bit with token k at nibble (k >> 1) | ((k & 1) << 2));
 *                page_size must be a multiple of T
 *   k/v scales   fp16   [num_blocks, Hkv, G, page_size]
 *   k/v biases   fp16   [num_blocks, Hkv, G, page_size]
 * Key words are packed as MLX packs them (element j of a word at bits
 * [j*bits,(j+1)*bits)); value w = scale * code + bias, with the codes, scales and
 * biases of mlx.core.quantize(mode="affine").
 */
#ifndef EMX_ATTN_H_
#define EMX_ATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Device ints the decode appends (emx_*_cache_append_rope) take as `counter`. */
#define EMX_APPEND_COUNTER_INTS 4

#define EMX_OK 0
#define EMX_ERR_INVALID (-1)     /* bad argument / shape (Python: ValueError) */
#define EMX_ERR_UNSUPPORTED (-2) /* valid but unsupported configuration (NotImplementedError) */
#define EMX_ERR_HIP (-3)         /* HIP runtime error (RuntimeError) */

#define EMX_DTYPE_F16 0
#define EMX_DTYPE_BF16 1
#define EMX_DTYPE_F32 2

/* Library version (major*10000 + minor*100 + patch). */
int emx_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* emx_last_error(void);

/*
 * Affine quantize, MLX layout: x fp16 [rows, head_dim] ->
 * codes uint32 [rows, head_dim*bits/32], scales/biases fp16 [rows, head_dim/group_size].
 * Replaces: mlx.core.quantize(w, group_size, bits) as called at
 *   lib/python/easymlx/infra/mixins/bridge.py:304,361 and
 *   lib/python/easymlx/layers/linears/_linear_moe.py:113 (format: infra/etils.py:74-94).
 */
int emx_affine_quantize(const void* x, long rows, int head_dim, int group_size, int bits, uint32_t* codes,
                        void* scales, void* biases, void* stream);

/*
 * Fused quantize-on-write of new K/V tokens into their pages.
 * keys/values fp16 [num_tokens, Hkv, head_dim]; slot_mapping int32 [num_tokens]
 * (block * page_size + offset, or -1 to skip the token).
 * Replaces the K/V write of PageCacheView.concatenate_to_cache
 *   lib/python/easymlx/caching/paged/cache.py:1088-1306 (decode :1155-1190,
 *   multi-token :1254-1290; its Metal reshape_and_cache :36-93) and the
 *   compiled-proxy write lib/python/easymlx/inference/esurge/runners/model_runner.py:139-189.
 */
int emx_affine_cache_write(const void* keys, const void* values, const int32_t* slot_mapping, int num_tokens,
                           int num_kv_heads, int head_dim, int group_size, int bits, int page_size, int num_blocks,
                           uint32_t* k_codes, void* k_scales, void* k_biases, uint32_t* v_codes, void* v_scales,
                           void* v_biases, void* stream);

/*
 * emx_affine_cache_write with rotary position embedding fused in: K rows turn
 * by theta = positions[t] * inv_freq[i] on pair i of the first rot_dims dims
 * ((i, i + rot_dims/2), or (2i, 2i+1) when traditional != 0), are rounded to
 * fp16 and then quantized exactly as emx_affine_cache_write does.  V is not
 * rotated.  positions int32 [num_tokens], inv_freq float32 [rot_dims/2].
 * queries (fp16 [num_tokens, num_q_heads, head_dim], or null) receive
 * queries_in turned by the same rotation (the dims past rot_dims copied), in
 * the same launch for decode-size writes; queries_in null turns queries in
 * place.
 * Replaces the RoPE applied to keys in PageCacheView.concatenate_to_cache
 *   lib/python/easymlx/caching/paged/cache.py:1161-1166 (multi-token :1208-1253)
 *   followed by the write :1186-1190, with the RoPE of
 *   lib/python/easymlx/layers/rotary/_rotary.py (mlx.core.fast.rope).
 */
int emx_affine_cache_write_rope(const void* keys, const void* values, const int32_t* slot_mapping, int num_tokens,
                                int num_kv_heads, int head_dim, int group_size, int bits, int page_size,
                                int num_blocks, uint32_t* k_codes, void* k_scales, void* k_biases, uint32_t* v_codes,
                                void* v_scales, void* v_biases, const int32_t* positions, const float* inv_freq,
                                int rot_dims, int traditional, const void* queries_in, void* queries,
                                int num_q_heads, void* stream);

/*
 * The decode-step append with RoPE in one launch: emx_cache_slots and
 * emx_affine_cache_write_rope together for one token per sequence.  Token t
 * (num_tokens <= 128) is the next token of sequence slot_ids[t]: its position
 * is kv_lens[slot_ids[t]], its slot block_tables[s, position / page_size] *
 * page_size + position % page_size (not written for a slot id outside
 * [0, num_seqs), a column past the table or a negative page id), K is rotated
 * at that position and quantized into the pages, queries_in rotated into
 * queries, and kv_lens[s] advances by one.  `counter` is EMX_APPEND_COUNTER_INTS
 * ints of device memory, zero before the first call; every call leaves them zero
 * (calls that share them must not overlap: give each stream its own, as the
 * Python views do; counters left nonzero, e.g. by a launch that never ran to its
 * end, make the later calls advance kv_lens at the wrong workgroup, so a caller
 * that aborts a launch zeroes them again).  A cache must not be appended to from two streams at
 * once (the pages and kv_lens would race).  head_dim and group_size multiples of 16,
 * group_size <= 64; otherwise EMX_ERR_UNSUPPORTED (use the two calls).
 * Replaces the decode branch of PageCacheView.concatenate_to_cache
 *   lib/python/easymlx/caching/paged/cache.py:1126-1190 (RoPE :1161-1166)
 * and the compiled decode proxy's write
 *   lib/python/easymlx/inference/esurge/runners/model_runner.py:139-189.
 */
int emx_affine_cache_append_rope(const void* keys, const void* values, const int32_t* slot_ids, int num_tokens,
                                 const int32_t* block_tables, int num_seqs, int max_blocks_per_seq, int32_t* kv_lens,
                                 int* counter, int num_kv_heads, int head_dim, int group_size, int bits,
                                 int page_size, int num_blocks, uint32_t* k_codes, void* k_scales, void* k_biases,
                                 uint32_t* v_codes, void* v_scales, void* v_biases, const float* inv_freq,
                                 int rot_dims, int traditional, const void* queries_in, void* queries,
                                 int num_q_heads, void* stream);

/*
 * The FP8 decode-step append with RoPE in one launch: emx_cache_slots and
 * emx_fp8_cache_write_rope together for one token per sequence, with the
 * positions, slots and kv_lens rule of emx_affine_cache_append_rope
 * (num_tokens <= 1024 and at most 65536 values per tensor; otherwise
 * EMX_ERR_UNSUPPORTED).  `counter`: EMX_APPEND_COUNTER_INTS device ints, zero
 * before the first call, left zero by every call (calls sharing them must not
 * overlap).  Besides the workgroup count they carry the call's K and V maxima
 * while its workgroups exchange them: the write workgroups wait (a bounded wait)
 * until every one of them has folded its maxima in, so all encode with the same
 * scales; their number is small (at most 128) and they are all resident at once.
 * Replaces the FP8 decode write of PageCacheView.concatenate_to_cache
 *   lib/python/easymlx/caching/paged/cache.py:1126-1184 (RoPE :1161-1166).
 */
int emx_fp8_cache_append_rope(const void* keys, const void* values, int dtype, const int32_t* slot_ids,
                              int num_tokens, const int32_t* block_tables, int num_seqs, int max_blocks_per_seq,
                              int32_t* kv_lens, int* counter, int num_kv_heads, int head_dim, int page_size,
                              int num_blocks, uint8_t* key_cache, uint8_t* value_cache, float* k_scales,
                              float* v_scales, const float* inv_freq, int rot_dims, int traditional,
                              const void* queries_in, void* queries, int num_q_heads, void* stream);

/*
 * Write positions of a cache write, on the device: token t of sequence i
 * (query_start_loc[i] <= t < query_start_loc[i+1], i < num_slots, int32 arrays
 * on the device) of slot s = slot_ids[i] goes to position
 * p = kv_lens[s] + t - query_start_loc[i], slot_mapping[t] =
 * block_tables[s, p / page_size] * page_size + p % page_size (-1 when s is
 * outside [0, num_seqs), the page column beyond max_blocks_per_seq or the
 * block id negative), positions[t] = p; then kv_lens[s] += query length of i
 * (in place).  num_tokens = query_start_loc[num_slots]; at most 4096 sequences.
 * One launch, no host round trip: usable under HIP graph capture.
 * Replaces the slot arithmetic of PageCacheView.concatenate_to_cache
 *   lib/python/easymlx/caching/paged/cache.py:1126-1170, 1211-1261, 1297
 *   and of the compiled decode proxy
 *   lib/python/easymlx/inference/esurge/runners/model_runner.py:164-184.
 */
int emx_cache_slots(const int32_t* slot_ids, const int32_t* query_start_loc, int num_slots, int num_tokens,
                    const int32_t* block_tables, int num_seqs, int max_blocks_per_seq, int page_size,
                    int32_t* kv_lens, int32_t* slot_mapping, int32_t* positions, void* stream);

/*
 * Unquantized cache write: token t's rows keys/values [num_tokens, Hkv,
 * head_dim] (dtype EMX_DTYPE_*) to slot slot_mapping[t] of key_cache /
 * value_cache [num_blocks, page_size, Hkv, head_dim] of the same dtype (-1 or a
 * page outside the pool skips the token).
 * Replaces reshape_and_cache lib/python/easymlx/caching/paged/cache.py:36-93
 *   (the cast-and-scatter of concatenate_to_cache :1186-1190, :1273-1277).
 */
int emx_dense_cache_write(const void* keys, const void* values, int dtype, const int32_t* slot_mapping,
                          int num_tokens, int num_kv_heads, int head_dim, int page_size, int num_blocks,
                          void* key_cache, void* value_cache, void* stream);

/*
 * Copy-on-write block copies over every array of a cache: arrays[k] holds
 * num_blocks blocks of block_bytes[k] bytes each (a positive multiple of 4;
 * host arrays of num_arrays <= 8 entries, e.g. codes, scales and biases of K
 * and V).  For each row (src, dst) of block_mapping int32 [num_pairs, 2] on the
 * device, block dst of every array becomes a copy of block src as it was
 * before the call, as the reference kernel reads its inputs and writes
 * separate outputs: swapped and chained pairs are well defined; of several
 * pairs with one destination the last counts.  Ids outside [0, num_blocks) are
 * skipped.  workspace: device staging of at least
 * emx_copy_blocks_workspace_bytes(...) bytes, 16-byte aligned (no zero-fill
 * needed); two launches (gather the sources, scatter to the destinations).
 * Replaces PageCacheView.copy_blocks / PageCache.copy_blocks
 *   lib/python/easymlx/caching/paged/cache.py:944-972, 1438-1445 (Metal kernel :95-136).
 */
int emx_copy_blocks(int num_arrays, void* const* arrays, const int64_t* block_bytes, int num_blocks,
                    const int32_t* block_mapping, int num_pairs, void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * Staging bytes emx_copy_blocks needs for num_pairs pairs over these arrays
 * (0 for an invalid description or no pairs).
 * No direct reference counterpart: the reference's kernel allocates whole
 * output arrays (cache.py:95-136).
 */
size_t emx_copy_blocks_workspace_bytes(int num_arrays, const int64_t* block_bytes, int num_pairs);

/*
 * Zero the blocks page_ids int32 [num_pages] (device) of every array of a cache
 * (same array description as emx_copy_blocks; ids outside [0, num_blocks) skipped).
 * Replaces the runner's _zero_pages
 *   lib/python/easymlx/inference/esurge/runners/model_runner.py:1058-1094 and the page
 *   zeroing of PageCacheView.reset lib/python/easymlx/caching/paged/cache.py:874-906.
 */
int emx_zero_blocks(int num_arrays, void* const* arrays, const int64_t* block_bytes, int num_blocks,
                    const int32_t* page_ids, int num_pages, void* stream);

/*
 * Affine cache layout conversion on the device, both directions (out-of-place;
 * every destination element written once).  Logical layout: what
 * mlx.core.quantize gives for the reference's dense cache [nb, bs, Hkv, D]
 * (lib/python/easymlx/caching/paged/cache.py:790-791; quantize at
 * lib/python/easymlx/infra/mixins/bridge.py:304,361): codes uint32
 * [nb, bs, Hkv, D*bits/32], scales / biases fp16 [nb, bs, Hkv, D/group_size].
 * Page layout: the one emx_paged_attention_affine and the writes use (above).
 * Lets a caller holding reference-layout affine caches hand them to this
 * library (and read pages back) without a host round trip.
 */
int emx_affine_pages_from_logical(const uint32_t* k_codes_in, const uint32_t* v_codes_in, const void* k_scales_in,
                                  const void* k_biases_in, const void* v_scales_in, const void* v_biases_in,
                                  int num_blocks, int page_size, int num_kv_heads, int head_dim, int bits,
                                  int group_size, uint32_t* k_codes, uint32_t* v_codes, void* k_scales,
                                  void* k_biases, void* v_scales, void* v_biases, void* stream);
int emx_affine_logical_from_pages(const uint32_t* k_codes, const uint32_t* v_codes, const void* k_scales,
                                  const void* k_biases, const void* v_scales, const void* v_biases, int num_blocks,
                                  int page_size, int num_kv_heads, int head_dim, int bits, int group_size,
                                  uint32_t* k_codes_out, uint32_t* v_codes_out, void* k_scales_out,
                                  void* k_biases_out, void* v_scales_out, void* v_biases_out, void* stream);

/*
 * Page-read probe (measurement only; no counterpart in the reference): reads
 * exactly the page bytes a decode call over these 4-bit or 8-bit affine pages
 * (head_dim 128, page_size a multiple of 64) reads -- K codes, V codes and the
 * four scale / bias runs of every 64-token slice of a page-head that holds a
 * token below kv_lens -- and nothing else, so bytes / time is the read
 * bandwidth this call's scattered pattern gets from the memory system.  Each
 * workgroup stores the XOR of the 32-bit words it read into sink[w]; it runs
 * min(sink_words, 8 x compute units) workgroups of 256 threads.
 */
int emx_probe_page_read(const uint32_t* k_codes, const void* k_scales, const void* k_biases, const uint32_t* v_codes,
                        const void* v_scales, const void* v_biases, int num_blocks, int page_size, int num_kv_heads,
                        int head_dim, int bits, int group_size, const int32_t* block_tables, int num_seqs,
                        int max_blocks_per_seq, const int32_t* kv_lens, uint32_t* sink, int sink_words, void* stream);

/*
 * The page-read probe over an FP8 (E4M3) cache in the reference layout
 * [num_blocks, page_size, Hkv, 128] uint8 with fp32 page scales (measurement
 * only; no counterpart in the reference): reads exactly what the FP8 decode
 * reads -- the 32-token row blocks of every kv head holding a token below
 * kv_lens, and their pages' two scales -- and nothing else.  page_size a
 * multiple of 32; sink and workgroups as emx_probe_page_read.
 */
int emx_probe_page_read_fp8(const uint8_t* key_cache, const uint8_t* value_cache, const float* k_scale,
                            const float* v_scale, int num_blocks, int page_size, int num_kv_heads, int head_dim,
                            const int32_t* block_tables, int num_seqs, int max_blocks_per_seq, const int32_t* kv_lens,
                            uint32_t* sink, int sink_words, void* stream);

/*
 * Dense K/V of a ragged batch gathered from pages: token t of sequence b
 * (cu_seq_lens[b] <= t < cu_seq_lens[b+1], int32 [num_seqs+1] on the device) at
 * offset j = t - cu_seq_lens[b] is entry j % page_size of page
 * block_table[b, j / page_size]; k_out/v_out [total_tokens, Hkv, head_dim] in
 * out_dtype (EMX_DTYPE_*).  Affine pages are dequantized (scale * code + bias
 * in fp32), FP8 pages decoded times their page scale, dense pages cast.  A page
 * id outside [0, num_blocks) or a column beyond the table yields zeros.
 * Replaces PageCacheView.gather_kv_cache
 *   lib/python/easymlx/caching/paged/cache.py:974-1027 (Metal kernel :138-193).
 */
int emx_gather_kv_affine(const uint32_t* k_codes, const void* k_scales, const void* k_biases, const uint32_t* v_codes,
                         const void* v_scales, const void* v_biases, int num_blocks, int page_size, int num_kv_heads,
                         int head_dim, int bits, int group_size, const int32_t* block_table, int num_seqs,
                         int max_blocks_per_seq, const int32_t* cu_seq_lens, int total_tokens, int out_dtype,
                         void* k_out, void* v_out, void* stream);
int emx_gather_kv_fp8(const uint8_t* key_cache, const uint8_t* value_cache, const float* k_scale,
                      const float* v_scale, int num_blocks, int page_size, int num_kv_heads, int head_dim,
                      const int32_t* block_table, int num_seqs, int max_blocks_per_seq, const int32_t* cu_seq_lens,
                      int total_tokens, int out_dtype, void* k_out, void* v_out, void* stream);
int emx_gather_kv_dense(const void* key_cache, const void* value_cache, int dtype, int num_blocks, int page_size,
                        int num_kv_heads, int head_dim, const int32_t* block_table, int num_seqs,
                        int max_blocks_per_seq, const int32_t* cu_seq_lens, int total_tokens, int out_dtype,
                        void* k_out, void* v_out, void* stream);

/*
 * Rotary position embedding in place on fp16 rows x [rows, heads, head_dim]
 * (row r at positions[r]), the same rotation as emx_affine_cache_write_rope.
 * Replaces the RoPE applied to queries in concatenate_to_cache
 *   lib/python/easymlx/caching/paged/cache.py:1161-1166.
 */
int emx_rope_rows(void* x, int rows, int heads, int head_dim, const int32_t* positions, const float* inv_freq,
                  int rot_dims, int traditional, void* stream);

/*
 * Bytes of device workspace emx_paged_attention_affine and
 * emx_paged_attention_fp8 need for split-K
 * partial results and arrival counters (0 if the call needs none).  The
 * workspace must be zero-filled before its first use; every call leaves its
 * counter region zeroed again, so one workspace serves any sequence of calls
 * (of any shape) that are ordered on one stream.  Calls sharing a workspace
 * must not overlap.  The workspace also carries the 4-bit decode's plan cache:
 * a pure decode call keeps its work split there, keyed by its shape and the
 * per-sequence counts of work items that kv_lens gives (an item: 256 tokens up
 * to GQA 4, 128 up to 8, 64 up to 16), and the next call with the same counts
 * (the next layer of the same decode step, and most next steps: a kv_len that
 * grows by one token keeps its count unless it crosses an item boundary)
 * starts from it; a call with other counts or another shape
 * computes its own.  Results are the same either way.
 * No direct reference counterpart: replaces the tmp_out/exp_sums/max_logits
 * allocation of lib/python/easymlx/operations/kernels/page_attention.py:2205-2272.
 */
size_t emx_paged_workspace_bytes(int num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                                 int max_blocks_per_seq, int page_size);

/*
 * Extra workspace bytes, after emx_paged_workspace_bytes(...), with which the
 * prefill kernel of emx_paged_attention_affine / emx_paged_attention_fp8 cuts
 * tiles of many keys into up to three parts (one workgroup each) and merges
 * them in-kernel (0 if the shape cannot split).  A call whose workspace_bytes
 * covers both sums splits; a smaller workspace runs every tile in one
 * workgroup.  Same zero-fill and ordering rules as the decode workspace.
 * No direct reference counterpart: the reference's prefill kernel runs one
 * threadgroup per query row (unified_attention.py:290-465).
 */
size_t emx_paged_prefill_workspace_bytes(int num_tokens, int num_seqs, int num_q_heads, int num_kv_heads,
                                         int head_dim);

/*
 * Paged attention over affine pages; queries/out fp16 [num_tokens, Hq, head_dim].
 * block_tables int32 [num_seqs, max_blocks_per_seq]; kv_lens int32 [num_seqs];
 * query_start_loc int32 [num_seqs+1].  single_token_decode != 0 means token i
 * belongs to sequence i (num_tokens == num_seqs) and selects the split-K MFMA
 * decode kernel when head_dim == 128 and page_size % 128 == 0.
 * Replaces: paged_attention(...) lib/python/easymlx/operations/kernels/unified_attention.py:1377-1512
 *   (kernels :290-609 and FP8 in-kernel dequant :776-1268), with
 *   k_scale/v_scale generalised to per-(token, group) scales and biases.
 */
int emx_paged_attention_affine(const void* queries, int num_tokens, int num_q_heads, int head_dim,
                               const uint32_t* k_codes, const void* k_scales, const void* k_biases,
                               const uint32_t* v_codes, const void* v_scales, const void* v_biases, int num_blocks,
                               int page_size, int num_kv_heads, int bits, int group_size,
                               const int32_t* block_tables, int num_seqs, int max_blocks_per_seq,
                               const int32_t* kv_lens, const int32_t* query_start_loc, float softmax_scale,
                               int sliding_window, int single_token_decode, void* workspace, size_t workspace_bytes,
                               void* out, void* stream);

/*
 * Paged attention over an unquantized cache in the reference layout
 * key/value [num_blocks, page_size, Hkv, head_dim] (dtype = queries' dtype).
 * Single-token decode calls (head_dim a multiple of 32 up to 256, page_size a
 * multiple of 8) run split-K over chunks of keys when the workspace holds
 * emx_paged_workspace_bytes(...) bytes (same rules as
 * emx_paged_attention_affine); otherwise, or with a null workspace, one
 * wave per (token, kv head) walks the keys.
 * Replaces: paged_attention(...) unified_attention.py:1377-1512 for fp16/bf16/fp32 caches
 *   (decode kernels :467-775, split-K precedent page_attention.py:1718-2059).
 */
int emx_paged_attention_dense(const void* queries, int num_tokens, int num_q_heads, int head_dim, int dtype,
                              const void* key_cache, const void* value_cache, int num_blocks, int page_size,
                              int num_kv_heads, const int32_t* block_tables, int num_seqs, int max_blocks_per_seq,
                              const int32_t* kv_lens, const int32_t* query_start_loc, float softmax_scale,
                              int sliding_window, int single_token_decode, void* workspace, size_t workspace_bytes,
                              void* out, void* stream);

/*
 * Bytes of device workspace emx_fp8_cache_write needs (per-workgroup maxima;
 * no zero fill needed).  Calls sharing a workspace must not overlap.
 * No direct reference counterpart (the reference reduces into an MLX output
 * array, lib/python/easymlx/caching/paged/cache.py:430-463).
 */
size_t emx_fp8_write_workspace_bytes(void);

/*
 * FP8 (E4M3) quantize-on-write into a page cache key/value [num_blocks,
 * page_size, Hkv, head_dim] uint8 with one fp32 scale per page (k_scales,
 * v_scales [num_blocks], zero-filled at allocation).  keys/values [num_tokens,
 * Hkv, head_dim] in dtype (EMX_DTYPE_*); slot_mapping int32 [num_tokens]
 * (block * page_size + offset, -1 to skip).  One scale per call,
 * max|x| / 240 over the written tokens; codes enc(x / max(scale, 1e-12));
 * each written page's scale becomes max(page scale, call scale).  At most
 * 2^33 - 4 values per tensor (EMX_ERR_UNSUPPORTED beyond).
 * Replaces the FP8 branch of PageCacheView.concatenate_to_cache
 *   lib/python/easymlx/caching/paged/cache.py:1171-1184 (compute_kv_scales
 *   :430-463, _fp8_quantize :466-478, encoder
 *   lib/python/easymlx/operations/kernels/_metal_header.py:339-419).
 */
int emx_fp8_cache_write(const void* keys, const void* values, int dtype, const int32_t* slot_mapping, int num_tokens,
                        int num_kv_heads, int head_dim, int page_size, int num_blocks, uint8_t* key_cache,
                        uint8_t* value_cache, float* k_scales, float* v_scales, void* workspace,
                        size_t workspace_bytes, void* stream);

/*
 * emx_fp8_cache_write that allocates nothing and takes no workspace: the
 * two-launch path keeps its per-workgroup maxima in a fixed device array of the
 * library, 8 slots of 2 KiB per GPU (held until the process ends), one slot per
 * stream that calls it: calls on one stream are ordered, calls on different
 * streams use different slots.  A ninth stream on one GPU is refused
 * (EMX_ERR_UNSUPPORTED).  Same arguments, results and limits as
 * emx_fp8_cache_write otherwise; calls no hipMalloc, hipFree or allocating
 * library routine.
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory or hold a workspace: code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation.
 */
int emx_fp8_cache_write_noalloc(const void* keys, const void* values, int dtype, const int32_t* slot_mapping,
                                int num_tokens, int num_kv_heads, int head_dim, int page_size, int num_blocks,
                                uint8_t* key_cache, uint8_t* value_cache, float* k_scales, float* v_scales,
                                void* stream);

/*
 * emx_fp8_cache_write with rotary position embedding fused in: the call's K
 * scale and codes are taken over the keys turned as in
 * emx_affine_cache_write_rope and rounded to dtype.  rot_dims a multiple of 8
 * (of 4 when traditional).  queries (fp16 [num_tokens, num_q_heads, head_dim],
 * or null) receive queries_in turned (null: queries turned in place), in the
 * same launch for decode-size writes.
 * Replaces the RoPE of PageCacheView.concatenate_to_cache
 *   lib/python/easymlx/caching/paged/cache.py:1161-1166 followed by its FP8 write :1171-1184.
 */
int emx_fp8_cache_write_rope(const void* keys, const void* values, int dtype, const int32_t* slot_mapping,
                             int num_tokens, int num_kv_heads, int head_dim, int page_size, int num_blocks,
                             uint8_t* key_cache, uint8_t* value_cache, float* k_scales, float* v_scales,
                             void* workspace, size_t workspace_bytes, const int32_t* positions, const float* inv_freq,
                             int rot_dims, int traditional, const void* queries_in, void* queries,
                             int num_q_heads, void* stream);

/*
 * Paged attention over an FP8 (E4M3) cache key/value [num_blocks, page_size,
 * Hkv, head_dim] uint8 with per-page fp32 scales k_scale/v_scale [num_blocks]:
 * K = dec(code) * k_scale[page].  queries/out in dtype (EMX_DTYPE_*).
 * With fp16 queries, head_dim 128 and page_size % 32 == 0, decode rows run on
 * the split-K decode kernel, which needs the workspace sized by
 * emx_paged_workspace_bytes (same rules as emx_paged_attention_affine);
 * other calls ignore it.
 * Replaces: paged_attention(..., k_scale=, v_scale=)
 *   lib/python/easymlx/operations/kernels/unified_attention.py:1377-1512 with the
 *   FP8 kernels :776-1268 (decoder :1275-1285).
 */
int emx_paged_attention_fp8(const void* queries, int num_tokens, int num_q_heads, int head_dim, int dtype,
                            const uint8_t* key_cache, const uint8_t* value_cache, const float* k_scale,
                            const float* v_scale, int num_blocks, int page_size, int num_kv_heads,
                            const int32_t* block_tables, int num_seqs, int max_blocks_per_seq, const int32_t* kv_lens,
                            const int32_t* query_start_loc, float softmax_scale, int sliding_window,
                            int single_token_decode, void* workspace, size_t workspace_bytes, void* out,
                            void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EMX_ATTN_H_ */
