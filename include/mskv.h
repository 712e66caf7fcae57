/*
 * mskv -- C ABI of the MI355X (gfx950) FP8 paged-KV library.
 *
 * Plain pointers and sizes only: every tensor argument is a device pointer to
 * contiguous memory, every stream argument is a hipStream_t passed as void*.
 * Launches are asynchronous on that stream; no entry point allocates device
 * memory, synchronizes, or reads device memory on the host, so all of them
 * may be captured into a HIP graph.
 *
 * Cache layout (the reference runner's, microserve/engine/model_runner.py:76-83):
 *   k_cache, v_cache           uint8 (OCP FP8 e4m3fn) [num_blocks, block_size, num_kv_heads, head_dim]
 *   k_scale_cache, v_scale_cache  float32             [num_blocks, block_size, num_kv_heads]
 * Cache row r = block * block_size + offset holds token slot r.
 *
 * Return value: 0 on success, a negative MSKV_E* code for rejected arguments,
 * or a positive hipError_t from the launch.  mskv_status_string() names it.
 */
#ifndef MSKV_H
#define MSKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* activation element types (query, key, value, output) */
#define MSKV_FLOAT16 0
#define MSKV_BFLOAT16 1
/* also accepted for the key/value rows of mskv_store_fp8_kvcache only */
#define MSKV_FLOAT32 2
/* slot_mapping element types */
#define MSKV_INT32 0
#define MSKV_INT64 1

#define MSKV_OK 0
#define MSKV_EINVAL (-1)       /* null pointer, bad size or inconsistent shape */
#define MSKV_EUNSUPPORTED (-2) /* valid shape the kernels do not implement     */
#define MSKV_EWORKSPACE (-3)   /* workspace missing or smaller than required   */

/* Library version (major * 10000 + minor * 100 + patch). */
int mskv_version(void);

/* Human-readable text for a status code returned by any entry point. */
const char* mskv_status_string(int status);

/*
 * Quantize K/V rows to FP8 e4m3fn with one fp32 scale per (token, kv head)
 * and scatter them through slot_mapping.
 *
 * Replaces store_fp8_kvcache, microserve/layers/fp8_kv_cache.py:42-61
 * (kernel :11-39): scale = max(amax_d |x|, 1e-8) / 448, byte =
 * e4m3fn(clamp(x / scale, -448, 448)) with IEEE fp32 division, written at
 * cache row slot_mapping[t].  key/value: [num_tokens, num_kv_heads, head_dim]
 * in act_dtype: MSKV_FLOAT16, MSKV_BFLOAT16 or MSKV_FLOAT32 (the reference
 * upcasts any float input to fp32, :22-23).  Slots outside [0, num_slots)
 * are skipped (num_slots = num_blocks * block_size); the reference never
 * produces them.  Supported: head_dim == 128.
 */
int mskv_store_fp8_kvcache(const void* key, const void* value,
                           void* k_cache, void* v_cache,
                           float* k_scale_cache, float* v_scale_cache,
                           const void* slot_mapping, int slot_dtype,
                           int64_t num_tokens, int num_kv_heads, int head_dim,
                           int64_t num_slots, int act_dtype, void* stream);

/*
 * Number of split-KV partitions mskv_fp8_decode_attention uses for a shape.
 * Depends on shapes only (never on device sequence lengths), so a captured
 * graph stays valid for any lengths up to max_blocks_per_seq * block_size.
 */
int mskv_decode_num_splits(int batch, int num_q_heads, int num_kv_heads,
                           int max_blocks_per_seq, int block_size);

/*
 * Scratch bytes mskv_fp8_decode_attention needs for num_splits (0 if 1):
 * the fp32 split partials and, for shapes of many workgroup rounds, the
 * longest-first work items that a pre-pass kernel writes.
 * Contents on entry do not matter.
 */
size_t mskv_decode_workspace_bytes(int batch, int num_q_heads,
                                   int num_kv_heads, int head_dim,
                                   int num_splits);


/*
 * Paged decode attention over the FP8 cache: one query token per sequence.
 *
 * Replaces fp8_decode_attention, microserve/layers/fp8_decode_attention.py:62-101
 * (kernel :8-59): q head h reads kv head h / (num_q_heads / num_kv_heads);
 * token p of sequence b is cache row block_tables[b][p / block_size] *
 * block_size + p % block_size for p < cache_seqlens[b]; scores are
 * q . (k * k_scale) * softmax_scale; out = softmax(scores) @ (v * v_scale),
 * or zeros when cache_seqlens[b] == 0.
 * query/out: [batch, num_q_heads, head_dim] in act_dtype; cache_seqlens:
 * int32 [batch]; block_tables: int32 [batch, max_blocks_per_seq], -1 padded.
 * Block ids outside [0, num_blocks) read as empty.  num_splits must be the
 * value mskv_decode_num_splits returns for the shape; when it is above 1 the
 * workspace must hold mskv_decode_workspace_bytes bytes, and a second
 * kernel merges the split partials.
 * Supported: head_dim == 128, block_size % 32 == 0, and a GQA group
 * (num_q_heads / num_kv_heads) of at most 16 or a multiple of 16.
 */
int mskv_fp8_decode_attention(const void* query, const void* k_cache,
                              const void* v_cache, const float* k_scale_cache,
                              const float* v_scale_cache,
                              const int32_t* cache_seqlens,
                              const int32_t* block_tables, void* out,
                              int batch, int num_q_heads, int num_kv_heads,
                              int head_dim, int block_size, int64_t num_blocks,
                              int max_blocks_per_seq, float softmax_scale,
                              int act_dtype, int num_splits, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Scratch (split partials, work items) the allocation-free decode holds per GPU. */
#define MSKV_DECODE_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

/*
 * mskv_fp8_decode_attention without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving
 * loops and harnesses that forbid hipMalloc).  It has no counterpart in the
 * reference.  The split partials (and, for batches of many workgroup
 * rounds, the pre-pass's work items) go to a library-owned device array of
 * MSKV_DECODE_NOALLOC_SCRATCH_BYTES (32 MiB) on each GPU, held until the
 * process ends; shapes whose mskv_decode_workspace_bytes exceeds it are
 * rejected with MSKV_EWORKSPACE (e.g. batch 64 x 4096 tokens at 32 q heads
 * needs 4.2 MB, batch 4 x 131072 at 64 q heads 16.9 MB).  The call makes no
 * hipMalloc/hipFree; the array's address on the current device is looked
 * up once, on that device's first call, which must therefore be an eager
 * call (not one under graph capture); later calls may be captured.  No part
 * of the array needs to start at zero.  Every call on one GPU shares that GPU's array: calls that
 * may overlap on one GPU (different streams, or one graph replayed while
 * another call runs) race on it and must be serialized by the caller.
 * Arguments and results are mskv_fp8_decode_attention's.
 */
int mskv_fp8_decode_attention_noalloc(const void* query, const void* k_cache,
                                      const void* v_cache,
                                      const float* k_scale_cache,
                                      const float* v_scale_cache,
                                      const int32_t* cache_seqlens,
                                      const int32_t* block_tables, void* out,
                                      int batch, int num_q_heads,
                                      int num_kv_heads, int head_dim,
                                      int block_size, int64_t num_blocks,
                                      int max_blocks_per_seq,
                                      float softmax_scale, int act_dtype,
                                      int num_splits, void* stream);

/*
 * Causal paged prefill over the FP8 cache for a varlen batch whose new
 * tokens are already stored in the cache.
 *
 * Replaces fp8_chunk_prefill_attention,
 * microserve/layers/fp8_chunk_prefill_attention.py:70-109 (kernel :8-67),
 * generalized from one sequence (block_table.view(-1), scalar prefix_len) to
 * the varlen batch the runner describes with cu_seqlens_q / cu_seqlens_k
 * (microserve/engine/model_runner.py:184-192).  Sequence s owns query rows
 * [cu_seqlens_q[s], cu_seqlens_q[s+1]) and context length
 * Lk = cu_seqlens_k[s+1] - cu_seqlens_k[s]; query i sees cache positions
 * p < (Lk - Lq) + i + 1 (fp8_chunk_prefill_attention.py:52-54).
 * When cu_seqlens_q and cu_seqlens_k are both NULL the batch is one
 * sequence of total_q queries over prefix_len + total_q positions, exactly
 * the reference's signature.  QK^T runs as FP8 MFMA contractions, the
 * query split into e4m3 parts under a power-of-two row scale; PV runs on
 * the fp16 MFMA with V converted exactly and weights p * v_scale rounded to
 * fp16 under a power-of-two scale.
 * query/out: [total_q, num_q_heads, head_dim] in act_dtype; block_tables:
 * int32 [num_seqs, max_blocks_per_seq].  max_seqlen_q must be at least
 * every sequence's query count: it sizes the grid, and query rows past it
 * are not written (flash-attn's contract for the same argument).
 * Supported: head_dim == 128, block_size % 128 == 0, GQA group <= 16 or a
 * multiple of 16, num_seqs <= 65535, max_seqlen_q <= 65535 query blocks
 * of 128 rows (2M tokens at GQA 4, 524k at GQA 16), and a positive, finite
 * softmax_scale; MSKV_EUNSUPPORTED otherwise.
 */
int mskv_fp8_prefill_attention(const void* query, const void* k_cache,
                               const void* v_cache, const float* k_scale_cache,
                               const float* v_scale_cache,
                               const int32_t* block_tables,
                               const int32_t* cu_seqlens_q,
                               const int32_t* cu_seqlens_k, int prefix_len,
                               void* out, int num_seqs, int64_t total_q,
                               int max_seqlen_q, int num_q_heads,
                               int num_kv_heads, int head_dim, int block_size,
                               int64_t num_blocks, int max_blocks_per_seq,
                               float softmax_scale, int act_dtype,
                               void* stream);

/*
 * Causal varlen attention over unquantized q/k/v: the fresh PREFILL of the
 * FP8-KV path.
 *
 * Replaces flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k,
 * max_seqlen_q, max_seqlen_k, softmax_scale, causal=True), called by
 * microserve/layers/attention.py:49-55 on the step's new tokens.  Sequence
 * s owns query rows [cu_seqlens_q[s], cu_seqlens_q[s+1]) and key rows
 * [cu_seqlens_k[s], cu_seqlens_k[s+1]); query i sees key j iff
 * j <= i + Lk - Lq (flash-attn's bottom-right causal alignment); a row that
 * sees no key is zero.  QK^T and PV run on 16-bit MFMA in act_dtype with
 * fp32 accumulation; the probabilities are rounded to act_dtype.
 * query/out: [total_q, num_q_heads, head_dim]; key/value:
 * [total_k, num_kv_heads, head_dim], all contiguous in act_dtype.
 * max_seqlen_q must be at least every sequence's query count: it sizes the
 * grid, and query rows past it are not written (as in flash-attn).
 * Supported: head_dim == 128, GQA group <= 16 or a multiple of 16,
 * num_seqs <= 65535, max_seqlen_q <= 65535 query blocks of 192 rows
 * (3.1M tokens at GQA 4), and a positive, finite softmax_scale;
 * MSKV_EUNSUPPORTED otherwise.
 */
int mskv_prefill_attention(const void* query, const void* key,
                           const void* value, void* out,
                           const int32_t* cu_seqlens_q,
                           const int32_t* cu_seqlens_k, int num_seqs,
                           int64_t total_q, int64_t total_k, int max_seqlen_q,
                           int num_q_heads, int num_kv_heads, int head_dim,
                           float softmax_scale, int act_dtype, void* stream);

/*
 * Expand one step's per-sequence scheduling state into its per-token inputs
 * and -1-padded block tables, in one launch.
 *
 * Replaces the element-by-element device writes of ModelRunner's
 * _compile_decode / _compile_prefill / _compile_chunk_prefill /
 * _make_block_tables (microserve/engine/model_runner.py:124-193, 208-216)
 * and the graph padding of _run_decode (:264-272).  Sequence b schedules
 * n_b = cu_seqlens_q[b+1] - cu_seqlens_q[b] positions p = seq_start[b] + j;
 * row r = cu_seqlens_q[b] + j gets input_ids[r] = token_ids[r],
 * positions[r] = p and slot_mapping[r] = table_b[p / block_size] *
 * block_size + p % block_size, or -1 when p / block_size is past the end of
 * table_b (the reference raises there; the store skips -1).  table_b is
 * tables[table_offsets[b] .. table_offsets[b+1]).  cache_seqlens[b] =
 * seq_start[b] + n_b; block_tables[b][c] = table_b[c] for c < len_b, else
 * -1, for c < table_width.  Rows b = num_seqs .. pad_seqs - 1 are padding
 * rows of a captured decode graph: slot_mapping / input_ids / positions row
 * total_q + (b - num_seqs) get garbage_slot / 0 / 0, cache_seqlens[b] = 0
 * and the table row is -1.
 * token_ids: int64 [total_q]; seq_start: int32 [num_seqs]; cu_seqlens_q and
 * table_offsets: nondecreasing int32 [num_seqs + 1] starting at 0, with
 * cu_seqlens_q[num_seqs] == total_q; tables: int32 [table_offsets[num_seqs]].
 * Outputs input_ids, positions, slot_mapping: int64 [total_q + pad_seqs -
 * num_seqs] (NULL allowed when that is 0); cache_seqlens: int32 [pad_seqs]
 * or NULL; block_tables: int32 [pad_seqs, table_width] or NULL.
 * max_seqlen_q only sizes the launch.
 */
int mskv_build_step_inputs(const int64_t* token_ids, const int32_t* seq_start,
                           const int32_t* cu_seqlens_q,
                           const int32_t* table_offsets, const int32_t* tables,
                           int num_seqs, int pad_seqs, int64_t total_q,
                           int block_size, int table_width,
                           int64_t garbage_slot, int64_t* input_ids,
                           int64_t* positions, int64_t* slot_mapping,
                           int32_t* cache_seqlens, int32_t* block_tables,
                           int max_seqlen_q, void* stream);

/*
 * Fused attention prologue: per-head RMSNorm of q and k, rotary embedding,
 * and the FP8 store of the rotated k and of v, in one launch.
 *
 * Replaces microserve/models/qwen3.py:49-53 (q_norm, k_norm, rotary_emb)
 * and the store_fp8_kvcache call that opens Attention.forward
 * (microserve/layers/attention.py:41-43).  For each token t and head row x
 * of q (num_q_heads rows) and k (num_kv_heads rows), in act_dtype T:
 *   RMSNorm (microserve/layers/layernorm.py:55-57, 80-81), skipped when both
 *   weights are NULL: var = (sum of x^2) / 128 in fp32, summed as eight
 *   partial sums (lane l: elements 8l..8l+7 then 64+8l..64+8l+7, in order)
 *   combined as ((s0+s1)+(s2+s3))+((s4+s5)+(s6+s7)); r = 1/sqrtf(var + eps)
 *   with IEEE fp32 sqrt and division; y = T(T(x * r) * w).
 *   Rotary (microserve/layers/rotary_embedding.py:24-31), p = positions[t],
 *   c = cos_cache[p], s = sin_cache[p], for d < 64:
 *   out[d] = T(T(y[d]*c[d]) + T(-y[d+64]*s[d])),
 *   out[d+64] = T(T(y[d+64]*c[d+64]) + T(y[d]*s[d+64])), sums in fp32 first.
 * q rows go to q_out; k rows to k_out (if not NULL) and, with the v rows, to
 * the FP8 cache at slot_mapping[t] with the bytes and scales of
 * mskv_store_fp8_kvcache.  A token with p outside [0, max_position) gets zero
 * q_out/k_out rows and is not stored; slots outside [0, num_slots) are
 * skipped.
 * q/k/v: [num_tokens, heads, 128] in act_dtype with heads contiguous and
 * the given token strides (elements; views of one qkv tensor allowed);
 * positions: int64 [num_tokens]; weights: act_dtype [128];
 * cos_cache/sin_cache: act_dtype [max_position, 128]; q_out: [num_tokens,
 * num_q_heads, 128]; k_out: [num_tokens, num_kv_heads, 128] or NULL.  Every
 * tensor must be 16-byte aligned and token strides multiples of 8.
 * Supported: head_dim == 128.
 */
int mskv_qk_norm_rope_store(const void* q, const void* k, const void* v,
                            int64_t q_token_stride, int64_t k_token_stride,
                            int64_t v_token_stride, const int64_t* positions,
                            const void* q_norm_weight, const void* k_norm_weight,
                            float eps, const void* cos_cache,
                            const void* sin_cache, int64_t max_position,
                            void* q_out, void* k_out, void* k_cache,
                            void* v_cache, float* k_scale_cache,
                            float* v_scale_cache, const void* slot_mapping,
                            int slot_dtype, int64_t num_tokens, int num_q_heads,
                            int num_kv_heads, int head_dim, int64_t num_slots,
                            int act_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MSKV_H */
