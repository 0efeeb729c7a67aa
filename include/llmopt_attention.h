/*
 * llmopt_attention.h -- C ABI of the paged KV cache writes and the decode attention in
 * libllmopt_qlinear.so (gfx950). Same conventions as llmopt_qlinear.h: device pointers owned by
 * the caller, `stream` a hipStream_t as void*, LLMOPT_OK or a negative LLMOPT_ERR_* code with
 * the message in llmopt_q_last_error(), dtype codes LLMOPT_DTYPE_*.
 *
 * Cache layout (the reference's, src/llmopt/cache/paged_cache.py:152-160): each layer's key and
 * value caches are [num_blocks, block_size, kv_heads, head_dim], row-major; callers pass the
 * layer's base pointers. Token t of sequence s lives in block block_ids[s * ldb + t / block_size]
 * at slot t % block_size. block_ids, token offsets and context lengths are int32.
 */
#ifndef LLMOPT_ATTENTION_H_
#define LLMOPT_ATTENTION_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * One new token per sequence into the cache. Replaces PagedKVCache.write_decode
 * (src/llmopt/cache/paged_cache.py:246-277). keys/values: [num_seqs, kv_heads, head_dim] of
 * src_dtype, row stride src_seq_stride elements; converted to cache_dtype with round-to-nearest-
 * even, as .to(dtype) does. A block id outside [0, num_blocks) writes block 0, as the reference
 * does; an offset whose block index is outside [0, ldb) writes nothing, where the reference
 * raises IndexError (index past the row) or writes the row's last block (negative offset,
 * through negative indexing).
 */
int llmopt_kv_write_decode(void* key_cache, void* value_cache, int cache_dtype, int64_t num_blocks,
                           int64_t block_size, int64_t kv_heads, int64_t head_dim, const int32_t* block_ids,
                           int64_t ldb, const int32_t* token_offsets, const void* keys, const void* values,
                           int src_dtype, int64_t src_seq_stride, int64_t num_seqs, void* stream);

/*
 * q_len new tokens per sequence, from token_offsets[s]. Replaces PagedKVCache.write / _write_one
 * (src/llmopt/cache/paged_cache.py:187-244): a sequence stops at its first -1 block or at the end
 * of its table row. keys/values: [num_seqs, q_len, kv_heads, head_dim] with element strides
 * src_seq_stride (sequence) and src_token_stride (token).
 */
int llmopt_kv_write(void* key_cache, void* value_cache, int cache_dtype, int64_t num_blocks, int64_t block_size,
                    int64_t kv_heads, int64_t head_dim, const int32_t* block_ids, int64_t ldb,
                    const int32_t* token_offsets, const void* keys, const void* values, int src_dtype,
                    int64_t src_seq_stride, int64_t src_token_stride, int64_t num_seqs, int64_t q_len,
                    void* stream);

/*
 * Bytes of workspace llmopt_paged_attention_decode uses to split the context (0: no split).
 */
size_t llmopt_paged_attention_workspace(int64_t num_seqs, int64_t num_heads, int64_t kv_heads, int64_t head_dim,
                                        int64_t ldb, int64_t block_size);

/*
 * Decode attention (one query token per sequence) read in place from the paged cache. Replaces
 * PagedAttention.forward with q_len == 1 (src/llmopt/attention/paged_attention.py:145-182,
 * 218-290), which gathers the K/V into a padded tensor first (paged_cache.py:279-324).
 * query: [num_seqs, num_heads, head_dim] of q_dtype, row stride q_seq_stride elements; it is
 * cast to the cache dtype as the reference does. out: [num_seqs, num_heads, head_dim] of
 * q_dtype. Query head h reads KV head h / (num_heads / kv_heads). Keys are the tokens
 * t < context_lens[s] whose block id is >= 0; a sequence without keys gets zeros. softcap > 0
 * applies tanh(x / softcap) * softcap to the scaled scores. Supported: cache_dtype F16/BF16,
 * head_dim 64 or 128, num_heads / kv_heads in {1, 2, 4, 8, 16}; otherwise
 * LLMOPT_ERR_UNSUPPORTED. With less workspace than llmopt_paged_attention_workspace asks for,
 * the context is not split (correct, slower for few sequences).
 */
int llmopt_paged_attention_decode(const void* query, int q_dtype, int64_t q_seq_stride, const void* key_cache,
                                  const void* value_cache, int cache_dtype, int64_t num_blocks, int64_t block_size,
                                  int64_t kv_heads, int64_t head_dim, const int32_t* block_ids, int64_t ldb,
                                  const int32_t* context_lens, int64_t num_seqs, int64_t num_heads, float scale,
                                  float softcap, void* out, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Prefill attention (q_len query tokens per sequence) read in place from the paged cache, after
 * this step's K/V were written. Replaces PagedAttention.forward with q_len > 1
 * (src/llmopt/attention/paged_attention.py:145-182, 210-290: the gather, the padding + causal
 * mask of _build_mask, and the dense or split softmax). Query token j of sequence s sits at
 * position context_lens[s] - q_len + j and sees the keys t <= that position (t < context_lens[s],
 * block id >= 0); a query with no keys gets zeros. query element (s, j, h, d) at
 * s * q_seq_stride + j * q_tok_stride + h * q_head_stride + d (q_dtype); out likewise with the
 * out_* strides, in q_dtype. Cache, table, scale, softcap and the supported shapes as in
 * llmopt_paged_attention_decode.
 */
int llmopt_paged_attention_prefill(const void* query, int q_dtype, int64_t q_seq_stride, int64_t q_tok_stride,
                                   int64_t q_head_stride, const void* key_cache, const void* value_cache,
                                   int cache_dtype, int64_t num_blocks, int64_t block_size, int64_t kv_heads,
                                   int64_t head_dim, const int32_t* block_ids, int64_t ldb,
                                   const int32_t* context_lens, int64_t num_seqs, int64_t num_heads, int64_t q_len,
                                   float scale, float softcap, void* out, int64_t out_seq_stride,
                                   int64_t out_tok_stride, int64_t out_head_stride, void* stream);

/*
 * The attention layer's decode step in one launch: llmopt_rope_kv_write_decode (include/
 * llmopt_model.h) followed by llmopt_paged_attention_decode. Replaces, for one token per
 * sequence, the rotary step (apply_rotary_pos_emb), PagedKVCache.write_decode and
 * PagedAttention.forward of the attention layer (src/llmopt/model/layers.py:118-140;
 * src/llmopt/cache/paged_cache.py:246-277; src/llmopt/attention/paged_attention.py:145-182).
 * q, k, v: the step's raw rows, [num_seqs, num_heads | kv_heads, head_dim] with token strides ldq,
 * ldk, ldv elements, of dtype = the cache dtype (BF16 or F16). positions (int64), cos_table /
 * sin_table ([table_rows, head_dim] fp32) and token_offsets (int32) as in
 * llmopt_rope_kv_write_decode: the rotated k and v are stored at the slot of token_offsets[s].
 * The cache, block table, context lengths, scale, softcap, out and workspace as in
 * llmopt_paged_attention_decode (the same workspace query). The new token's key and value enter
 * the softmax from registers, so the results are those of the two calls bit for bit whenever the
 * slot a sequence writes is not also a key of another sequence of the call -- which holds for
 * the reference's block pool, where only full (immutable) blocks are shared
 * (src/llmopt/cache/block_pool.py:65-70).
 */
int llmopt_paged_attention_decode_rope(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                                       int64_t ldv, const int64_t* positions, const float* cos_table,
                                       const float* sin_table, int64_t table_rows, int dtype, void* key_cache,
                                       void* value_cache, int64_t num_blocks, int64_t block_size, int64_t kv_heads,
                                       int64_t head_dim, const int32_t* block_ids, int64_t ldb,
                                       const int32_t* token_offsets, const int32_t* context_lens, int64_t num_seqs,
                                       int64_t num_heads, float scale, float softcap, void* out, void* workspace,
                                       size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LLMOPT_ATTENTION_H_ */
