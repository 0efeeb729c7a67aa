/*
 * llmopt_model.h -- C ABI of the decoder's elementwise steps in libllmopt_qlinear.so (gfx950):
 * RMSNorm with an optional fused residual add, and the rotary embedding of q and k. Same
 * conventions as llmopt_qlinear.h: device pointers owned by the caller, `stream` a hipStream_t
 * as void*, LLMOPT_OK or a negative LLMOPT_ERR_* code with the message in llmopt_q_last_error(),
 * dtype codes LLMOPT_DTYPE_* (F16 or BF16 here; other dtypes return LLMOPT_ERR_UNSUPPORTED and
 * the Python layer runs the reference's torch sequence).
 */
#ifndef LLMOPT_MODEL_H_
#define LLMOPT_MODEL_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * y = x * rsqrt(mean(x^2) + eps) * weight, per row, computed in fp32 and rounded once to dtype.
 * Replaces RMSNorm.forward (src/llmopt/model/layers.py:14-31). With residual != NULL the input
 * is first h = residual + x, rounded to dtype (the residual add of DecoderLayer.forward,
 * layers.py:185-195), and h is written to h_out. x, residual, h_out, y: [rows, hidden] with row
 * strides ldx, ldr, ldh, ldy elements; weight: [hidden] of dtype. Needs hidden % 8 == 0, row
 * strides % 8 == 0 and 16-byte aligned pointers (else LLMOPT_ERR_UNSUPPORTED).
 */
int llmopt_rmsnorm(const void* x, int64_t ldx, const void* residual, int64_t ldr, void* h_out, int64_t ldh,
                   const void* weight, void* y, int64_t ldy, int64_t rows, int64_t hidden, float eps, int dtype,
                   void* stream);

/*
 * llmopt_rmsnorm with a residual, whose x is a linear's K-split partial sums left by
 * llmopt_q_linear_deferred: planes [splits][rows][hidden] fp32 (16-byte aligned), x = their sum
 * in slice order plus bias ([hidden] of dtype, may be NULL), rounded to dtype; then h = residual
 * + x and y = RMSNorm(h) as llmopt_rmsnorm computes them. Bit for bit llmopt_q_linear's
 * split-K reduction followed by llmopt_rmsnorm (the residual add + RMSNorm of
 * src/llmopt/model/layers.py:185-195 after the down projection), in one launch instead of two.
 */
int llmopt_rmsnorm_planes(const float* planes, int64_t splits, const void* bias, const void* residual, int64_t ldr,
                          void* h_out, int64_t ldh, const void* weight, void* y, int64_t ldy, int64_t rows,
                          int64_t hidden, float eps, int dtype, void* stream);

/*
 * Rotary embedding of q and k at positions[t] (int64): out = x * cos + rotate_half(x) * sin,
 * rotate_half([a, b]) = [-b, a] over the two halves of each head; cos_table / sin_table are the
 * fp32 [table_rows, head_dim] tables, cast to dtype as the reference casts them. Replaces
 * apply_rotary_pos_emb with RotaryEmbedding.forward (src/llmopt/model/rotary.py:23-45,85-102);
 * every product and sum is rounded to dtype as torch rounds it, so the result is identical.
 * q: [tokens, heads, head_dim] with token stride ldq; k: [tokens, kv_heads, head_dim] with token
 * stride ldk; q_out, k_out: contiguous. v (optional, may be NULL): [tokens, kv_heads, head_dim]
 * with token stride ldv, copied unchanged to the contiguous v_out (the layer's cache write then
 * reads contiguous rows). Positions outside [0, table_rows) are clamped (the Python layer raises
 * for them first, as the reference does).
 */
int llmopt_rope(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv, void* q_out,
                void* k_out, void* v_out, const int64_t* positions, const float* cos_table, const float* sin_table,
                int64_t table_rows, int64_t tokens, int64_t heads, int64_t kv_heads, int64_t head_dim, int dtype,
                void* stream);

/*
 * llmopt_rope for a decode step (one token per sequence, tokens = seqs) fused with the cache
 * write that follows it: the rotated k and the unchanged v go straight into this layer's paged
 * cache (key_cache / value_cache [num_blocks, block_size, kv_heads, head_dim], of dtype) at the
 * slot of token_offsets[s] in block block_ids[s, token_offsets[s] / block_size] (int32, row
 * stride ldb); a block id outside [0, num_blocks) is replaced by block 0, as the reference does.
 * Replaces the rotary step of the attention layer followed by PagedKVCache.write_decode
 * (src/llmopt/cache/paged_cache.py:246-277), whose results it gives bit for bit for offsets
 * whose block index lies in [0, ldb). Outside that range it differs: such a token's k and v
 * are not written, where the reference raises IndexError (index past the row) or, through
 * negative indexing, writes into the row's last block (negative offset). The offsets live on
 * the device, so checking them would need a host sync; callers that can hold such offsets
 * check them first. q_out as in llmopt_rope.
 */
int llmopt_rope_kv_write_decode(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                                void* q_out, const int64_t* positions, const float* cos_table,
                                const float* sin_table, int64_t table_rows, int64_t seqs, int64_t heads,
                                int64_t kv_heads, int64_t head_dim, int dtype, void* key_cache, void* value_cache,
                                int64_t num_blocks, int64_t block_size, const int32_t* block_ids, int64_t ldb,
                                const int32_t* token_offsets, void* stream);

/*
 * Greedy sampling's argmax of each row: out[r] = the index of the first maximum of row r of
 * x ([rows, cols] of dtype F32 / F16 / BF16, row stride ldx elements), a NaN counting as larger
 * than every number (the first NaN wins) -- torch.argmax(logits, dim=-1) of the reference's
 * greedy sampler (src/llmopt/engine/sampler.py:94-95). out: int64 [rows] on the device.
 */
int llmopt_argmax_rows(const void* x, int dtype, int64_t rows, int64_t cols, int64_t ldx, int64_t* out,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif  // LLMOPT_MODEL_H_
