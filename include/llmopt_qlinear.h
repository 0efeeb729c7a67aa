/*
 * llmopt_qlinear.h -- C ABI of libllmopt_qlinear.so, the gfx950 (MI355X)
 * fused dequantize-and-multiply library behind llmopt.quantization.QuantLinear.
 *
 * Storage layout consumed (identical to the reference's, quantizers.py:83-97,
 * 100-142, 204-239):
 *   qweight, bits 1 - 7  : uint8 [N, ldq], two codes per byte; column k is in
 *                          byte k>>1, even k in bits 0-3, odd k in bits 4-7.
 *   qweight, bits 8      : uint8 (asymmetric) or int8 (symmetric) [N, ldq].
 *   scales, zeros        : fp32 [N, K/group], row-major, contiguous.
 *   dequantized weight   : w[n,k] = (q[n,k] - z) * s   evaluated in fp32 with a
 *                          single rounding, z = zeros[n, k/group] (asymmetric),
 *                          2^(bits-1) (symmetric, bits < 8) or 0 (symmetric 8-bit).
 *
 * Conventions:
 *   - Every pointer is a device pointer on the current HIP device, owned by the
 *     caller. The library keeps no tensors; scratch space (split-K partial sums,
 *     the dense weight of the two-pass path) comes in through `workspace`. The
 *     one allocation it makes is hipBLASLt's handle, created by the first
 *     two-pass call on a device (so that call must not run under stream capture).
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream). Work is
 *     enqueued asynchronously; nothing synchronises the host, except the first
 *     two-pass call of a size class (M rounded up to 2^k or 3 * 2^(k-1), up to
 *     6144 tokens) on a stream that is not being captured: it times hipBLASLt's
 *     candidate algorithms on its own inputs and waits for them, once.
 *   - Return value: LLMOPT_OK (0) or a negative LLMOPT_ERR_* code. The message of
 *     the last failure on the calling thread is llmopt_q_last_error().
 *   - Reentrant: the mutable global state is the per-thread error text, the
 *     static device scratch of llmopt_q_linear_noalloc (below), and the two-pass
 *     path's hipBLASLt handles and plan cache, guarded by a mutex; every other
 *     entry point's calls from several host threads on different streams are
 *     independent.
 *   - group_size <= 0 means one group spanning the whole row.
 *   - dtype codes: LLMOPT_DTYPE_F32 / F16 / BF16.
 *
 * The reference (Python on torch) has no C interface; each entry point below
 * names the Python function whose work it replaces.
 */
#ifndef LLMOPT_QLINEAR_H_
#define LLMOPT_QLINEAR_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LLMOPT_QLINEAR_ABI_VERSION 1

#define LLMOPT_DTYPE_F32 0
#define LLMOPT_DTYPE_F16 1
#define LLMOPT_DTYPE_BF16 2

#define LLMOPT_OK 0
#define LLMOPT_ERR_INVALID_ARG (-1)
#define LLMOPT_ERR_UNSUPPORTED (-2)
#define LLMOPT_ERR_HIP (-3)
#define LLMOPT_ERR_WORKSPACE (-4)

/* Kernel selection for llmopt_q_linear_ex. AUTO is what llmopt_q_linear uses. */
#define LLMOPT_ALGO_AUTO 0
#define LLMOPT_ALGO_GENERIC 1 /* any shape and dtype; scalar dequant + fp32 dot */
#define LLMOPT_ALGO_DECODE 2  /* MFMA skinny GEMM, M <= 64 */
#define LLMOPT_ALGO_PREFILL 3 /* MFMA GEMM with weight tiles dequantized into LDS */
#define LLMOPT_ALGO_DENSE 4   /* the weight dequantized into the workspace, then hipBLASLt */

/* ABI version of the loaded library (LLMOPT_QLINEAR_ABI_VERSION). */
int llmopt_q_abi_version(void);

/* Message describing the last failed call on this thread ("" if none). */
const char* llmopt_q_last_error(void);

/*
 * Split packed bytes into nibble codes.
 * Replaces unpack_int4 (src/llmopt/quantization/quantizers.py:92-97):
 *   codes[r, c] = (packed[r, c>>1] >> (4*(c&1))) & 0xF   for c < columns.
 * packed: uint8 [rows, packed_cols]; codes: uint8 [rows, columns], columns <= 2*packed_cols.
 */
int llmopt_q_unpack(const uint8_t* packed, uint8_t* codes, int64_t rows, int64_t packed_cols,
                    int64_t columns, void* stream);

/*
 * Dense weight from the packed form, bit-identical to the reference.
 * Replaces dequantize + dequantize_codes (quantizers.py:204-239):
 *   out[n, k] = dtype((q[n,k] - z) * s)   (fp32 arithmetic, round-to-nearest-even cast).
 * qweight: [N, ldq] bytes; zeros may be NULL when symmetric; signed_codes = 1 when
 * an 8-bit qweight is int8. out: [N, K] of out_dtype.
 */
int llmopt_q_dequant(const void* qweight, int64_t ldq, const float* scales, const float* zeros,
                     void* out, int out_dtype, int64_t N, int64_t K, int bits, int group_size,
                     int symmetric, int signed_codes, void* stream);

/*
 * Round-to-nearest quantization of a dense weight into the packed layout, in one pass.
 * Replaces RoundToNearestQuantizer.quantize (src/llmopt/quantization/quantizers.py:285-305),
 * i.e. choose_qparams (:100-142), quantize_to_codes (:167-201) and pack_int4 (:83-89),
 * bit-exact with their fp32 arithmetic on finite weights.
 * weight: [N, ldw] of w_dtype; bits in {2, 4, 8}; group_size divides K (even below 8 bits).
 * qweight: [N, ldq] bytes -- uint8 two codes per byte (bits < 8), uint8 (asymmetric 8-bit) or
 * int8 (symmetric 8-bit); scales, zeros: [N, K/group] fp32 (zeros are 0 when symmetric).
 */
int llmopt_q_quantize_rtn(const void* weight, int w_dtype, int64_t ldw, int64_t N, int64_t K, int bits,
                          int group_size, int symmetric, void* qweight, int64_t ldq, float* scales,
                          float* zeros, void* stream);

/*
 * Bytes of workspace llmopt_q_linear may use for these sizes (0 if none): fp32 partial sums of
 * a K split, splits * M * N * 4 bytes, for the prefill GEMM and for the decode kernels that
 * split K over fewer than 1024 tiles of 16 features (5-64 tokens on rows of K >= 8192, 33-64 on
 * shorter rows; none at 5-32 tokens over K = 4096 in groups of 128); from 1024 tokens, the
 * two-pass path's llmopt_q_linear_dense_workspace bytes (or the split's, if larger). With less,
 * those shapes run on the other kernels: correct, slower.
 */
size_t llmopt_q_linear_workspace(int64_t M, int64_t N, int64_t K, int bits, int group_size);

/*
 * llmopt_q_linear_workspace for an activation dtype: the same for LLMOPT_DTYPE_BF16 / F16; for
 * LLMOPT_DTYPE_F32 the bytes of the fp32 path -- each activation split exactly into three bf16
 * pieces (3 * M * K * 2 bytes), the decode kernels' fp32 sums of a chunk of up to 21 tokens
 * (3 * chunk * N * 4) and their K-split partial sums; from 65 tokens, the two-pass path's fp32
 * llmopt_q_linear_dense_workspace bytes (or the pieces', if larger). With less, fp32 runs on the
 * generic kernel.
 * Sizes the workspace of QuantLinear.forward with compute_dtype float32
 * (src/llmopt/quantization/quant_linear.py:93-113), the reference engine's quantized model
 * (engine/llm_engine.py:258-264).
 */
size_t llmopt_q_linear_workspace_ex(int64_t M, int64_t N, int64_t K, int bits, int group_size, int act_dtype);

/*
 * Bytes of workspace of the two-pass path (LLMOPT_ALGO_DENSE, and AUTO from 1024 tokens, 65 with
 * fp32 activations): the dense [N, K] weight in the activation dtype, 256-byte aligned, then
 * 32 MiB for hipBLASLt. The two passes are the reference's own computation,
 * QuantLinear._dequantized_weight then F.linear (src/llmopt/quantization/quant_linear.py:93-113),
 * with the dense weight rebuilt in the workspace by every call instead of cached in the module.
 */
size_t llmopt_q_linear_dense_workspace(int64_t N, int64_t K, int act_dtype);

/*
 * y = x @ dequant(qweight)^T + bias, without materialising the dense weight.
 * Replaces QuantLinear.forward (src/llmopt/quantization/quant_linear.py:93-113):
 * the reference dequantizes into a cached dense weight and calls F.linear.
 * x: [M, K] act_dtype with row stride ldx; y: [M, N] act_dtype with row stride ldy;
 * bias: [N] act_dtype or NULL. Accumulation is fp32. M == 0 is a no-op.
 */
int llmopt_q_linear(const void* x, int64_t M, int64_t K, int64_t ldx, const void* qweight,
                    int64_t ldq, const float* scales, const float* zeros, const void* bias,
                    void* y, int64_t N, int64_t ldy, int act_dtype, int bits, int group_size,
                    int symmetric, int signed_codes, void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * llmopt_q_linear whose K-split partial sums may be left for the consumer to add up. When the
 * plan for these sizes is the K-sliced decode kernel with S > 1 slices (llmopt_q_linear_workspace
 * reports S * M * N * 4 bytes), no reduction runs, y is left untouched, and *planes = S: the
 * fp32 partial sums [S][M][N] (bias not added) sit at the start of the workspace, and
 * llmopt_rmsnorm_planes (llmopt_model.h) adds them up inside the residual add + RMSNorm that
 * follows. Otherwise *planes = 0 and y holds the result, as from llmopt_q_linear. 16-bit
 * activations only defer (fp32 finishes as usual). The pair replaces the down projection's
 * QuantLinear.forward and the next layer's residual add + RMSNorm
 * (src/llmopt/quantization/quant_linear.py:110-113; src/llmopt/model/layers.py:185-195) with
 * one launch fewer and the same bits.
 */
int llmopt_q_linear_deferred(const void* x, int64_t M, int64_t K, int64_t ldx, const void* qweight,
                             int64_t ldq, const float* scales, const float* zeros, const void* bias,
                             void* y, int64_t N, int64_t ldy, int act_dtype, int bits, int group_size,
                             int symmetric, int signed_codes, void* workspace, size_t workspace_bytes,
                             void* stream, int* planes);

/*
 * llmopt_q_linear without a workspace argument and without any allocation: the K-split
 * partial sums that llmopt_q_linear keeps in the caller's workspace live in a static device
 * array of the library instead, llmopt_q_linear_noalloc_max_scratch() bytes (32 MiB) per
 * device, held until the process ends. Below 1024 tokens, results are those of llmopt_q_linear
 * with a workspace of llmopt_q_linear_workspace(...) bytes, bit for bit; from 1024 tokens it runs
 * the fused GEMM (the two-pass path's dense weight does not fit the scratch): the results of
 * llmopt_q_linear_ex with LLMOPT_ALGO_PREFILL. A shape whose plan needs more scratch than that
 * returns LLMOPT_ERR_WORKSPACE and launches nothing. Calls that overlap on one
 * device (other streams, other threads) share that device's array and race on it; serialize
 * them. Run it with the stream's device current.
 * No counterpart in the reference: for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 */
int llmopt_q_linear_noalloc(const void* x, int64_t M, int64_t K, int64_t ldx, const void* qweight,
                            int64_t ldq, const float* scales, const float* zeros, const void* bias,
                            void* y, int64_t N, int64_t ldy, int act_dtype, int bits, int group_size,
                            int symmetric, int signed_codes, void* stream);

/* Bytes of the static scratch behind llmopt_q_linear_noalloc (the largest plan it takes). */
size_t llmopt_q_linear_noalloc_max_scratch(void);

/*
 * llmopt_q_linear with an explicit kernel choice (LLMOPT_ALGO_*). Returns
 * LLMOPT_ERR_UNSUPPORTED when the chosen kernel cannot take these arguments.
 * No counterpart in the reference: lets tests and benchmarks pin one kernel.
 */
int llmopt_q_linear_ex(const void* x, int64_t M, int64_t K, int64_t ldx, const void* qweight,
                       int64_t ldq, const float* scales, const float* zeros, const void* bias,
                       void* y, int64_t N, int64_t ldy, int act_dtype, int bits, int group_size,
                       int symmetric, int signed_codes, void* workspace, size_t workspace_bytes,
                       void* stream, int algo);

/*
 * Bytes of workspace llmopt_q_linear_swiglu may use for these sizes (N = fused rows),
 * assuming 16-byte aligned, contiguous tensors (0 if none).
 */
size_t llmopt_q_linear_swiglu_workspace(int64_t M, int64_t N, int64_t K, int bits, int group_size);

/*
 * llmopt_q_linear_swiglu_workspace for an activation dtype (LLMOPT_DTYPE_F32: the [M, N] fp32
 * product and the fp32 path's workspace, as llmopt_q_linear_workspace_ex). Sizes the workspace
 * of SwiGLUMLP.forward (src/llmopt/model/layers.py:43-44) in a float32 model.
 */
size_t llmopt_q_linear_swiglu_workspace_ex(int64_t M, int64_t N, int64_t K, int bits, int group_size,
                                           int act_dtype);

/*
 * The gated activation of the reference's MLP, silu(gate(x)) * up(x), from one quantized
 * weight holding both projections. Replaces the gate_proj / up_proj / silu / multiply part of
 * SwiGLUMLP.forward (src/llmopt/model/layers.py:43-44): two F.linear calls and two
 * elementwise passes over [M, intermediate].
 * Fused row 8p + r (r < 4) is gate row 4p + r and fused row 8p + 4 + r is up row 4p + r;
 * scales, zeros and bias follow the same order. N (fused rows) must be a multiple of 8.
 * y: [M, N/2] act_dtype, row stride ldy. Rounding as the reference's sequence: gate and up
 * rounded to act_dtype, silu in fp32 on the rounded gate and rounded, the product rounded.
 * Kernels without the fused activation write the full product into `workspace` first;
 * when that is too small the call returns LLMOPT_ERR_WORKSPACE and names the size.
 */
int llmopt_q_linear_swiglu(const void* x, int64_t M, int64_t K, int64_t ldx, const void* qweight,
                           int64_t ldq, const float* scales, const float* zeros, const void* bias,
                           void* y, int64_t N, int64_t ldy, int act_dtype, int bits, int group_size,
                           int symmetric, int signed_codes, void* workspace, size_t workspace_bytes,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LLMOPT_QLINEAR_H_ */
