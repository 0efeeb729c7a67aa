// Host-side launchers shared between the kernel files and the C ABI (capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llmopt {

// Everything a linear kernel needs. Pointers are device pointers.
struct LinearArgs {
  const void* x;        // [M, K] activations, row stride ldx (elements)
  const uint8_t* qw;    // [N, ldq] packed codes
  const float* scales;  // [N, G]
  const float* zeros;   // [N, G] or nullptr (symmetric)
  const void* bias;     // [N] activation dtype or nullptr
  void* y;              // [M, N] activation dtype, row stride ldy (elements)
  int64_t ldx, ldq, ldy;
  int64_t M, N, K;
  int64_t group;        // resolved group size (> 0)
  int64_t G;            // groups per row
  int act;              // kDtF32 / kDtF16 / kDtBf16
  int fmt;              // kNibble / kByte
  int bits;
  int symmetric;
  int signed_codes;
  float zero_const;     // code offset used when symmetric
  void* workspace;      // caller-owned device scratch (split-K partial sums), may be null
  size_t workspace_bytes;
  // kEpiSwiglu: the weight rows are gate and up projections interleaved in blocks of four
  // (fused rows 8p .. 8p+3 = gate features 4p .. 4p+3, rows 8p+4 .. 8p+7 = up features
  // 4p .. 4p+3) and y[m, 4p + r] = silu(gate) * up; y then has N / 2 columns.
  int epilogue;
  // 1: y is fp32 and takes the sums unrounded (the fp32-activation path's products of its
  // bf16 pieces); only the decode kernels and the K-split reduction take it, with no bias
  // and no epilogue.
  int out_f32;
  // Host side only. defer_reduce = 1: a K-sliced decode plan leaves its fp32 partial sums
  // [slices][M][N] at the start of the workspace, launches no reduction, leaves y untouched and
  // stores the slice count in *deferred_planes (which the caller zeroes first); other plans
  // finish as usual. Only without an epilogue (with out_f32 = 1: the fp32-activation path,
  // whose combining kernel then adds the slices as well as the pieces).
  int defer_reduce;
  int* deferred_planes;
};
enum : int { kEpiNone = 0, kEpiSwiglu = 1 };

#ifdef __HIPCC__
// Stores output element `idx` of a linear kernel: rounded to the activation dtype, or (out_f32)
// the fp32 sum itself.
template <class Act>
__device__ __forceinline__ void put_y(const LinearArgs& a, int64_t idx, float v) {
  if (a.out_f32)
    static_cast<float*>(a.y)[idx] = v;
  else
    static_cast<typename Act::raw*>(a.y)[idx] = Act::store(v);
}
#endif

// Each launcher returns hipSuccess or the launch error; `why` is set when the arguments do not
// fit the kernel (then hipErrorInvalidValue is returned and nothing is launched).
hipError_t launch_unpack(const uint8_t* packed, uint8_t* codes, int64_t rows, int64_t packed_cols,
                         int64_t columns, hipStream_t stream);
hipError_t launch_dequant(const LinearArgs& a, void* out, int out_dtype, hipStream_t stream);

// Round-to-nearest quantization of a dense weight into the packed layout.
struct RtnArgs {
  const void* w;   // [N, ldw] weight of w_dtype
  int w_dtype;     // kDtF32 / kDtF16 / kDtBf16
  int64_t ldw;     // row stride of w, elements
  int64_t N, K;
  int bits;        // 2, 4 or 8
  int64_t group;   // columns per group (divides K; even)
  int64_t G;       // K / group
  int symmetric;
  uint8_t* q;      // [N, ldq] codes: two per byte below 8 bits
  int64_t ldq;     // row stride of q, bytes
  float* scales;   // [N, G]
  float* zeros;    // [N, G] (zeros written even for symmetric grids)
};
hipError_t launch_quantize_rtn(const RtnArgs& a, hipStream_t stream);

// Paged KV cache: one layer's caches [num_blocks, block_size, kv_heads, head_dim].
struct KvWriteArgs {
  void* key_cache;
  void* value_cache;
  int cache_dtype;
  int64_t num_blocks, block_size, kv_heads, head_dim;
  const int32_t* block_ids;  // [num_seqs, ldb]
  int64_t ldb;
  const int32_t* offsets;    // [num_seqs] first position written
  const void* keys;          // [num_seqs, (q_len,) kv_heads, head_dim] of src_dtype
  const void* values;
  int src_dtype;
  int64_t src_seq_stride, src_token_stride;  // elements
  int64_t num_seqs;
};
hipError_t launch_kv_write(const KvWriteArgs& a, int64_t q_len, bool decode, hipStream_t stream);

struct PagedDecodeArgs {
  const void* query;  // [num_seqs, num_heads, head_dim] rows of q_seq_stride elements
  int q_dtype;
  int64_t q_seq_stride;
  const void* key_cache;
  const void* value_cache;
  int cache_dtype;
  int64_t num_blocks, block_size, kv_heads, head_dim;
  const int32_t* block_ids;
  int64_t ldb;
  const int32_t* context_lens;
  int64_t num_seqs, num_heads;
  float scale, softcap;
  void* out;  // [num_seqs, num_heads, head_dim] of out_dtype
  int out_dtype;
  float* part_out;  // [splits, num_seqs, num_heads, head_dim]
  float* part_lse;  // [splits, num_seqs, num_heads]
  int splits;
  int64_t tiles_per_split;  // 16-token tiles per split (per workgroup)
  int waves;                // waves per workgroup: 1, 2, 4 or 8 (8 only below 16 heads per KV head)
  int q_vec;                // query rows 16-byte aligned: vector loads
  // Rotary step in the same launch (rope != 0; query, caches and new rows all of cache_dtype):
  // `query` holds the step's raw q rows; new_k / new_v the raw k and v rows [num_seqs, kv_heads,
  // head_dim] (token strides ldk / ldv). q and k are rotated at positions[s] from the fp32
  // tables, k and v are stored into the cache slot of offsets[s] (k_store / v_store: the same
  // caches), and the new token's key and value enter the softmax from registers.
  int rope;
  const void* new_k;
  const void* new_v;
  int64_t ldk, ldv;
  const int64_t* positions;
  const float* cos_table;
  const float* sin_table;
  int64_t table_rows;
  const int32_t* offsets;
  void* k_store;
  void* v_store;
  // Prefill (launch_paged_prefill): q_len query tokens per sequence at positions
  // context_lens[s] - q_len + j, each seeing the keys up to its own position. query element
  // (s, j, h, d) at s * q_seq_stride + j * q_tok_stride + h * q_head_stride + d; out likewise
  // with the out_* strides.
  int64_t q_len;
  int64_t q_tok_stride, q_head_stride;
  int64_t out_seq_stride, out_tok_stride, out_head_stride;
};
hipError_t launch_paged_decode(const PagedDecodeArgs& a, hipStream_t stream);
hipError_t launch_paged_prefill(const PagedDecodeArgs& a, hipStream_t stream);

struct RmsNormArgs {
  const void* x;         // [rows, hidden], row stride ldx
  const void* residual;  // optional [rows, hidden], row stride ldr: h = residual + x
  void* h_out;           // with residual: h, row stride ldh
  const void* weight;    // [hidden], the activation dtype
  void* y;               // [rows, hidden], row stride ldy
  int64_t rows, hidden, ldx, ldr, ldh, ldy;
  float eps;
  int dtype;             // kDtBf16 or kDtF16
  // Optional, in place of x (needs the residual): the K-sliced decode kernel's partial sums
  // [splits][rows][hidden] fp32, x = their sum in slice order plus plane_bias ([hidden] of the
  // activation dtype, may be null), rounded to the activation dtype -- the split-K reduction's
  // result, bit for bit.
  const float* planes;
  int64_t splits;
  const void* plane_bias;
};
hipError_t launch_rmsnorm(const RmsNormArgs& a, hipStream_t stream);

struct RopeArgs {
  const void* q;  // [tokens, heads, head_dim], token stride ldq
  const void* k;  // [tokens, kv_heads, head_dim], token stride ldk
  void* q_out;    // [tokens, heads, head_dim], contiguous
  void* k_out;    // [tokens, kv_heads, head_dim], contiguous
  const void* v;  // optional [tokens, kv_heads, head_dim], token stride ldv: copied to v_out
  void* v_out;
  int64_t ldv;
  const int64_t* positions;  // [tokens]
  const float* cos_table;    // [table_rows, head_dim] fp32
  const float* sin_table;
  int64_t table_rows, tokens, heads, kv_heads, head_dim, ldq, ldk;
  int dtype;
  // Optional (decode, one token per sequence): k and v go straight to this layer's paged
  // cache [num_blocks, block_size, kv_heads, head_dim] of the same dtype, at the slot of
  // offsets[t] in block_ids[t, :], instead of k_out / v_out.
  void* key_cache;
  void* value_cache;
  const int32_t* block_ids;  // [tokens, ldb]
  const int32_t* offsets;    // [tokens]
  int64_t ldb, num_blocks, block_size;
  int vec;  // rows and tables 16-byte aligned, head_dim % 16 == 0: 16-byte loads and stores
};
hipError_t launch_rope(const RopeArgs& a, hipStream_t stream);

struct ArgmaxArgs {
  const void* x;  // [rows, cols] of dtype, row stride ldx elements
  int dtype;
  int64_t rows, cols, ldx;
  int vec;        // rows 16-byte aligned: 16-byte loads
  int64_t* out;   // [rows]
};
hipError_t launch_argmax_rows(const ArgmaxArgs& a, hipStream_t stream);
hipError_t launch_linear_generic(const LinearArgs& a, hipStream_t stream);
// Decode and prefill report `fits = false` (and launch nothing) when the shape, alignment or
// dtype is outside what the kernel handles.
hipError_t launch_linear_decode(const LinearArgs& a, hipStream_t stream, bool* fits);
hipError_t launch_linear_prefill(const LinearArgs& a, hipStream_t stream, bool* fits);
hipError_t launch_linear_gemm(const LinearArgs& a, hipStream_t stream, bool* fits);
// y[m, 4p + r] = silu(t[m, 8p + r]) * t[m, 8p + 4 + r] for a full fused output t [M, N]
// (row stride ldt) in the activation dtype: the path for kernels without the fused epilogue.
hipError_t launch_swiglu_combine(const void* t, int64_t ldt, void* y, int64_t ldy, int64_t M, int64_t N,
                                 int act, hipStream_t stream);
// Workspace the prefill GEMM's split-K plan uses for these sizes (0 when it does not split).
size_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group, int fmt);
// y = bias + the fixed-order sum of `splits` fp32 partial products [splits][M][N] (with the
// SwiGLU epilogue when a.epilogue asks for it).
hipError_t launch_splitk_reduce(const LinearArgs& a, const float* partials, int splits, hipStream_t stream);
// Workspace the decode path's K-split kernels (N-split, K-sliced) use for these sizes (0 when
// they do not split); with less, the decode path takes its other kernels.
size_t decode_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group, int bits);
// Whether the decode path's K-sliced kernel takes this size (given its workspace).
bool ks_takes(int64_t M, int64_t N, int64_t K, int64_t group, int bits);
// Whether the decode path's N-split kernel takes this 33-64-token size (grids of >= 1024 tiles).
bool nx_takes_wide(int64_t M, int64_t N, int64_t K, int64_t group, int bits);
// fp32 activations as three bf16 pieces per token on the decode kernels (chunks of up to 21
// tokens), then a combining kernel; *fits is false when the workspace is smaller than
// f32_workspace_bytes (the caller then takes the generic kernel).
hipError_t launch_linear_f32_pieces(const LinearArgs& a, hipStream_t stream, bool* fits);
// One or two fp32 tokens on the one-shot kernel with the split into pieces and their sum inside
// it (no workspace); *fits is false for the shapes it does not take.
hipError_t launch_linear_oneshot_f32(const LinearArgs& a, hipStream_t stream, bool* fits);
size_t f32_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group, int bits);
// Long batches in two passes: the weight dequantized into the workspace, then hipBLASLt's dense
// GEMM. *fits is false (nothing launched) when the workspace is smaller than
// dense_workspace_bytes, for an epilogue, or when hipBLASLt offers no algorithm for the shape.
hipError_t launch_linear_dense(const LinearArgs& a, hipStream_t stream, bool* fits);
size_t dense_workspace_bytes(int64_t N, int64_t K, int act);
// Batches from this many tokens take the two-pass path (given its workspace).
int64_t dense_min_tokens(int act);

}  // namespace llmopt
