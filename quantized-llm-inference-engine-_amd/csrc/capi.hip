// C ABI of libllmopt_qlinear.so (declared in include/llmopt_qlinear.h).
//
// Validates arguments the way the reference's torch code would reject them, fills the
// kernel argument block and picks the kernel: the decode kernels for M <= 32, the MFMA
// register-dequant GEMM (split over K on small grids) above, from 1024 tokens (65 with fp32
// activations) the weight dequantized into the workspace and hipBLASLt's dense GEMM, the
// LDS-dequant GEMM for the shapes the register-dequant one does not take, and the generic kernel
// for shapes, alignments or dtypes the fast kernels do not take. Error text is kept per host
// thread.
#include <stdarg.h>
#include <algorithm>
#include <stdio.h>

#include <mutex>
#include <string>

#include "../../include/llmopt_attention.h"
#include "../../include/llmopt_model.h"
#include "../../include/llmopt_qlinear.h"
#include "qcommon.hpp"
#include "qkernels.hpp"

namespace {

// Batches of up to this many tokens go to the decode kernels; above it the prefill GEMM with a
// K split is faster (measured on the Llama-3-8B projections: at M = 48 gate_up takes ~58 us in
// the GEMM against 105 us in the multi-tile decode kernel; at M = 32 the decode kernels lead).
constexpr int64_t kDecodeMaxTokens = 32;

// Whether the split-K GEMM takes a plain product of this size: every batch above
// kDecodeMaxTokens, and from 24 tokens the long rows (K >= 8192), unless the decode path's
// kernels that split K themselves take them (given a workspace: the caller checks).
// Batches of 33-64 tokens stay on the decode path where it streams them faster than the split-K
// GEMM: over at least 1024 tiles of 16 features (gate_up) its N-split kernel (gate_up at M = 64:
// 36.5 against 43 us), on smaller grids its K-sliced kernel -- each only for the weight formats
// it takes (2/4-bit codes, groups of a multiple of 128); other formats stay on the GEMM.
bool gemm_first(int64_t M, int64_t K, int64_t N, int64_t group, int bits) {
  if (M > kDecodeMaxTokens && M <= 64) {
    if (N >= 16 * 1024 && K < 8192 && llmopt::nx_takes_wide(M, N, K, group, bits)) return false;
    if (llmopt::ks_takes(M, N, K, group, bits)) return false;
  }
  return M > kDecodeMaxTokens || (M >= 24 && K >= 8192);
}

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list args;
  va_start(args, fmt);
  vsnprintf(buf, sizeof(buf), fmt, args);
  va_end(args);
  g_last_error = buf;
  return code;
}

int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return LLMOPT_OK;
  return fail(LLMOPT_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
}

bool valid_dtype(int dt) {
  return dt == LLMOPT_DTYPE_F32 || dt == LLMOPT_DTYPE_F16 || dt == LLMOPT_DTYPE_BF16;
}

// Shared validation of the packed-weight description; fills the format fields of `a`.
int describe_weight(llmopt::LinearArgs& a, const void* qweight, int64_t ldq, const float* scales,
                    const float* zeros, int64_t N, int64_t K, int bits, int group_size,
                    int symmetric, int signed_codes) {
  // Widths below 8 share the two-codes-per-byte storage (quantizers.py:236,273).
  if (bits < 1 || bits > 8) return fail(LLMOPT_ERR_INVALID_ARG, "unsupported bit width: %d", bits);
  if (N < 0 || K < 0) return fail(LLMOPT_ERR_INVALID_ARG, "negative shape N=%lld K=%lld",
                                  (long long)N, (long long)K);
  const int64_t group = group_size <= 0 ? K : group_size;
  if (K > 0 && (group <= 0 || K % group != 0))
    return fail(LLMOPT_ERR_INVALID_ARG, "in_features=%lld not divisible by group_size=%lld",
                (long long)K, (long long)group);
  const int fmt = bits == 8 ? llmopt::kByte : llmopt::kNibble;
  const int64_t need = fmt == llmopt::kNibble ? (K + 1) / 2 : K;
  if (ldq < need)
    return fail(LLMOPT_ERR_INVALID_ARG, "packed row of %lld bytes cannot hold %lld columns",
                (long long)ldq, (long long)K);
  if (fmt == llmopt::kNibble && signed_codes)
    return fail(LLMOPT_ERR_UNSUPPORTED, "sub-byte codes must be stored as uint8");
  if (N > 0 && K > 0) {
    if (!qweight || !scales) return fail(LLMOPT_ERR_INVALID_ARG, "null qweight or scales");
    if (!symmetric && !zeros) return fail(LLMOPT_ERR_INVALID_ARG, "asymmetric grid needs zeros");
  }
  a.qw = static_cast<const uint8_t*>(qweight);
  a.ldq = ldq;
  a.scales = scales;
  a.zeros = symmetric ? nullptr : zeros;
  a.N = N;
  a.K = K;
  a.group = group > 0 ? group : 1;
  a.G = group > 0 ? K / group : 0;
  a.fmt = fmt;
  a.bits = bits;
  a.symmetric = symmetric ? 1 : 0;
  a.signed_codes = signed_codes ? 1 : 0;
  a.zero_const = (symmetric && bits < 8) ? float(1 << (bits - 1)) : 0.0f;
  return LLMOPT_OK;
}


// The full [M, N] product that the combining kernel reads, in the activation dtype.
size_t swiglu_temp_bytes(int64_t M, int64_t N, int act) {
  return (size_t(M) * size_t(N) * (act == LLMOPT_DTYPE_F32 ? 4 : 2) + 255) / 256 * 256;
}

// Workspace of the fused kernels' plan (16-bit activations): the decode path's K split when it
// has one for these sizes (a call given that much takes it), else the split-K GEMM's when the
// GEMM takes the shape.
size_t fused_workspace_bytes(int64_t M, int64_t N, int64_t K, int bits, int group_size) {
  if (M <= 0 || N <= 0 || K <= 0 || bits < 1 || bits > 8) return 0;
  const int64_t g = group_size <= 0 ? K : group_size;
  const size_t dec = M <= 64 ? llmopt::decode_workspace_bytes(M, N, K, g, bits) : 0;
  if (dec > 0 || !gemm_first(M, K, N, g, bits)) return dec;
  return llmopt::gemm_workspace_bytes(M, N, K, g, bits == 8 ? llmopt::kByte : llmopt::kNibble);
}

// Whether a call of this size with this workspace takes the two-pass path (dequantize, then
// hipBLASLt) when hipBLASLt has an algorithm for it.
bool dense_first(int64_t M, int64_t N, int64_t K, int act, const void* workspace, size_t workspace_bytes) {
  return M >= llmopt::dense_min_tokens(act) && workspace != nullptr &&
         reinterpret_cast<uintptr_t>(workspace) % 256 == 0 &&
         workspace_bytes >= llmopt::dense_workspace_bytes(N, K, act);
}

// Dispatch shared by llmopt_q_linear_ex and llmopt_q_linear_swiglu. With the SwiGLU epilogue,
// `y` is [M, N/2]; kernels that cannot apply it themselves write the full [M, N] product into
// the workspace and a combining kernel finishes.
int run_linear(const void* x, int64_t M, int64_t K, int64_t ldx, const void* qweight, int64_t ldq,
               const float* scales, const float* zeros, const void* bias, void* y, int64_t N,
               int64_t ldy, int act_dtype, int bits, int group_size, int symmetric, int signed_codes,
               void* workspace, size_t workspace_bytes, void* stream, int algo, int epilogue,
               int* deferred = nullptr) {
  if (deferred) *deferred = 0;
  if (!valid_dtype(act_dtype)) return fail(LLMOPT_ERR_INVALID_ARG, "bad dtype code %d", act_dtype);
  if (M < 0) return fail(LLMOPT_ERR_INVALID_ARG, "negative M=%lld", (long long)M);
  llmopt::LinearArgs a{};
  int rc = describe_weight(a, qweight, ldq, scales, zeros, N, K, bits, group_size, symmetric,
                           signed_codes);
  if (rc != LLMOPT_OK) return rc;
  if (M == 0 || N == 0) return LLMOPT_OK;
  const int64_t ycols = epilogue == llmopt::kEpiSwiglu ? N / 2 : N;
  if (ldx < K || ldy < ycols)
    return fail(LLMOPT_ERR_INVALID_ARG, "row strides ldx=%lld ldy=%lld below K=%lld N=%lld",
                (long long)ldx, (long long)ldy, (long long)K, (long long)ycols);
  if (!x || !y) return fail(LLMOPT_ERR_INVALID_ARG, "null activation or output");
  a.x = x;
  a.bias = bias;
  a.y = y;
  a.ldx = ldx;
  a.ldy = ldy;
  a.M = M;
  a.act = act_dtype;
  a.workspace = workspace;
  a.workspace_bytes = workspace ? workspace_bytes : 0;
  a.epilogue = epilogue;
  a.defer_reduce = deferred != nullptr && epilogue == llmopt::kEpiNone && act_dtype != LLMOPT_DTYPE_F32;
  a.deferred_planes = a.defer_reduce ? deferred : nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);

  if (K == 0 && epilogue == llmopt::kEpiNone) {
    // An empty reduction: the reference's F.linear returns the bias (or zeros).
    a.K = 0;
    return hip_status(llmopt::launch_linear_generic(a, s), "linear launch");
  }

  bool fits = false;
  hipError_t err = hipSuccess;
  if (epilogue != llmopt::kEpiNone) {
    // Kernels with the fused epilogue first, unless the batch is long enough for the two-pass
    // path and the workspace holds its product and dense weight.
    const size_t temp = swiglu_temp_bytes(M, N, act_dtype);
    const bool dense = algo == LLMOPT_ALGO_AUTO && workspace_bytes >= temp &&
                       dense_first(M, N, K, act_dtype, workspace, workspace_bytes - temp);
    if (K > 0 && algo == LLMOPT_ALGO_AUTO && !dense) {
      if (M <= kDecodeMaxTokens || !gemm_first(M, K, N, a.group, bits)) {
        err = llmopt::launch_linear_decode(a, s, &fits);
        if (!fits && M > kDecodeMaxTokens) err = llmopt::launch_linear_gemm(a, s, &fits);
      } else {
        err = llmopt::launch_linear_gemm(a, s, &fits);
        if (!fits && M <= 64) err = llmopt::launch_linear_decode(a, s, &fits);
      }
      if (fits) return hip_status(err, "linear launch");
    }
    // Then the plain product into the workspace, and the combining kernel.
    if (!workspace || workspace_bytes < temp || reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
      return fail(LLMOPT_ERR_WORKSPACE, "this shape needs a workspace of at least %zu bytes",
                  temp + llmopt_q_linear_workspace_ex(M, N, K, bits, group_size, act_dtype));
    void* t = workspace;
    rc = run_linear(x, M, K, ldx, qweight, ldq, scales, zeros, bias, t, N, N, act_dtype, bits,
                    group_size, symmetric, signed_codes, static_cast<uint8_t*>(workspace) + temp,
                    workspace_bytes - temp, stream, algo, llmopt::kEpiNone);
    if (rc != LLMOPT_OK) return rc;
    return hip_status(llmopt::launch_swiglu_combine(t, N, y, ldy, M, N, act_dtype, s), "swiglu launch");
  }

  if (algo == LLMOPT_ALGO_DENSE || (algo == LLMOPT_ALGO_AUTO && dense_first(M, N, K, act_dtype, a.workspace,
                                                                               a.workspace_bytes))) {
    // Long batches: the weight dequantized into the workspace, then hipBLASLt's dense GEMM.
    err = llmopt::launch_linear_dense(a, s, &fits);
    if (fits) return hip_status(err, "dense linear");
    if (algo == LLMOPT_ALGO_DENSE) {
      const size_t need = llmopt::dense_workspace_bytes(N, K, act_dtype);
      if (!a.workspace || a.workspace_bytes < need || reinterpret_cast<uintptr_t>(a.workspace) % 256 != 0)
        return fail(LLMOPT_ERR_WORKSPACE, "the dense path needs a 256-byte aligned workspace of at least %zu bytes",
                    need);
      return fail(LLMOPT_ERR_UNSUPPORTED, "hipBLASLt offers no algorithm for M=%lld N=%lld K=%lld", (long long)M,
                  (long long)N, (long long)K);
    }
  }

  if (act_dtype == LLMOPT_DTYPE_F32 && algo == LLMOPT_ALGO_AUTO) {
    // fp32 activations: three bf16 pieces per token on the decode kernels (given the workspace
    // llmopt_q_linear_workspace_ex asks for), else the generic kernel below.
    err = llmopt::launch_linear_f32_pieces(a, s, &fits);
    if (fits) return hip_status(err, "linear launch");
  }

  switch (algo) {
    case LLMOPT_ALGO_AUTO: {
      bool gemm = gemm_first(M, K, N, a.group, bits);
      if (gemm && M <= kDecodeMaxTokens) {
        // The decode path's K-split kernel first, then the GEMM, which is worth it only with
        // its own K split; each needs its workspace.
        const size_t nx = llmopt::decode_workspace_bytes(M, N, K, a.group, bits);
        const size_t need = llmopt::gemm_workspace_bytes(M, N, K, a.group, a.fmt);
        const bool ws_nx = nx > 0 && a.workspace != nullptr && a.workspace_bytes >= nx;
        gemm = !ws_nx && need > 0 && a.workspace != nullptr && a.workspace_bytes >= need;
      }
      if (!gemm) {
        err = llmopt::launch_linear_decode(a, s, &fits);
        // A batch above the decode threshold that no decode kernel took (an alignment or a
        // workspace the planner assumed): the GEMMs before the generic kernel.
        if (!fits && M > kDecodeMaxTokens) err = llmopt::launch_linear_gemm(a, s, &fits);
        if (!fits && M > kDecodeMaxTokens) err = llmopt::launch_linear_prefill(a, s, &fits);
      } else {
        err = llmopt::launch_linear_gemm(a, s, &fits);
        if (!fits && M <= 64) err = llmopt::launch_linear_decode(a, s, &fits);
        if (!fits) err = llmopt::launch_linear_prefill(a, s, &fits);
      }
      if (!fits) err = llmopt::launch_linear_generic(a, s);
      break;
    }
    case LLMOPT_ALGO_GENERIC:
      err = llmopt::launch_linear_generic(a, s);
      break;
    case LLMOPT_ALGO_DECODE:
      err = llmopt::launch_linear_decode(a, s, &fits);
      if (!fits) return fail(LLMOPT_ERR_UNSUPPORTED, "decode kernel does not take these arguments");
      break;
    case LLMOPT_ALGO_PREFILL:
      err = llmopt::launch_linear_gemm(a, s, &fits);
      if (!fits) err = llmopt::launch_linear_prefill(a, s, &fits);
      if (!fits) return fail(LLMOPT_ERR_UNSUPPORTED, "prefill kernel does not take these arguments");
      break;
    default:
      return fail(LLMOPT_ERR_INVALID_ARG, "unknown algo %d", algo);
  }
  return hip_status(err, "linear launch");
}

// ---- the allocation-free linear's scratch ------------------------------------------------------
//
// llmopt_q_linear_noalloc takes its K-split partial sums from this file-scope device array
// instead of a caller's workspace. Each device the library runs on holds its own copy, of
// kNoAllocScratchBytes, until the process ends. Host code never uses the array's name as an
// address (on the host it is only a stand-in for the symbol): the device address of each
// device's copy comes from hipGetSymbolAddress, once per device, with that device current,
// and only that address is handed to kernels. Every call on a device shares its copy, so
// calls that overlap on one device (several streams, several threads) race on it; the
// kernels write every partial sum they later read, so nothing needs clearing between calls.
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) static uint8_t scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxDevices] = {};

// Device address of the current device's scratch (set up on the first call on that device).
int current_scratch(void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return hip_status(err, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(LLMOPT_ERR_UNSUPPORTED, "device %d beyond the scratch table", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_address[dev] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return hip_status(err, "hipGetSymbolAddress(scratch)");
    if (ptr == nullptr) return fail(LLMOPT_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_address[dev] = ptr;
  }
  *out = g_scratch_address[dev];
  return LLMOPT_OK;
}

}  // namespace

extern "C" {

int llmopt_q_abi_version(void) { return LLMOPT_QLINEAR_ABI_VERSION; }

const char* llmopt_q_last_error(void) { return g_last_error.c_str(); }

int llmopt_q_unpack(const uint8_t* packed, uint8_t* codes, int64_t rows, int64_t packed_cols,
                    int64_t columns, void* stream) {
  if (rows < 0 || packed_cols < 0 || columns < 0)
    return fail(LLMOPT_ERR_INVALID_ARG, "negative unpack shape");
  if (columns > 2 * packed_cols)
    return fail(LLMOPT_ERR_INVALID_ARG, "columns=%lld exceeds 2 * packed_cols=%lld",
                (long long)columns, (long long)(2 * packed_cols));
  if (rows > 0 && columns > 0 && (!packed || !codes))
    return fail(LLMOPT_ERR_INVALID_ARG, "null unpack pointer");
  return hip_status(llmopt::launch_unpack(packed, codes, rows, packed_cols, columns,
                                          static_cast<hipStream_t>(stream)),
                    "unpack launch");
}

int llmopt_q_dequant(const void* qweight, int64_t ldq, const float* scales, const float* zeros,
                     void* out, int out_dtype, int64_t N, int64_t K, int bits, int group_size,
                     int symmetric, int signed_codes, void* stream) {
  if (!valid_dtype(out_dtype)) return fail(LLMOPT_ERR_INVALID_ARG, "bad dtype code %d", out_dtype);
  llmopt::LinearArgs a{};
  const int rc = describe_weight(a, qweight, ldq, scales, zeros, N, K, bits, group_size,
                                 symmetric, signed_codes);
  if (rc != LLMOPT_OK) return rc;
  if (N > 0 && K > 0 && !out) return fail(LLMOPT_ERR_INVALID_ARG, "null output");
  return hip_status(llmopt::launch_dequant(a, out, out_dtype, static_cast<hipStream_t>(stream)),
                    "dequant launch");
}

int llmopt_q_quantize_rtn(const void* weight, int w_dtype, int64_t ldw, int64_t N, int64_t K, int bits,
                          int group_size, int symmetric, void* qweight, int64_t ldq, float* scales,
                          float* zeros, void* stream) {
  if (!valid_dtype(w_dtype)) return fail(LLMOPT_ERR_INVALID_ARG, "bad dtype code %d", w_dtype);
  // Quantizer validation (quantizers.py:252-255) and choose_qparams' divisibility check (:123-124).
  if (bits != 2 && bits != 4 && bits != 8) return fail(LLMOPT_ERR_INVALID_ARG, "unsupported bit width: %d", bits);
  if (N < 0 || K < 0) return fail(LLMOPT_ERR_INVALID_ARG, "negative shape N=%lld K=%lld", (long long)N, (long long)K);
  const int64_t group = group_size <= 0 ? K : group_size;
  if (K > 0 && K % group != 0)
    return fail(LLMOPT_ERR_INVALID_ARG, "in_features=%lld not divisible by group_size=%lld", (long long)K,
                (long long)group);
  if (bits < 8 && group % 2 != 0)  // pack_int4 needs whole bytes (quantizers.py:85-86)
    return fail(LLMOPT_ERR_INVALID_ARG, "4-bit packing requires an even number of columns");
  if (ldw < K) return fail(LLMOPT_ERR_INVALID_ARG, "weight row stride %lld < in_features %lld", (long long)ldw,
                           (long long)K);
  const int64_t need = bits == 8 ? K : K / 2;
  if (ldq < need)
    return fail(LLMOPT_ERR_INVALID_ARG, "packed row of %lld bytes cannot hold %lld columns", (long long)ldq,
                (long long)K);
  if (N == 0 || K == 0) return LLMOPT_OK;
  if (!weight || !qweight || !scales || !zeros) return fail(LLMOPT_ERR_INVALID_ARG, "null pointer argument");
  if (N * K / 8 >= (int64_t(1) << 38)) return fail(LLMOPT_ERR_UNSUPPORTED, "weight too large for one launch");
  llmopt::RtnArgs a{};
  a.w = weight;
  a.w_dtype = w_dtype;
  a.ldw = ldw;
  a.N = N;
  a.K = K;
  a.bits = bits;
  a.group = group;
  a.G = K / group;
  a.symmetric = symmetric ? 1 : 0;
  a.q = static_cast<uint8_t*>(qweight);
  a.ldq = ldq;
  a.scales = scales;
  a.zeros = zeros;
  return hip_status(llmopt::launch_quantize_rtn(a, static_cast<hipStream_t>(stream)), "quantize launch");
}

size_t llmopt_q_linear_workspace(int64_t M, int64_t N, int64_t K, int bits, int group_size) {
  // The GEMM's K split, and the decode path's kernels that split K over workgroups (5-64 tokens
  // on grids of fewer than 1024 tiles of 16 features); the other decode kernels reduce in LDS.
  // From 1024 tokens the dense weight and hipBLASLt's workspace, and at least the fused plan's
  // (what runs if hipBLASLt has no algorithm for the shape).
  if (M <= 0 || N <= 0 || K <= 0 || bits < 1 || bits > 8) return 0;
  const size_t fused = fused_workspace_bytes(M, N, K, bits, group_size);
  if (M < llmopt::dense_min_tokens(LLMOPT_DTYPE_BF16)) return fused;
  return std::max(fused, llmopt::dense_workspace_bytes(N, K, LLMOPT_DTYPE_BF16));
}

size_t llmopt_q_linear_workspace_ex(int64_t M, int64_t N, int64_t K, int bits, int group_size, int act_dtype) {
  if (act_dtype != LLMOPT_DTYPE_F32) return llmopt_q_linear_workspace(M, N, K, bits, group_size);
  if (M <= 0 || N <= 0 || K <= 0 || bits < 1 || bits > 8) return 0;
  const size_t pieces = llmopt::f32_workspace_bytes(M, N, K, group_size <= 0 ? K : group_size, bits);
  if (M < llmopt::dense_min_tokens(LLMOPT_DTYPE_F32)) return pieces;
  return std::max(pieces, llmopt::dense_workspace_bytes(N, K, LLMOPT_DTYPE_F32));
}

size_t llmopt_q_linear_dense_workspace(int64_t N, int64_t K, int act_dtype) {
  if (!valid_dtype(act_dtype)) return 0;
  return llmopt::dense_workspace_bytes(N, K, act_dtype);
}

int llmopt_q_linear_ex(const void* x, int64_t M, int64_t K, int64_t ldx, const void* qweight,
                       int64_t ldq, const float* scales, const float* zeros, const void* bias,
                       void* y, int64_t N, int64_t ldy, int act_dtype, int bits, int group_size,
                       int symmetric, int signed_codes, void* workspace, size_t workspace_bytes,
                       void* stream, int algo) {
  return run_linear(x, M, K, ldx, qweight, ldq, scales, zeros, bias, y, N, ldy, act_dtype, bits,
                    group_size, symmetric, signed_codes, workspace, workspace_bytes, stream, algo,
                    llmopt::kEpiNone);
}

size_t llmopt_q_linear_swiglu_workspace(int64_t M, int64_t N, int64_t K, int bits, int group_size) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const int64_t g = group_size <= 0 ? K : group_size;
  // Long batches: the [M, N] product and the two-pass path's workspace, then the combining kernel.
  if (M >= llmopt::dense_min_tokens(LLMOPT_DTYPE_BF16) && bits >= 1 && bits <= 8)
    return swiglu_temp_bytes(M, N, LLMOPT_DTYPE_BF16) + llmopt_q_linear_workspace(M, N, K, bits, group_size);
  const bool nibble = bits == 2 || bits == 4;
  // Sizes whose kernels apply the activation themselves (assuming aligned, contiguous tensors):
  // the decode path's partial sums where its plan splits K, else nothing.
  if (nibble && (M <= kDecodeMaxTokens || !gemm_first(M, K, N, g, bits)) && g % 128 == 0 && K % 128 == 0 &&
      (K / g) % 4 == 0 && (M <= 4 || K <= 8192))
    return M <= 64 ? llmopt::decode_workspace_bytes(M, N, K, g, bits) : 0;
  if (M > kDecodeMaxTokens && bits >= 1 && bits <= 8 && g % 32 == 0 && K % 64 == 0)
    return llmopt::gemm_workspace_bytes(M, N, K, g, bits == 8 ? llmopt::kByte : llmopt::kNibble);
  // Otherwise: the full [M, N] output, then the combining kernel.
  return swiglu_temp_bytes(M, N, LLMOPT_DTYPE_BF16) + llmopt_q_linear_workspace(M, N, K, bits, group_size);
}

size_t llmopt_q_linear_swiglu_workspace_ex(int64_t M, int64_t N, int64_t K, int bits, int group_size,
                                           int act_dtype) {
  if (act_dtype != LLMOPT_DTYPE_F32) return llmopt_q_linear_swiglu_workspace(M, N, K, bits, group_size);
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  // No fp32 kernel applies the activation itself: the product into the workspace, then the
  // combining kernel.
  return swiglu_temp_bytes(M, N, act_dtype) + llmopt_q_linear_workspace_ex(M, N, K, bits, group_size, act_dtype);
}

int llmopt_q_linear_swiglu(const void* x, int64_t M, int64_t K, int64_t ldx, const void* qweight,
                           int64_t ldq, const float* scales, const float* zeros, const void* bias,
                           void* y, int64_t N, int64_t ldy, int act_dtype, int bits, int group_size,
                           int symmetric, int signed_codes, void* workspace, size_t workspace_bytes,
                           void* stream) {
  if (N % 8 != 0)
    return fail(LLMOPT_ERR_INVALID_ARG, "fused gate/up rows N=%lld are not a multiple of 8", (long long)N);
  return run_linear(x, M, K, ldx, qweight, ldq, scales, zeros, bias, y, N, ldy, act_dtype, bits,
                    group_size, symmetric, signed_codes, workspace, workspace_bytes, stream,
                    LLMOPT_ALGO_AUTO, llmopt::kEpiSwiglu);
}

int llmopt_q_linear_deferred(const void* x, int64_t M, int64_t K, int64_t ldx, const void* qweight,
                             int64_t ldq, const float* scales, const float* zeros, const void* bias,
                             void* y, int64_t N, int64_t ldy, int act_dtype, int bits, int group_size,
                             int symmetric, int signed_codes, void* workspace, size_t workspace_bytes,
                             void* stream, int* planes) {
  if (!planes) return fail(LLMOPT_ERR_INVALID_ARG, "null planes pointer");
  return run_linear(x, M, K, ldx, qweight, ldq, scales, zeros, bias, y, N, ldy, act_dtype, bits,
                    group_size, symmetric, signed_codes, workspace, workspace_bytes, stream,
                    LLMOPT_ALGO_AUTO, llmopt::kEpiNone, planes);
}

int llmopt_q_linear(const void* x, int64_t M, int64_t K, int64_t ldx, const void* qweight,
                    int64_t ldq, const float* scales, const float* zeros, const void* bias,
                    void* y, int64_t N, int64_t ldy, int act_dtype, int bits, int group_size,
                    int symmetric, int signed_codes, void* workspace, size_t workspace_bytes,
                    void* stream) {
  return llmopt_q_linear_ex(x, M, K, ldx, qweight, ldq, scales, zeros, bias, y, N, ldy, act_dtype,
                            bits, group_size, symmetric, signed_codes, workspace, workspace_bytes,
                            stream, LLMOPT_ALGO_AUTO);
}

size_t llmopt_q_linear_noalloc_max_scratch(void) { return kNoAllocScratchBytes; }

int llmopt_q_linear_noalloc(const void* x, int64_t M, int64_t K, int64_t ldx, const void* qweight,
                            int64_t ldq, const float* scales, const float* zeros, const void* bias,
                            void* y, int64_t N, int64_t ldy, int act_dtype, int bits, int group_size,
                            int symmetric, int signed_codes, void* stream) {
  // The fused kernels' plan: the two-pass path's dense weight does not fit the scratch.
  const size_t need = fused_workspace_bytes(M, N, K, bits, group_size);
  if (need > kNoAllocScratchBytes)
    return fail(LLMOPT_ERR_WORKSPACE,
                "llmopt_q_linear_noalloc: M=%lld N=%lld K=%lld needs %zu bytes of scratch, beyond the %zu "
                "bytes of the static scratch; call llmopt_q_linear with a workspace",
                (long long)M, (long long)N, (long long)K, need, kNoAllocScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = current_scratch(&ws);
    if (rc != LLMOPT_OK) return rc;
  }
  return run_linear(x, M, K, ldx, qweight, ldq, scales, zeros, bias, y, N, ldy, act_dtype, bits,
                    group_size, symmetric, signed_codes, ws, ws ? need : 0, stream,
                    LLMOPT_ALGO_AUTO, llmopt::kEpiNone);
}

}  // extern "C"

namespace {

int describe_cache(llmopt::KvWriteArgs& a, void* key_cache, void* value_cache, int cache_dtype, int64_t num_blocks,
                   int64_t block_size, int64_t kv_heads, int64_t head_dim, const int32_t* block_ids, int64_t ldb) {
  if (!valid_dtype(cache_dtype)) return fail(LLMOPT_ERR_INVALID_ARG, "bad cache dtype code %d", cache_dtype);
  if (num_blocks < 1 || block_size < 1 || kv_heads < 1 || head_dim < 1 || ldb < 0)
    return fail(LLMOPT_ERR_INVALID_ARG, "bad cache geometry: blocks %lld, block_size %lld, kv_heads %lld, "
                "head_dim %lld, table width %lld", (long long)num_blocks, (long long)block_size, (long long)kv_heads,
                (long long)head_dim, (long long)ldb);
  a.key_cache = key_cache;
  a.value_cache = value_cache;
  a.cache_dtype = cache_dtype;
  a.num_blocks = num_blocks;
  a.block_size = block_size;
  a.kv_heads = kv_heads;
  a.head_dim = head_dim;
  a.block_ids = block_ids;
  a.ldb = ldb;
  return LLMOPT_OK;
}

// Work split for decode attention. Each (sequence, KV head) gets `parts` waves, about 2048 in
// all (two per SIMD), each with at least four 16-token tiles. Up to 8 of them (4 for groups of 16
// query heads, whose merge buffer in LDS is larger) form one workgroup and merge in LDS; beyond
// that the context is cut into `splits` workgroups, at most 64, which a second kernel merges.
struct DecodePlan {
  int splits;
  int waves;
  int64_t tiles_per_split;
};
DecodePlan plan_decode(int64_t num_seqs, int64_t kv_heads, int64_t group, int64_t ldb, int64_t block_size) {
  const int64_t tiles = (ldb * block_size + 15) / 16;
  const int64_t pairs = num_seqs * kv_heads;
  const int64_t want = pairs > 0 ? (2048 + pairs - 1) / pairs : 1;
  int64_t parts = (tiles + 3) / 4;
  if (parts > want) parts = want;
  if (parts < 1) parts = 1;
  const int wmax = group >= 16 ? 4 : 8;
  int waves = 1;
  while (waves < wmax && waves < parts) waves *= 2;
  int64_t splits = (parts + waves - 1) / waves;
  if (splits > 64) splits = 64;
  int64_t per = (tiles + splits - 1) / splits;
  if (per < 1) per = 1;
  splits = tiles > 0 ? (tiles + per - 1) / per : 1;  // no empty split
  return DecodePlan{int(splits), waves, per};
}

}  // namespace

extern "C" {

int llmopt_kv_write_decode(void* key_cache, void* value_cache, int cache_dtype, int64_t num_blocks,
                           int64_t block_size, int64_t kv_heads, int64_t head_dim, const int32_t* block_ids,
                           int64_t ldb, const int32_t* token_offsets, const void* keys, const void* values,
                           int src_dtype, int64_t src_seq_stride, int64_t num_seqs, void* stream) {
  llmopt::KvWriteArgs a{};
  int rc = describe_cache(a, key_cache, value_cache, cache_dtype, num_blocks, block_size, kv_heads, head_dim,
                          block_ids, ldb);
  if (rc != LLMOPT_OK) return rc;
  if (!valid_dtype(src_dtype)) return fail(LLMOPT_ERR_INVALID_ARG, "bad dtype code %d", src_dtype);
  if (num_seqs < 0) return fail(LLMOPT_ERR_INVALID_ARG, "negative sequence count");
  if (num_seqs == 0) return LLMOPT_OK;
  if (!key_cache || !value_cache || !block_ids || !token_offsets || !keys || !values)
    return fail(LLMOPT_ERR_INVALID_ARG, "null pointer argument");
  a.offsets = token_offsets;
  a.keys = keys;
  a.values = values;
  a.src_dtype = src_dtype;
  a.src_seq_stride = src_seq_stride;
  a.src_token_stride = 0;
  a.num_seqs = num_seqs;
  return hip_status(llmopt::launch_kv_write(a, 1, true, static_cast<hipStream_t>(stream)), "kv write launch");
}

int llmopt_kv_write(void* key_cache, void* value_cache, int cache_dtype, int64_t num_blocks, int64_t block_size,
                    int64_t kv_heads, int64_t head_dim, const int32_t* block_ids, int64_t ldb,
                    const int32_t* token_offsets, const void* keys, const void* values, int src_dtype,
                    int64_t src_seq_stride, int64_t src_token_stride, int64_t num_seqs, int64_t q_len,
                    void* stream) {
  llmopt::KvWriteArgs a{};
  int rc = describe_cache(a, key_cache, value_cache, cache_dtype, num_blocks, block_size, kv_heads, head_dim,
                          block_ids, ldb);
  if (rc != LLMOPT_OK) return rc;
  if (!valid_dtype(src_dtype)) return fail(LLMOPT_ERR_INVALID_ARG, "bad dtype code %d", src_dtype);
  if (num_seqs < 0 || q_len < 0) return fail(LLMOPT_ERR_INVALID_ARG, "negative sequence count or q_len");
  if (num_seqs == 0 || q_len == 0) return LLMOPT_OK;
  if (q_len > 65535 || num_seqs > 65535)
    return fail(LLMOPT_ERR_UNSUPPORTED, "q_len %lld x sequences %lld exceed one launch", (long long)q_len,
                (long long)num_seqs);
  if (!key_cache || !value_cache || !block_ids || !token_offsets || !keys || !values)
    return fail(LLMOPT_ERR_INVALID_ARG, "null pointer argument");
  a.offsets = token_offsets;
  a.keys = keys;
  a.values = values;
  a.src_dtype = src_dtype;
  a.src_seq_stride = src_seq_stride;
  a.src_token_stride = src_token_stride;
  a.num_seqs = num_seqs;
  return hip_status(llmopt::launch_kv_write(a, q_len, false, static_cast<hipStream_t>(stream)), "kv write launch");
}

size_t llmopt_paged_attention_workspace(int64_t num_seqs, int64_t num_heads, int64_t kv_heads, int64_t head_dim,
                                        int64_t ldb, int64_t block_size) {
  if (num_seqs <= 0 || num_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || ldb <= 0 || block_size <= 0) return 0;
  if (num_heads % kv_heads != 0) return 0;
  const DecodePlan plan = plan_decode(num_seqs, kv_heads, num_heads / kv_heads, ldb, block_size);
  if (plan.splits <= 1) return 0;
  return size_t(plan.splits) * size_t(num_seqs) * size_t(num_heads) * size_t(head_dim + 1) * sizeof(float);
}

}  // extern "C"

namespace {

// Checks and work split shared by the decode attention entry points; fills `a` (its launch fields
// included) and returns LLMOPT_OK, or the error to return. num_seqs == 0 returns LLMOPT_OK with
// a.num_seqs == 0 (nothing to launch).
int prepare_paged_decode(llmopt::PagedDecodeArgs& a, const void* query, int q_dtype, int64_t q_seq_stride,
                         const void* key_cache, const void* value_cache, int cache_dtype, int64_t num_blocks,
                         int64_t block_size, int64_t kv_heads, int64_t head_dim, const int32_t* block_ids,
                         int64_t ldb, const int32_t* context_lens, int64_t num_seqs, int64_t num_heads, float scale,
                         float softcap, void* out, void* workspace, size_t workspace_bytes) {
  if (!valid_dtype(q_dtype) || !valid_dtype(cache_dtype))
    return fail(LLMOPT_ERR_INVALID_ARG, "bad dtype code %d / %d", q_dtype, cache_dtype);
  if (num_seqs < 0 || num_heads < 1 || kv_heads < 1 || num_heads % kv_heads != 0)
    return fail(LLMOPT_ERR_INVALID_ARG, "num_heads %lld must be a positive multiple of kv_heads %lld",
                (long long)num_heads, (long long)kv_heads);
  if (num_blocks < 1 || block_size < 1 || ldb < 0 || head_dim < 1)
    return fail(LLMOPT_ERR_INVALID_ARG, "bad cache geometry");
  const int64_t group = num_heads / kv_heads;
  if (cache_dtype == LLMOPT_DTYPE_F32 || (head_dim != 64 && head_dim != 128) ||
      (group != 1 && group != 2 && group != 4 && group != 8 && group != 16))
    return fail(LLMOPT_ERR_UNSUPPORTED, "decode attention kernel: cache dtype %d, head_dim %lld, %lld heads per KV "
                "head", cache_dtype, (long long)head_dim, (long long)group);
  if (num_blocks * block_size * kv_heads * head_dim * 2 >= (int64_t(1) << 31) || num_seqs > 65535 ||
      kv_heads > 65535)
    return fail(LLMOPT_ERR_UNSUPPORTED, "cache layer (2 GiB at most) or batch too large for one launch");
  if (ldb >= (int64_t(1) << 31) / (block_size + 16))
    return fail(LLMOPT_ERR_UNSUPPORTED, "block table row of %lld blocks too long", (long long)ldb);
  if (q_seq_stride < num_heads * head_dim)
    return fail(LLMOPT_ERR_INVALID_ARG, "query row stride %lld < heads x head_dim", (long long)q_seq_stride);
  a = llmopt::PagedDecodeArgs{};
  if (num_seqs == 0) return LLMOPT_OK;
  if (!query || !key_cache || !value_cache || !block_ids || !context_lens || !out)
    return fail(LLMOPT_ERR_INVALID_ARG, "null pointer argument");
  if (reinterpret_cast<uintptr_t>(key_cache) % 16 != 0 || reinterpret_cast<uintptr_t>(value_cache) % 16 != 0)
    return fail(LLMOPT_ERR_UNSUPPORTED, "caches must be 16-byte aligned");
  a.query = query;
  a.q_dtype = q_dtype;
  a.q_seq_stride = q_seq_stride;
  a.key_cache = key_cache;
  a.value_cache = value_cache;
  a.cache_dtype = cache_dtype;
  a.num_blocks = num_blocks;
  a.block_size = block_size;
  a.kv_heads = kv_heads;
  a.head_dim = head_dim;
  a.block_ids = block_ids;
  a.ldb = ldb;
  a.context_lens = context_lens;
  a.num_seqs = num_seqs;
  a.num_heads = num_heads;
  a.scale = scale;
  a.softcap = softcap;
  a.out = out;
  a.out_dtype = q_dtype;
  const int64_t q_esize = q_dtype == LLMOPT_DTYPE_F32 ? 4 : 2;
  a.q_vec = reinterpret_cast<uintptr_t>(query) % 16 == 0 && (q_seq_stride * q_esize) % 16 == 0;
  const DecodePlan plan = plan_decode(num_seqs, kv_heads, group, ldb, block_size);
  int splits = plan.splits;
  int64_t per = plan.tiles_per_split;
  const size_t need = llmopt_paged_attention_workspace(num_seqs, num_heads, kv_heads, head_dim, ldb, block_size);
  if (splits > 1 && (workspace == nullptr || workspace_bytes < need ||
                     reinterpret_cast<uintptr_t>(workspace) % 16 != 0)) {
    splits = 1;
    per = (ldb * block_size + 15) / 16;
  }
  a.splits = splits;
  a.tiles_per_split = per < 1 ? 1 : per;
  a.waves = plan.waves;
  if (splits > 1) {
    a.part_out = static_cast<float*>(workspace);
    a.part_lse = a.part_out + size_t(splits) * size_t(num_seqs) * size_t(num_heads) * size_t(head_dim);
  }
  return LLMOPT_OK;
}

}  // namespace

extern "C" {

int llmopt_paged_attention_decode(const void* query, int q_dtype, int64_t q_seq_stride, const void* key_cache,
                                  const void* value_cache, int cache_dtype, int64_t num_blocks, int64_t block_size,
                                  int64_t kv_heads, int64_t head_dim, const int32_t* block_ids, int64_t ldb,
                                  const int32_t* context_lens, int64_t num_seqs, int64_t num_heads, float scale,
                                  float softcap, void* out, void* workspace, size_t workspace_bytes, void* stream) {
  llmopt::PagedDecodeArgs a{};
  const int rc = prepare_paged_decode(a, query, q_dtype, q_seq_stride, key_cache, value_cache, cache_dtype, num_blocks,
                                      block_size, kv_heads, head_dim, block_ids, ldb, context_lens, num_seqs,
                                      num_heads, scale, softcap, out, workspace, workspace_bytes);
  if (rc != LLMOPT_OK || a.num_seqs == 0) return rc;
  return hip_status(llmopt::launch_paged_decode(a, static_cast<hipStream_t>(stream)), "paged attention launch");
}

int llmopt_paged_attention_prefill(const void* query, int q_dtype, int64_t q_seq_stride, int64_t q_tok_stride,
                                   int64_t q_head_stride, const void* key_cache, const void* value_cache,
                                   int cache_dtype, int64_t num_blocks, int64_t block_size, int64_t kv_heads,
                                   int64_t head_dim, const int32_t* block_ids, int64_t ldb,
                                   const int32_t* context_lens, int64_t num_seqs, int64_t num_heads, int64_t q_len,
                                   float scale, float softcap, void* out, int64_t out_seq_stride,
                                   int64_t out_tok_stride, int64_t out_head_stride, void* stream) {
  if (q_len < 1 || q_len > 0x7FFFFFFF)
    return fail(LLMOPT_ERR_INVALID_ARG, "prefill attention: q_len %lld", (long long)q_len);
  if (q_tok_stride < 1 || q_head_stride < 1 || out_seq_stride < 1 || out_tok_stride < 1 || out_head_stride < 1)
    return fail(LLMOPT_ERR_INVALID_ARG, "prefill attention: strides must be positive");
  llmopt::PagedDecodeArgs a{};
  const int rc = prepare_paged_decode(a, query, q_dtype, q_seq_stride, key_cache, value_cache, cache_dtype, num_blocks,
                                      block_size, kv_heads, head_dim, block_ids, ldb, context_lens, num_seqs,
                                      num_heads, scale, softcap, out, nullptr, 0);
  if (rc != LLMOPT_OK || a.num_seqs == 0) return rc;
  const int64_t esize = q_dtype == LLMOPT_DTYPE_F32 ? 4 : 2;
  a.q_vec = a.q_vec && (q_tok_stride * esize) % 16 == 0 && (q_head_stride * esize) % 16 == 0;
  a.q_len = q_len;
  a.q_tok_stride = q_tok_stride;
  a.q_head_stride = q_head_stride;
  a.out_seq_stride = out_seq_stride;
  a.out_tok_stride = out_tok_stride;
  a.out_head_stride = out_head_stride;
  // Waves per workgroup, each with its own 16 / group query tokens over the same key tiles.
  a.splits = 1;
  a.waves = q_len >= 64 ? 4 : q_len >= 16 ? 2 : 1;
  return hip_status(llmopt::launch_paged_prefill(a, static_cast<hipStream_t>(stream)), "prefill attention launch");
}

int llmopt_paged_attention_decode_rope(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                                       int64_t ldv, const int64_t* positions, const float* cos_table,
                                       const float* sin_table, int64_t table_rows, int dtype, void* key_cache,
                                       void* value_cache, int64_t num_blocks, int64_t block_size, int64_t kv_heads,
                                       int64_t head_dim, const int32_t* block_ids, int64_t ldb,
                                       const int32_t* token_offsets, const int32_t* context_lens, int64_t num_seqs,
                                       int64_t num_heads, float scale, float softcap, void* out, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  if (dtype != LLMOPT_DTYPE_BF16 && dtype != LLMOPT_DTYPE_F16)
    return fail(LLMOPT_ERR_UNSUPPORTED, "fused rotary + decode attention: dtype %d (bf16 and fp16 only)", dtype);
  if (table_rows < 1 || kv_heads < 1 || ldk < kv_heads * head_dim || ldv < kv_heads * head_dim)
    return fail(LLMOPT_ERR_INVALID_ARG, "bad rotary table or k / v token stride");
  llmopt::PagedDecodeArgs a{};
  const int rc = prepare_paged_decode(a, q, dtype, ldq, key_cache, value_cache, dtype, num_blocks, block_size,
                                      kv_heads, head_dim, block_ids, ldb, context_lens, num_seqs, num_heads, scale,
                                      softcap, out, workspace, workspace_bytes);
  if (rc != LLMOPT_OK || a.num_seqs == 0) return rc;
  if (!k || !v || !positions || !cos_table || !sin_table || !token_offsets)
    return fail(LLMOPT_ERR_INVALID_ARG, "null rotary / cache-write pointer");
  auto aligned = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (!a.q_vec || !aligned(k) || !aligned(v) || ldk % 8 != 0 || ldv % 8 != 0 || !aligned(cos_table) ||
      !aligned(sin_table))
    return fail(LLMOPT_ERR_UNSUPPORTED, "fused rotary + decode attention: q, k, v rows and the rotary tables must "
                "be 16-byte aligned");
  a.rope = 1;
  a.new_k = k;
  a.new_v = v;
  a.ldk = ldk;
  a.ldv = ldv;
  a.positions = positions;
  a.cos_table = cos_table;
  a.sin_table = sin_table;
  a.table_rows = table_rows;
  a.offsets = token_offsets;
  a.k_store = key_cache;
  a.v_store = value_cache;
  return hip_status(llmopt::launch_paged_decode(a, static_cast<hipStream_t>(stream)), "paged attention launch");
}

int llmopt_rmsnorm(const void* x, int64_t ldx, const void* residual, int64_t ldr, void* h_out, int64_t ldh,
                   const void* weight, void* y, int64_t ldy, int64_t rows, int64_t hidden, float eps, int dtype,
                   void* stream) {
  if (dtype != LLMOPT_DTYPE_BF16 && dtype != LLMOPT_DTYPE_F16)
    return fail(LLMOPT_ERR_UNSUPPORTED, "rmsnorm kernel: dtype %d (bf16 and fp16 only)", dtype);
  if (rows < 0 || hidden < 1 || rows > 0x7FFFFFFF) return fail(LLMOPT_ERR_INVALID_ARG, "bad rmsnorm shape");
  if (rows == 0) return LLMOPT_OK;
  if (!x || !weight || !y || (residual && !h_out)) return fail(LLMOPT_ERR_INVALID_ARG, "null rmsnorm pointer");
  if (ldx < hidden || ldy < hidden || (residual && (ldr < hidden || ldh < hidden)))
    return fail(LLMOPT_ERR_INVALID_ARG, "rmsnorm row stride below hidden=%lld", (long long)hidden);
  auto aligned = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (hidden % 8 || ldx % 8 || ldy % 8 || (residual && (ldr % 8 || ldh % 8)) || !aligned(x) || !aligned(y) ||
      !aligned(weight) || (residual && (!aligned(residual) || !aligned(h_out))))
    return fail(LLMOPT_ERR_UNSUPPORTED, "rmsnorm kernel: needs hidden and row strides % 8 == 0, 16-byte aligned rows");
  llmopt::RmsNormArgs a{};
  a.x = x;
  a.residual = residual;
  a.h_out = h_out;
  a.weight = weight;
  a.y = y;
  a.rows = rows;
  a.hidden = hidden;
  a.ldx = ldx;
  a.ldr = ldr;
  a.ldh = ldh;
  a.ldy = ldy;
  a.eps = eps;
  a.dtype = dtype;
  return hip_status(llmopt::launch_rmsnorm(a, static_cast<hipStream_t>(stream)), "rmsnorm launch");
}

int llmopt_rmsnorm_planes(const float* planes, int64_t splits, const void* bias, const void* residual, int64_t ldr,
                          void* h_out, int64_t ldh, const void* weight, void* y, int64_t ldy, int64_t rows,
                          int64_t hidden, float eps, int dtype, void* stream) {
  if (dtype != LLMOPT_DTYPE_BF16 && dtype != LLMOPT_DTYPE_F16)
    return fail(LLMOPT_ERR_UNSUPPORTED, "rmsnorm kernel: dtype %d (bf16 and fp16 only)", dtype);
  if (rows < 0 || hidden < 1 || rows > 0x7FFFFFFF || splits < 1 || splits > 4096)
    return fail(LLMOPT_ERR_INVALID_ARG, "bad rmsnorm shape");
  if (rows == 0) return LLMOPT_OK;
  if (!planes || !residual || !h_out || !weight || !y) return fail(LLMOPT_ERR_INVALID_ARG, "null rmsnorm pointer");
  if (ldy < hidden || ldr < hidden || ldh < hidden)
    return fail(LLMOPT_ERR_INVALID_ARG, "rmsnorm row stride below hidden=%lld", (long long)hidden);
  auto aligned = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (hidden % 8 || ldy % 8 || ldr % 8 || ldh % 8 || !aligned(planes) || !aligned(y) || !aligned(weight) ||
      !aligned(residual) || !aligned(h_out))
    return fail(LLMOPT_ERR_UNSUPPORTED, "rmsnorm kernel: needs hidden and row strides % 8 == 0, 16-byte aligned rows");
  llmopt::RmsNormArgs a{};
  a.planes = planes;
  a.splits = splits;
  a.plane_bias = bias;
  a.residual = residual;
  a.h_out = h_out;
  a.weight = weight;
  a.y = y;
  a.rows = rows;
  a.hidden = hidden;
  a.ldx = hidden;
  a.ldr = ldr;
  a.ldh = ldh;
  a.ldy = ldy;
  a.eps = eps;
  a.dtype = dtype;
  return hip_status(llmopt::launch_rmsnorm(a, static_cast<hipStream_t>(stream)), "rmsnorm launch");
}

int llmopt_argmax_rows(const void* x, int dtype, int64_t rows, int64_t cols, int64_t ldx, int64_t* out,
                       void* stream) {
  if (!valid_dtype(dtype)) return fail(LLMOPT_ERR_INVALID_ARG, "bad dtype code %d", dtype);
  if (rows < 0 || rows > 0x7FFFFFFF || cols < 1 || ldx < cols)
    return fail(LLMOPT_ERR_INVALID_ARG, "bad argmax shape: rows %lld, cols %lld, ldx %lld", (long long)rows,
                (long long)cols, (long long)ldx);
  if (rows == 0) return LLMOPT_OK;
  if (!x || !out) return fail(LLMOPT_ERR_INVALID_ARG, "null argmax pointer");
  const int64_t esize = dtype == LLMOPT_DTYPE_F32 ? 4 : 2;
  llmopt::ArgmaxArgs a{};
  a.x = x;
  a.dtype = dtype;
  a.rows = rows;
  a.cols = cols;
  a.ldx = ldx;
  a.vec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && (ldx * esize) % 16 == 0;
  a.out = out;
  return hip_status(llmopt::launch_argmax_rows(a, static_cast<hipStream_t>(stream)), "argmax launch");
}

int llmopt_rope(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv, void* q_out,
                void* k_out, void* v_out, const int64_t* positions, const float* cos_table, const float* sin_table,
                int64_t table_rows, int64_t tokens, int64_t heads, int64_t kv_heads, int64_t head_dim, int dtype,
                void* stream) {
  if (dtype != LLMOPT_DTYPE_BF16 && dtype != LLMOPT_DTYPE_F16)
    return fail(LLMOPT_ERR_UNSUPPORTED, "rope kernel: dtype %d (bf16 and fp16 only)", dtype);
  if (tokens < 0 || tokens > 0x7FFFFFFF || heads < 1 || kv_heads < 0 || head_dim < 2 || head_dim % 2 ||
      table_rows < 1)
    return fail(LLMOPT_ERR_INVALID_ARG, "bad rope shape");
  if (tokens == 0) return LLMOPT_OK;
  if (!q || !q_out || !positions || !cos_table || !sin_table || (kv_heads > 0 && (!k || !k_out)))
    return fail(LLMOPT_ERR_INVALID_ARG, "null rope pointer");
  if (ldq < heads * head_dim || (kv_heads > 0 && ldk < kv_heads * head_dim))
    return fail(LLMOPT_ERR_INVALID_ARG, "rope token stride below heads x head_dim");
  if (v && (!v_out || ldv < kv_heads * head_dim)) return fail(LLMOPT_ERR_INVALID_ARG, "bad rope v arguments");
  llmopt::RopeArgs a{};
  a.q = q;
  a.k = k;
  a.q_out = q_out;
  a.k_out = k_out;
  a.v = kv_heads > 0 ? v : nullptr;
  a.v_out = v_out;
  a.ldv = ldv;
  a.positions = positions;
  a.cos_table = cos_table;
  a.sin_table = sin_table;
  a.table_rows = table_rows;
  a.tokens = tokens;
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.head_dim = head_dim;
  a.ldq = ldq;
  a.ldk = ldk;
  a.dtype = dtype;
  auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  a.vec = head_dim % 16 == 0 && ldq % 8 == 0 && al(q) && al(q_out) && al(cos_table) && al(sin_table) &&
          (kv_heads == 0 || (ldk % 8 == 0 && al(k) && al(k_out))) && (!a.v || (ldv % 8 == 0 && al(v) && al(v_out)));
  return hip_status(llmopt::launch_rope(a, static_cast<hipStream_t>(stream)), "rope launch");
}

int llmopt_rope_kv_write_decode(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                                void* q_out, const int64_t* positions, const float* cos_table,
                                const float* sin_table, int64_t table_rows, int64_t seqs, int64_t heads,
                                int64_t kv_heads, int64_t head_dim, int dtype, void* key_cache, void* value_cache,
                                int64_t num_blocks, int64_t block_size, const int32_t* block_ids, int64_t ldb,
                                const int32_t* token_offsets, void* stream) {
  if (dtype != LLMOPT_DTYPE_BF16 && dtype != LLMOPT_DTYPE_F16)
    return fail(LLMOPT_ERR_UNSUPPORTED, "rope kernel: dtype %d (bf16 and fp16 only)", dtype);
  if (seqs < 0 || seqs > 0x7FFFFFFF || heads < 1 || kv_heads < 1 || head_dim < 2 || head_dim % 2 ||
      table_rows < 1 || num_blocks < 1 || block_size < 1 || ldb < 1)
    return fail(LLMOPT_ERR_INVALID_ARG, "bad rope / cache shape");
  if (seqs == 0) return LLMOPT_OK;
  if (!q || !k || !v || !q_out || !positions || !cos_table || !sin_table || !key_cache || !value_cache ||
      !block_ids || !token_offsets)
    return fail(LLMOPT_ERR_INVALID_ARG, "null rope / cache pointer");
  if (ldq < heads * head_dim || ldk < kv_heads * head_dim || ldv < kv_heads * head_dim)
    return fail(LLMOPT_ERR_INVALID_ARG, "rope token stride below heads x head_dim");
  llmopt::RopeArgs a{};
  a.q = q;
  a.k = k;
  a.q_out = q_out;
  a.v = v;
  a.ldv = ldv;
  a.positions = positions;
  a.cos_table = cos_table;
  a.sin_table = sin_table;
  a.table_rows = table_rows;
  a.tokens = seqs;
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.head_dim = head_dim;
  a.ldq = ldq;
  a.ldk = ldk;
  a.dtype = dtype;
  a.key_cache = key_cache;
  a.value_cache = value_cache;
  a.block_ids = block_ids;
  a.offsets = token_offsets;
  a.ldb = ldb;
  a.num_blocks = num_blocks;
  a.block_size = block_size;
  return hip_status(llmopt::launch_rope(a, static_cast<hipStream_t>(stream)), "rope launch");
}

}  // extern "C"
