// C ABI of libllmopt_qlinear.so (declared in include/llmopt_qlinear.h).
//
// Validates arguments the way the reference's torch code would reject them, fills the
// kernel argument block and picks the kernel: the MFMA skinny GEMM for M <= 64, the MFMA
// LDS-dequant GEMM for larger M, and the generic kernel for shapes, alignments or dtypes
// the fast kernels do not take. Error text is kept per host thread.
#include <stdarg.h>
#include <stdio.h>

#include <string>

#include "../../include/llmopt_qlinear.h"
#include "qcommon.hpp"
#include "qkernels.hpp"

namespace {

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


size_t swiglu_temp_bytes(int64_t M, int64_t N) { return (size_t(M) * size_t(N) * 4 + 255) / 256 * 256; }

// Dispatch shared by llmopt_q_linear_ex and llmopt_q_linear_swiglu. With the SwiGLU epilogue,
// `y` is [M, N/2]; kernels that cannot apply it themselves write the full [M, N] product into
// the workspace and a combining kernel finishes.
int run_linear(const void* x, int64_t M, int64_t K, int64_t ldx, const void* qweight, int64_t ldq,
               const float* scales, const float* zeros, const void* bias, void* y, int64_t N,
               int64_t ldy, int act_dtype, int bits, int group_size, int symmetric, int signed_codes,
               void* workspace, size_t workspace_bytes, void* stream, int algo, int epilogue) {
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
  hipStream_t s = static_cast<hipStream_t>(stream);

  if (K == 0 && epilogue == llmopt::kEpiNone) {
    // An empty reduction: the reference's F.linear returns the bias (or zeros).
    a.K = 0;
    return hip_status(llmopt::launch_linear_generic(a, s), "linear launch");
  }

  bool fits = false;
  hipError_t err = hipSuccess;
  if (epilogue != llmopt::kEpiNone) {
    // Kernels with the fused epilogue first.
    if (K > 0 && algo == LLMOPT_ALGO_AUTO) {
      if (M <= 64)
        err = llmopt::launch_linear_decode(a, s, &fits);
      else
        err = llmopt::launch_linear_gemm(a, s, &fits);
      if (fits) return hip_status(err, "linear launch");
    }
    // Then the plain product into the workspace, and the combining kernel.
    const size_t temp = swiglu_temp_bytes(M, N);
    if (!workspace || workspace_bytes < temp || reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
      return fail(LLMOPT_ERR_WORKSPACE, "this shape needs a workspace of at least %zu bytes",
                  temp + llmopt_q_linear_workspace(M, N, K, bits, group_size));
    void* t = workspace;
    rc = run_linear(x, M, K, ldx, qweight, ldq, scales, zeros, bias, t, N, N, act_dtype, bits,
                    group_size, symmetric, signed_codes, static_cast<uint8_t*>(workspace) + temp,
                    workspace_bytes - temp, stream, algo, llmopt::kEpiNone);
    if (rc != LLMOPT_OK) return rc;
    return hip_status(llmopt::launch_swiglu_combine(t, N, y, ldy, M, N, act_dtype, s), "swiglu launch");
  }

  switch (algo) {
    case LLMOPT_ALGO_AUTO:
      if (M <= 64) {
        err = llmopt::launch_linear_decode(a, s, &fits);
      } else {
        err = llmopt::launch_linear_gemm(a, s, &fits);
        if (!fits) err = llmopt::launch_linear_prefill(a, s, &fits);
      }
      if (!fits) err = llmopt::launch_linear_generic(a, s);
      break;
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
  // Only the prefill GEMM (M > 64) splits K; the decode kernels reduce in LDS.
  if (M <= 64 || N <= 0 || K <= 0 || bits < 1 || bits > 8) return 0;
  const int64_t g = group_size <= 0 ? K : group_size;
  return llmopt::gemm_workspace_bytes(M, N, K, g, bits == 8 ? llmopt::kByte : llmopt::kNibble);
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
  const bool nibble = bits == 2 || bits == 4;
  // Sizes whose kernels apply the activation themselves (assuming aligned, contiguous tensors).
  if (nibble && M <= 64 && g % 128 == 0 && K % 128 == 0 && (K / g) % 4 == 0 && (M <= 4 || K <= 8192))
    return 0;
  if (M > 64 && bits >= 1 && bits <= 8 && g % 32 == 0 && K % 64 == 0)
    return llmopt::gemm_workspace_bytes(M, N, K, g, bits == 8 ? llmopt::kByte : llmopt::kNibble);
  // Otherwise: the full [M, N] output in fp32-sized slots, then the combining kernel.
  return swiglu_temp_bytes(M, N) + llmopt_q_linear_workspace(M, N, K, bits, group_size);
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

int llmopt_q_linear(const void* x, int64_t M, int64_t K, int64_t ldx, const void* qweight,
                    int64_t ldq, const float* scales, const float* zeros, const void* bias,
                    void* y, int64_t N, int64_t ldy, int act_dtype, int bits, int group_size,
                    int symmetric, int signed_codes, void* workspace, size_t workspace_bytes,
                    void* stream) {
  return llmopt_q_linear_ex(x, M, K, ldx, qweight, ldq, scales, zeros, bias, y, N, ldy, act_dtype,
                            bits, group_size, symmetric, signed_codes, workspace, workspace_bytes,
                            stream, LLMOPT_ALGO_AUTO);
}

}  // extern "C"
