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
};

// Each launcher returns hipSuccess or the launch error; `why` is set when the arguments do not
// fit the kernel (then hipErrorInvalidValue is returned and nothing is launched).
hipError_t launch_unpack(const uint8_t* packed, uint8_t* codes, int64_t rows, int64_t packed_cols,
                         int64_t columns, hipStream_t stream);
hipError_t launch_dequant(const LinearArgs& a, void* out, int out_dtype, hipStream_t stream);
hipError_t launch_linear_generic(const LinearArgs& a, hipStream_t stream);
// Decode and prefill report `fits = false` (and launch nothing) when the shape, alignment or
// dtype is outside what the kernel handles.
hipError_t launch_linear_decode(const LinearArgs& a, hipStream_t stream, bool* fits);
hipError_t launch_linear_prefill(const LinearArgs& a, hipStream_t stream, bool* fits);
hipError_t launch_linear_gemm(const LinearArgs& a, hipStream_t stream, bool* fits);
// Workspace the prefill GEMM's split-K plan uses for these sizes (0 when it does not split).
size_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group);

}  // namespace llmopt
