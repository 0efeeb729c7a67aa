// Generic quantized linear: any shape, alignment, group size, storage format and activation
// dtype (fp32 included). It follows the reference's QuantLinear.forward literally
// (src/llmopt/quantization/quant_linear.py:93-113): each weight is dequantized exactly,
// rounded to the compute dtype as the reference's cached dense weight is, and multiplied
// with fp32 accumulation. One wave owns one output feature and up to kRows activation rows;
// lanes stride over K and reduce with cross-lane shuffles.
#include "qcommon.hpp"
#include "qkernels.hpp"

namespace llmopt {
namespace {

constexpr int kWaves = 4;
constexpr int kRows = 8;

template <class Act>
__global__ void __launch_bounds__(kWaves * 64) qlinear_generic_kernel(const LinearArgs a) {
  using Raw = typename Act::raw;
  const int lane = threadIdx.x & 63;
  const int64_t n = int64_t(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (n >= a.N) return;
  const int64_t m0 = int64_t(blockIdx.y) * kRows;
  const Raw* x = static_cast<const Raw*>(a.x);
  const uint8_t* row = a.qw + n * a.ldq;
  const float* srow = a.scales + n * a.G;
  const float* zrow = a.symmetric ? nullptr : a.zeros + n * a.G;

  float acc[kRows];
#pragma unroll
  for (int i = 0; i < kRows; ++i) acc[i] = 0.0f;

  for (int64_t k = lane; k < a.K; k += 64) {
    const int64_t g = k / a.group;
    const float q = code_value(row, k, a.fmt, a.signed_codes);
    const float z = zrow ? zrow[g] : a.zero_const;
    // The dense weight as the reference caches it: fp32 dequant, then compute dtype.
    const float w = Act::load(Act::store(dequant_exact(q, z, srow[g])));
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      if (m0 + i < a.M) acc[i] = __builtin_fmaf(w, Act::load(x[(m0 + i) * a.ldx + k]), acc[i]);
    }
  }

#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    float v = acc[i];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    acc[i] = v;
  }
  if (lane < kRows && m0 + lane < a.M) {
    float v = 0.0f;
#pragma unroll
    for (int i = 0; i < kRows; ++i) v = (lane == i) ? acc[i] : v;
    if (a.bias) v += Act::load(static_cast<const Raw*>(a.bias)[n]);
    static_cast<Raw*>(a.y)[(m0 + lane) * a.ldy + n] = Act::store(v);
  }
}

}  // namespace

hipError_t launch_linear_generic(const LinearArgs& a, hipStream_t stream) {
  if (a.M == 0 || a.N == 0) return hipSuccess;
  const int64_t gx = (a.N + kWaves - 1) / kWaves;
  const int64_t gy = (a.M + kRows - 1) / kRows;
  if (gx > 0x7FFFFFFF || gy > 65535) return hipErrorInvalidValue;
  const dim3 grid{unsigned(gx), unsigned(gy), 1u};
  const dim3 block(kWaves * 64);
  switch (a.act) {
    case kDtF32:
      hipLaunchKernelGGL(qlinear_generic_kernel<ActF32>, grid, block, 0, stream, a);
      break;
    case kDtF16:
      hipLaunchKernelGGL(qlinear_generic_kernel<ActF16>, grid, block, 0, stream, a);
      break;
    case kDtBf16:
      hipLaunchKernelGGL(qlinear_generic_kernel<ActBf16>, grid, block, 0, stream, a);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace llmopt
