// fp32 activations on the bf16 decode kernels: QuantLinear.forward with compute_dtype float32
// (src/llmopt/quantization/quant_linear.py:93-113; the reference engine quantizes a float32 model,
// engine/llm_engine.py:258-264, and QuantLinear takes its layer's dtype, quant_linear.py:199-201).
//
// Each fp32 activation is split into three bf16 pieces, x = hi + mid + lo, exactly: hi is x
// rounded to bf16, mid the rounded remainder, lo the rest, and the remainders are exact in fp32
// (an fp32 significand has 24 bits, a bf16 one 8). The pieces of token m become rows 3m, 3m + 1,
// 3m + 2 of a bf16 batch, which the decode kernels multiply with the packed weight as they do any
// bf16 batch: codes are exact MFMA operands, products of bf16 values are exact in fp32, sums are
// fp32, and the group's scale is applied in fp32. The kernels write those three rows' sums in
// fp32 (LinearArgs::out_f32), and the combining kernel adds them, in a fixed order, with the
// bias: y = (t_hi + t_mid) + t_lo + b, an fp32 result within fp32 rounding of the reference's
// fp32 dequantize-then-F.linear. The weight is streamed once per chunk of up to 21 tokens
// (63 rows, the decode kernels' limit of 64; 16 tokens with groups of 64), so the memory-bound
// cost is that of a bf16 batch three times as tall.
#include <algorithm>

#include "qcommon.hpp"
#include "qkernels.hpp"

namespace llmopt {
namespace {

constexpr int kThreads = 256;
// Tokens per decode launch: 3 x 21 = 63 piece rows; with groups of 64, 3 x 16 = 48 (the
// K-sliced kernel's two-group form stops at 48 rows).
int64_t chunk_tokens(int64_t group) { return group == 64 ? 16 : 21; }

// xs[3m + p][k] = piece p of x[m][k]. Four columns per thread (16-byte loads where aligned).
__global__ void __launch_bounds__(kThreads) split_pieces_kernel(const float* x, int64_t ldx, uint16_t* xs,
                                                                int64_t M, int64_t K) {
  const int64_t kq = (K + 3) / 4;
  const int64_t e = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= M * kq) return;
  const int64_t m = e / kq;
  const int64_t k0 = (e - m * kq) * 4;
  const float* src = x + m * ldx + k0;
  uint16_t* d0 = xs + (3 * m) * K + k0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (k0 + j >= K) break;
    const float v = src[j];
    const uint16_t hi = f32_to_bf16_rne(v);
    const float r1 = v - bf16_to_f32(hi);  // exact
    const uint16_t mid = f32_to_bf16_rne(r1);
    const float r2 = r1 - bf16_to_f32(mid);  // exact
    d0[j] = hi;
    d0[K + j] = mid;
    d0[2 * K + j] = f32_to_bf16_rne(r2);  // exact for normal x
  }
}

// y[m][n] = (t[3m][n] + t[3m + 1][n]) + t[3m + 2][n] + bias[n], rows m0 .. m0 + rows of y.
__global__ void __launch_bounds__(kThreads) combine_pieces_kernel(const float* t, int64_t N, const float* bias,
                                                                  float* y, int64_t ldy, int64_t rows) {
  const int64_t e = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= rows * N) return;
  const int64_t m = e / N;
  const int64_t n = e - m * N;
  const float* r = t + 3 * m * N + n;
  float v = (r[0] + r[N]) + r[2 * N];
  if (bias) v += bias[n];
  y[m * ldy + n] = v;
}

// The same from a K-sliced launch's partial sums P[s][3 rows][N] (slices not yet added): each
// piece row's slices in slice order, as the split-K reduction adds them, then the pieces as above
// -- one kernel instead of the reduction and the combining kernel, with the same sums.
__global__ void __launch_bounds__(kThreads) combine_slices_kernel(const float* partials, int splits, int64_t N,
                                                                  const float* bias, float* y, int64_t ldy,
                                                                  int64_t rows) {
  const int64_t e = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= rows * N) return;
  const int64_t m = e / N;
  const int64_t n = e - m * N;
  const size_t plane = size_t(3 * rows) * size_t(N);
  const float* r = partials + size_t(3 * m) * size_t(N) + n;
  float t[3] = {r[0], r[N], r[2 * N]};
#pragma unroll 4
  for (int s = 1; s < splits; ++s) {
    const float* q = r + size_t(s) * plane;
    t[0] += q[0];
    t[1] += q[N];
    t[2] += q[2 * N];
  }
  float v = (t[0] + t[1]) + t[2];
  if (bias) v += bias[n];
  y[m * ldy + n] = v;
}

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

struct F32Plan {
  int64_t chunk = 0;   // tokens per decode launch
  size_t xs = 0, t = 0, inner = 0;
  size_t total() const { return xs + t + inner; }
};

F32Plan plan_f32(int64_t M, int64_t N, int64_t K, int64_t group, int bits) {
  F32Plan p;
  const int64_t most = chunk_tokens(group);
  const int64_t chunks = (M + most - 1) / most;
  p.chunk = (M + chunks - 1) / chunks;
  const int64_t last = M - (chunks - 1) * p.chunk;
  p.xs = align256(size_t(3) * M * K * 2);
  p.t = align256(size_t(3) * p.chunk * N * 4);
  p.inner = std::max(decode_workspace_bytes(3 * p.chunk, N, K, group, bits),
                     decode_workspace_bytes(3 * last, N, K, group, bits));
  return p;
}

}  // namespace

size_t f32_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group, int bits) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return plan_f32(M, N, K, group, bits).total();
}

hipError_t launch_linear_f32_pieces(const LinearArgs& a, hipStream_t stream, bool* fits) {
  *fits = false;
  if (a.act != kDtF32 || a.epilogue != kEpiNone || a.M < 1 || a.K < 1) return hipSuccess;
  // One or two tokens: the one-shot kernel splits and sums the pieces itself.
  const hipError_t e1 = launch_linear_oneshot_f32(a, stream, fits);
  if (*fits) return e1;
  const F32Plan p = plan_f32(a.M, a.N, a.K, a.group, a.bits);
  if (!a.workspace || a.workspace_bytes < p.total() || reinterpret_cast<uintptr_t>(a.workspace) % 256 != 0)
    return hipSuccess;
  if (3 * a.M * a.K >= (int64_t(1) << 40)) return hipSuccess;
  uint8_t* ws = static_cast<uint8_t*>(a.workspace);
  uint16_t* xs = reinterpret_cast<uint16_t*>(ws);
  float* t = reinterpret_cast<float*>(ws + p.xs);
  void* inner = p.inner ? ws + p.xs + p.t : nullptr;

  // The bf16 batch of one chunk: its piece rows, fp32 sums into t, no bias, no epilogue.
  auto chunk_args = [&](int64_t m0, int64_t rows) {
    LinearArgs b = a;
    b.x = xs + 3 * m0 * a.K;
    b.ldx = a.K;
    b.M = 3 * rows;
    b.act = kDtBf16;
    b.bias = nullptr;
    b.y = t;
    b.ldy = a.N;
    b.out_f32 = 1;
    b.workspace = inner;
    b.workspace_bytes = p.inner;
    b.defer_reduce = 1;  // a K-sliced plan's slices are added by the combining kernel below
    b.deferred_planes = nullptr;
    return b;
  };
  // A chunk whose shape the decode path refuses (an alignment or a format it does not take)
  // runs the generic kernel on its fp32 rows instead.
  *fits = true;
  const int64_t kq = (a.K + 3) / 4;
  hipLaunchKernelGGL(split_pieces_kernel, dim3(unsigned((a.M * kq + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     stream, static_cast<const float*>(a.x), a.ldx, xs, a.M, a.K);
  hipError_t err = hipGetLastError();
  for (int64_t m0 = 0; m0 < a.M && err == hipSuccess; m0 += p.chunk) {
    const int64_t rows = std::min(p.chunk, a.M - m0);
    LinearArgs b = chunk_args(m0, rows);
    int planes = 0;
    b.deferred_planes = &planes;
    bool taken = false;
    err = launch_linear_decode(b, stream, &taken);
    if (err != hipSuccess) break;
    if (!taken) {
      LinearArgs g = a;
      g.x = static_cast<const float*>(a.x) + m0 * a.ldx;
      g.y = static_cast<float*>(a.y) + m0 * a.ldy;
      g.M = rows;
      err = launch_linear_generic(g, stream);
      continue;
    }
    const dim3 grid(unsigned((rows * a.N + kThreads - 1) / kThreads));
    if (planes > 0)
      hipLaunchKernelGGL(combine_slices_kernel, grid, dim3(kThreads), 0, stream, static_cast<const float*>(inner),
                         planes, a.N, static_cast<const float*>(a.bias), static_cast<float*>(a.y) + m0 * a.ldy,
                         a.ldy, rows);
    else
      hipLaunchKernelGGL(combine_pieces_kernel, grid, dim3(kThreads), 0, stream, t, a.N,
                         static_cast<const float*>(a.bias), static_cast<float*>(a.y) + m0 * a.ldy, a.ldy, rows);
    err = hipGetLastError();
  }
  return err;
}

}  // namespace llmopt
