// Prefill-regime quantized linear (large M): an MFMA GEMM whose weight tiles are
// dequantized into LDS.
//
// Replaces QuantLinear.forward (src/llmopt/quantization/quant_linear.py:93-113) for long
// batches. The reference dequantizes the whole weight to a dense compute-dtype matrix and
// calls F.linear; here each BN x 64 weight tile is read packed from HBM, dequantized in
// registers with the reference's exact fp32 arithmetic ((q - z) * s, one rounding, then a
// round-to-nearest-even cast to bf16/fp16), written to LDS, and consumed by
// v_mfma_f32_32x32x16_{bf16,f16} together with the matching activation tile. The dense
// weight exists only as a 64-column slice in LDS.
//
// Block tile BM x BN x 64, 256 threads = 4 waves in a 2x2 grid, each wave (BM/2) x (BN/2)
// built from 32x32 MFMA tiles. LDS holds two stages (double buffering), rows padded by 16
// bytes so the 16-byte fragment reads of 16 consecutive rows hit distinct banks. Tiles are
// ordered in column groups so workgroups that run together share activation and weight
// tiles in L2, and the id space is split evenly over the 8 XCDs.
#include "qcommon.hpp"
#include "qkernels.hpp"

namespace llmopt {
namespace {

constexpr int kBK = 64;
constexpr int kStride = kBK + 8;  // LDS row stride in 16-bit elements
constexpr int kThreads = 256;
constexpr int kGroupM = 8;

template <class Act>
struct Mfma32;
template <>
struct Mfma32<ActBf16> {
  __device__ static f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static uint32_t pack(float lo, float hi) {
    return uint32_t(__builtin_bit_cast(uint16_t, __bf16(lo))) |
           (uint32_t(__builtin_bit_cast(uint16_t, __bf16(hi))) << 16);
  }
};
template <>
struct Mfma32<ActF16> {
  __device__ static f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static uint32_t pack(float lo, float hi) {
    return uint32_t(f32_to_f16_rne(lo)) | (uint32_t(f32_to_f16_rne(hi)) << 16);
  }
};

// Eight dequantized weights -> one 16-byte LDS store.
template <class Act>
__device__ __forceinline__ u32x4 pack8(const float (&v)[8]) {
  u32x4 r;
  r.x = Mfma32<Act>::pack(v[0], v[1]);
  r.y = Mfma32<Act>::pack(v[2], v[3]);
  r.z = Mfma32<Act>::pack(v[4], v[5]);
  r.w = Mfma32<Act>::pack(v[6], v[7]);
  return r;
}

template <class Act, int FMT, int BM, int BN>
__global__ void __launch_bounds__(kThreads)
    qlinear_prefill_kernel(const LinearArgs a, int tiles_m, int tiles_n, uint32_t group_magic) {
  using Raw = typename Act::raw;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  // Activation tile: BM rows x 8 pieces of 16 bytes.
  constexpr int kXLoads = BM * 8 / kThreads;
  // Weight tile: BN rows x (32 or 64) packed bytes in 16-byte pieces.
  constexpr int kPiecesPerRow = FMT == kNibble ? 2 : 4;
  constexpr int kPieceK = kBK / kPiecesPerRow;  // codes per piece
  constexpr int kWLoads = BN * kPiecesPerRow / kThreads;
  static_assert(kXLoads * kThreads == BM * 8, "activation tile split");
  static_assert(kWLoads * kThreads == BN * kPiecesPerRow, "weight tile split");

  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (BM + BN) * kStride];

  // Tile order: split ids evenly over the XCDs, then walk kGroupM row-tiles per column sweep.
  int bid = blockIdx.x;
  const int nblk = gridDim.x;
  if (nblk % 8 == 0) bid = (bid % 8) * (nblk / 8) + bid / 8;
  const int per_group = kGroupM * tiles_n;
  const int first_m = (bid / per_group) * kGroupM;
  const int rows_in_group = min(tiles_m - first_m, kGroupM);
  const int tm = first_m + (bid % per_group) % rows_in_group;
  const int tn = (bid % per_group) / rows_in_group;
  const int64_t m0 = int64_t(tm) * BM;
  const int64_t n0 = int64_t(tn) * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;

  // Per-thread global sources.
  const Raw* xsrc[kXLoads];
  bool xok[kXLoads];
  int xdst[kXLoads];
#pragma unroll
  for (int i = 0; i < kXLoads; ++i) {
    const int e = tid + kThreads * i;
    const int row = e >> 3;
    const int piece = e & 7;
    const int64_t m = m0 + row;
    xok[i] = m < a.M;
    xsrc[i] = static_cast<const Raw*>(a.x) + (xok[i] ? m : 0) * a.ldx + piece * 8;
    xdst[i] = row * kStride + piece * 8;
  }
  const uint8_t* wsrc[kWLoads];
  int64_t wmeta[kWLoads];
  int wk[kWLoads];
  int wdst[kWLoads];
#pragma unroll
  for (int i = 0; i < kWLoads; ++i) {
    const int e = tid + kThreads * i;
    const int row = e / kPiecesPerRow;
    const int piece = e % kPiecesPerRow;
    int64_t n = n0 + row;
    n = n < a.N ? n : a.N - 1;
    wsrc[i] = a.qw + n * a.ldq + piece * 16;
    wmeta[i] = n * a.G;
    wk[i] = piece * kPieceK;
    wdst[i] = (BM + row) * kStride + piece * kPieceK;
  }

  const bool asym = !a.symmetric;
  const uint32_t flip = (FMT == kByte && a.signed_codes) ? 0x80808080u : 0u;
  const float z_adj = (FMT == kByte && a.signed_codes) ? 128.0f : 0.0f;

  u32x4 xreg[kXLoads];
  u32x4 wreg[kWLoads];
  float sreg[kWLoads], zreg[kWLoads];

  auto fetch = [&](int kt) {
    const int64_t k0 = int64_t(kt) * kBK;
#pragma unroll
    for (int i = 0; i < kXLoads; ++i)
      xreg[i] = xok[i] ? *reinterpret_cast<const u32x4*>(xsrc[i] + k0) : u32x4{0u, 0u, 0u, 0u};
    const int64_t boff = FMT == kNibble ? k0 / 2 : k0;
#pragma unroll
    for (int i = 0; i < kWLoads; ++i) {
      wreg[i] = *reinterpret_cast<const u32x4*>(wsrc[i] + boff);
      const uint32_t g = div_small(uint32_t(k0 + wk[i]), group_magic);
      sreg[i] = a.scales[wmeta[i] + g];
      zreg[i] = asym ? a.zeros[wmeta[i] + g] : a.zero_const;
    }
  };

  auto stash = [&](int buf) {
    uint16_t* base = smem + buf * (BM + BN) * kStride;
#pragma unroll
    for (int i = 0; i < kXLoads; ++i) *reinterpret_cast<u32x4*>(base + xdst[i]) = xreg[i];
#pragma unroll
    for (int i = 0; i < kWLoads; ++i) {
      const float s = sreg[i];
      const float z = zreg[i] + z_adj;
      const uint32_t words[4] = {wreg[i].x ^ flip, wreg[i].y ^ flip, wreg[i].z ^ flip,
                                 wreg[i].w ^ flip};
      if constexpr (FMT == kNibble) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t lo = words[d] & 0x0F0F0F0Fu;
          const uint32_t hi = (words[d] >> 4) & 0x0F0F0F0Fu;
          float v[8];
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            v[2 * b] = dequant_exact(float((lo >> (8 * b)) & 0xFFu), z, s);
            v[2 * b + 1] = dequant_exact(float((hi >> (8 * b)) & 0xFFu), z, s);
          }
          *reinterpret_cast<u32x4*>(base + wdst[i] + 8 * d) = pack8<Act>(v);
        }
      } else {
#pragma unroll
        for (int d = 0; d < 2; ++d) {
          float v[8];
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            v[b] = dequant_exact(float((words[2 * d] >> (8 * b)) & 0xFFu), z, s);
            v[4 + b] = dequant_exact(float((words[2 * d + 1] >> (8 * b)) & 0xFFu), z, s);
          }
          *reinterpret_cast<u32x4*>(base + wdst[i] + 8 * d) = pack8<Act>(v);
        }
      }
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int ktiles = int(a.K / kBK);
  fetch(0);
  stash(0);
  __syncthreads();

  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * 8;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ktiles) fetch(kt + 1);
    const uint16_t* as = smem + buf * (BM + BN) * kStride;
    const uint16_t* bs = as + BM * kStride;
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 16) {
      u32x4 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const u32x4*>(as + (wm * WM + 32 * i + frag_row) * kStride + kk + frag_k);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bfr[j] = *reinterpret_cast<const u32x4*>(bs + (wn * WN + 32 * j + frag_row) * kStride + kk + frag_k);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Mfma32<Act>::run(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < ktiles) stash(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds column n = lane % 32 of each 32x32 tile and rows 8q + 4(lane/32) + r.
  const Raw* bias = static_cast<const Raw*>(a.bias);
  Raw* y = static_cast<Raw*>(a.y);
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t n = n0 + wn * WN + 32 * j + (lane & 31);
    if (n >= a.N) continue;
    const float b = bias ? Act::load(bias[n]) : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t m = m0 + wm * WM + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (m < a.M) y[m * a.ldy + n] = Act::store(acc[i][j][v] + b);
      }
    }
  }
}

template <class Act, int FMT, int BM, int BN>
hipError_t launch_tiles(const LinearArgs& a, uint32_t magic, hipStream_t stream) {
  const int64_t tm = (a.M + BM - 1) / BM;
  const int64_t tn = (a.N + BN - 1) / BN;
  if (tm * tn > 0x7FFFFFFF) return hipErrorInvalidValue;
  hipLaunchKernelGGL((qlinear_prefill_kernel<Act, FMT, BM, BN>), dim3(unsigned(tm * tn)),
                     dim3(kThreads), 0, stream, a, int(tm), int(tn), magic);
  return hipGetLastError();
}

template <class Act, int FMT>
hipError_t launch_fmt(const LinearArgs& a, uint32_t magic, hipStream_t stream) {
  // Largest tile that still gives every CU at least one workgroup.
  const int64_t big = ((a.M + 255) / 256) * ((a.N + 255) / 256);
  if (big >= 256) return launch_tiles<Act, FMT, 256, 256>(a, magic, stream);
  return launch_tiles<Act, FMT, 128, 128>(a, magic, stream);
}

}  // namespace

hipError_t launch_linear_prefill(const LinearArgs& a, hipStream_t stream, bool* fits) {
  *fits = false;
  if (a.act != kDtBf16 && a.act != kDtF16) return hipSuccess;
  if (a.M < 1 || a.epilogue != kEpiNone) return hipSuccess;
  const int piece_k = a.fmt == kNibble ? 32 : 16;
  if (a.K % kBK != 0 || a.K >= 65536 || a.group % piece_k != 0) return hipSuccess;
  if (a.ldq % 16 != 0 || reinterpret_cast<uintptr_t>(a.qw) % 16 != 0) return hipSuccess;
  if (a.ldx % 8 != 0 || reinterpret_cast<uintptr_t>(a.x) % 16 != 0) return hipSuccess;
  const uint32_t g = uint32_t(a.group);
  const uint32_t magic =
      g == 1 ? 0u : uint32_t((uint64_t(1) << 32) / g + ((uint64_t(1) << 32) % g != 0));
  *fits = true;
  if (a.act == kDtBf16) {
    if (a.fmt == kNibble) return launch_fmt<ActBf16, kNibble>(a, magic, stream);
    return launch_fmt<ActBf16, kByte>(a, magic, stream);
  }
  if (a.fmt == kNibble) return launch_fmt<ActF16, kNibble>(a, magic, stream);
  return launch_fmt<ActF16, kByte>(a, magic, stream);
}

}  // namespace llmopt
