// Decode-regime quantized linear (M <= 64): an HBM-streaming split-K skinny GEMM on MFMA.
//
// Replaces QuantLinear.forward (src/llmopt/quantization/quant_linear.py:93-113) for small
// batches: the packed codes are read once, straight from HBM with 16-byte loads, turned
// into MFMA operands in registers, and never written back as a dense weight.
//
// Work split. A workgroup owns 16*NT consecutive output features and all of K. Its NW waves
// take K in chunks, interleaved (chunk c goes to wave c % NW), so at any moment the waves
// of a workgroup read adjacent bytes of the same rows. A chunk is 4 lane groups x CB bytes
// per row; the lane with (col, kq) = (lane % 16, lane / 16) reads CB contiguous bytes of
// row n0 + col at offset kq*CB. The per-wave partial sums are added in a fixed order
// through LDS at the end, so results are deterministic.
//
// Arithmetic. v_mfma_f32_16x16x32_{bf16,f16} with A = activations (rows m) and B = codes
// (columns n). A code q becomes an exact MFMA operand without any float math: OR-ing a
// nibble into the mantissa of 128.0 (bf16) or 1024.0 (fp16) gives OFF + q. The scale and
// zero point are applied once per chunk (a chunk never straddles a group):
//     sum_k (q_k - z) s x_k = s * (sum_k (OFF + q_k) x_k - (OFF + z) * sum_k x_k)
// where sum_k x_k comes from one extra MFMA against a ones operand. The codes land in the
// operand in the order (k0,k4,k1,k5,k2,k6,k3,k7); the activations are permuted to match.
#include "qcommon.hpp"
#include "qkernels.hpp"

namespace llmopt {
namespace {

template <class Act>
struct Mfma16;
template <>
struct Mfma16<ActBf16> {
  __device__ static f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma16<ActF16> {
  __device__ static f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// Geometry of one chunk: CB bytes per lane and row, four lane groups per chunk.
template <int FMT, int CB>
struct Chunk {
  static constexpr int kWords = CB / 4;
  static constexpr int kLaneK = FMT == kNibble ? 2 * CB : CB;  // codes per lane
  static constexpr int kK = 4 * kLaneK;                        // codes per row per chunk
  static constexpr int kBytes = 4 * CB;                        // bytes per row per chunk
  static constexpr int kMfma = kLaneK / 8;                     // MFMAs per chunk
};

// MFMA operand j (8 codes) of one lane, plus the constant added to every code on the way.
template <class Act, int FMT>
struct Codes;

template <class Act>
struct Codes<Act, kNibble> {
  static constexpr float kOffset = Act::kNibbleOffset;
  template <int W>
  __device__ static u32x4 operand(const uint32_t (&w)[W], int j, uint32_t) {
    constexpr uint32_t kMagic = Act::kNibbleMagic2;
    const uint32_t d = w[j];
    u32x4 r;
    r.x = (d & 0x000F000Fu) | kMagic;          // k0, k4
    r.y = ((d >> 4) & 0x000F000Fu) | kMagic;   // k1, k5
    r.z = ((d >> 8) & 0x000F000Fu) | kMagic;   // k2, k6
    r.w = ((d >> 12) & 0x000F000Fu) | kMagic;  // k3, k7
    return r;
  }
};

template <>
struct Codes<ActF16, kByte> {
  static constexpr float kOffset = 1024.0f;
  template <int W>
  __device__ static u32x4 operand(const uint32_t (&w)[W], int j, uint32_t flip) {
    const uint32_t a = w[2 * j] ^ flip;
    const uint32_t b = w[2 * j + 1] ^ flip;
    u32x4 r;
    r.x = (a & 0x00FF00FFu) | 0x64006400u;         // k0, k2
    r.y = ((a >> 8) & 0x00FF00FFu) | 0x64006400u;  // k1, k3
    r.z = (b & 0x00FF00FFu) | 0x64006400u;         // k4, k6
    r.w = ((b >> 8) & 0x00FF00FFu) | 0x64006400u;  // k5, k7
    return r;
  }
};

template <>
struct Codes<ActBf16, kByte> {
  static constexpr float kOffset = 0.0f;
  // Bytes are exact in fp32 with at most 8 significant bits, so the top half of the fp32
  // pattern is the exact bf16.
  __device__ static uint32_t pair(uint32_t lo, uint32_t hi) {
    return (__float_as_uint(float(lo)) >> 16) | (__float_as_uint(float(hi)) & 0xFFFF0000u);
  }
  template <int W>
  __device__ static u32x4 operand(const uint32_t (&w)[W], int j, uint32_t flip) {
    const uint32_t a = w[2 * j] ^ flip;
    const uint32_t b = w[2 * j + 1] ^ flip;
    u32x4 r;
    r.x = pair(a & 0xFFu, (a >> 8) & 0xFFu);
    r.y = pair((a >> 16) & 0xFFu, a >> 24);
    r.z = pair(b & 0xFFu, (b >> 8) & 0xFFu);
    r.w = pair((b >> 16) & 0xFFu, b >> 24);
    return r;
  }
};

// Eight consecutive activations (x0..x7 in d) rearranged into the code order above.
template <class Act, int FMT>
__device__ __forceinline__ u32x4 arrange(u32x4 d) {
  u32x4 o;
  if constexpr (FMT == kNibble) {  // (x0,x4) (x1,x5) (x2,x6) (x3,x7)
    o.x = (d.x & 0xFFFFu) | (d.z << 16);
    o.y = (d.x >> 16) | (d.z & 0xFFFF0000u);
    o.z = (d.y & 0xFFFFu) | (d.w << 16);
    o.w = (d.y >> 16) | (d.w & 0xFFFF0000u);
  } else if constexpr (Act::id == kDtF16) {  // (x0,x2) (x1,x3) (x4,x6) (x5,x7)
    o.x = (d.x & 0xFFFFu) | (d.y << 16);
    o.y = (d.x >> 16) | (d.y & 0xFFFF0000u);
    o.z = (d.z & 0xFFFFu) | (d.w << 16);
    o.w = (d.z >> 16) | (d.w & 0xFFFF0000u);
  } else {  // natural order
    o = d;
  }
  return o;
}

template <int CB>
__device__ __forceinline__ void load_codes(uint32_t (&dst)[CB / 4], const uint8_t* p) {
  if constexpr (CB == 16) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
    dst[0] = v.x;
    dst[1] = v.y;
    dst[2] = v.z;
    dst[3] = v.w;
  } else if constexpr (CB == 8) {
    const u32x2 v = *reinterpret_cast<const u32x2*>(p);
    dst[0] = v.x;
    dst[1] = v.y;
  } else {
    dst[0] = *reinterpret_cast<const uint32_t*>(p);
  }
}

template <int NT, int MB, int CB, int NM>
struct Stage {
  uint32_t w[NT][CB / 4];
  u32x4 x[MB][NM];
  float s[NT];
  float z[NT];
};

template <class Act, int FMT, int CB, int MB, int NT, int NW>
__global__ void __launch_bounds__(NW * 64)
    qlinear_decode_kernel(const LinearArgs a, uint32_t group_magic) {
  using C = Chunk<FMT, CB>;
  using Raw = typename Act::raw;
  using Op = Codes<Act, FMT>;
  constexpr int NM = C::kMfma;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int kq = lane >> 4;
  const int64_t n_base = int64_t(blockIdx.x) * (16 * NT);
  const bool asym = !a.symmetric;

  const uint8_t* wrow[NT];
  int64_t meta[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int64_t n = n_base + 16 * t + col;
    n = n < a.N ? n : a.N - 1;
    wrow[t] = a.qw + n * a.ldq + kq * CB;
    meta[t] = n * a.G;
  }
  const Raw* xrow[MB];
  bool xok[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int64_t m = 16 * mb + col;
    xok[mb] = m < a.M;
    xrow[mb] = static_cast<const Raw*>(a.x) + (xok[mb] ? m : 0) * a.ldx + kq * C::kLaneK;
  }

  const uint32_t flip = (FMT == kByte && a.signed_codes) ? 0x80808080u : 0u;
  const float z_shift = Op::kOffset + ((FMT == kByte && a.signed_codes) ? 128.0f : 0.0f);
  const float z_const = a.zero_const + z_shift;
  const int chunks = int(a.K / C::kK);

  f32x4 tot[NT][MB];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) tot[t][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto load = [&](Stage<NT, MB, CB, NM>& st, int c) {
    const int64_t boff = int64_t(c) * C::kBytes;
#pragma unroll
    for (int t = 0; t < NT; ++t) load_codes<CB>(st.w[t], wrow[t] + boff);
    const int64_t koff = int64_t(c) * C::kK;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < NM; ++j)
        st.x[mb][j] = xok[mb] ? *reinterpret_cast<const u32x4*>(xrow[mb] + koff + 8 * j)
                              : u32x4{0u, 0u, 0u, 0u};
    const uint32_t g = div_small(uint32_t(c), group_magic);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      st.s[t] = a.scales[meta[t] + g];
      st.z[t] = asym ? a.zeros[meta[t] + g] : 0.0f;
    }
  };

  auto compute = [&](const Stage<NT, MB, CB, NM>& st) {
    const u32x4 ones = {Act::kOne2, Act::kOne2, Act::kOne2, Act::kOne2};
    u32x4 xa[MB][NM];
    f32x4 xsum[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      xsum[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NM; ++j) {
        xa[mb][j] = arrange<Act, FMT>(st.x[mb][j]);
        xsum[mb] = Mfma16<Act>::run(xa[mb][j], ones, xsum[mb]);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      u32x4 wb[NM];
#pragma unroll
      for (int j = 0; j < NM; ++j) wb[j] = Op::operand(st.w[t], j, flip);
      const float s = st.s[t];
      const float zc = asym ? st.z[t] + z_shift : z_const;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NM; ++j) acc = Mfma16<Act>::run(xa[mb][j], wb[j], acc);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          tot[t][mb][r] = __builtin_fmaf(s, __builtin_fmaf(-zc, xsum[mb][r], acc[r]), tot[t][mb][r]);
      }
    }
  };

  Stage<NT, MB, CB, NM> s0, s1;
  int c = wave;
  if (c < chunks) load(s0, c);
  for (; c < chunks; c += 2 * NW) {
    const int c1 = c + NW;
    if (c1 < chunks) load(s1, c1);
    compute(s0);
    if (c1 < chunks) {
      if (c1 + NW < chunks) load(s0, c1 + NW);
      compute(s1);
    }
  }

  // Fixed-order reduction of the per-wave partial sums.
  constexpr int kElems = NT * MB * 4 * 64;
  __shared__ float partial[NW * kElems];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) partial[wave * kElems + ((t * MB + mb) * 4 + r) * 64 + lane] = tot[t][mb][r];
  __syncthreads();

  const Raw* bias = static_cast<const Raw*>(a.bias);
  Raw* y = static_cast<Raw*>(a.y);
  for (int e = threadIdx.x; e < kElems; e += NW * 64) {
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += partial[w * kElems + e];
    const int ln = e & 63;
    const int r = (e >> 6) & 3;
    const int tm = e >> 8;
    const int t = tm / MB;
    const int mb = tm - t * MB;
    const int64_t m = 16 * mb + 4 * (ln >> 4) + r;
    const int64_t n = n_base + 16 * t + (ln & 15);
    if (m < a.M && n < a.N) {
      if (bias) v += Act::load(bias[n]);
      y[m * a.ldy + n] = Act::store(v);
    }
  }
}

// ---- dispatch ----------------------------------------------------------------------------------

template <class Act, int FMT, int CB, int MB, int NT, int NW>
hipError_t launch_cfg(const LinearArgs& a, uint32_t magic, hipStream_t stream) {
  const int64_t blocks = (a.N + 16 * NT - 1) / (16 * NT);
  hipLaunchKernelGGL((qlinear_decode_kernel<Act, FMT, CB, MB, NT, NW>), dim3(unsigned(blocks)),
                     dim3(NW * 64), 0, stream, a, magic);
  return hipGetLastError();
}

template <class Act, int FMT, int CB, int MB>
hipError_t launch_mb(const LinearArgs& a, uint32_t magic, hipStream_t stream) {
  // Two output tiles per workgroup once there are enough rows to keep every CU busy.
  if (a.N >= 8192) return launch_cfg<Act, FMT, CB, MB, 2, 8>(a, magic, stream);
  return launch_cfg<Act, FMT, CB, MB, 1, 8>(a, magic, stream);
}

template <class Act, int FMT, int CB>
hipError_t launch_cb(const LinearArgs& a, uint32_t magic, hipStream_t stream) {
  if (a.M <= 16) return launch_mb<Act, FMT, CB, 1>(a, magic, stream);
  if (a.M <= 32) return launch_mb<Act, FMT, CB, 2>(a, magic, stream);
  if constexpr (FMT == kNibble && CB == 16) {
    return hipErrorInvalidValue;  // M > 32 is routed to 8-byte chunks by the caller
  } else {
    return launch_mb<Act, FMT, CB, 4>(a, magic, stream);
  }
}

template <class Act>
hipError_t launch_act(const LinearArgs& a, int cb, uint32_t magic, hipStream_t stream) {
  if (a.fmt == kNibble) {
    if (cb == 16) return launch_cb<Act, kNibble, 16>(a, magic, stream);
    return launch_cb<Act, kNibble, 8>(a, magic, stream);
  }
  return launch_cb<Act, kByte, 16>(a, magic, stream);
}

}  // namespace

hipError_t launch_linear_decode(const LinearArgs& a, hipStream_t stream, bool* fits) {
  *fits = false;
  if (a.act != kDtBf16 && a.act != kDtF16) return hipSuccess;
  if (a.M < 1 || a.M > 64) return hipSuccess;
  // Bytes per lane per chunk: the widest that a group and the row alignment allow.
  int cb = 0;
  int chunk_k = 0;
  if (a.fmt == kNibble) {
    if (a.group % 128 == 0 && a.ldq % 16 == 0) {
      cb = 16;
      chunk_k = 128;
    } else if (a.group % 64 == 0 && a.ldq % 8 == 0) {
      cb = 8;
      chunk_k = 64;
    }
  } else if (a.group % 64 == 0 && a.ldq % 16 == 0) {
    cb = 16;
    chunk_k = 64;
  }
  if (cb == 0) return hipSuccess;
  // Four 16-column activation blocks with 16-byte nibble chunks exceed the register file;
  // 8-byte chunks keep them resident.
  if (a.fmt == kNibble && cb == 16 && a.M > 32) {
    cb = 8;
    chunk_k = 64;
  }
  if (a.K % chunk_k != 0 || a.K / chunk_k >= 65536) return hipSuccess;
  if (reinterpret_cast<uintptr_t>(a.qw) % 16 != 0) return hipSuccess;
  if (reinterpret_cast<uintptr_t>(a.x) % 16 != 0 || a.ldx % 8 != 0) return hipSuccess;
  if (a.N > int64_t(0x7FFFFFFF) * 16) return hipSuccess;
  const uint32_t per_group = uint32_t(a.group / chunk_k);
  const uint32_t magic =
      per_group == 1 ? 0u : uint32_t((uint64_t(1) << 32) / per_group + ((uint64_t(1) << 32) % per_group != 0));
  *fits = true;
  if (a.act == kDtBf16) return launch_act<ActBf16>(a, cb, magic, stream);
  return launch_act<ActF16>(a, cb, magic, stream);
}

}  // namespace llmopt
