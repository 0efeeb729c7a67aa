// On-device round-to-nearest quantizer: the device form of RoundToNearestQuantizer.quantize,
// i.e. choose_qparams + quantize_to_codes + pack_int4 in one pass over the weight
// (src/llmopt/quantization/quantizers.py:83-89, 100-142, 167-201, 285-305).
//
// Bit-exact with the reference's fp32 torch arithmetic on finite weights:
//   * per (row, group): lo = min(w), hi = max(w) (exact; the weight's own dtype converts to
//     fp32 exactly and monotonically, so min/max commute with the conversion);
//   * asymmetric: lo = min(lo, 0), hi = max(hi, 0), s = max((hi - lo) / (2^b - 1), 1e-8),
//     z = rne(-lo / s); symmetric: s = max(|lo|, |hi|, 1e-8) / (2^(b-1) - 1), z = 0;
//   * codes: asymmetric clamp(rne(w / s) + z, 0, 2^b - 1) as uint8; symmetric
//     clamp(rne(w / s), -2^(b-1), 2^(b-1) - 1), as int8 for 8 bits, else + 2^(b-1) as uint8;
//   * every operation rounds once in fp32 (correctly rounded division, round-half-even,
//     no contraction), as torch does on the host;
//   * codes of widths below 8 are packed two per byte, even column in the low nibble.
// NaN weights propagate into their group's scale as with torch.amin/amax; the codes of such a
// group are then unspecified (the reference converts NaN to uint8).
//
// Layout of the work: a team of T lanes owns one (row, group); each lane takes 8-column chunks
// of the group (one 16-byte load for 2-byte weights, two for fp32), the team reduces min/max
// with lane shuffles, and every lane writes its chunk's codes (4 bytes of nibbles or 8 bytes)
// -- one coalesced pass that reads the weight once and writes codes, scales and zeros once.
// Groups that are not a power-of-two number of chunks up to 256 (or a multiple of 64 chunks)
// and unaligned tensors take a one-thread-per-group kernel with the same arithmetic.
#include "qcommon.hpp"
#include "qkernels.hpp"

namespace llmopt {
namespace {

// torch.amin / amax propagate NaN, and so do IEEE 754-2019 minimum / maximum, which gfx950
// executes as v_minimum3_f32 / v_maximum3_f32 (two new weights per instruction). Their choice
// between -0 and +0 does not reach the results: both grids clamp or take |.| of lo and hi first.
__device__ __forceinline__ float nan_min(float a, float b) { return __builtin_elementwise_minimum(a, b); }
__device__ __forceinline__ float nan_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }

struct Grid {
  float s, z;
  float r;  // RN(1 / s), for the quotients in rint_quotients
};

// choose_qparams for one group (quantizers.py:100-142).
__device__ __forceinline__ Grid group_grid(float lo, float hi, int bits, bool symmetric) {
  const float tiny = 1e-8f;
  if (symmetric) {
    float m = nan_max(fabsf(lo), fabsf(hi));
    m = nan_max(m, tiny);  // clamp(min=1e-8)
    const float s = __fdiv_rn(m, float((1 << (bits - 1)) - 1));
    return {s, 0.0f, __fdiv_rn(1.0f, s)};
  }
  // clamp(max=0) / clamp(min=0); a NaN stays NaN.
  lo = (lo != lo) ? lo : (lo < 0.0f ? lo : 0.0f);
  hi = (hi != hi) ? hi : (hi > 0.0f ? hi : 0.0f);
  float s = __fdiv_rn(__fsub_rn(hi, lo), float((1 << bits) - 1));
  s = (s != s) ? s : (s > tiny ? s : tiny);
  const float z = __builtin_rintf(__fdiv_rn(-lo, s));  // -lo is exact
  return {s, z, __fdiv_rn(1.0f, s)};
}

// rne(RN(w / s)) for the eight weights of a chunk without a division: Markstein's correction.
// With r = RN(1/s) and q0 = RN(w r), one fma gives the remainder e = RN(w - s q0) and a second
// q1 = RN(q0 + e r), which is RN(w / s) (Markstein, "Computation of elementary functions on the
// IBM RISC System/6000 processor", IBM J. Res. Dev. 34(1), 1990; Muller et al., Handbook of
// Floating-Point Arithmetic, ch. 4). rne(q1) can only differ from rne(w / s) when w / s lies
// within an ulp of a half-integer; tests/test_quotient_exactness.py checks every fp32 s in
// [1, 2), every half-integer below 256 and the w within 4 ulps of s times it (all agree), and
// the steps scale exactly with s and w (by powers of two) while the remainder stays exactly
// representable: for every s from 2^-100 to 2^120 once |w / s| >= 1/4 (below that both sides
// round to zero). The quantizers' smallest scale is 1e-8 / 127 (about 7.9e-11: the amax floor
// of an 8-bit symmetric grid), inside that range. Larger or non-finite scales
// (r near the subnormal range, or 0) take the correctly rounded division, behind a branch that
// is wave-uniform in practice.
__device__ __forceinline__ void rint_quotients(const float* v, const Grid& g, float* ratio) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float q0 = __fmul_rn(v[j], g.r);
    const float e = __builtin_fmaf(-g.s, q0, v[j]);
    ratio[j] = __builtin_rintf(__builtin_fmaf(e, g.r, q0));
  }
  const bool divide = !(g.s <= 0x1p120f);
  if (__builtin_amdgcn_ballot_w64(divide) != 0) {
    if (divide) {
#pragma unroll
      for (int j = 0; j < 8; ++j) ratio[j] = __builtin_rintf(__fdiv_rn(v[j], g.s));
    }
  }
}

// quantize_to_codes for one weight, given rne(w / s) (quantizers.py:167-201): the stored byte.
template <int BITS, bool SYM>
__device__ __forceinline__ uint32_t code_of(float ratio, const Grid& g) {
  if constexpr (SYM) {
    constexpr float top = float((1 << (BITS - 1)) - 1);
    const float c = fminf(fmaxf(ratio, -top - 1.0f), top);
    if constexpr (BITS == 8) return uint32_t(int32_t(c)) & 0xFFu;  // int8, two's complement
    return uint32_t(__fadd_rn(c, float(1 << (BITS - 1))));
  }
  const float c = fminf(fmaxf(__fadd_rn(ratio, g.z), 0.0f), float((1 << BITS) - 1));
  return uint32_t(c);
}

__device__ __forceinline__ uint32_t code_of(float w, const Grid& g, int bits, bool symmetric) {
  const float ratio = __builtin_rintf(__fdiv_rn(w, g.s));
  if (symmetric) {
    const float top = float((1 << (bits - 1)) - 1);
    const float c = fminf(fmaxf(ratio, -top - 1.0f), top);
    if (bits == 8) return uint32_t(int32_t(c)) & 0xFFu;
    return uint32_t(__fadd_rn(c, float(1 << (bits - 1))));
  }
  const float c = fminf(fmaxf(__fadd_rn(ratio, g.z), 0.0f), float((1 << bits) - 1));
  return uint32_t(c);
}

template <class In>
__device__ __forceinline__ void load_chunk(const typename In::raw* p, float* v) {
  if constexpr (sizeof(typename In::raw) == 4) {
    const u32x4 a = *reinterpret_cast<const u32x4*>(p);
    const u32x4 b = *reinterpret_cast<const u32x4*>(p + 4);
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = __uint_as_float(w[j]);
  } else {
    const u32x4 a = *reinterpret_cast<const u32x4*>(p);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = In::load(typename In::raw(w[j] & 0xFFFFu));
      v[2 * j + 1] = In::load(typename In::raw(w[j] >> 16));
    }
  }
}

// Codes of one 8-column chunk (columns col .. col + 7 of the packed row).
template <int BITS, bool SYM>
__device__ __forceinline__ void store_chunk(uint8_t* qrow, int64_t col, const float* v, const Grid& g) {
  float ratio[8];
  rint_quotients(v, g, ratio);
  if constexpr (BITS < 8) {
    uint32_t packed = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) packed |= code_of<BITS, SYM>(ratio[j], g) << (4 * j);
    *reinterpret_cast<uint32_t*>(qrow + col / 2) = packed;
  } else {
    u32x2 packed = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      packed.x |= code_of<BITS, SYM>(ratio[j], g) << (8 * j);
      packed.y |= code_of<BITS, SYM>(ratio[4 + j], g) << (8 * j);
    }
    *reinterpret_cast<u32x2*>(qrow + col) = packed;
  }
}

// min/max of a team's weights (lane values lo, hi already folded over the lane's own weights),
// NaN-propagating; every lane of the team ends with the team's values.
__device__ __forceinline__ void team_reduce(float& lo, float& hi, int T) {
  for (int off = T >> 1; off > 0; off >>= 1) {
    lo = nan_min(lo, __shfl_xor(lo, off, 64));
    hi = nan_max(hi, __shfl_xor(hi, off, 64));
  }
}

__device__ __forceinline__ void fold(const float* v, float& lo, float& hi) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    lo = nan_min(lo, v[j]);
    hi = nan_max(hi, v[j]);
  }
}

// Groups of T * CPL chunks, T = 2^team_log2: a team of T lanes per (row, group), CPL adjacent
// chunks per lane, and each lane serves U teams -- rows r, r + R, ..., r + (U - 1) R of the same
// group, R = ceil(N / U) -- whose loads are all issued before any is used, so a wave keeps
// U * CPL kilobytes in flight. Four adjacent chunks per lane (64 bytes of 2-byte weights) cut
// the per-weight share of the group's scale and zero point (three divisions per lane) and of
// the team's shuffles; with eight, a lane's loads no longer coalesce with its neighbours'.
template <class In, int BITS, bool SYM, int U, int CPL>
__global__ void __launch_bounds__(256) rtn_team_kernel(const RtnArgs a, int team_log2, int64_t rows_per_unit) {
  using Raw = typename In::raw;
  const int T = 1 << team_log2;
  const int64_t gtid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t team0 = gtid >> team_log2;
  const int tl = int(gtid & (T - 1));
  // Lanes past the last team work on row 0 without storing, so every lane of a wave takes part
  // in the shuffles.
  const int64_t row0 = team0 / a.G;
  const int64_t grp = team0 - row0 * a.G;
  const int64_t col = grp * a.group + int64_t(tl) * (8 * CPL);
  const float inf = __int_as_float(0x7F800000);

  float v[U][8 * CPL];
  int64_t row[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    row[u] = row0 + u * rows_per_unit;
    const int64_t r = row[u] < a.N ? row[u] : 0;
#pragma unroll
    for (int c = 0; c < CPL; ++c) load_chunk<In>(static_cast<const Raw*>(a.w) + r * a.ldw + col + 8 * c, v[u] + 8 * c);
  }
  // The U reductions run side by side (one basic block).
  float lo[U], hi[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    lo[u] = inf;
    hi[u] = -inf;
#pragma unroll
    for (int c = 0; c < CPL; ++c) fold(v[u] + 8 * c, lo[u], hi[u]);
  }
  for (int off = T >> 1; off > 0; off >>= 1) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      lo[u] = nan_min(lo[u], __shfl_xor(lo[u], off, 64));
      hi[u] = nan_max(hi[u], __shfl_xor(hi[u], off, 64));
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const Grid g = group_grid(lo[u], hi[u], BITS, SYM);
    if (row[u] < a.N && row0 < rows_per_unit) {
      if (tl == 0) {
        a.scales[row[u] * a.G + grp] = g.s;
        a.zeros[row[u] * a.G + grp] = g.z;
      }
#pragma unroll
      for (int c = 0; c < CPL; ++c) store_chunk<BITS, SYM>(a.q + row[u] * a.ldq, col + 8 * c, v[u] + 8 * c, g);
    }
  }
}

// Groups of a multiple of 64 chunks: a whole wave per (row, group), each lane taking
// `per_lane` chunks; the codes pass reads the chunks again (from cache).
template <class In, int BITS, bool SYM>
__global__ void __launch_bounds__(256) rtn_wave_kernel(const RtnArgs a, int per_lane) {
  using Raw = typename In::raw;
  const int64_t gtid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t teams = a.N * a.G;
  const int64_t team = gtid >> 6;
  const bool live = team < teams;
  const int64_t t = live ? team : 0;
  const int tl = int(gtid & 63);
  const int64_t row = t / a.G;
  const int64_t grp = t - row * a.G;
  const Raw* wg = static_cast<const Raw*>(a.w) + row * a.ldw + grp * a.group;
  const float inf = __int_as_float(0x7F800000);
  float v[8];
  float lo = inf, hi = -inf;
  for (int p = 0; p < per_lane; ++p) {
    load_chunk<In>(wg + int64_t(tl + p * 64) * 8, v);
    fold(v, lo, hi);
  }
  team_reduce(lo, hi, 64);
  const Grid g = group_grid(lo, hi, BITS, SYM);
  if (!live) return;
  if (tl == 0) {
    a.scales[row * a.G + grp] = g.s;
    a.zeros[row * a.G + grp] = g.z;
  }
  for (int p = 0; p < per_lane; ++p) {
    const int64_t c = int64_t(tl + p * 64) * 8;
    load_chunk<In>(wg + c, v);
    store_chunk<BITS, SYM>(a.q + row * a.ldq, grp * a.group + c, v, g);
  }
}

// Any geometry: one thread per (row, group), element by element (groups are even, so a
// group's codes fill whole bytes).
template <class In>
__global__ void __launch_bounds__(256) rtn_generic_kernel(const RtnArgs a) {
  using Raw = typename In::raw;
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= a.N * a.G) return;
  const int64_t row = t / a.G;
  const int64_t grp = t - row * a.G;
  const Raw* wg = static_cast<const Raw*>(a.w) + row * a.ldw + grp * a.group;
  float lo = __int_as_float(0x7F800000), hi = -__int_as_float(0x7F800000);
  for (int64_t k = 0; k < a.group; ++k) {
    const float w = In::load(wg[k]);
    lo = nan_min(lo, w);
    hi = nan_max(hi, w);
  }
  const bool symmetric = a.symmetric != 0;
  const Grid g = group_grid(lo, hi, a.bits, symmetric);
  a.scales[t] = g.s;
  a.zeros[t] = g.z;
  uint8_t* const qrow = a.q + row * a.ldq;
  const int64_t col0 = grp * a.group;
  if (a.bits == 8) {
    for (int64_t k = 0; k < a.group; ++k) qrow[col0 + k] = uint8_t(code_of(In::load(wg[k]), g, 8, symmetric));
  } else {
    for (int64_t k = 0; k < a.group; k += 2) {
      const uint32_t c0 = code_of(In::load(wg[k]), g, a.bits, symmetric);
      const uint32_t c1 = code_of(In::load(wg[k + 1]), g, a.bits, symmetric);
      qrow[(col0 + k) / 2] = uint8_t(c0 | (c1 << 4));
    }
  }
}

template <class In>
hipError_t launch_in(const RtnArgs& a, hipStream_t stream) {
  const int64_t teams = a.N * a.G;
  const int64_t chunks = a.group / 8;  // per group
  const bool chunked = a.group % 8 == 0 && a.ldw % 8 == 0 && reinterpret_cast<uintptr_t>(a.w) % 16 == 0;
  const bool nibble = a.bits < 8;
  const bool out_aligned = nibble ? (a.ldq % 4 == 0 && reinterpret_cast<uintptr_t>(a.q) % 4 == 0)
                                  : (a.ldq % 8 == 0 && reinterpret_cast<uintptr_t>(a.q) % 8 == 0);
  int team_log2 = -1, per_lane = 1, cpl = 1;
  if (chunked && out_aligned) {
    if (chunks <= 256 && chunks >= 4 && (chunks & (chunks - 1)) == 0) {
      cpl = 4;
      team_log2 = __builtin_ctzll(uint64_t(chunks / 4));
    } else if (chunks == 2) {
      cpl = 2;
      team_log2 = 0;
    } else if (chunks <= 64 && (chunks & (chunks - 1)) == 0) {
      team_log2 = __builtin_ctzll(uint64_t(chunks));
    } else if (chunks % 64 == 0) {
      team_log2 = 6;
      per_lane = int(chunks / 64);
    }
  }
  if (team_log2 < 0) {
    const dim3 grid(unsigned((teams + 255) / 256));
    hipLaunchKernelGGL(rtn_generic_kernel<In>, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
  }
  const bool sym = a.symmetric != 0;
  // One row per lane: measured on MI355X (gate_up, bf16 -> W4 g128), one row of four chunks
  // per lane 56 us, two rows of two chunks 61 us, one row of two 57 us, eight chunks (each
  // lane a whole line, uncoalesced across the wave) 77 us.
  constexpr int kUnits = 1;
  const int64_t rows_per_unit = (a.N + kUnits - 1) / kUnits;
  const dim3 team_grid(unsigned((((rows_per_unit * a.G) << team_log2) + 255) / 256));
  const dim3 wave_grid(unsigned((teams * 64 + 255) / 256));
#define LLMOPT_RTN(B, S)                                                                           \
  if (a.bits == B && sym == S) {                                                                \
    if (per_lane == 1 && cpl == 4)                                                              \
      hipLaunchKernelGGL((rtn_team_kernel<In, B, S, kUnits, 4>), team_grid, dim3(256), 0, stream, a, \
                         team_log2, rows_per_unit);                                             \
    else if (per_lane == 1 && cpl == 2)                                                         \
      hipLaunchKernelGGL((rtn_team_kernel<In, B, S, kUnits, 2>), team_grid, dim3(256), 0, stream, a, \
                         team_log2, rows_per_unit);                                             \
    else if (per_lane == 1)                                                                     \
      hipLaunchKernelGGL((rtn_team_kernel<In, B, S, kUnits, 1>), team_grid, dim3(256), 0, stream, a, \
                         team_log2, rows_per_unit);                                             \
    else                                                                                        \
      hipLaunchKernelGGL((rtn_wave_kernel<In, B, S>), wave_grid, dim3(256), 0, stream, a,        \
                         per_lane);                                                             \
  }
  LLMOPT_RTN(2, false) LLMOPT_RTN(2, true) LLMOPT_RTN(4, false) LLMOPT_RTN(4, true)
  LLMOPT_RTN(8, false) LLMOPT_RTN(8, true)
#undef LLMOPT_RTN
  return hipGetLastError();
}

}  // namespace

hipError_t launch_quantize_rtn(const RtnArgs& a, hipStream_t stream) {
  if (a.N == 0 || a.K == 0) return hipSuccess;
  switch (a.w_dtype) {
    case kDtF32: return launch_in<ActF32>(a, stream);
    case kDtF16: return launch_in<ActF16>(a, stream);
    case kDtBf16: return launch_in<ActBf16>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace llmopt
