// Unpack and dequantize kernels: the device form of unpack_int4 / dequantize
// (src/llmopt/quantization/quantizers.py:92-97, 204-239). Both are bit-exact with the
// reference's torch arithmetic: codes are pure bit operations, and the dense weight is
// (q - z) * s in fp32 with one rounding per operation, then a round-to-nearest-even cast.
#include "qcommon.hpp"
#include "qkernels.hpp"

namespace llmopt {
namespace {

// Four packed bytes -> eight codes, low nibble first.
__device__ __forceinline__ u32x2 split_nibbles(uint32_t w) {
  const uint32_t lo = w & 0x0F0F0F0Fu;
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
  u32x2 out;
  out.x = (lo & 0xFFu) | ((hi & 0xFFu) << 8) | ((lo & 0xFF00u) << 8) | ((hi & 0xFF00u) << 16);
  out.y = ((lo >> 16) & 0xFFu) | (((hi >> 16) & 0xFFu) << 8) | ((lo >> 24) << 16) | ((hi >> 24) << 24);
  return out;
}

// Rows whose full packed width is unpacked, with 4-byte-aligned packed rows and 8-byte-aligned
// output rows: each thread turns one packed dword into eight codes.
__global__ void __launch_bounds__(256) unpack_words_kernel(const uint32_t* packed, u32x2* codes,
                                                           int64_t words) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < words;
       i += int64_t(gridDim.x) * blockDim.x) {
    codes[i] = split_nibbles(packed[i]);
  }
}

// Any geometry: one thread per packed byte, writing the one or two codes that fall below
// `columns`.
__global__ void __launch_bounds__(256) unpack_bytes_kernel(const uint8_t* packed, uint8_t* codes,
                                                           int64_t rows, int64_t packed_cols,
                                                           int64_t columns) {
  const int64_t total = rows * packed_cols;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = i / packed_cols;
    const int64_t j = i - r * packed_cols;
    const uint8_t b = packed[i];
    const int64_t c = 2 * j;
    uint8_t* out = codes + r * columns;
    if (c < columns) out[c] = b & 0x0F;
    if (c + 1 < columns) out[c + 1] = b >> 4;
  }
}

template <class Out>
__device__ __forceinline__ void store_elem(void* out, int64_t idx, float v) {
  static_cast<typename Out::raw*>(out)[idx] = Out::store(v);
}

// Dense weight, any geometry: each thread produces eight consecutive columns of one row.
template <class Out>
__global__ void __launch_bounds__(256) dequant_kernel(const LinearArgs a, void* out) {
  const int64_t chunks = (a.K + 7) / 8;
  const int64_t total = a.N * chunks;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t n = i / chunks;
    const int64_t k0 = (i - n * chunks) * 8;
    const uint8_t* row = a.qw + n * a.ldq;
    const float* srow = a.scales + n * a.G;
    const float* zrow = a.symmetric ? nullptr : a.zeros + n * a.G;
    int64_t g = k0 / a.group;
    int64_t in_group = k0 - g * a.group;
    const int64_t k_end = k0 + 8 < a.K ? k0 + 8 : a.K;
    for (int64_t k = k0; k < k_end; ++k) {
      if (in_group == a.group) {
        ++g;
        in_group = 0;
      }
      const float q = code_value(row, k, a.fmt, a.signed_codes);
      const float z = zrow ? zrow[g] : a.zero_const;
      store_elem<Out>(out, n * a.K + k, dequant_exact(q, z, srow[g]));
      ++in_group;
    }
  }
}

// Dense weight, vectorized: rows of whole 8-code chunks (K % 8 == 0, group % 8 == 0, rows of
// packed codes 4-byte (nibbles) or 8-byte (bytes) aligned). Thread (chunk c, row n) reads the
// chunk's 4 or 8 code bytes and its group's scale and zero, and writes eight consecutive
// outputs with 16-byte stores, so a wave moves one contiguous run of each row. Grid: x covers
// a row's chunks, y strides over rows.
template <class Out, int FMT>
__global__ void __launch_bounds__(256) dequant_chunks_kernel(const LinearArgs a, void* out) {
  using Raw = typename Out::raw;
  const int64_t chunks = a.K >> 3;
  const int64_t c = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= chunks) return;
  const int64_t g = (c * 8) / a.group;
  for (int64_t n = blockIdx.y; n < a.N; n += gridDim.y) {
    const uint8_t* row = a.qw + n * a.ldq;
    float q[8];
    if constexpr (FMT == kNibble) {
      const uint32_t w = *reinterpret_cast<const uint32_t*>(row + c * 4);
#pragma unroll
      for (int j = 0; j < 8; ++j) q[j] = float((w >> (4 * j)) & 0xFu);
    } else {
      const u32x2 w = *reinterpret_cast<const u32x2*>(row + c * 8);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t b = ((j < 4 ? w.x : w.y) >> (8 * (j & 3))) & 0xFFu;
        q[j] = a.signed_codes ? float(int8_t(b)) : float(b);
      }
    }
    const float s = a.scales[n * a.G + g];
    const float z = a.symmetric ? a.zero_const : a.zeros[n * a.G + g];
    Raw v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = Out::store(dequant_exact(q[j], z, s));
    u32x4* dst = reinterpret_cast<u32x4*>(static_cast<Raw*>(out) + n * a.K + c * 8);
#pragma unroll
    for (int h = 0; h < int(sizeof(v) / 16); ++h) {
      u32x4 piece;
      __builtin_memcpy(&piece, reinterpret_cast<const char*>(v) + 16 * h, 16);
      dst[h] = piece;
    }
  }
}

// Dense 16-bit weight from nibble codes, whole lines both ways: one wave owns 2048 codes of a
// row (1 KB of codes, 4 KB of output). Lane l takes codes 512 h + 8 l .. + 7 for h < 4: each of
// the wave's four code loads reads 256 contiguous bytes and each of its four stores writes 1 KB
// of whole lines, against the chunk kernel's 16-byte pieces of 64 bytes per lane. Scales and
// zeros: one 4-byte load each per lane and h (16 lanes share a group of 128). Every load is
// issued before the first conversion. K % 2048 == 0, group % 8 == 0.
template <class Out>
__global__ void __launch_bounds__(256) dequant_lines_kernel(const LinearArgs a, void* out) {
  using Raw = typename Out::raw;
  static_assert(sizeof(Raw) == 2, "16-bit outputs");
  const int lane = threadIdx.x & 63;
  const int64_t chunks = a.K >> 11;
  const int64_t task = int64_t(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (task >= a.N * chunks) return;
  const int64_t n = task / chunks;
  const int64_t k0 = (task - n * chunks) * 2048 + 8 * lane;
  const uint8_t* row = a.qw + n * a.ldq;
  uint32_t w[4];
  float sc[4], zr[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const int64_t k = k0 + 512 * h;
    w[h] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(row + k / 2));
    const int64_t g = n * a.G + k / a.group;
    sc[h] = a.scales[g];
    zr[h] = a.symmetric ? a.zero_const : a.zeros[g];
  }
  Raw* dst = static_cast<Raw*>(out) + n * a.K + k0;
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    Raw v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = Out::store(dequant_exact(float((w[h] >> (4 * j)) & 0xFu), zr[h], sc[h]));
    u32x4 piece;
    __builtin_memcpy(&piece, v, 16);
    *reinterpret_cast<u32x4*>(dst + 512 * h) = piece;
  }
}

int grid_for(int64_t work, int per_block) {
  int64_t blocks = (work + per_block - 1) / per_block;
  if (blocks > 65536) blocks = 65536;
  return blocks < 1 ? 1 : int(blocks);
}

}  // namespace

hipError_t launch_unpack(const uint8_t* packed, uint8_t* codes, int64_t rows, int64_t packed_cols,
                         int64_t columns, hipStream_t stream) {
  if (rows == 0 || columns == 0) return hipSuccess;
  const bool whole_rows = columns == 2 * packed_cols;
  const bool aligned = (reinterpret_cast<uintptr_t>(packed) % 4 == 0) &&
                       (reinterpret_cast<uintptr_t>(codes) % 8 == 0) && (packed_cols % 4 == 0);
  if (whole_rows && aligned) {
    const int64_t words = rows * packed_cols / 4;
    hipLaunchKernelGGL(unpack_words_kernel, dim3(grid_for(words, 256)), dim3(256), 0, stream,
                       reinterpret_cast<const uint32_t*>(packed), reinterpret_cast<u32x2*>(codes),
                       words);
  } else {
    hipLaunchKernelGGL(unpack_bytes_kernel, dim3(grid_for(rows * packed_cols, 256)), dim3(256), 0,
                       stream, packed, codes, rows, packed_cols, columns);
  }
  return hipGetLastError();
}

template <class Out>
void launch_dequant_chunks(const LinearArgs& a, void* out, hipStream_t stream) {
  const int64_t chunks = a.K >> 3;
  const dim3 grid(unsigned((chunks + 255) / 256), unsigned(a.N < 65535 ? a.N : 65535));
  if (a.fmt == kNibble)
    hipLaunchKernelGGL((dequant_chunks_kernel<Out, kNibble>), grid, dim3(256), 0, stream, a, out);
  else
    hipLaunchKernelGGL((dequant_chunks_kernel<Out, kByte>), grid, dim3(256), 0, stream, a, out);
}

hipError_t launch_dequant(const LinearArgs& a, void* out, int out_dtype, hipStream_t stream) {
  if (a.N == 0 || a.K == 0) return hipSuccess;
  const uintptr_t qa = reinterpret_cast<uintptr_t>(a.qw);
  const int64_t code_align = a.fmt == kNibble ? 4 : 8;
  const bool chunked = a.K % 8 == 0 && a.group % 8 == 0 && a.ldq % code_align == 0 &&
                       qa % code_align == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                       (a.K >> 3) <= int64_t(65535) * 256;
  // Nibble codes into a 16-bit dense weight, rows of whole 2048-code chunks: the line kernel.
  const bool lines = a.fmt == kNibble && out_dtype != kDtF32 && a.K % 2048 == 0 && a.group % 8 == 0 &&
                     a.ldq % 4 == 0 && qa % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                     a.N * (a.K >> 11) <= int64_t(0x7FFFFFFF) * 4;
  if (lines) {
    const int64_t tasks = a.N * (a.K >> 11);
    const dim3 grid(unsigned((tasks + 3) / 4));
    if (out_dtype == kDtBf16)
      hipLaunchKernelGGL(dequant_lines_kernel<ActBf16>, grid, dim3(256), 0, stream, a, out);
    else
      hipLaunchKernelGGL(dequant_lines_kernel<ActF16>, grid, dim3(256), 0, stream, a, out);
    return hipGetLastError();
  }
  if (chunked) {
    switch (out_dtype) {
      case kDtF32: launch_dequant_chunks<ActF32>(a, out, stream); break;
      case kDtF16: launch_dequant_chunks<ActF16>(a, out, stream); break;
      case kDtBf16: launch_dequant_chunks<ActBf16>(a, out, stream); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  const dim3 grid(grid_for(a.N * ((a.K + 7) / 8), 256));
  switch (out_dtype) {
    case kDtF32:
      hipLaunchKernelGGL(dequant_kernel<ActF32>, grid, dim3(256), 0, stream, a, out);
      break;
    case kDtF16:
      hipLaunchKernelGGL(dequant_kernel<ActF16>, grid, dim3(256), 0, stream, a, out);
      break;
    case kDtBf16:
      hipLaunchKernelGGL(dequant_kernel<ActBf16>, grid, dim3(256), 0, stream, a, out);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

namespace {
template <class Act>
__global__ void __launch_bounds__(256) swiglu_combine_kernel(const typename Act::raw* t, int64_t ldt,
                                                             typename Act::raw* y, int64_t ldy, int64_t M,
                                                             int64_t I) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= M * I) return;
  const int64_t m = i / I;
  const int64_t f = i - m * I;
  const int64_t col = (f >> 2) * 8 + (f & 3);  // gate; the matching up column is col + 4
  y[m * ldy + f] = Act::store(swiglu<Act>(Act::load(t[m * ldt + col]), Act::load(t[m * ldt + col + 4])));
}
// The same with one thread per block of eight fused columns (four gate, four up): one 16-byte
// load (two for fp32) and one 8-byte store (16 for fp32) instead of eight 2-byte loads and four
// stores -- the product of a long prefill batch is hundreds of MB, read once.
template <class Act>
__global__ void __launch_bounds__(256) swiglu_combine_vec_kernel(const typename Act::raw* t, int64_t ldt,
                                                                 typename Act::raw* y, int64_t ldy, int64_t M,
                                                                 int64_t P) {
  using Raw = typename Act::raw;
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= M * P) return;
  const int64_t m = i / P;
  const int64_t p = i - m * P;
  const Raw* src = t + m * ldt + 8 * p;
  float g[4], u[4];
  if constexpr (sizeof(Raw) == 2) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(src);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      g[2 * r] = Act::load(Raw(w[r] & 0xFFFFu));
      g[2 * r + 1] = Act::load(Raw(w[r] >> 16));
      u[2 * r] = Act::load(Raw(w[2 + r] & 0xFFFFu));
      u[2 * r + 1] = Act::load(Raw(w[2 + r] >> 16));
    }
    uint32_t o[2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
      o[r] = uint32_t(Act::store(swiglu<Act>(g[2 * r], u[2 * r]))) |
             (uint32_t(Act::store(swiglu<Act>(g[2 * r + 1], u[2 * r + 1]))) << 16);
    *reinterpret_cast<u32x2*>(y + m * ldy + 4 * p) = u32x2{o[0], o[1]};
  } else {
    const f32x4 gv = *reinterpret_cast<const f32x4*>(src);
    const f32x4 uv = *reinterpret_cast<const f32x4*>(src + 4);
    f32x4 o;
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = Act::store(swiglu<Act>(gv[r], uv[r]));
    *reinterpret_cast<f32x4*>(y + m * ldy + 4 * p) = o;
  }
}
// Sixteen fused columns per thread for 16-bit activations (two 16-byte loads, one 16-byte
// store): twice the bytes in flight per thread of swiglu_combine_vec_kernel.
template <class Act>
__global__ void __launch_bounds__(256) swiglu_combine_vec2_kernel(const typename Act::raw* t, int64_t ldt,
                                                                  typename Act::raw* y, int64_t ldy, int64_t M,
                                                                  int64_t P2) {
  using Raw = typename Act::raw;
  static_assert(sizeof(Raw) == 2, "16-bit activations");
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= M * P2) return;
  const int64_t m = i / P2;
  const int64_t p = i - m * P2;
  const Raw* src = t + m * ldt + 16 * p;
  const u32x4 v0 = *reinterpret_cast<const u32x4*>(src);
  const u32x4 v1 = *reinterpret_cast<const u32x4*>(src + 8);
  const uint32_t w[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
  uint32_t o[4];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      // Block b: gate words 4b, 4b + 1, up words 4b + 2, 4b + 3 (four gate, four up columns).
      const uint32_t gw = w[4 * b + r], uw = w[4 * b + 2 + r];
      const float lo = swiglu<Act>(Act::load(Raw(gw & 0xFFFFu)), Act::load(Raw(uw & 0xFFFFu)));
      const float hi = swiglu<Act>(Act::load(Raw(gw >> 16)), Act::load(Raw(uw >> 16)));
      o[2 * b + r] = uint32_t(Act::store(lo)) | (uint32_t(Act::store(hi)) << 16);
    }
  *reinterpret_cast<u32x4*>(y + m * ldy + 8 * p) = u32x4{o[0], o[1], o[2], o[3]};
}
}  // namespace

hipError_t launch_swiglu_combine(const void* t, int64_t ldt, void* y, int64_t ldy, int64_t M, int64_t N,
                                 int act, hipStream_t stream) {
  const int64_t I = N / 2;
  const int64_t total = M * I;
  if (total == 0) return hipSuccess;
  const size_t es = act == kDtF32 ? 4 : 2;
  const bool vec = N % 8 == 0 && reinterpret_cast<uintptr_t>(t) % 16 == 0 && (ldt * es) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(y) % (4 * es) == 0 && (ldy * es) % (4 * es) == 0;
  if (vec && es == 2 && N % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0 && (ldy * es) % 16 == 0) {
    const int64_t P2 = N / 16;
    const dim3 grid(unsigned((M * P2 + 255) / 256)), block(256);
    if (act == kDtBf16)
      hipLaunchKernelGGL(swiglu_combine_vec2_kernel<ActBf16>, grid, block, 0, stream,
                         static_cast<const uint16_t*>(t), ldt, static_cast<uint16_t*>(y), ldy, M, P2);
    else
      hipLaunchKernelGGL(swiglu_combine_vec2_kernel<ActF16>, grid, block, 0, stream,
                         static_cast<const uint16_t*>(t), ldt, static_cast<uint16_t*>(y), ldy, M, P2);
    return hipGetLastError();
  }
  if (vec) {
    const int64_t P = N / 8;
    const dim3 grid(unsigned((M * P + 255) / 256)), block(256);
    if (act == kDtBf16)
      hipLaunchKernelGGL(swiglu_combine_vec_kernel<ActBf16>, grid, block, 0, stream,
                         static_cast<const uint16_t*>(t), ldt, static_cast<uint16_t*>(y), ldy, M, P);
    else if (act == kDtF16)
      hipLaunchKernelGGL(swiglu_combine_vec_kernel<ActF16>, grid, block, 0, stream,
                         static_cast<const uint16_t*>(t), ldt, static_cast<uint16_t*>(y), ldy, M, P);
    else
      hipLaunchKernelGGL(swiglu_combine_vec_kernel<ActF32>, grid, block, 0, stream, static_cast<const float*>(t),
                         ldt, static_cast<float*>(y), ldy, M, P);
    return hipGetLastError();
  }
  const dim3 grid(unsigned((total + 255) / 256)), block(256);
  if (act == kDtBf16)
    hipLaunchKernelGGL(swiglu_combine_kernel<ActBf16>, grid, block, 0, stream,
                       static_cast<const uint16_t*>(t), ldt, static_cast<uint16_t*>(y), ldy, M, I);
  else if (act == kDtF16)
    hipLaunchKernelGGL(swiglu_combine_kernel<ActF16>, grid, block, 0, stream,
                       static_cast<const uint16_t*>(t), ldt, static_cast<uint16_t*>(y), ldy, M, I);
  else
    hipLaunchKernelGGL(swiglu_combine_kernel<ActF32>, grid, block, 0, stream, static_cast<const float*>(t),
                       ldt, static_cast<float*>(y), ldy, M, I);
  return hipGetLastError();
}

}  // namespace llmopt
