// The decoder's per-token elementwise steps as single kernels, with the reference's roundings.
//
// Replaces, on HIP devices:
//   * RMSNorm.forward (src/llmopt/model/layers.py:14-31): y = x * rsqrt(mean(x^2) + eps) * w in
//     fp32, rounded once to the activation dtype -- and, fused in front of it, the residual add
//     of DecoderLayer.forward (layers.py:185-195), h = x + r rounded to the activation dtype as
//     torch's bf16/fp16 add rounds it, with h written out as the new residual stream;
//   * apply_rotary_pos_emb with RotaryEmbedding.forward (src/llmopt/model/rotary.py:23-45,
//     85-102) for q and k together: the fp32 cos/sin tables cast to the activation dtype, then
//     q * cos + rotate_half(q) * sin with each product and the sum rounded to the activation
//     dtype, as torch evaluates the expression op by op -- so the result is bit-identical; v is
//     copied alongside k into a contiguous buffer for the cache write.
// torch runs these as about 8 (norm) and 14 (rotary) separate kernels per layer and step.
#include "qcommon.hpp"
#include "qkernels.hpp"

namespace llmopt {
namespace {

template <class Act>
__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = Act::load(typename Act::raw(w[i] & 0xFFFFu));
    f[2 * i + 1] = Act::load(typename Act::raw(w[i] >> 16));
  }
}

template <class Act>
__device__ __forceinline__ u32x4 pack8(const float* f) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = uint32_t(Act::store(f[2 * i])) | (uint32_t(Act::store(f[2 * i + 1])) << 16);
  return u32x4{w[0], w[1], w[2], w[3]};
}

// One workgroup of 256 threads per row; 16-byte accesses (the host checks hidden % 8 == 0 and
// 16-byte aligned rows). Pass 1 forms h (with the residual, if any), stores it and sums h^2;
// pass 2 re-reads h (from L2) and normalizes.
template <class Act>
__global__ void __launch_bounds__(256) rmsnorm_kernel(const RmsNormArgs a) {
  using Raw = typename Act::raw;
  const int64_t row = blockIdx.x;
  const Raw* x = a.x ? static_cast<const Raw*>(a.x) + row * a.ldx : nullptr;
  const Raw* r = a.residual ? static_cast<const Raw*>(a.residual) + row * a.ldr : nullptr;
  Raw* h_out = a.h_out ? static_cast<Raw*>(a.h_out) + row * a.ldh : nullptr;
  Raw* y = static_cast<Raw*>(a.y) + row * a.ldy;
  const Raw* w = static_cast<const Raw*>(a.weight);
  const int tid = threadIdx.x;

  float ss = 0.0f;
  for (int64_t e = int64_t(tid) * 8; e < a.hidden; e += 256 * 8) {
    float h[8];
    if (a.planes) {
      // x = the partial sums added in slice order, plus the bias, rounded: the split-K
      // reduction's arithmetic.
      const size_t plane = size_t(a.rows) * size_t(a.hidden);
      const float* p = a.planes + size_t(row) * size_t(a.hidden) + e;
      f32x4 lo = *reinterpret_cast<const f32x4*>(p), hi = *reinterpret_cast<const f32x4*>(p + 4);
      for (int64_t s = 1; s < a.splits; ++s) {
        const f32x4 l2 = *reinterpret_cast<const f32x4*>(p + s * plane);
        const f32x4 h2 = *reinterpret_cast<const f32x4*>(p + s * plane + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lo[i] += l2[i];
          hi[i] += h2[i];
        }
      }
      const Raw* pb = static_cast<const Raw*>(a.plane_bias);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        h[i] = Act::load(Act::store(pb ? lo[i] + Act::load(pb[e + i]) : lo[i]));
        h[4 + i] = Act::load(Act::store(pb ? hi[i] + Act::load(pb[e + 4 + i]) : hi[i]));
      }
    } else {
      unpack8<Act>(*reinterpret_cast<const u32x4*>(x + e), h);
    }
    if (r) {
      float rv[8];
      unpack8<Act>(*reinterpret_cast<const u32x4*>(r + e), rv);
#pragma unroll
      for (int i = 0; i < 8; ++i) h[i] = Act::load(Act::store(rv[i] + h[i]));
      *reinterpret_cast<u32x4*>(h_out + e) = pack8<Act>(h);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(h[i], h[i], ss);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  __shared__ float part[4];
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  const float total = (part[0] + part[1]) + (part[2] + part[3]);
  const float inv = __frsqrt_rn(total / float(a.hidden) + a.eps);

  const Raw* src = r ? h_out : x;
  for (int64_t e = int64_t(tid) * 8; e < a.hidden; e += 256 * 8) {
    float h[8], wv[8], o[8];
    unpack8<Act>(*reinterpret_cast<const u32x4*>(src + e), h);
    unpack8<Act>(*reinterpret_cast<const u32x4*>(w + e), wv);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = __fmul_rn(__fmul_rn(h[i], inv), wv[i]);
    *reinterpret_cast<u32x4*>(y + e) = pack8<Act>(o);
  }
}

// The same for rows of 512 to 8192 elements (hidden % 512 == 0): one thread per 8 elements,
// hidden / 8 threads per row, h kept in registers between the two passes, every load of a row
// issued before the first wait. Rows of a linear's partial sums (a.planes) read S planes per
// element: one launch with all of them in flight instead of a reduction kernel and a norm.
template <class Act>
__global__ void __launch_bounds__(1024) rmsnorm_rows_kernel(const RmsNormArgs a) {
  using Raw = typename Act::raw;
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t e = int64_t(tid) * 8;
  const Raw* w = static_cast<const Raw*>(a.weight);
  float h[8];
  if (a.planes) {
    const size_t plane = size_t(a.rows) * size_t(a.hidden);
    const float* p = a.planes + size_t(row) * size_t(a.hidden) + e;
    f32x4 lo = *reinterpret_cast<const f32x4*>(p), hi = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll 4
    for (int64_t s = 1; s < a.splits; ++s) {
      const f32x4 l2 = *reinterpret_cast<const f32x4*>(p + s * plane);
      const f32x4 h2 = *reinterpret_cast<const f32x4*>(p + s * plane + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lo[i] += l2[i];
        hi[i] += h2[i];
      }
    }
    const Raw* pb = static_cast<const Raw*>(a.plane_bias);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h[i] = Act::load(Act::store(pb ? lo[i] + Act::load(pb[e + i]) : lo[i]));
      h[4 + i] = Act::load(Act::store(pb ? hi[i] + Act::load(pb[e + 4 + i]) : hi[i]));
    }
  } else {
    unpack8<Act>(*reinterpret_cast<const u32x4*>(static_cast<const Raw*>(a.x) + row * a.ldx + e), h);
  }
  if (a.residual) {
    float rv[8];
    unpack8<Act>(*reinterpret_cast<const u32x4*>(static_cast<const Raw*>(a.residual) + row * a.ldr + e), rv);
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = Act::load(Act::store(rv[i] + h[i]));
    *reinterpret_cast<u32x4*>(static_cast<Raw*>(a.h_out) + row * a.ldh + e) = pack8<Act>(h);
  }
  float wv[8];
  unpack8<Act>(*reinterpret_cast<const u32x4*>(w + e), wv);
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(h[i], h[i], ss);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  __shared__ float part[16];
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  const int nw = int(blockDim.x) >> 6;
  float total = part[0];
  for (int i = 1; i < nw; ++i) total += part[i];
  const float inv = __frsqrt_rn(total / float(a.hidden) + a.eps);
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = __fmul_rn(__fmul_rn(h[i], inv), wv[i]);
  *reinterpret_cast<u32x4*>(static_cast<Raw*>(a.y) + row * a.ldy + e) = pack8<Act>(o);
}

// Grid (token, chunk of 256 pairs); a thread per (head, i < D/2) pair rotates dims i and
// i + D/2 of q or k, and for the KV heads also copies v's dims i and i + D/2 (when v is given),
// so that the cache write that follows reads contiguous rows.
template <class Act>
__global__ void __launch_bounds__(256) rope_kernel(const RopeArgs a) {
  using Raw = typename Act::raw;
  const int64_t t = blockIdx.x;
  const int half = int(a.head_dim / 2);
  const int64_t j = int64_t(blockIdx.y) * 256 + threadIdx.x;
  if (j >= (a.heads + a.kv_heads) * half) return;
  int64_t p = a.positions[t];
  p = p < 0 ? 0 : (p >= a.table_rows ? a.table_rows - 1 : p);  // the host checks the range
  const float* cs = a.cos_table + p * a.head_dim;
  const float* sn = a.sin_table + p * a.head_dim;
  const int64_t head = j / half;
  const int i = int(j - head * half);
  const bool is_q = head < a.heads;
  const int64_t hh = is_q ? head : head - a.heads;
  const Raw* src = static_cast<const Raw*>(is_q ? a.q : a.k) + t * (is_q ? a.ldq : a.ldk) + hh * a.head_dim;
  Raw* dst = static_cast<Raw*>(is_q ? a.q_out : a.k_out) + (t * (is_q ? a.heads : a.kv_heads) + hh) * a.head_dim;
  Raw* vd = a.v_out ? static_cast<Raw*>(a.v_out) + (t * a.kv_heads + hh) * a.head_dim : nullptr;
  if (!is_q && a.key_cache) {
    // The decode cache write (paged_cache.py:246-277): block block_ids[t, off / B], replaced by
    // block 0 outside [0, num_blocks); an offset past the table row writes nothing.
    const int64_t off = a.offsets[t];
    const int64_t index = off >= 0 ? off / a.block_size : -1;
    if (index < 0 || index >= a.ldb) return;
    int64_t block = a.block_ids[t * a.ldb + index];
    if (block < 0 || block >= a.num_blocks) block = 0;
    const int64_t row = ((block * a.block_size + off % a.block_size) * a.kv_heads + hh) * a.head_dim;
    dst = static_cast<Raw*>(a.key_cache) + row;
    vd = static_cast<Raw*>(a.value_cache) + row;
  }
  const float x1 = Act::load(src[i]), x2 = Act::load(src[i + half]);
  // The tables are cast to the activation dtype first (cos.to(q.dtype)).
  const float c1 = Act::load(Act::store(cs[i])), s1 = Act::load(Act::store(sn[i]));
  const float c2 = Act::load(Act::store(cs[i + half])), s2 = Act::load(Act::store(sn[i + half]));
  // rotate_half(x) = [-x2, x1]; every product and the sum rounded as torch rounds them.
  const float lo = Act::load(Act::store(Act::load(Act::store(x1 * c1)) + Act::load(Act::store(-x2 * s1))));
  const float hi = Act::load(Act::store(Act::load(Act::store(x2 * c2)) + Act::load(Act::store(x1 * s2))));
  dst[i] = Act::store(lo);
  dst[i + half] = Act::store(hi);
  if (!is_q && a.v) {
    const Raw* vs = static_cast<const Raw*>(a.v) + t * a.ldv + hh * a.head_dim;
    vd[i] = vs[i];
    vd[i + half] = vs[i + half];
  }
}

// rope_kernel for 16-byte aligned rows (a.vec, checked on the host; head_dim % 16 == 0): a thread
// per (head, 8 consecutive pairs i0 .. i0 + 7), the same arithmetic on 16-byte loads and stores.
template <class Act>
__global__ void __launch_bounds__(256) rope_vec_kernel(const RopeArgs a) {
  using Raw = typename Act::raw;
  const int64_t t = blockIdx.x;
  const int half = int(a.head_dim / 2);
  const int64_t g = int64_t(blockIdx.y) * 256 + threadIdx.x;
  if (g * 8 >= (a.heads + a.kv_heads) * half) return;
  int64_t p = a.positions[t];
  p = p < 0 ? 0 : (p >= a.table_rows ? a.table_rows - 1 : p);  // the host checks the range
  const int64_t head = (g * 8) / half;
  const int i0 = int(g * 8 - head * half);
  const bool is_q = head < a.heads;
  const int64_t hh = is_q ? head : head - a.heads;
  const Raw* src = static_cast<const Raw*>(is_q ? a.q : a.k) + t * (is_q ? a.ldq : a.ldk) + hh * a.head_dim;
  Raw* dst = static_cast<Raw*>(is_q ? a.q_out : a.k_out) + (t * (is_q ? a.heads : a.kv_heads) + hh) * a.head_dim;
  float x1[8], x2[8], c1[8], s1[8], c2[8], s2[8];
  unpack8<Act>(*reinterpret_cast<const u32x4*>(src + i0), x1);
  unpack8<Act>(*reinterpret_cast<const u32x4*>(src + i0 + half), x2);
  const float* cs = a.cos_table + p * a.head_dim;
  const float* sn = a.sin_table + p * a.head_dim;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const f32x4 ca = *reinterpret_cast<const f32x4*>(cs + i0 + 4 * h);
    const f32x4 sa = *reinterpret_cast<const f32x4*>(sn + i0 + 4 * h);
    const f32x4 cb = *reinterpret_cast<const f32x4*>(cs + i0 + half + 4 * h);
    const f32x4 sb = *reinterpret_cast<const f32x4*>(sn + i0 + half + 4 * h);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // The tables are cast to the activation dtype first (cos.to(q.dtype)).
      c1[4 * h + e] = Act::load(Act::store(ca[e]));
      s1[4 * h + e] = Act::load(Act::store(sa[e]));
      c2[4 * h + e] = Act::load(Act::store(cb[e]));
      s2[4 * h + e] = Act::load(Act::store(sb[e]));
    }
  }
  float lo[8], hi[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    // rotate_half(x) = [-x2, x1]; every product and the sum rounded as torch rounds them.
    lo[e] = Act::load(Act::store(Act::load(Act::store(x1[e] * c1[e])) + Act::load(Act::store(-x2[e] * s1[e]))));
    hi[e] = Act::load(Act::store(Act::load(Act::store(x2[e] * c2[e])) + Act::load(Act::store(x1[e] * s2[e]))));
  }
  *reinterpret_cast<u32x4*>(dst + i0) = pack8<Act>(lo);
  *reinterpret_cast<u32x4*>(dst + i0 + half) = pack8<Act>(hi);
  if (!is_q && a.v) {
    const Raw* vs = static_cast<const Raw*>(a.v) + t * a.ldv + hh * a.head_dim;
    Raw* vd = static_cast<Raw*>(a.v_out) + (t * a.kv_heads + hh) * a.head_dim;
    *reinterpret_cast<u32x4*>(vd + i0) = *reinterpret_cast<const u32x4*>(vs + i0);
    *reinterpret_cast<u32x4*>(vd + i0 + half) = *reinterpret_cast<const u32x4*>(vs + i0 + half);
  }
}

// Greedy sampling's argmax over each row (the reference's greedy sampler, torch.argmax(logits,
// dim=-1), src/llmopt/engine/sampler.py:94-95): the index of the first maximum, a NaN counting
// as larger than every number (the first NaN wins), as torch returns it. One workgroup of 1024
// threads per row; thread t takes the 8-element pieces t, t + 1024, ... of the row, sixteen loads
// in flight at a time, then the workgroup combines the threads' winners.
__device__ __forceinline__ bool argmax_gt(float a, float b) { return (a != a && b == b) || a > b; }

__device__ __forceinline__ void argmax_take(float& v, int64_t& i, float v2, int64_t i2) {
  if (argmax_gt(v2, v) || (!argmax_gt(v, v2) && i2 < i)) v = v2, i = i2;
}

template <class T>
__device__ __forceinline__ float argmax_load(const void* x, int64_t idx, int dtype) {
  if constexpr (sizeof(T) == 4) return static_cast<const float*>(x)[idx];
  const uint16_t h = static_cast<const uint16_t*>(x)[idx];
  return dtype == kDtF16 ? f16_to_f32(h) : bf16_to_f32(h);
}

template <class T>
__global__ void __launch_bounds__(1024) argmax_rows_kernel(const ArgmaxArgs a) {
  constexpr int kPer = 16 / sizeof(T);  // elements per 16-byte piece
  constexpr int kAhead = 16;
  const int64_t row = blockIdx.x;
  const int tid = int(threadIdx.x);
  const T* x = static_cast<const T*>(a.x) + row * a.ldx;
  float best = -__int_as_float(0x7F800000);
  int64_t at = INT64_MAX;
  const int64_t pieces = a.vec ? a.cols / kPer : 0;
  for (int64_t base = 0; base < pieces; base += 1024 * kAhead) {
    u32x4 v[kAhead];
#pragma unroll
    for (int u = 0; u < kAhead; ++u) {
      const int64_t c = base + tid + 1024 * u;
      v[u] = *reinterpret_cast<const u32x4*>(x + kPer * (c < pieces ? c : 0));
    }
#pragma unroll
    for (int u = 0; u < kAhead; ++u) {
      const int64_t c = base + tid + 1024 * u;
      const bool in = c < pieces;  // a predicate, not a branch: the loads above stay in flight together
      const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        float f;
        if constexpr (sizeof(T) == 4)
          f = __uint_as_float(w[e]);
        else {
          const uint16_t h = uint16_t(w[e / 2] >> (16 * (e % 2)));
          f = a.dtype == kDtF16 ? f16_to_f32(h) : bf16_to_f32(h);
        }
        // Pieces and their elements come in increasing index order: a strict comparison keeps
        // the first of equal values.
        const bool take = in && argmax_gt(f, best);
        best = take ? f : best;
        at = take ? kPer * c + e : at;
      }
    }
  }
  for (int64_t j = pieces * kPer + tid; j < a.cols; j += 1024) {  // the tail, or every element
    const float f = argmax_load<T>(x, j, a.dtype);
    if (argmax_gt(f, best)) best = f, at = j;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float v2 = __shfl_xor(best, off, 64);
    const int64_t i2 = __shfl_xor(at, off, 64);
    argmax_take(best, at, v2, i2);
  }
  __shared__ float wv[16];
  __shared__ int64_t wi[16];
  const int lane = tid & 63, wave = tid >> 6;
  if (lane == 0) wv[wave] = best, wi[wave] = at;
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < int(blockDim.x >> 6); ++w) argmax_take(best, at, wv[w], wi[w]);
    a.out[row] = at == INT64_MAX ? 0 : at;
  }
}

}  // namespace

hipError_t launch_rmsnorm(const RmsNormArgs& a, hipStream_t stream) {
  if (a.rows == 0) return hipSuccess;
  if (a.hidden % 512 == 0 && a.hidden <= 8192) {
    const dim3 block(unsigned(a.hidden / 8));
    if (a.dtype == kDtBf16)
      hipLaunchKernelGGL(rmsnorm_rows_kernel<ActBf16>, dim3(unsigned(a.rows)), block, 0, stream, a);
    else
      hipLaunchKernelGGL(rmsnorm_rows_kernel<ActF16>, dim3(unsigned(a.rows)), block, 0, stream, a);
    return hipGetLastError();
  }
  if (a.dtype == kDtBf16)
    hipLaunchKernelGGL(rmsnorm_kernel<ActBf16>, dim3(unsigned(a.rows)), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<ActF16>, dim3(unsigned(a.rows)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_rope(const RopeArgs& a, hipStream_t stream) {
  if (a.tokens == 0) return hipSuccess;
  if (a.vec && !a.key_cache) {
    const dim3 grid(unsigned(a.tokens), unsigned(((a.heads + a.kv_heads) * (a.head_dim / 16) + 255) / 256));
    if (a.dtype == kDtBf16)
      hipLaunchKernelGGL(rope_vec_kernel<ActBf16>, grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL(rope_vec_kernel<ActF16>, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
  }
  const dim3 grid(unsigned(a.tokens), unsigned(((a.heads + a.kv_heads) * (a.head_dim / 2) + 255) / 256));
  if (a.dtype == kDtBf16)
    hipLaunchKernelGGL(rope_kernel<ActBf16>, grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(rope_kernel<ActF16>, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_argmax_rows(const ArgmaxArgs& a, hipStream_t stream) {
  if (a.rows == 0) return hipSuccess;
  if (a.dtype == kDtF32)
    hipLaunchKernelGGL(argmax_rows_kernel<float>, dim3(unsigned(a.rows)), dim3(1024), 0, stream, a);
  else
    hipLaunchKernelGGL(argmax_rows_kernel<uint16_t>, dim3(unsigned(a.rows)), dim3(1024), 0, stream, a);
  return hipGetLastError();
}

}  // namespace llmopt
