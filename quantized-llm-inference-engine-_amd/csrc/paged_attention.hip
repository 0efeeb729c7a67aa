// Paged KV-cache writes and decode attention straight from the block table.
//
// Replaces, on the decode path (one query token per sequence):
//   * PagedKVCache.write_decode / write (src/llmopt/cache/paged_cache.py:187-277): one kernel
//     scatters each sequence's new K/V rows into their blocks, instead of an indexed assignment
//     (decode) or a Python loop over sequences and blocks (prefill);
//   * PagedAttention.forward with q_len == 1 (src/llmopt/attention/paged_attention.py:145-182,
//     218-290): the reference first gathers every sequence's K/V into a padded dense tensor
//     (paged_cache.py:279-324), repeats each KV head for its query heads, and runs matmul /
//     softmax / matmul. Here each workgroup reads its sequence's blocks in place, once per KV
//     head for all the query heads that share it.
//
// Cache layout (the reference's): [num_blocks, block_size, kv_heads, head_dim] per layer, so one
// token of one KV head is a contiguous head_dim row. Token t of sequence s sits in block
// block_ids[s, t / block_size] at slot t % block_size; it is a key of the query iff
// t < context_lens[s] and that block id is >= 0.
//
// Decode attention, per workgroup = one wave = (sequence, KV head, context split):
//   * 16-token tiles. Scores S[token][head] = K Q^T * scale on v_mfma_f32_16x16x32: the A operand
//     is 16 tokens x 32 dims of K (16 bytes per lane, read straight from the cache), the B operand
//     the group's query heads (columns >= group are zero), HD / 32 MFMAs per tile;
//   * online softmax per head in fp32 (running max and sum), masked tokens contribute nothing;
//   * P V on the VALU with lanes over head dims (HD / 64 dims per lane): each token's V row is one
//     coalesced 256-byte read per wave, the tile's probabilities come from LDS as broadcasts;
//   * two or three tiles of K and V, and the block ids of as many after them, are in flight
//     while a tile is computed;
//   * with several splits each wave writes its normalized partial output and log-sum-exp, and a
//     merge kernel combines them (the reference's merge_states, paged_attention.py:30-56).
// Everything is computed in fp32 and rounded once into the query dtype; the reference rounds
// its scores, probabilities and partial outputs to the cache dtype on the way.
#include "qcommon.hpp"
#include "qkernels.hpp"

namespace llmopt {
namespace {

template <class C>
struct Mfma16x32;
template <>
struct Mfma16x32<ActBf16> {
  __device__ static f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
};
template <>
struct Mfma16x32<ActF16> {
  __device__ static f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
};

__device__ __forceinline__ float load_any(const void* p, int64_t i, int dtype) {
  switch (dtype) {
    case kDtF32: return static_cast<const float*>(p)[i];
    case kDtF16: return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
    default: return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
}

__device__ __forceinline__ void store_any(void* p, int64_t i, int dtype, float v) {
  switch (dtype) {
    case kDtF32: static_cast<float*>(p)[i] = v; break;
    case kDtF16: static_cast<uint16_t*>(p)[i] = f32_to_f16_rne(v); break;
    default: static_cast<uint16_t*>(p)[i] = f32_to_bf16_rne(v); break;
  }
}

// ---- cache writes ------------------------------------------------------------------------------

// One token of one sequence: copy (and convert) its kv_heads x head_dim row of K and V.
__device__ __forceinline__ void copy_token(const KvWriteArgs& a, int64_t src_row, int64_t block, int64_t slot) {
  const int64_t width = a.kv_heads * a.head_dim;
  const int64_t dst = (block * a.block_size + slot) * width;
  for (int64_t e = threadIdx.x; e < width; e += blockDim.x) {
    store_any(a.key_cache, dst + e, a.cache_dtype, load_any(a.keys, src_row + e, a.src_dtype));
    store_any(a.value_cache, dst + e, a.cache_dtype, load_any(a.values, src_row + e, a.src_dtype));
  }
}

// write_decode (paged_cache.py:246-277): token offsets[s] of sequence s. A block id outside
// [0, num_blocks) is replaced by block 0, as the reference does; an offset outside the table
// (which makes the reference raise) writes nothing.
__global__ void __launch_bounds__(256) kv_write_decode_kernel(const KvWriteArgs a) {
  const int64_t s = blockIdx.x;
  const int64_t off = a.offsets[s];
  const int64_t index = off >= 0 ? off / a.block_size : -1;
  if (index < 0 || index >= a.ldb) return;
  int64_t block = a.block_ids[s * a.ldb + index];
  if (block < 0 || block >= a.num_blocks) block = 0;
  copy_token(a, s * a.src_seq_stride, block, off % a.block_size);
}

// write (paged_cache.py:187-244): tokens offsets[s] + j, j < q_len; a sequence stops at the
// end of its table row or at its first -1 block (the reference's loop breaks there).
__global__ void __launch_bounds__(256) kv_write_kernel(const KvWriteArgs a) {
  const int64_t s = blockIdx.y;
  const int64_t j = blockIdx.x;
  const int64_t start = a.offsets[s];
  if (start < 0) return;
  const int64_t pos = start + j;
  const int64_t index = pos / a.block_size;
  if (index >= a.ldb) return;
  for (int64_t i = start / a.block_size; i <= index; ++i)
    if (a.block_ids[s * a.ldb + i] < 0) return;
  const int64_t block = a.block_ids[s * a.ldb + index];
  if (block >= a.num_blocks) return;
  copy_token(a, s * a.src_seq_stride + j * a.src_token_stride, block, pos % a.block_size);
}

// ---- decode attention --------------------------------------------------------------------------

template <class C, int HD, int GQ>
__global__ void __launch_bounds__(64) paged_decode_kernel(const PagedDecodeArgs a) {
  using Raw = typename C::raw;
  constexpr int kNm = HD / 32;  // MFMAs per tile (32 dims each)
  constexpr int kDpl = HD / 64;  // head dims per lane in P V
  const int lane = threadIdx.x;
  const int col = lane & 15;
  const int kb = lane >> 4;
  const int64_t split = blockIdx.x, kvh = blockIdx.y, s = blockIdx.z;
  const int64_t ctx = a.context_lens[s];
  const int64_t t_begin = split * a.tiles_per_split * 16;
  const int64_t t_end = ctx < t_begin + a.tiles_per_split * 16 ? ctx : t_begin + a.tiles_per_split * 16;
  const int64_t row_stride = a.kv_heads * HD;  // elements between two slots
  const uint32_t cache_bytes = uint32_t(a.num_blocks * a.block_size * row_stride * int64_t(sizeof(Raw)));
  const auto krs = make_rsrc(a.key_cache, cache_bytes);
  const auto vrs = make_rsrc(a.value_cache, cache_bytes);
  const uint32_t row_bytes = uint32_t(row_stride * int64_t(sizeof(Raw)));
  const uint32_t head_off = uint32_t(kvh * HD * int64_t(sizeof(Raw)));
  const uint32_t v_lane_off = uint32_t(kDpl * lane * int(sizeof(Raw)));
  const int32_t* const table = a.block_ids + s * a.ldb;

  __shared__ float p_lds[16][GQ < 4 ? 4 : GQ];  // [token][head]
  __shared__ float a_lds[GQ < 4 ? 4 : GQ];      // per-head rescale of the running output
  __shared__ float l_lds[GQ < 4 ? 4 : GQ];

  // Query heads kvh * GQ + col (col < GQ) as the B operand, cast to the cache dtype (q.to(k.dtype)).
  u32x4 qf[kNm];
  {
    const bool hv = col < GQ;
    const int64_t h = kvh * GQ + (hv ? col : 0);
#pragma unroll
    for (int m = 0; m < kNm; ++m) {
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t d = 32 * m + 8 * kb + 2 * e;
        const float x0 = hv ? load_any(a.query, s * a.q_seq_stride + h * HD + d, a.q_dtype) : 0.0f;
        const float x1 = hv ? load_any(a.query, s * a.q_seq_stride + h * HD + d + 1, a.q_dtype) : 0.0f;
        w[e] = uint32_t(C::store(x0)) | (uint32_t(C::store(x1)) << 16);
      }
      qf[m] = u32x4{w[0], w[1], w[2], w[3]};
    }
  }

  // Slot row (block * block_size + slot) of token t0 + col, or -1 when that token is not a key.
  // 32-bit arithmetic: contexts, table widths and slot rows stay below 2^31 (checked on the host).
  const uint32_t bsz = uint32_t(a.block_size);
  const uint32_t ldb32 = uint32_t(a.ldb);
  const uint32_t nblk = uint32_t(a.num_blocks);
  const uint32_t t_end32 = uint32_t(t_end > 0 ? t_end : 0);
  auto fetch_row = [&](int64_t t0) -> int32_t {
    const uint32_t t = uint32_t(t0) + uint32_t(col);
    const uint32_t bi = t / bsz;
    int32_t block = -1;
    if (t < t_end32 && bi < ldb32) block = table[bi];  // past the row: no key
    const bool ok = block >= 0 && uint32_t(block) < nblk;
    return ok ? int32_t(uint32_t(block) * bsz + (t - bi * bsz)) : -1;
  };
  // K of token t0 + col (dims 8kb .. of each 32-dim slice) and this lane's dims of V for all 16
  // tokens (slot rows broadcast with readlane, so each V row address is a scalar); masked tokens
  // read slot row 0. Buffer loads with 32-bit offsets (the host keeps a layer's cache under
  // 2 GiB), marked to stay in program order so that the ring below keeps them in flight.
  auto fetch_kv = [&](int32_t row, u32x4* kf, uint32_t* vf, uint32_t& valid_bits) {
    valid_bits = uint32_t(__builtin_amdgcn_ballot_w64(row >= 0) & 0xFFFFu);
    const uint32_t r_own = uint32_t(row >= 0 ? row : 0);
#pragma unroll
    for (int m = 0; m < kNm; ++m)
      kf[m] = buf_load16(krs, (r_own * row_bytes) + uint32_t(2 * (32 * m + 8 * kb)), head_off);
    const int32_t row0 = row >= 0 ? row : 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t r = uint32_t(__builtin_amdgcn_readlane(row0, j));
      if constexpr (kDpl == 2)
        vf[j] = __builtin_amdgcn_raw_buffer_load_b32(vrs, v_lane_off, int(r * row_bytes + head_off), kLoadInOrder);
      else
        vf[j] = uint32_t(__builtin_amdgcn_raw_buffer_load_b16(vrs, v_lane_off, int(r * row_bytes + head_off),
                                                              kLoadInOrder));
    }
  };

  const float neg_inf = -__int_as_float(0x7F800000);
  float m_run = neg_inf, l_run = 0.0f;  // for head `col`, replicated over the four lane rows
  float o[GQ][kDpl];
#pragma unroll
  for (int h = 0; h < GQ; ++h)
#pragma unroll
    for (int d = 0; d < kDpl; ++d) o[h][d] = 0.0f;

  // One tile: scores on the MFMA, online softmax, P V on the VALU.
  auto compute = [&](const u32x4* kf, const uint32_t* vf, uint32_t bits) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < kNm; ++m) acc = Mfma16x32<C>::run(kf[m], qf[m], acc);

    // Rows 4kb .. 4kb + 3 of the tile, column = head `col`.
    float sc[4];
    float tmax = neg_inf;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float x = acc[r] * a.scale;
      if (a.softcap > 0.0f) x = tanhf(x / a.softcap) * a.softcap;
      sc[r] = ((bits >> (4 * kb + r)) & 1u) ? x : neg_inf;
      tmax = fmaxf(tmax, sc[r]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const bool live = m_new != neg_inf;
    const float alpha = live ? __expf(m_run - m_new) : 1.0f;
    float psum = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float p = live ? __expf(sc[r] - m_new) : 0.0f;
      psum += p;
      if (col < GQ) p_lds[4 * kb + r][col] = p;
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = alpha * l_run + psum;
    m_run = m_new;
    if (lane < GQ) a_lds[lane] = alpha;
    __syncthreads();

#pragma unroll
    for (int h = 0; h < GQ; ++h) {
      const float al = a_lds[h];
#pragma unroll
      for (int d = 0; d < kDpl; ++d) o[h][d] *= al;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float v[kDpl];
      if constexpr (kDpl == 2) {
        v[0] = C::load(Raw(vf[j] & 0xFFFFu));
        v[1] = C::load(Raw(vf[j] >> 16));
      } else {
        v[0] = C::load(Raw(vf[j]));
      }
      if (!((bits >> j) & 1u)) {  // masked token: its slot may hold anything
#pragma unroll
        for (int d = 0; d < kDpl; ++d) v[d] = 0.0f;
      }
#pragma unroll
      for (int h = 0; h < GQ; ++h) {
        const float p = p_lds[j][h];
#pragma unroll
        for (int d = 0; d < kDpl; ++d) o[h][d] = __builtin_fmaf(p, v[d], o[h][d]);
      }
    }
    __syncthreads();
  };

  // A ring of kDepth tiles in flight. Slot u holds tile g + u of the current group; after it is
  // computed it is refilled with tile g + u + kDepth, whose slot rows were loaded kDepth tiles
  // earlier (rows[u]); the rows for the refill after that are loaded at the same time. The main
  // loop runs whole groups with unconditional loads (past the last tile they read slot row 0 and
  // are never used), so the loads keep one static order; the last partial group has no refills.
  constexpr int kDepth = GQ >= 16 ? 1 : GQ >= 8 ? 2 : 3;  // registers: larger groups keep more accumulators
  u32x4 kf[kDepth][kNm];
  uint32_t vf[kDepth][16];
  uint32_t bits[kDepth];
  int32_t rows[kDepth];
  const int64_t n_tiles = t_end > t_begin ? (t_end - t_begin + 15) / 16 : 0;
  if (n_tiles > 0) {
    int32_t first[kDepth];
#pragma unroll
    for (int u = 0; u < kDepth; ++u) first[u] = fetch_row(t_begin + 16 * u);
#pragma unroll
    for (int u = 0; u < kDepth; ++u) rows[u] = fetch_row(t_begin + 16 * (u + kDepth));
#pragma unroll
    for (int u = 0; u < kDepth; ++u) fetch_kv(first[u], kf[u], vf[u], bits[u]);
  }
  int64_t g = 0;
  for (; g + kDepth <= n_tiles; g += kDepth) {
#pragma unroll
    for (int u = 0; u < kDepth; ++u) {
      compute(kf[u], vf[u], bits[u]);
      const int32_t next = rows[u];
      rows[u] = fetch_row(t_begin + 16 * (g + u + 2 * kDepth));
      fetch_kv(next, kf[u], vf[u], bits[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < kDepth; ++u)
    if (g + u < n_tiles) compute(kf[u], vf[u], bits[u]);

  // Normalize; one split writes the output, several write partials for the merge.
  if (lane < GQ) l_lds[lane] = l_run;
  __syncthreads();
  const int64_t h0 = kvh * GQ;
  if (a.splits == 1) {
#pragma unroll
    for (int h = 0; h < GQ; ++h) {
      const float l = l_lds[h];
#pragma unroll
      for (int d = 0; d < kDpl; ++d)
        store_any(a.out, (s * a.num_heads + h0 + h) * HD + kDpl * lane + d, a.out_dtype,
                  l > 0.0f ? o[h][d] / l : 0.0f);
    }
    return;
  }
  const int64_t base = split * a.num_seqs + s;
#pragma unroll
  for (int h = 0; h < GQ; ++h) {
    const float l = l_lds[h];
#pragma unroll
    for (int d = 0; d < kDpl; ++d)
      a.part_out[((base * a.num_heads + h0 + h) * HD) + kDpl * lane + d] = l > 0.0f ? o[h][d] / l : 0.0f;
  }
  if (lane < GQ) a.part_lse[base * a.num_heads + h0 + lane] = l_run > 0.0f ? m_run + __logf(l_run) : neg_inf;
}

// Combine the splits of one (sequence, head): weights exp(lse_i - max lse). The lanes first
// share the max over the splits, then every lane sums its dims over all splits, four at a time
// so that their loads overlap.
template <int HD>
__global__ void __launch_bounds__(64) paged_merge_kernel(const PagedDecodeArgs a) {
  constexpr int kDpl = HD / 64;
  const int64_t h = blockIdx.x, s = blockIdx.y;
  const int lane = threadIdx.x;
  const float neg_inf = -__int_as_float(0x7F800000);
  auto lse_of = [&](int i) { return a.part_lse[(int64_t(i) * a.num_seqs + s) * a.num_heads + h]; };
  float top = neg_inf;
  for (int i = lane; i < a.splits; i += 64) top = fmaxf(top, lse_of(i));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) top = fmaxf(top, __shfl_xor(top, off, 64));
  float acc[kDpl] = {};
  float wsum = 0.0f;
  if (top != neg_inf) {
    int i = 0;
    for (; i + 4 <= a.splits; i += 4) {
      float w[4], v[4][kDpl];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t base = (int64_t(i + u) * a.num_seqs + s) * a.num_heads + h;
        const float lse = a.part_lse[base];
        w[u] = lse == neg_inf ? 0.0f : __expf(lse - top);
#pragma unroll
        for (int d = 0; d < kDpl; ++d) v[u][d] = a.part_out[base * HD + kDpl * lane + d];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        wsum += w[u];
#pragma unroll
        for (int d = 0; d < kDpl; ++d) acc[d] = __builtin_fmaf(w[u], v[u][d], acc[d]);
      }
    }
    for (; i < a.splits; ++i) {
      const int64_t base = (int64_t(i) * a.num_seqs + s) * a.num_heads + h;
      const float lse = a.part_lse[base];
      const float w = lse == neg_inf ? 0.0f : __expf(lse - top);
      wsum += w;
#pragma unroll
      for (int d = 0; d < kDpl; ++d) acc[d] = __builtin_fmaf(w, a.part_out[base * HD + kDpl * lane + d], acc[d]);
    }
  }
#pragma unroll
  for (int d = 0; d < kDpl; ++d)
    store_any(a.out, (s * a.num_heads + h) * HD + kDpl * lane + d, a.out_dtype, wsum > 0.0f ? acc[d] / wsum : 0.0f);
}

template <class C, int HD>
hipError_t launch_decode_hd(const PagedDecodeArgs& a, hipStream_t stream) {
  const dim3 grid(unsigned(a.splits), unsigned(a.kv_heads), unsigned(a.num_seqs));
  const int g = int(a.num_heads / a.kv_heads);
  switch (g) {
    case 1: hipLaunchKernelGGL((paged_decode_kernel<C, HD, 1>), grid, dim3(64), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((paged_decode_kernel<C, HD, 2>), grid, dim3(64), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((paged_decode_kernel<C, HD, 4>), grid, dim3(64), 0, stream, a); break;
    case 8: hipLaunchKernelGGL((paged_decode_kernel<C, HD, 8>), grid, dim3(64), 0, stream, a); break;
    case 16: hipLaunchKernelGGL((paged_decode_kernel<C, HD, 16>), grid, dim3(64), 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  if (a.splits > 1)
    hipLaunchKernelGGL((paged_merge_kernel<HD>), dim3(unsigned(a.num_heads), unsigned(a.num_seqs)), dim3(64), 0,
                       stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_kv_write(const KvWriteArgs& a, int64_t q_len, bool decode, hipStream_t stream) {
  if (a.num_seqs == 0 || q_len == 0) return hipSuccess;
  if (decode)
    hipLaunchKernelGGL(kv_write_decode_kernel, dim3(unsigned(a.num_seqs)), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(kv_write_kernel, dim3(unsigned(q_len), unsigned(a.num_seqs)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_paged_decode(const PagedDecodeArgs& a, hipStream_t stream) {
  if (a.num_seqs == 0) return hipSuccess;
  if (a.cache_dtype == kDtBf16)
    return a.head_dim == 128 ? launch_decode_hd<ActBf16, 128>(a, stream) : launch_decode_hd<ActBf16, 64>(a, stream);
  return a.head_dim == 128 ? launch_decode_hd<ActF16, 128>(a, stream) : launch_decode_hd<ActF16, 64>(a, stream);
}

}  // namespace llmopt
