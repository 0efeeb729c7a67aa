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
// Decode attention: one workgroup per (context split, KV head, sequence) with W = 1..8 waves that
// take its 16-token tiles in turn:
//   * scores S[token][head] = K Q^T * scale on v_mfma_f32_16x16x32: the A operand is 16 tokens x
//     32 dims of K (16 bytes per lane, read straight from the cache), the B operand the group's
//     query heads (columns >= group are zero), HD / 32 MFMAs per tile;
//   * online softmax per head in fp32 (running max and sum); masked tokens contribute nothing;
//   * O^T += V^T P on v_mfma_f32_16x16x16, HD / 16 MFMAs per tile: the probabilities, rounded to
//     the cache dtype as the reference's softmax output is, are the B operand exactly as the
//     score MFMA left them in the lanes, and each lane reads HD / 8 contiguous bytes of four V rows;
//   * two tiles of K and V, and the block ids of two more, are in flight while a tile is computed;
//   * the W waves merge their partial results in LDS; with several splits each workgroup writes
//     its normalized partial output and log-sum-exp, and a merge kernel combines them (the
//     reference's merge_states, paged_attention.py:30-56).
// Scores, softmax and the output accumulate in fp32; the output is rounded once into the query
// dtype.
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

// v_mfma_f32_16x16x16 (four 16-bit elements per lane) for P V, and the probabilities rounded to
// the cache dtype as its operand (the reference's softmax output is in that dtype too).
template <class C>
struct Mfma16x16;
template <>
struct Mfma16x16<ActBf16> {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  __device__ static f32x4 run(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                     0, 0, 0);
  }
  __device__ static uint32_t pack(float lo, float hi) {
    return uint32_t(__builtin_bit_cast(uint16_t, __bf16(lo))) | (uint32_t(__builtin_bit_cast(uint16_t, __bf16(hi))) << 16);
  }
};
template <>
struct Mfma16x16<ActF16> {
  typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
  __device__ static f32x4 run(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0,
                                                 0);
  }
  __device__ static uint32_t pack(float lo, float hi) {
    return uint32_t(__builtin_bit_cast(uint16_t, _Float16(lo))) |
           (uint32_t(__builtin_bit_cast(uint16_t, _Float16(hi))) << 16);
  }
};

// One wave per (context split, KV head, sequence). Lane l: col = l % 16, kb = l / 16.
//   S = K Q^T on v_mfma_f32_16x16x32: lane l supplies K of token col (dims 32m + 8kb ..) and q of
//   head col; it receives S[token 4kb + r][head col], r = 0..3.
//   O^T += V^T P on v_mfma_f32_16x16x16 (M = 16 head dims, K = the 16 tokens, N = 16 heads): the
//   B operand P[token 4kb + r][head col] is exactly what lane l holds after the softmax, so the
//   probabilities never leave registers; the A operand is V of tokens 4kb .. 4kb + 3 at dims
//   (HD/16) col + i for MFMA i, i.e. one contiguous HD/16-dim piece of four V rows per lane.
//   Lane l accumulates O[head col][dims (HD/16)(4kb + r) + i]: HD/4 contiguous dims of one head,
//   so the per-head rescale of the online softmax needs no data from other lanes.
//
// ROPE: the step's rotary embedding and cache write in the same launch (the reference's
// apply_rotary_pos_emb, then PagedKVCache.write_decode, then the attention). Every lane rotates
// its q dims and the new token's k dims (dims i and i + HD/2 are m and m + kNm/2 of one lane) with
// the roundings of the rotary kernel; the first split's wave 0 stores k and v into the slot of
// offsets[s]; and the tile that holds that token takes its key and value from these registers
// instead of the cache, so no workgroup waits for the store. The slot a sequence writes must not be
// a key of another sequence in the same call (a block being filled is never shared).
//
// PRE: prefill, q_len query tokens per sequence. A wave holds NCB blocks of 16 B-operand columns,
// each kTpt = 16 / GQ consecutive query tokens x the GQ heads of the KV head (block cb, column c:
// token j0 + cb kTpt + c / GQ, head c % GQ); wave w of workgroup x takes tokens j0 = (x W + w)
// kTpt NCB .. and every key tile up to its last token's position, so the W waves walk the same
// key tiles together (their loads meet in the CU's L1) and each stores its own columns. A key
// tile's K operand, slot rows and rearranged V serve all NCB blocks; each block keeps its own
// softmax state and output. Key t enters column c's softmax iff it is a key and
// t <= ctx - q_len + token (the reference's causal mask).
template <class C, int HD, int GQ, int W, bool ROPE = false, bool PRE = false, int NCB = 1>
__global__ void __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2))) paged_decode_kernel(const PagedDecodeArgs a) {
  static_assert(!(ROPE && PRE), "the rotary step is a decode-step fusion");
  static_assert(NCB == 1 || PRE, "several column blocks per wave: prefill");
  constexpr int kNc = PRE ? 16 : GQ;  // columns of the B operand that carry queries
  constexpr int kTpt = 16 / GQ;       // PRE: query tokens per workgroup
  constexpr int kNm = HD / 32;  // score MFMAs per tile (32 dims each)
  constexpr int kNv = HD / 16;  // P V MFMAs per tile; also V dims per lane per token
  constexpr int kVw = kNv / 2;  // 32-bit words of V per lane per token
  const int lane = threadIdx.x & 63;
  const int wave = W > 1 ? int(threadIdx.x >> 6) : 0;
  const int col = lane & 15;
  const int kb = lane >> 4;
  // PRE: grid (KV head, sequence, query block), the blocks latest in the prompt (the longest
  // walks under the causal mask) dispatched first: 32 x 512-token prompts 476 -> 448 us against
  // query blocks innermost.
  const int64_t split = PRE ? int64_t(gridDim.z) - 1 - blockIdx.z : blockIdx.x;
  const int64_t kvh = PRE ? blockIdx.x : blockIdx.y, s = PRE ? blockIdx.y : blockIdx.z;
  const int64_t ctx = a.context_lens[s];
  // PRE: the wave's NCB blocks of 16 columns; block cb holds query tokens j0 + cb kTpt .. + kTpt
  // (column col: token j0 + cb kTpt + col / GQ, head col % GQ) and the last key position each
  // column sees (-1: none).
  const int64_t j0 = PRE ? (split * W + wave) * kTpt * NCB : 0;
  int64_t q_tok[NCB], q_pos[NCB];
  bool q_ok[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    q_tok[cb] = PRE ? j0 + cb * kTpt + col / GQ : 0;
    q_ok[cb] = !PRE || q_tok[cb] < a.q_len;
    q_pos[cb] = PRE && q_ok[cb] ? ctx - a.q_len + q_tok[cb] : -1;
  }
  int64_t t_begin, t_end;
  if constexpr (PRE) {
    const int64_t last = j0 + kTpt * NCB < a.q_len ? j0 + kTpt * NCB : a.q_len;  // tokens j0 .. last - 1
    const int64_t lim = ctx - a.q_len + last;                         // keys t < lim
    t_begin = 0;
    t_end = j0 >= a.q_len ? 0 : ctx < lim ? ctx : lim;  // a wave past the prompt walks no tiles
  } else {
    t_begin = split * a.tiles_per_split * 16;
    t_end = ctx < t_begin + a.tiles_per_split * 16 ? ctx : t_begin + a.tiles_per_split * 16;
  }
  // The workgroup's tiles are dealt to its waves in turn: wave w takes tiles w, w + W, ...
  auto tile_t0 = [&](int64_t j) -> int64_t { return PRE ? 16 * j : t_begin + 16 * (wave + int64_t(W) * j); };
  const int64_t row_stride = a.kv_heads * HD;  // elements between two slots
  const uint32_t cache_bytes = uint32_t(a.num_blocks * a.block_size * row_stride * 2);
  const auto krs = make_rsrc(a.key_cache, cache_bytes);
  const auto vrs = make_rsrc(a.value_cache, cache_bytes);
  const uint32_t row_bytes = uint32_t(row_stride * 2);
  const uint32_t head_off = uint32_t(kvh * HD * 2);
  const uint32_t v_lane_off = uint32_t(kNv * col * 2);
  const int32_t* const table = a.block_ids + s * a.ldb;

  // Query heads kvh * GQ + col (col < GQ) as the B operand of the scores, cast to the cache dtype
  // (q.to(k.dtype)); columns >= GQ are zero. One branch on the dtype, then independent loads.
  // ROPE: the group's rotated q heads and the rotated new key, [GQ + 1][HD] of the cache dtype.
  __shared__ __align__(16) typename C::raw rot_lds[ROPE ? (GQ + 1) * HD : 8];
  u32x4 qf[NCB][kNm];
  u32x4 knew[ROPE ? kNm : 1];     // the new key, dims 32m + 8kb .. + 8 (the K operand's order)
  uint32_t vnew[ROPE ? kVw : 1];  // the new value, dims kNv col .. + kNv (the V operand's order)
  int64_t off_new = -1;           // its position in the sequence
  // The query (and with ROPE the new key and value): converted, rotated, in the operand order.
  auto load_query = [&]() {
    if constexpr (ROPE) {
      // Each (head, pair i < HD/2) of the group's q heads and of the new k is rotated once per
      // workgroup, one pair per thread, into LDS; the lanes then read their operand pieces.
      using Raw = typename C::raw;
      constexpr int kHalf = HD / 2;
      int64_t p = a.positions[s];
      p = p < 0 ? 0 : (p >= a.table_rows ? a.table_rows - 1 : p);  // the host checks the range
      const Raw* qrow = static_cast<const Raw*>(a.query) + s * a.q_seq_stride + kvh * GQ * HD;
      const Raw* krow = static_cast<const Raw*>(a.new_k) + s * a.ldk + kvh * HD;
      const float* ct = a.cos_table + p * HD;
      const float* st = a.sin_table + p * HD;
      for (int j = int(threadIdx.x); j < (GQ + 1) * kHalf; j += 64 * W) {
        const int h = j / kHalf;
        const int i = j - h * kHalf;
        const Raw* src = h < GQ ? qrow + h * HD : krow;
        const float x1 = C::load(src[i]), x2 = C::load(src[i + kHalf]);
        // The tables are cast to the activation dtype first (cos.to(q.dtype)); rotate_half(x) =
        // [-x2, x1]; every product and the sum rounded as torch rounds them.
        const float c1 = C::load(C::store(ct[i])), s1 = C::load(C::store(st[i]));
        const float c2 = C::load(C::store(ct[i + kHalf])), s2 = C::load(C::store(st[i + kHalf]));
        rot_lds[h * HD + i] = C::store(C::load(C::store(x1 * c1)) + C::load(C::store(-x2 * s1)));
        rot_lds[h * HD + i + kHalf] = C::store(C::load(C::store(x2 * c2)) + C::load(C::store(x1 * s2)));
      }
      __syncthreads();
#pragma unroll
      for (int m = 0; m < kNm; ++m) {
        qf[0][m] = col < GQ ? *reinterpret_cast<const u32x4*>(rot_lds + col * HD + 32 * m + 8 * kb) : u32x4{0u, 0u, 0u, 0u};
        knew[m] = *reinterpret_cast<const u32x4*>(rot_lds + GQ * HD + 32 * m + 8 * kb);
      }
      const Raw* vr = static_cast<const Raw*>(a.new_v) + s * a.ldv + kvh * HD + kNv * col;
      if constexpr (kVw == 4) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(vr);
        vnew[0] = w.x, vnew[1] = w.y, vnew[2] = w.z, vnew[3] = w.w;
      } else {
        const u32x2 w = *reinterpret_cast<const u32x2*>(vr);
        vnew[0] = w.x, vnew[1] = w.y;
      }
      off_new = a.offsets[s];
      // The cache write (paged_cache.py:246-277): block block_ids[s, off / B], replaced by block 0
      // outside [0, num_blocks); an offset outside the table row writes nothing.
      if (split == 0 && wave == 0) {
        const int64_t index = off_new >= 0 ? off_new / a.block_size : -1;
        if (index >= 0 && index < a.ldb) {
          int64_t block = a.block_ids[s * a.ldb + index];
          if (block < 0 || block >= a.num_blocks) block = 0;
          const int64_t row = ((block * a.block_size + off_new % a.block_size) * a.kv_heads + kvh) * HD;
          Raw* kd = static_cast<Raw*>(a.k_store) + row;
          Raw* vd = static_cast<Raw*>(a.v_store) + row + kNv * col;
          if (col == 0) {
#pragma unroll
            for (int m = 0; m < kNm; ++m) *reinterpret_cast<u32x4*>(kd + 32 * m + 8 * kb) = knew[m];
          }
          if (kb == 0) {
            if constexpr (kVw == 4)
              *reinterpret_cast<u32x4*>(vd) = u32x4{vnew[0], vnew[1], vnew[2], vnew[3]};
            else
              *reinterpret_cast<u32x2*>(vd) = u32x2{vnew[0], vnew[1]};
          }
        }
      }
    } else {
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        const bool hv = PRE ? q_ok[cb] : col < GQ;
        const int64_t q0 = PRE ? s * a.q_seq_stride + (q_ok[cb] ? q_tok[cb] : 0) * a.q_tok_stride +
                                     (kvh * GQ + col % GQ) * a.q_head_stride + 8 * kb
                               : s * a.q_seq_stride + (kvh * GQ + (hv ? col : 0)) * HD + 8 * kb;
        float x[kNm][8];
        // Eight consecutive dims per lane and m: one or two 16-byte loads when the rows are
        // 16-byte aligned (a.q_vec, checked on the host), else element loads.
        if (a.q_dtype == kDtF32) {
          const float* q = static_cast<const float*>(a.query) + q0;
          if (a.q_vec) {
#pragma unroll
            for (int m = 0; m < kNm; ++m) {
              const f32x4 v0 = *reinterpret_cast<const f32x4*>(q + 32 * m);
              const f32x4 v1 = *reinterpret_cast<const f32x4*>(q + 32 * m + 4);
#pragma unroll
              for (int e = 0; e < 4; ++e) x[m][e] = v0[e], x[m][e + 4] = v1[e];
            }
          } else {
#pragma unroll
            for (int m = 0; m < kNm; ++m)
#pragma unroll
              for (int e = 0; e < 8; ++e) x[m][e] = q[32 * m + e];
          }
        } else {
          const uint16_t* q = static_cast<const uint16_t*>(a.query) + q0;
          const bool half = a.q_dtype == kDtF16;
          auto cvt = [&](uint16_t h) { return half ? f16_to_f32(h) : bf16_to_f32(h); };
          if (a.q_vec) {
#pragma unroll
            for (int m = 0; m < kNm; ++m) {
              const u32x4 w = *reinterpret_cast<const u32x4*>(q + 32 * m);
              const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
              for (int e = 0; e < 4; ++e)
                x[m][2 * e] = cvt(uint16_t(ws[e])), x[m][2 * e + 1] = cvt(uint16_t(ws[e] >> 16));
            }
          } else {
#pragma unroll
            for (int m = 0; m < kNm; ++m)
#pragma unroll
              for (int e = 0; e < 8; ++e) x[m][e] = cvt(q[32 * m + e]);
          }
        }
#pragma unroll
        for (int m = 0; m < kNm; ++m) {
          uint32_t w[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            w[e] = hv ? uint32_t(C::store(x[m][2 * e])) | (uint32_t(C::store(x[m][2 * e + 1])) << 16) : 0u;
          qf[cb][m] = u32x4{w[0], w[1], w[2], w[3]};
        }
      }
    }
  };
  load_query();
  // Slot row (block * block_size + slot) of token t0 + col, or -1 when that token is not a key.
  // 32-bit arithmetic: contexts, table widths and slot rows stay below 2^31 (checked on the host).
  const uint32_t bsz = uint32_t(a.block_size);
  const uint32_t ldb32 = uint32_t(a.ldb);
  const uint32_t nblk = uint32_t(a.num_blocks);
  const uint32_t t_end32 = uint32_t(t_end > 0 ? t_end : 0);
  // The table entry is loaded a full ring turn before its slot row is needed: fetch_block
  // issues the load and row_of turns the entry into a slot row when the tile's K/V loads are
  // issued.
  const auto trs = make_rsrc(table, uint32_t(a.ldb * 4));
  auto fetch_block = [&](int64_t t0) -> int32_t {
    const uint32_t bi = (uint32_t(t0) + uint32_t(col)) / bsz;
    return int32_t(__builtin_amdgcn_raw_buffer_load_b32(trs, (bi < ldb32 ? bi : 0u) * 4u, 0, kLoadPolicy));
  };
  auto row_of = [&](int64_t t0, int32_t block) -> int32_t {
    const uint32_t t = uint32_t(t0) + uint32_t(col);
    const uint32_t bi = t / bsz;
    const bool ok = t < t_end32 && bi < ldb32 && block >= 0 && uint32_t(block) < nblk;  // else no key
    return ok ? int32_t(uint32_t(block) * bsz + (t - bi * bsz)) : -1;
  };
  // K of token t0 + col (masked tokens read slot row 0; their scores are dropped) and V of tokens
  // t0 + 4kb .. t0 + 4kb + 3, whose slot rows come from the lanes that computed them. A masked
  // token's V is read at an offset past the cache (which the host keeps under 2 GiB), where
  // buffer loads return zeros, so its product with a zero probability stays zero whatever the
  // slot holds.
  constexpr uint32_t kPastCache = 0x80000000u;
  auto fetch_kv = [&](int32_t row, u32x4* kf, uint32_t (*vf)[kVw], uint32_t& valid_bits) {
    valid_bits = uint32_t(__builtin_amdgcn_ballot_w64(row >= 0) & 0xFFFFu);
    const uint32_t r_own = uint32_t(row >= 0 ? row : 0);
#pragma unroll
    for (int m = 0; m < kNm; ++m) kf[m] = buf_load16(krs, r_own * row_bytes + uint32_t(2 * (32 * m + 8 * kb)), head_off);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int32_t rv = __shfl(row, 4 * kb + k, 64);
      const uint32_t off = rv >= 0 ? uint32_t(rv) * row_bytes + v_lane_off : kPastCache;
      if constexpr (kVw == 4) {
        const u32x4 w = buf_load16(vrs, off, head_off);
        vf[k][0] = w.x, vf[k][1] = w.y, vf[k][2] = w.z, vf[k][3] = w.w;
      } else {
        const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(vrs, int(off), int(head_off), kLoadPolicy));
        vf[k][0] = w.x, vf[k][1] = w.y;
      }
    }
  };

  const float neg_inf = -__int_as_float(0x7F800000);
  float m_run[NCB], l_run[NCB];  // per column block: running max of column col (the same on
                                 // the four lanes of a column) and this lane's share of its sum
  f32x4 o[NCB][kNv];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    m_run[cb] = neg_inf;
    l_run[cb] = 0.0f;
#pragma unroll
    for (int i = 0; i < kNv; ++i) o[cb][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // One tile (tokens t0 .. t0 + 15): scores, online softmax, P V, all on 64 lanes without LDS.
  auto compute = [&](const u32x4* kf_in, const uint32_t (*vf_in)[kVw], uint32_t bits, int64_t t0) {
    u32x4 kf[kNm];
    uint32_t vf[4][kVw];
#pragma unroll
    for (int m = 0; m < kNm; ++m) kf[m] = kf_in[m];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int w = 0; w < kVw; ++w) vf[k][w] = vf_in[k][w];
    if constexpr (ROPE) {
      // The new token, when it is a key of this tile: its key and value from registers.
      const int64_t rel = off_new - t0;
      if (rel >= 0 && rel < 16 && ((bits >> rel) & 1u)) {
        if (col == int(rel)) {
#pragma unroll
          for (int m = 0; m < kNm; ++m) kf[m] = knew[m];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (4 * kb + k == int(rel)) {
#pragma unroll
            for (int w = 0; w < kVw; ++w) vf[k][w] = vnew[w];
          }
      }
    }
    // Scores of every column block against the tile's keys (the K operand shared), then each
    // block's online softmax; the V operand is rearranged once and multiplies every block's P.
    f32x4 acc[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < kNm; ++m) acc[cb] = Mfma16x32<C>::run(kf[m], qf[cb][m], acc[cb]);
    }
    u32x2 pb[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      float sc[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[r] = acc[cb][r] * a.scale;
      if (a.softcap > 0.0f) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[r] = tanhf(sc[r] / a.softcap) * a.softcap;
      }
      float tmax = neg_inf;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool key = ((bits >> (4 * kb + r)) & 1u) && (!PRE || t0 + 4 * kb + r <= q_pos[cb]);
        sc[r] = key ? sc[r] : neg_inf;
        tmax = fmaxf(tmax, sc[r]);
      }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float m_new = fmaxf(m_run[cb], tmax);
      const bool live = m_new != neg_inf;
      const float alpha = live ? __expf(m_run[cb] - m_new) : 1.0f;
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) p[r] = live ? __expf(sc[r] - m_new) : 0.0f;
      l_run[cb] = alpha * l_run[cb] + ((p[0] + p[1]) + (p[2] + p[3]));
      m_run[cb] = m_new;
      // Rescale only when some column's max moved (alpha is exactly 1 otherwise).
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
        for (int i = 0; i < kNv; ++i) o[cb][i] *= alpha;
      }
      pb[cb] = u32x2{Mfma16x16<C>::pack(p[0], p[1]), Mfma16x16<C>::pack(p[2], p[3])};
    }
#pragma unroll
    for (int i = 0; i < kNv; ++i) {
      // Dim (HD/16) col + i of tokens 4kb + 0..3: half i % 2 of word i / 2 of each V piece.
      const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
      const u32x2 va = {__builtin_amdgcn_perm(vf[1][i >> 1], vf[0][i >> 1], sel),
                        __builtin_amdgcn_perm(vf[3][i >> 1], vf[2][i >> 1], sel)};
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) o[cb][i] = Mfma16x16<C>::run(va, pb[cb], o[cb][i]);
    }
  };

  // A ring of kDepth tiles in flight. Slot u holds the wave's tile g + u of the current group;
  // after it is computed it is refilled with tile g + u + kDepth, whose table entries were loaded
  // kDepth tiles earlier (rows[u]); the entries for the refill after that are loaded at the same
  // time. The main loop runs whole groups with unconditional loads (past the last tile they read
  // slot row 0 or nothing and are never used), so the loads keep one static order; the last
  // partial group has no refills.
  constexpr int kDepth = PRE && NCB > 2 ? 1 : 2;  // three column blocks fit with one tile in flight
  u32x4 kf[kDepth][kNm];
  uint32_t vf[kDepth][4][kVw];
  uint32_t bits[kDepth];
  int32_t rows[kDepth];
  const int64_t n_all = t_end > t_begin ? (t_end - t_begin + 15) / 16 : 0;
  const int64_t n_tiles = PRE ? n_all : n_all > wave ? (n_all - wave + W - 1) / W : 0;
  if (n_tiles > 0) {
    int32_t first[kDepth];
#pragma unroll
    for (int u = 0; u < kDepth; ++u) first[u] = fetch_block(tile_t0(u));
#pragma unroll
    for (int u = 0; u < kDepth; ++u) rows[u] = fetch_block(tile_t0(u + kDepth));
#pragma unroll
    for (int u = 0; u < kDepth; ++u) fetch_kv(row_of(tile_t0(u), first[u]), kf[u], vf[u], bits[u]);
  }
  int64_t g = 0;
  for (; g + kDepth <= n_tiles; g += kDepth) {
#pragma unroll
    for (int u = 0; u < kDepth; ++u) {
      compute(kf[u], vf[u], bits[u], tile_t0(g + u));
      const int32_t next = row_of(tile_t0(g + u + kDepth), rows[u]);
      rows[u] = fetch_block(tile_t0(g + u + 2 * kDepth));
      fetch_kv(next, kf[u], vf[u], bits[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < kDepth; ++u)
    if (g + u < n_tiles) compute(kf[u], vf[u], bits[u], tile_t0(g + u));

  // Lane l holds column col of each column block, dims (HD/4) kb + (HD/16) r + i, unnormalized,
  // with the wave's running max m_run and (after this sum) its running sum l_run of that column.
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    l_run[cb] += __shfl_xor(l_run[cb], 16, 64);
    l_run[cb] += __shfl_xor(l_run[cb], 32, 64);
  }
  const int64_t h0 = kvh * GQ;
  const int64_t d0 = (HD / 4) * kb;
  if constexpr (PRE) {
    const int64_t h = h0 + col % GQ;
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      if (!q_ok[cb]) continue;
      float v[4][kNv];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < kNv; ++i) v[r][i] = l_run[cb] > 0.0f ? o[cb][i][r] / l_run[cb] : 0.0f;
      const int64_t base = s * a.out_seq_stride + q_tok[cb] * a.out_tok_stride + h * a.out_head_stride + d0;
      if (a.out_dtype == kDtF32) {
        float* out = static_cast<float*>(a.out) + base;
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int i = 0; i < kNv; ++i) out[kNv * r + i] = v[r][i];
      } else {
        uint16_t* out = static_cast<uint16_t*>(a.out) + base;
        const bool half = a.out_dtype == kDtF16;
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int i = 0; i < kNv; ++i) out[kNv * r + i] = half ? f32_to_f16_rne(v[r][i]) : f32_to_bf16_rne(v[r][i]);
      }
    }
    return;
  }
  if constexpr (W == 1 && !PRE) {
    if (col >= GQ) return;
    const int64_t h = h0 + col;
    float v[4][kNv];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int i = 0; i < kNv; ++i) v[r][i] = l_run[0] > 0.0f ? o[0][i][r] / l_run[0] : 0.0f;
    if (a.splits == 1) {
      const int64_t base = (s * a.num_heads + h) * HD + d0;
      if (a.out_dtype == kDtF32) {
        float* out = static_cast<float*>(a.out) + base;
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int i = 0; i < kNv; ++i) out[kNv * r + i] = v[r][i];
      } else {
        uint16_t* out = static_cast<uint16_t*>(a.out) + base;
        const bool half = a.out_dtype == kDtF16;
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int i = 0; i < kNv; ++i) out[kNv * r + i] = half ? f32_to_f16_rne(v[r][i]) : f32_to_bf16_rne(v[r][i]);
      }
      return;
    }
    const int64_t base = (split * a.num_seqs + s) * a.num_heads + h;
    float* part = a.part_out + base * HD + d0;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int i = 0; i < kNv; ++i) part[kNv * r + i] = v[r][i];
    if (kb == 0) a.part_lse[base] = l_run[0] > 0.0f ? m_run[0] + __logf(l_run[0]) : neg_inf;
  } else if constexpr (!PRE) {
    // Merge the W waves in LDS (the reference's merge_states over W parts): weights
    // exp(m_w - max m), then one (head, dim) element per thread.
    __shared__ float m_lds[W][kNc];
    __shared__ float l_lds[W][kNc];
    __shared__ float o_lds[W][kNc][HD];
    if (col < kNc) {
      if (kb == 0) m_lds[wave][col] = m_run[0], l_lds[wave][col] = l_run[0];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < kNv; ++i) o_lds[wave][col][d0 + kNv * r + i] = o[0][i][r];
    }
    __syncthreads();
    for (int e = int(threadIdx.x); e < kNc * HD; e += 64 * W) {
      const int hh = e / HD, d = e % HD;  // hh: the column (PRE: token j0 + hh / GQ, head hh % GQ)
      if (PRE && j0 + hh / GQ >= a.q_len) continue;
      float top = neg_inf;
#pragma unroll
      for (int w = 0; w < W; ++w) top = fmaxf(top, m_lds[w][hh]);
      float lsum = 0.0f, acc = 0.0f;
      if (top != neg_inf) {
#pragma unroll
        for (int w = 0; w < W; ++w) {
          const float mw = m_lds[w][hh];
          const float f = mw == neg_inf ? 0.0f : __expf(mw - top);
          lsum = __builtin_fmaf(f, l_lds[w][hh], lsum);
          acc = __builtin_fmaf(f, o_lds[w][hh][d], acc);
        }
      }
      const float val = lsum > 0.0f ? acc / lsum : 0.0f;
      const int64_t h = h0 + (PRE ? hh % GQ : hh);
      if (PRE || a.splits == 1) {
        const int64_t i = PRE ? s * a.out_seq_stride + (j0 + hh / GQ) * a.out_tok_stride + h * a.out_head_stride + d
                              : (s * a.num_heads + h) * HD + d;
        if (a.out_dtype == kDtF32)
          static_cast<float*>(a.out)[i] = val;
        else if (a.out_dtype == kDtF16)
          static_cast<uint16_t*>(a.out)[i] = f32_to_f16_rne(val);
        else
          static_cast<uint16_t*>(a.out)[i] = f32_to_bf16_rne(val);
      } else {
        const int64_t base = (split * a.num_seqs + s) * a.num_heads + h;
        a.part_out[base * HD + d] = val;
        if (d == 0) a.part_lse[base] = lsum > 0.0f ? top + __logf(lsum) : neg_inf;
      }
    }
  }
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

template <class C, int HD, int GQ, bool ROPE>
void launch_decode_group(const PagedDecodeArgs& a, dim3 grid, hipStream_t stream) {
  switch (a.waves) {
    case 1: hipLaunchKernelGGL((paged_decode_kernel<C, HD, GQ, 1, ROPE>), grid, dim3(64), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((paged_decode_kernel<C, HD, GQ, 2, ROPE>), grid, dim3(128), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((paged_decode_kernel<C, HD, GQ, 4, ROPE>), grid, dim3(256), 0, stream, a); break;
    default:
      if constexpr (GQ < 16)
        hipLaunchKernelGGL((paged_decode_kernel<C, HD, GQ, 8, ROPE>), grid, dim3(512), 0, stream, a);
      break;
  }
}

template <class C, int HD, int GQ>
void launch_decode_group(const PagedDecodeArgs& a, dim3 grid, hipStream_t stream) {
  if (a.rope)
    launch_decode_group<C, HD, GQ, true>(a, grid, stream);
  else
    launch_decode_group<C, HD, GQ, false>(a, grid, stream);
}

template <class C, int HD>
hipError_t launch_decode_hd(const PagedDecodeArgs& a, hipStream_t stream) {
  const dim3 grid(unsigned(a.splits), unsigned(a.kv_heads), unsigned(a.num_seqs));
  const int g = int(a.num_heads / a.kv_heads);
  if (a.waves != 1 && a.waves != 2 && a.waves != 4 && !(a.waves == 8 && g < 16)) return hipErrorInvalidValue;
  switch (g) {
    case 1: launch_decode_group<C, HD, 1>(a, grid, stream); break;
    case 2: launch_decode_group<C, HD, 2>(a, grid, stream); break;
    case 4: launch_decode_group<C, HD, 4>(a, grid, stream); break;
    case 8: launch_decode_group<C, HD, 8>(a, grid, stream); break;
    case 16: launch_decode_group<C, HD, 16>(a, grid, stream); break;
    default: return hipErrorInvalidValue;
  }
  if (a.splits > 1)
    hipLaunchKernelGGL((paged_merge_kernel<HD>), dim3(unsigned(a.num_heads), unsigned(a.num_seqs)), dim3(64), 0,
                       stream, a);
  return hipGetLastError();
}

// Blocks of 16 query columns per wave in the prefill form (two or four waves): a key tile's
// loads, block lookups and V operand serve all of them. Measured on MI355X, 32 x 512-token
// prompts: one block 741 us, two 520 (558 with a one-tile ring), three with a one-tile ring 476
// (249 VGPRs), four 818 (spilling).
constexpr int kPrefillColumnBlocks = 3;

template <class C, int HD, int GQ>
void launch_prefill_group(const PagedDecodeArgs& a, hipStream_t stream) {
  constexpr int kTpt = 16 / GQ;
  constexpr int kNcb = kPrefillColumnBlocks;
  const int64_t per = int64_t(kTpt) * kNcb * a.waves;  // query tokens per workgroup
  const dim3 grid(unsigned(a.kv_heads), unsigned(a.num_seqs), unsigned((a.q_len + per - 1) / per));
  const int64_t per1 = int64_t(kTpt) * a.waves;
  const dim3 grid1(unsigned(a.kv_heads), unsigned(a.num_seqs), unsigned((a.q_len + per1 - 1) / per1));
  switch (a.waves) {
    case 1: hipLaunchKernelGGL((paged_decode_kernel<C, HD, GQ, 1, false, true, 1>), grid1, dim3(64), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((paged_decode_kernel<C, HD, GQ, 2, false, true, kNcb>), grid, dim3(128), 0, stream, a); break;
    default: hipLaunchKernelGGL((paged_decode_kernel<C, HD, GQ, 4, false, true, kNcb>), grid, dim3(256), 0, stream, a); break;
  }
}

template <class C, int HD>
hipError_t launch_prefill_hd(const PagedDecodeArgs& a, hipStream_t stream) {
  switch (a.num_heads / a.kv_heads) {
    case 1: launch_prefill_group<C, HD, 1>(a, stream); break;
    case 2: launch_prefill_group<C, HD, 2>(a, stream); break;
    case 4: launch_prefill_group<C, HD, 4>(a, stream); break;
    case 8: launch_prefill_group<C, HD, 8>(a, stream); break;
    case 16: launch_prefill_group<C, HD, 16>(a, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_paged_prefill(const PagedDecodeArgs& a, hipStream_t stream) {
  if (a.num_seqs == 0 || a.q_len == 0) return hipSuccess;
  if (a.cache_dtype == kDtBf16)
    return a.head_dim == 128 ? launch_prefill_hd<ActBf16, 128>(a, stream) : launch_prefill_hd<ActBf16, 64>(a, stream);
  return a.head_dim == 128 ? launch_prefill_hd<ActF16, 128>(a, stream) : launch_prefill_hd<ActF16, 64>(a, stream);
}

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
