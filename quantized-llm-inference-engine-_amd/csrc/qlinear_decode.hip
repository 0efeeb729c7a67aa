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
#include <algorithm>
#include <utility>

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
      put_y<Act>(a, m * a.ldy + n, v);
    }
  }
}

// ---- streaming kernel (small M) ---------------------------------------------------------------
//
// One workgroup owns NTT tiles of 16 output features and all of K; its NW waves split K by
// steps (one step = 64 packed bytes per row), interleaved so that at any moment the waves
// read adjacent bytes of the same rows.
//
// * Everything but the codes is staged into LDS once, at the start, with wide coalesced loads:
//   the activation block x[M, K] (permuted into the MFMA operand order), the per-step sums
//   sum_k x[m, k] that the zero-point correction needs, and the workgroup's slice of scales
//   and zeros (a contiguous block of rows, interleaved as (s, z) pairs). Reading scales and
//   zeros from memory per step instead -- one 4-byte lane load per row and step -- doubles the
//   kernel time: those loads touch as many cache lines as the codes themselves.
// * Codes stream through a ring of P = NTT*Q register slots per lane: a slot holds the 16
//   bytes of one (step, tile) item and is refilled with the item P positions ahead as soon as
//   it has been consumed. Every refill is issued unconditionally (positions past the end
//   re-read the last step), so the loads form one static sequence and the in-order completion
//   counter lets each wave keep P items (P KB) in flight.
// * Per-wave partial sums are combined through LDS in a fixed wave order.
constexpr size_t kStreamLds = 96 * 1024;
constexpr int kStageBatch = 8;  // 16-byte activation pieces staged per thread, at most
constexpr int kMetaBatch = 2;   // 16-byte scale (and zero) pieces staged per thread, at most

template <int FMT>
struct StreamGeom {
  using C = Chunk<FMT, 16>;
  static constexpr int kNM = C::kMfma;         // 16-byte activation pieces per lane and step
  static constexpr int kStepPieces = 4 * kNM;  // pieces per activation row and step
  // LDS layout: x [M][steps*kStepPieces + 1] 16-byte pieces, then kNM zero pieces that lanes
  // of rows m >= M read instead | xsum [steps][16] floats (rows m >= M zero) |
  // meta [rows][2G + 2] floats. Row paddings keep lanes of different rows on different banks.
  __host__ __device__ static size_t x_pieces(int64_t M, int64_t steps) {
    return size_t(M) * size_t(steps * kStepPieces + 1) + kNM;
  }
  __host__ __device__ static size_t xsum_floats(int64_t steps) { return size_t(steps) * 16; }
  static size_t lds_bytes(int64_t M, int64_t steps, int64_t G, int ntt) {
    return x_pieces(M, steps) * 16 + xsum_floats(steps) * 4 + size_t(ntt) * 16 * (2 * G + 2) * 4;
  }
};

// RM: output rows per lane that carry data (1 when M == 1, else 4; the MFMA output gives each
// lane rows 4*(lane/16) + r, r < 4).
template <class Act, int FMT, int NTT, int Q, int NW, int RM>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(4, 8)))
    decode_stream_kernel(const LinearArgs a, int steps, uint32_t group_magic) {
  using Geo = StreamGeom<FMT>;
  using C = typename Geo::C;
  using Raw = typename Act::raw;
  using Op = Codes<Act, FMT>;
  constexpr int NM = Geo::kNM;
  constexpr int P = NTT * Q;
  constexpr int kThreads = NW * 64;

  extern __shared__ u32x4 lds[];
  const int M = int(a.M);
  const int G = int(a.G);
  const int row_pieces = steps * Geo::kStepPieces;
  const int kRow = row_pieces + 1;
  u32x4* const zero_lds = lds + Geo::x_pieces(M, steps) - NM;
  float* const xsum_lds = reinterpret_cast<float*>(lds + Geo::x_pieces(M, steps));  // [steps][16]
  float* const meta_lds = xsum_lds + Geo::xsum_floats(steps);  // [NTT*16][2G+2]: (s, z) pairs
  const int meta_row = 2 * G + 2;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;
  const int kq = lane >> 4;
  const int64_t tile0 = int64_t(blockIdx.x) * NTT;
  const bool asym = !a.symmetric;
  const int my_steps = steps / NW;  // the host guarantees NW | steps

  // Per-lane byte offset of this lane's row in each tile (rows past N repeat row N-1; their
  // sums are never stored). The step offset is wave-uniform and goes in the scalar slot.
  const auto wq = make_rsrc(a.qw, uint32_t(a.N * a.ldq));
  uint32_t qoff[NTT];
#pragma unroll
  for (int t = 0; t < NTT; ++t) {
    int64_t n = (tile0 + t) * 16 + col;
    n = n < a.N ? n : a.N - 1;
    qoff[t] = uint32_t(n * a.ldq + kq * 16);
  }

  u32x4 ring[P];
  // Item (q, t): this wave's q-th step (global step q*NW + wave) of tile t.
  auto load_item = [&](int p, int q) {
    q = q < my_steps ? q : my_steps - 1;
    ring[p] = buf_load16(wq, qoff[p % NTT], uint32_t(q * NW + wave) * C::kBytes);
  };

  // ---- prologue: the ring's first P items, then the activation and metadata loads ----
  // (the staging data is waited for once, behind the ring loads, which are then in hand
  // when the main loop starts)
#pragma unroll
  for (int p = 0; p < P; ++p) load_item(p, p / NTT);
  const Raw* xg = static_cast<const Raw*>(a.x);
  const int pieces = M * row_pieces;
  u32x4 xv[kStageBatch];
#pragma unroll
  for (int e = 0; e < kStageBatch; ++e) {
    if (e * kThreads < pieces) {  // uniform
      int idx = tid + e * kThreads;
      idx = idx < pieces ? idx : pieces - 1;
      const int m = idx / row_pieces;
      const int c = idx - m * row_pieces;
      xv[e] = *reinterpret_cast<const u32x4*>(xg + m * a.ldx + 8 * c);
    }
  }
  // The workgroup's scales/zeros: rows [tile0*16, tile0*16 + 16*NTT) are one contiguous run of
  // 16*NTT*G floats. Pieces past the end of the tensors read as zero (buffer range check).
  const int meta_pieces = (NTT * 16 * G + 3) / 4;
  const uint32_t meta_base = uint32_t(tile0 * 16 * G * 4);
  const auto ms = make_rsrc(a.scales, uint32_t(a.N * a.G * 4));
  const auto mz = make_rsrc(asym ? a.zeros : a.scales, uint32_t(a.N * a.G * 4));
  u32x4 sv[kMetaBatch], zv[kMetaBatch];
#pragma unroll
  for (int e = 0; e < kMetaBatch; ++e) {
    if (e * kThreads < meta_pieces) {  // uniform
      const uint32_t off = meta_base + uint32_t(tid + e * kThreads) * 16;
      sv[e] = buf_load16(ms, off, 0);
      zv[e] = buf_load16(mz, off, 0);
    }
  }

  // ---- write the staged data to LDS ----
  for (int i = tid; i < NM; i += kThreads) zero_lds[i] = u32x4{0u, 0u, 0u, 0u};
  for (int i = tid; i < steps * 16; i += kThreads)
    if ((i & 15) >= M) xsum_lds[i] = 0.0f;
#pragma unroll
  for (int e = 0; e < kStageBatch; ++e) {
    if (e * kThreads < pieces) {  // uniform
      const int idx = tid + e * kThreads;
      const int m = idx / row_pieces;
      const int c = idx - m * row_pieces;
      // Sum of this piece's 8 activations, then over the kStepPieces consecutive lanes that
      // hold the pieces of one step (kThreads and row_pieces are multiples of kStepPieces).
      const uint32_t w4[4] = {xv[e].x, xv[e].y, xv[e].z, xv[e].w};
      float sum = 0.0f;
#pragma unroll
      for (int h = 0; h < 4; ++h)
        sum += Act::load(Raw(w4[h] & 0xFFFFu)) + Act::load(Raw(w4[h] >> 16));
#pragma unroll
      for (int off = 1; off < Geo::kStepPieces; off <<= 1) sum += __shfl_xor(sum, off, 64);
      if (idx < pieces) {
        lds[m * kRow + c] = arrange<Act, FMT>(xv[e]);
        if ((c & (Geo::kStepPieces - 1)) == 0) xsum_lds[(c / Geo::kStepPieces) * 16 + m] = sum;
      }
    }
  }
#pragma unroll
  for (int e = 0; e < kMetaBatch; ++e) {
    if (e * kThreads < meta_pieces) {  // uniform
      const int first = (tid + e * kThreads) * 4;
      const uint32_t s4[4] = {sv[e].x, sv[e].y, sv[e].z, sv[e].w};
      const uint32_t z4[4] = {zv[e].x, zv[e].y, zv[e].z, zv[e].w};
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int f = first + h;
        if (f < NTT * 16 * G) {
          const int row = f / G;
          const int g = f - row * G;
          float2 sz;
          sz.x = __uint_as_float(s4[h]);
          sz.y = __uint_as_float(z4[h]);
          *reinterpret_cast<float2*>(meta_lds + row * meta_row + 2 * g) = sz;
        }
      }
    }
  }
  __syncthreads();

  const uint32_t flip = (FMT == kByte && a.signed_codes) ? 0x80808080u : 0u;
  const float z_shift = Op::kOffset + ((FMT == kByte && a.signed_codes) ? 128.0f : 0.0f);
  const float z_const = a.zero_const + z_shift;

  f32x4 tot[NTT];
#pragma unroll
  for (int t = 0; t < NTT; ++t) tot[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const NibbleConsts nib = NibbleConsts::make<Act>(uint32_t(a.ldq) & 0u);
  // Lanes of rows m >= M read the zero pieces.
  const u32x4* const xrow = col < M ? lds + col * kRow + kq * NM : zero_lds;
  const int xstep = col < M ? 4 * NM : 0;

  for (int q0 = 0; q0 < my_steps; q0 += Q) {  // the host guarantees Q | my_steps
#pragma unroll
    for (int qq = 0; qq < Q; ++qq) {
      const int q = q0 + qq;
      const int step = q * NW + wave;
      const int g = int(div_small(uint32_t(step), group_magic));
      u32x4 xa[NM];
#pragma unroll
      for (int j = 0; j < NM; ++j) xa[j] = xrow[step * xstep + j];
      float xsum[RM];
      if constexpr (RM == 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(xsum_lds + step * 16 + 4 * kq);
#pragma unroll
        for (int r = 0; r < 4; ++r) xsum[r] = v[r];
      } else {
        xsum[0] = xsum_lds[step * 16 + 4 * kq];
      }
#pragma unroll
      for (int t = 0; t < NTT; ++t) {
        const int p = qq * NTT + t;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        if constexpr (FMT == kNibble) {
          const uint32_t words[4] = {ring[p].x, ring[p].y, ring[p].z, ring[p].w};
#pragma unroll
          for (int j = 0; j < NM; ++j) acc = Mfma16<Act>::run(xa[j], nib.operand(words[j]), acc);
        } else {
          const uint32_t words[4] = {ring[p].x, ring[p].y, ring[p].z, ring[p].w};
#pragma unroll
          for (int j = 0; j < NM; ++j) acc = Mfma16<Act>::run(xa[j], Op::operand(words, j, flip), acc);
        }
        const float2 sz = *reinterpret_cast<const float2*>(meta_lds + (t * 16 + col) * meta_row + 2 * g);
        const float zc = asym ? sz.y + z_shift : z_const;
#pragma unroll
        for (int r = 0; r < RM; ++r)
          tot[t][r] = __builtin_fmaf(sz.x, __builtin_fmaf(-zc, xsum[r], acc[r]), tot[t][r]);
      }
#pragma unroll
      for (int t = 0; t < NTT; ++t) load_item(qq * NTT + t, q + Q);
    }
  }

  // ---- fixed-order reduction over the waves: red[wave][t][m][16] ----
  __syncthreads();  // every wave is done reading the staged data
  float* red = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int t = 0; t < NTT; ++t)
#pragma unroll
    for (int r = 0; r < RM; ++r) {
      const int m = 4 * kq + r;
      if (m < M) red[((wave * NTT + t) * M + m) * 16 + col] = tot[t][r];
    }
  __syncthreads();
  const Raw* bias = static_cast<const Raw*>(a.bias);
  const int outs = NTT * M * 16;
  for (int e = tid; e < outs; e += kThreads) {
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += red[w * outs + e];
    const int t = e / (M * 16);
    const int rem = e - t * M * 16;
    const int m = rem >> 4;
    const int64_t n = (tile0 + t) * 16 + (rem & 15);
    if (n < a.N) {
      if (bias) v += Act::load(bias[n]);
      put_y<Act>(a, m * a.ldy + n, v);
    }
  }
}

// ---- one-shot kernel (M <= 8, nibble codes, group 128) ------------------------------------------
//
// One workgroup owns one tile of 16 output features; its waves split K into contiguous chunks of
// C steps (C*128 codes per row), one chunk per wave. A wave issues every load it needs up front
// -- its share of the tile's scales and zeros, its activation slice, then its C code loads --
// and only then starts waiting, so the whole chunk (C KB of codes) is in flight at once and the
// grid as a whole streams the weight at the rate HBM can deliver.
// * The tile's scales and zeros (16 rows x G floats each, one contiguous run of the [N, G]
//   tensors) are loaded once per workgroup with coalesced 16-byte lane loads into LDS; loading
//   each wave's groups separately costs about as much time again as all the codes' latency.
// * The activation slice goes through a wave-private LDS region, permuted into the MFMA operand
//   order; the per-step sums for the zero-point term are staged with it for one token and come
//   from MFMAs against ones for two to four.
// * One barrier makes the staged data visible; the final cross-wave reduction needs two more.
template <int C, int MMAX>
struct OneShotGeom {
  static constexpr int kStepPieces = 16;                     // 16-byte x pieces per row and step
  static constexpr int kRowPieces = C * kStepPieces + 1;     // padded LDS row of a wave's slice
  static constexpr int kWavePieces = MMAX * kRowPieces + 4;  // + four zero pieces
  static constexpr int kXPerLane = (MMAX * C * kStepPieces + 63) / 64;
  // Scale / zero rows of the tile in LDS: G + 4 floats (keeps 16-byte alignment and puts the
  // 16 rows on distinct banks for the per-step reads).
  __host__ __device__ static int meta_stride(int64_t G) { return int(G) + 4; }
  static size_t lds_bytes(int nw, int64_t G) {
    const size_t stage = size_t(nw) * (kWavePieces * 16 + C * 16 * 4) + size_t(2) * 16 * meta_stride(G) * 4;
    const size_t red = size_t(nw) * 4 * 64 * 4;
    return stage > red ? stage : red;
  }
};

// GS: groups per 128-code step, 1 (groups of 128) or 2 (groups of 64). With two, each lane's
// four code words are transposed across the four 16-lane rows of the wave (two permlane
// swaps of each kind), so that MFMA e multiplies codes 32e .. 32e + 31 of the step -- within
// group e / 2 -- and the step's two groups keep accumulators, activation sums and scales of
// their own; the activation fragments are read in the matching order.
// F32X: fp32 activations (a.x fp32, a.M tokens) taken as three bf16 pieces per token, rows 3m,
// 3m + 1, 3m + 2 of the staged slice (hi, mid, lo: x = hi + mid + lo exactly), and each token's
// output the fp32 sum of its three rows, (t_hi + t_mid) + t_lo + bias, stored in fp32 -- the
// split and the sum of the fp32 path in one launch.
// FMT = kByte: 8-bit codes, one per byte. Lane (col, kq) then loads 32 bytes of the step (two
// 16-byte loads: codes 32kq .. 32kq + 31), and MFMA j takes the exact byte operand of codes
// 32kq + 8j .. + 8 (bf16: the code itself; fp16: 1024 + code); signed codes are read with the
// sign bit flipped and 128 added to the zero point. Groups of 128, 16-bit activations.
template <class Act, int C, int MMAX, int RM, bool INTER = false, int GS = 1, bool F32X = false,
          int FMT = kNibble>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4, 8)))
    decode_oneshot_kernel(const LinearArgs a) {
  static_assert(GS == 1 || GS == 2, "one or two groups per step");
  static_assert(!F32X || Act::id == kDtBf16, "fp32 pieces are bf16");
  static_assert(FMT == kNibble || (GS == 1 && !F32X), "byte codes: groups of 128, 16-bit activations");
  constexpr int kCB = FMT == kNibble ? 1 : 2;  // 16-byte code loads per lane and step
  using Geo = OneShotGeom<C, MMAX>;
  using Raw = typename Act::raw;
  constexpr int NM = 4;

  extern __shared__ u32x4 lds[];
  const int M = F32X ? 3 * int(a.M) : int(a.M);  // rows of the staged slice
  const int G = int(a.G);
  const int nw = int(blockDim.x) >> 6;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;
  const int kq = lane >> 4;
  const int64_t tile = blockIdx.x;
  const bool asym = !a.symmetric;
  // Item i of this wave is step `step0 + i * sstride`: a contiguous chunk per wave, or (INTER)
  // interleaved over the waves. Measured on MI355X, contiguous chunks are as fast or faster.
  const int step0 = INTER ? wave : wave * C;
  const int sstride = INTER ? nw : 1;

  int64_t n = tile * 16 + col;
  n = n < a.N ? n : a.N - 1;  // rows past N repeat row N-1; their sums are never stored

  // LDS: [wave x slices | wave xsums | scales [16][G+4] | zeros [16][G+4]]
  u32x4* const xw = lds + wave * Geo::kWavePieces;
  u32x4* const zero4 = xw + MMAX * Geo::kRowPieces;
  float* const xsum = reinterpret_cast<float*>(lds + nw * Geo::kWavePieces) + wave * C * 16;  // [C][16]
  const int mstride = Geo::meta_stride(G);
  float* const s_lds = reinterpret_cast<float*>(lds + nw * Geo::kWavePieces) + nw * C * 16;
  float* const z_lds = s_lds + 16 * mstride;

  // ---- issue every load: the tile's scales/zeros, the activation slice, the chunk's codes ----
  const int meta_pieces = 16 * G / 4;  // the host guarantees G % 4 == 0
  const bool meta_loader = tid < meta_pieces;
  const uint32_t meta_bytes = uint32_t(a.N * a.G * 4);
  const auto ms = make_rsrc(a.scales, meta_bytes);
  const auto mz = make_rsrc(asym ? a.zeros : a.scales, meta_bytes);
  const uint32_t mo = uint32_t(tile * 16 * a.G * 4) + uint32_t(meta_loader ? tid : 0) * 16;
  const u32x4 sv = buf_load16(ms, mo, 0);  // past the end of the tensors: zeros
  const u32x4 zv = buf_load16(mz, mo, 0);

  u32x4 xv[Geo::kXPerLane];
  // F32X: eight fp32 activations of a token per (token, piece column), loaded once; all three
  // piece rows are made from them when the slice is staged.
  constexpr int kTok = (MMAX + 2) / 3;
  constexpr int kXTok = (kTok * C * 16 + 63) / 64;
  const int ntok = int(a.M);
  f32x4 xf[F32X ? kXTok : 1][2];
  if constexpr (F32X) {
    const float* xg = static_cast<const float*>(a.x) + int64_t(step0) * 128;
#pragma unroll
    for (int e = 0; e < kXTok; ++e) {
      int idx = lane + 64 * e;
      idx = idx < ntok * C * 16 ? idx : 0;
      const int tok = idx / (C * 16);
      const int c = idx - tok * (C * 16);
      const float* src = xg + tok * a.ldx + (c >> 4) * (sstride * 128) + 8 * (c & 15);
      xf[e][0] = *reinterpret_cast<const f32x4*>(src);
      xf[e][1] = *reinterpret_cast<const f32x4*>(src + 4);
    }
  } else {
    const Raw* xg = static_cast<const Raw*>(a.x) + int64_t(step0) * 128;
#pragma unroll
    for (int e = 0; e < Geo::kXPerLane; ++e) {
      int idx = lane + 64 * e;
      idx = idx < M * C * 16 ? idx : 0;
      const int m = idx / (C * 16);
      const int c = idx - m * (C * 16);
      xv[e] = *reinterpret_cast<const u32x4*>(xg + m * a.ldx + (c >> 4) * (sstride * 128) + 8 * (c & 15));
    }
  }
  const auto wq = make_rsrc(a.qw, uint32_t(a.N * a.ldq));
  u32x4 w[C][kCB];
  const uint32_t qoff = uint32_t(n * a.ldq + kq * 16 * kCB);
#pragma unroll
  for (int i = 0; i < C; ++i)
#pragma unroll
    for (int c = 0; c < kCB; ++c) w[i][c] = buf_load16(wq, qoff + 16 * c, uint32_t(step0 + i * sstride) * 64 * kCB);

  // ---- stage scales/zeros and this wave's activation slice in LDS ----
  if (meta_loader) {
    const int row = (tid * 4) / G;
    const int g = tid * 4 - row * G;
    *reinterpret_cast<u32x4*>(s_lds + row * mstride + g) = sv;
    *reinterpret_cast<u32x4*>(z_lds + row * mstride + g) = zv;
  }
  if (lane < NM) zero4[lane] = u32x4{0u, 0u, 0u, 0u};
  // Per-step activation sums: staged here for one token; from two tokens on, the staging work
  // grows with the rows while one MFMA against a ones operand per fragment gives every lane its
  // rows' sums in the compute loop (measured on MI355X at three and four tokens: qkv 7.2 ->
  // 6.5-6.7 us, o 5.5 -> 5.2; at one token the staged sums stay 0.5-1 % ahead).
  constexpr bool kMfmaSums = MMAX >= 2 || GS == 2;
  if constexpr (!kMfmaSums) {
#pragma unroll
    for (int i = lane; i < C * 16; i += 64)
      if ((i & 15) >= M) xsum[i] = 0.0f;
  }
  if constexpr (F32X) {
    // Rows 3t, 3t + 1, 3t + 2: the hi, mid and lo pieces of token t (x = hi + mid + lo exactly).
#pragma unroll
    for (int e = 0; e < kXTok; ++e) {
      const int idx = lane + 64 * e;
      const int tok = idx / (C * 16);
      const int c = idx - tok * (C * 16);
      const float v[8] = {xf[e][0][0], xf[e][0][1], xf[e][0][2], xf[e][0][3],
                          xf[e][1][0], xf[e][1][1], xf[e][1][2], xf[e][1][3]};
      uint32_t hi[8], mid[8], lo[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        hi[j] = f32_to_bf16_rne(v[j]);
        const float r1 = v[j] - bf16_to_f32(uint16_t(hi[j]));  // exact
        mid[j] = f32_to_bf16_rne(r1);
        lo[j] = f32_to_bf16_rne(r1 - bf16_to_f32(uint16_t(mid[j])));  // exact remainder
      }
      if (idx < ntok * C * 16) {
        const uint32_t* parts[3] = {hi, mid, lo};
#pragma unroll
        for (int p = 0; p < 3; ++p) {
          const uint32_t* h = parts[p];
          xw[(3 * tok + p) * Geo::kRowPieces + c] = arrange<Act, FMT>(
              u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)});
        }
      }
    }
  }
#pragma unroll
  for (int e = 0; e < (F32X ? 0 : Geo::kXPerLane); ++e) {
    const int idx = lane + 64 * e;
    const int m = idx / (C * 16);
    const int c = idx - m * (C * 16);
    float sum = 0.0f;
    if constexpr (!kMfmaSums) {
      const uint32_t w4[4] = {xv[e].x, xv[e].y, xv[e].z, xv[e].w};
#pragma unroll
      for (int h = 0; h < 4; ++h) sum += Act::load(Raw(w4[h] & 0xFFFFu)) + Act::load(Raw(w4[h] >> 16));
      // The 16 pieces of one step sit in 16 consecutive lanes.
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) sum += __shfl_xor(sum, off, 64);
    }
    if (idx < M * C * 16) {
      xw[m * Geo::kRowPieces + c] = arrange<Act, FMT>(xv[e]);
      if (!kMfmaSums && (c & 15) == 0) xsum[(c >> 4) * 16 + m] = sum;
    }
  }
  __syncthreads();

  // ---- compute ----
  const NibbleConsts nib = NibbleConsts::make<Act>(uint32_t(a.ldq) & 0u);
  const bool flipped = FMT == kByte && a.signed_codes;
  const uint32_t flip = flipped ? 0x80808080u : 0u;
  const float z_shift = Codes<Act, FMT>::kOffset + (flipped ? 128.0f : 0.0f);
  const float z_const = a.zero_const + z_shift;
  // Lane (col, kq) reads activation pieces 4 kq + j of a step (GS = 1), or 4 j + kq (GS = 2:
  // codes 32 j + 8 kq of the transposed words); rows past M read the zero pieces.
  const u32x4* const xrow = col < M ? xw + col * Geo::kRowPieces + (GS == 1 ? kq * NM : kq) : zero4;
  const int xstep = col < M ? 4 * NM : 0;
  const int jstride = GS == 1 ? 1 : (col < M ? 4 : 0);
  const float* const srow = s_lds + col * mstride + GS * step0;
  const float* const zrow = z_lds + col * mstride + GS * step0;
  f32x4 tot = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < C; ++i) {
    u32x4 xa[NM];
#pragma unroll
    for (int j = 0; j < NM; ++j) xa[j] = xrow[i * xstep + j * jstride];
    if constexpr (GS == 2) {
      // One step's work at a time: hoisting the swaps and sums of later steps would keep their
      // values live across the chunk and spill.
      __builtin_amdgcn_sched_barrier(0);
      const u32x4 ones = {Act::kOne2, Act::kOne2, Act::kOne2, Act::kOne2};
      // Words of the step's codes, transposed: T[e] in row kq = word kq of row e.
      const auto p02 = __builtin_amdgcn_permlane32_swap(w[i][0].x, w[i][0].z, false, false);
      const auto p13 = __builtin_amdgcn_permlane32_swap(w[i][0].y, w[i][0].w, false, false);
      const auto r01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
      const auto r23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
      const uint32_t tw[4] = {r01[0], r01[1], r23[0], r23[1]};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 2 * h; j < 2 * h + 2; ++j) {
          v = Mfma16<Act>::run(xa[j], ones, v);
          acc = Mfma16<Act>::run(xa[j], nib.operand(tw[j]), acc);
        }
        const float s = srow[2 * i * sstride + h];
        const float zc = asym ? zrow[2 * i * sstride + h] + z_shift : z_const;
#pragma unroll
        for (int r = 0; r < RM; ++r) tot[r] = __builtin_fmaf(s, __builtin_fmaf(-zc, v[r], acc[r]), tot[r]);
      }
      continue;
    }
    float xs[RM];
    if constexpr (kMfmaSums) {
      const u32x4 ones = {Act::kOne2, Act::kOne2, Act::kOne2, Act::kOne2};
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NM; ++j) v = Mfma16<Act>::run(xa[j], ones, v);
#pragma unroll
      for (int r = 0; r < RM; ++r) xs[r] = v[r];
    } else if constexpr (RM == 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(xsum + i * 16 + 4 * kq);
#pragma unroll
      for (int r = 0; r < 4; ++r) xs[r] = v[r];
    } else {
#pragma unroll
      for (int r = 0; r < RM; ++r) xs[r] = xsum[i * 16 + 4 * kq + r];
    }
    const float s = srow[i * sstride];
    const float zc = asym ? zrow[i * sstride] + z_shift : z_const;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (FMT == kNibble) {
      const uint32_t words[4] = {w[i][0].x, w[i][0].y, w[i][0].z, w[i][0].w};
#pragma unroll
      for (int j = 0; j < NM; ++j) acc = Mfma16<Act>::run(xa[j], nib.operand(words[j]), acc);
    } else {
      const uint32_t words[8] = {w[i][0].x, w[i][0].y, w[i][0].z, w[i][0].w,
                                 w[i][1].x, w[i][1].y, w[i][1].z, w[i][1].w};
#pragma unroll
      for (int j = 0; j < NM; ++j) acc = Mfma16<Act>::run(xa[j], Codes<Act, kByte>::operand(words, j, flip), acc);
    }
#pragma unroll
    for (int r = 0; r < RM; ++r) tot[r] = __builtin_fmaf(s, __builtin_fmaf(-zc, xs[r], acc[r]), tot[r]);
  }

  // ---- fixed-order reduction over the waves (the K chunks): red[wave][r][lane] ----
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int r = 0; r < RM; ++r) red[(wave * 4 + r) * 64 + lane] = tot[r];
  __syncthreads();
  if constexpr (F32X) {
    // Token m's three rows, each summed over the waves in order, then hi + mid + lo.
    if (tid < 16 * int(a.M)) {
      const int m = tid >> 4;
      const int c = tid & 15;
      float part[3];
#pragma unroll
      for (int p = 0; p < 3; ++p) {
        const int row = 3 * m + p;
        const int src_lane = c + 16 * (row >> 2);
        float v = 0.0f;
        for (int w2 = 0; w2 < nw; ++w2) v += red[(w2 * 4 + (row & 3)) * 64 + src_lane];
        part[p] = v;
      }
      const int64_t nn = tile * 16 + c;
      if (nn < a.N) {
        float v = (part[0] + part[1]) + part[2];
        if (a.bias) v += static_cast<const float*>(a.bias)[nn];
        static_cast<float*>(a.y)[m * a.ldy + nn] = v;
      }
    }
    return;
  }
  if (tid < 16 * M) {
    const int m = tid >> 4;
    const int c = tid & 15;
    const int src_lane = c + 16 * (m >> 2);
    const int r = m & 3;
    float v = 0.0f;
    for (int w2 = 0; w2 < nw; ++w2) v += red[(w2 * 4 + r) * 64 + src_lane];
    const int64_t nn = tile * 16 + c;
    if (nn < a.N) {
      if (a.bias) v += Act::load(static_cast<const Raw*>(a.bias)[nn]);
      if (a.epilogue == kEpiSwiglu) {
        // Gate rows 8p .. 8p+3 and up rows 8p+4 .. 8p+7 sit four lanes apart (N % 8 == 0).
        const float up = __shfl_xor(v, 4, 64);
        if ((c & 4) == 0)
          static_cast<Raw*>(a.y)[m * a.ldy + (nn >> 3) * 4 + (c & 3)] = Act::store(swiglu<Act>(v, up));
      } else {
        put_y<Act>(a, m * a.ldy + nn, v);
      }
    }
  }
}


// ---- line-streaming kernel (M <= 4, nibble codes, group 128) -----------------------------------
//
// The one-shot kernel's work split (one workgroup per tile of 16 output features, its waves
// taking contiguous runs of K), with the codes brought in whole cache lines. The unit is a
// block of 256 codes: 128 bytes of each of the tile's 16 rows, 2 KB. A wave loads a block with
// two direct-to-LDS loads, each covering 8 rows x 128 B (every lane 16 bytes), non-temporal,
// into its own LDS ring of D blocks; the first D blocks are issued before anything else is
// waited for, and a slot is refilled with the block D further on as soon as it has been read.
// Inside a load, lane l fetches chunk (l % 8) ^ (l / 8) of row l / 8, so that the MFMA-layout
// reads that follow (lane (col, kq) reads chunk 4h + kq of row col, one 16-byte read per
// 128-code step h) hit distinct LDS banks. From there on everything is the one-shot kernel's:
// the same activation slices, per-step sums, scales and cross-wave reduction.
template <int I, class F>
__device__ __forceinline__ void static_for_one(F& f) {
  f(std::integral_constant<int, I>{});
}
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (static_for_one<I>(f), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <int NB, int D, int MMAX, int SPB = 2>
struct LineGeom {
  static constexpr int kSteps = SPB * NB;                    // 128-code steps per wave
  static constexpr int kStepPieces = 16;                     // 16-byte x pieces per row and step
  static constexpr int kRowPieces = kSteps * kStepPieces + 1;  // padded LDS row of a wave's slice
  static constexpr int kWavePieces = MMAX * kRowPieces + 4;  // + four zero pieces
  static constexpr int kXPerLane = (MMAX * kSteps * kStepPieces + 63) / 64;
  __host__ __device__ static int meta_stride(int64_t G) { return int(G) + 4; }
  // [x slices | x sums | scales | zeros | code rings (256-byte aligned)]
  __host__ __device__ static size_t code_offset(int nw, int64_t G) {
    const size_t stage = size_t(nw) * (kWavePieces * 16 + kSteps * 16 * 4) + size_t(2) * 16 * meta_stride(G) * 4;
    return (stage + 255) / 256 * 256;
  }
  static size_t lds_bytes(int nw, int64_t G) {
    const size_t all = code_offset(nw, G) + size_t(nw) * D * 2048;
    const size_t red = size_t(nw) * 4 * 64 * 4;
    return all > red ? all : red;
  }
};

// FMT = kByte: 8-bit codes. A block of 128 bytes per row is then one 128-code step, and lane
// (col, kq) reads its 32 codes of the step as chunks 2kq and 2kq + 1 of row col; the byte
// operands, flipped signs and zero-point offset are the one-shot kernel's.
// GS = 2: groups of 64 (nibble codes), as in the one-shot kernel: the step's code words
// transposed across the wave's 16-lane rows, per-group accumulators, activation sums (MFMAs
// against ones) and scales.
template <class Act, int NB, int D, int MMAX, int RM, int FMT = kNibble, int GS = 1>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4, 8)))
    decode_line_kernel(const LinearArgs a) {
  static_assert(GS == 1 || (GS == 2 && FMT == kNibble), "groups of 64: nibble codes");
  constexpr int SPB = FMT == kNibble ? 2 : 1;  // 128-code steps per block
  using Geo = LineGeom<NB, D, MMAX, SPB>;
  using Raw = typename Act::raw;
  constexpr int NM = 4;
  constexpr int C = SPB * NB;

  extern __shared__ u32x4 lds[];
  const int M = int(a.M);
  const int G = int(a.G);
  const int nw = int(blockDim.x) >> 6;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;
  const int kq = lane >> 4;
  const int64_t tile = blockIdx.x;
  const bool asym = !a.symmetric;
  const int step0 = wave * C;
  const int block0 = wave * NB;

  u32x4* const xw = lds + wave * Geo::kWavePieces;
  u32x4* const zero4 = xw + MMAX * Geo::kRowPieces;
  float* const xsum = reinterpret_cast<float*>(lds + nw * Geo::kWavePieces) + wave * C * 16;  // [C][16]
  const int mstride = Geo::meta_stride(G);
  float* const s_lds = reinterpret_cast<float*>(lds + nw * Geo::kWavePieces) + nw * C * 16;
  float* const z_lds = s_lds + 16 * mstride;
  uint8_t* const ring = reinterpret_cast<uint8_t*>(lds) + Geo::code_offset(nw, G) + size_t(wave) * D * 2048;

  // ---- the tile's scales/zeros and the wave's activation slice, into registers ----
  const int meta_pieces = 16 * G / 4;  // the host guarantees G % 4 == 0
  const bool meta_loader = tid < meta_pieces;
  const uint32_t meta_bytes = uint32_t(a.N * a.G * 4);
  const auto ms = make_rsrc(a.scales, meta_bytes);
  const auto mz = make_rsrc(asym ? a.zeros : a.scales, meta_bytes);
  const uint32_t mo = uint32_t(tile * 16 * a.G * 4) + uint32_t(meta_loader ? tid : 0) * 16;
  const u32x4 sv = buf_load16(ms, mo, 0);  // past the end of the tensors: zeros
  const u32x4 zv = buf_load16(mz, mo, 0);
  const Raw* xg = static_cast<const Raw*>(a.x) + int64_t(step0) * 128;
  u32x4 xv[Geo::kXPerLane];
#pragma unroll
  for (int e = 0; e < Geo::kXPerLane; ++e) {
    int idx = lane + 64 * e;
    idx = idx < M * C * 16 ? idx : 0;
    const int m = idx / (C * 16);
    const int c = idx - m * (C * 16);
    xv[e] = *reinterpret_cast<const u32x4*>(xg + m * a.ldx + (c >> 4) * 128 + 8 * (c & 15));
  }

  // ---- the first D code blocks, straight into the LDS ring, issued after the loads above so
  //      that staging those does not wait for the codes ----
  __builtin_amdgcn_sched_barrier(0);
  const auto wq = make_rsrc(a.qw, uint32_t(a.N * a.ldq));
  const int r8 = lane >> 3;
  const uint32_t chunk = uint32_t((lane & 7) ^ r8);
  uint32_t qoff[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    int64_t n = tile * 16 + 8 * h + r8;
    n = n < a.N ? n : a.N - 1;  // rows past N repeat row N-1; their sums are never stored
    qoff[h] = uint32_t(n * a.ldq) + chunk * 16;
  }
  auto issue = [&](int ib) {
    uint8_t* dst = ring + (ib % D) * 2048;
    const uint32_t so = uint32_t(block0 + ib) * 128;
    load_lds16(wq, dst, qoff[0], so);
    load_lds16(wq, dst + 1024, qoff[1], so);
  };
#pragma unroll
  for (int ib = 0; ib < (D < NB ? D : NB); ++ib) issue(ib);
  __builtin_amdgcn_sched_barrier(0);

  // ---- stage scales/zeros and this wave's activation slice in LDS ----
  if (meta_loader) {
    const int row = (tid * 4) / G;
    const int g = tid * 4 - row * G;
    *reinterpret_cast<u32x4*>(s_lds + row * mstride + g) = sv;
    *reinterpret_cast<u32x4*>(z_lds + row * mstride + g) = zv;
  }
  if (lane < NM) zero4[lane] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = lane; i < C * 16; i += 64)
    if ((i & 15) >= M) xsum[i] = 0.0f;
#pragma unroll
  for (int e = 0; e < Geo::kXPerLane; ++e) {
    const int idx = lane + 64 * e;
    const int m = idx / (C * 16);
    const int c = idx - m * (C * 16);
    const uint32_t w4[4] = {xv[e].x, xv[e].y, xv[e].z, xv[e].w};
    float sum = 0.0f;
#pragma unroll
    for (int h = 0; h < 4; ++h) sum += Act::load(Raw(w4[h] & 0xFFFFu)) + Act::load(Raw(w4[h] >> 16));
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) sum += __shfl_xor(sum, off, 64);
    if (idx < M * C * 16) {
      xw[m * Geo::kRowPieces + c] = arrange<Act, FMT>(xv[e]);
      if ((c & 15) == 0) xsum[(c >> 4) * 16 + m] = sum;
    }
  }
  // A plain barrier once this wave's LDS writes are done: __syncthreads() would also wait for
  // every outstanding direct-to-LDS load (its release fence covers them), i.e. for the codes.
  wait_lgkmcnt0();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // ---- compute, block by block as the ring fills ----
  const NibbleConsts nib = NibbleConsts::make<Act>(uint32_t(a.ldq) & 0u);
  const bool flipped = FMT == kByte && a.signed_codes;
  const uint32_t flip = flipped ? 0x80808080u : 0u;
  const float z_shift = Codes<Act, FMT>::kOffset + (flipped ? 128.0f : 0.0f);
  const float z_const = a.zero_const + z_shift;
  // Activation pieces 4 kq + j of a step (GS = 1), or 4 j + kq (GS = 2, the transposed words).
  const u32x4* const xrow = col < M ? xw + col * Geo::kRowPieces + (GS == 1 ? kq * NM : kq) : zero4;
  const int xstep = col < M ? 4 * NM : 0;
  const int jstride = GS == 1 ? 1 : (col < M ? 4 : 0);
  const float* const srow = s_lds + col * mstride + GS * step0;
  const float* const zrow = z_lds + col * mstride + GS * step0;
  // Byte offset, within a block, of chunk 4h + kq of row col (nibbles: step h of the block), or
  // of chunk 2kq + h (bytes: half h of the lane's 32 codes of the block's one step).
  uint32_t rd_off[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int chunk = FMT == kNibble ? 4 * h + kq : 2 * kq + h;
    rd_off[h] = uint32_t((col >> 3) * 1024 + ((col & 7) * 8 + (chunk ^ (col & 7))) * 16);
  }
  f32x4 tot = {0.f, 0.f, 0.f, 0.f};
  static_for<NB>([&](auto IB) {
    constexpr int ib = decltype(IB)::value;
    constexpr int after = 2 * ((ib + D < NB ? ib + D : NB) - 1 - ib);  // loads issued after block ib's
    wait_vmcnt<after>();
    const uint8_t* blk = ring + (ib % D) * 2048;
#pragma unroll
    for (int h = 0; h < SPB; ++h) {
      const int i = SPB * ib + h;
      const u32x4 w = *reinterpret_cast<const u32x4*>(blk + rd_off[h]);
      const u32x4 w2 = FMT == kByte ? *reinterpret_cast<const u32x4*>(blk + rd_off[1]) : w;
      u32x4 xa[NM];
#pragma unroll
      for (int j = 0; j < NM; ++j) xa[j] = xrow[i * xstep + j * jstride];
      if constexpr (GS == 2) {
        const u32x4 ones = {Act::kOne2, Act::kOne2, Act::kOne2, Act::kOne2};
        // Words of the step's codes, transposed: T[e] in row kq = word kq of row e.
        const auto p02 = __builtin_amdgcn_permlane32_swap(w.x, w.z, false, false);
        const auto p13 = __builtin_amdgcn_permlane32_swap(w.y, w.w, false, false);
        const auto r01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
        const auto r23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
        const uint32_t tw[4] = {r01[0], r01[1], r23[0], r23[1]};
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          f32x4 v = {0.f, 0.f, 0.f, 0.f};
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 2 * g; j < 2 * g + 2; ++j) {
            v = Mfma16<Act>::run(xa[j], ones, v);
            acc = Mfma16<Act>::run(xa[j], nib.operand(tw[j]), acc);
          }
          const float sg = srow[2 * i + g];
          const float zg = asym ? zrow[2 * i + g] + z_shift : z_const;
#pragma unroll
          for (int r = 0; r < RM; ++r) tot[r] = __builtin_fmaf(sg, __builtin_fmaf(-zg, v[r], acc[r]), tot[r]);
        }
        continue;
      }
      float xs[RM];
      if constexpr (RM == 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(xsum + i * 16 + 4 * kq);
#pragma unroll
        for (int r = 0; r < 4; ++r) xs[r] = v[r];
      } else {
        xs[0] = xsum[i * 16 + 4 * kq];
      }
      const float sc = srow[i];
      const float zc = asym ? zrow[i] + z_shift : z_const;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if constexpr (FMT == kNibble) {
        const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < NM; ++j) acc = Mfma16<Act>::run(xa[j], nib.operand(words[j]), acc);
      } else {
        const uint32_t words[8] = {w.x, w.y, w.z, w.w, w2.x, w2.y, w2.z, w2.w};
#pragma unroll
        for (int j = 0; j < NM; ++j)
          acc = Mfma16<Act>::run(xa[j], Codes<Act, kByte>::operand(words, j, flip), acc);
      }
#pragma unroll
      for (int r = 0; r < RM; ++r) tot[r] = __builtin_fmaf(sc, __builtin_fmaf(-zc, xs[r], acc[r]), tot[r]);
    }
    if constexpr (ib + D < NB) {
      wait_lgkmcnt0();  // the slot's reads are done before the load overwrites it
      issue(ib + D);
    }
  });

  // ---- fixed-order reduction over the waves (the K runs): red[wave][r][lane] ----
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int r = 0; r < RM; ++r) red[(wave * 4 + r) * 64 + lane] = tot[r];
  __syncthreads();
  if (tid < 16 * M) {
    const int m = tid >> 4;
    const int c = tid & 15;
    const int src_lane = c + 16 * (m >> 2);
    const int r = m & 3;
    float v = 0.0f;
    for (int w2 = 0; w2 < nw; ++w2) v += red[(w2 * 4 + r) * 64 + src_lane];
    const int64_t nn = tile * 16 + c;
    if (nn < a.N) {
      if (a.bias) v += Act::load(static_cast<const Raw*>(a.bias)[nn]);
      if (a.epilogue == kEpiSwiglu) {
        // Gate rows 8p .. 8p+3 and up rows 8p+4 .. 8p+7 sit four lanes apart (N % 8 == 0).
        const float up = __shfl_xor(v, 4, 64);
        if ((c & 4) == 0)
          static_cast<Raw*>(a.y)[m * a.ldy + (nn >> 3) * 4 + (c & 3)] = Act::store(swiglu<Act>(v, up));
      } else {
        put_y<Act>(a, m * a.ldy + nn, v);
      }
    }
  }
}


// ---- persistent line-streaming kernel (M <= 8, nibble codes, group 128, many tiles) -------------
//
// For grids of thousands of 16-feature tiles (gate_up: 1792) one workgroup per tile pays, for
// every tile, a workgroup launch and a first-data latency that nothing overlaps: measured on
// MI355X, workgroups of such a grid live ~2.3 us of which ~1.9 us is the wait for their first
// bytes, and the grid's launches spread over the whole kernel. Here one workgroup per CU walks a
// strided list of tiles (tile blockIdx.x + j * gridDim.x). Its 8 waves split K (NB blocks of 256
// codes each per tile). Each wave's LDS ring holds R tiles of its blocks; a slot is refilled with
// the block R tiles ahead as soon as it has been read, so R tiles stream in while one is
// computed. The activations and the workgroup's bias values are staged once. Each tile's scales
// and zeros come in one tile ahead, by direct-to-LDS 4-byte loads laid out [group][row] (so the
// 16 rows of one group are 16 consecutive floats: conflict-free reads), double-buffered. The
// per-wave partial sums go to a double-buffered reduction area; one barrier per tile publishes
// them and the next tile's metadata. Inside the tile loop the only memory loads are these
// direct-to-LDS loads, issued by every wave in the same order, so every wait is a static count
// (near the end of the list, where nothing more is loaded ahead, the waits are for everything).
template <int NB, int R, int MMAX>
struct PLineGeom {
  static constexpr int kStepPieces = 16;  // 16-byte x pieces per row and step
  // LDS: [x: MMAX rows x (steps*16 + 1) pieces][zero pieces: 4][xsum: steps x 16 floats]
  //      [meta: 2 buffers x (s, z) x G x 16 floats][red: 2 x S x 4 x 64 floats][bias: 16 x tiles]
  //      [rings: S x R*NB x 2 KB, 256-byte aligned]
  __host__ __device__ static int row_pieces(int steps) { return steps * kStepPieces + 1; }
  __host__ __device__ static size_t x_bytes(int steps) { return size_t(MMAX * row_pieces(steps) + 4) * 16; }
  __host__ __device__ static size_t xsum_bytes(int steps) { return size_t(steps) * 16 * 4; }
  __host__ __device__ static size_t meta_bytes(int64_t G) { return size_t(2) * 2 * 16 * G * 4; }
  __host__ __device__ static size_t red_bytes(int nw) { return size_t(2) * nw * 4 * 64 * 4; }
  __host__ __device__ static size_t bias_bytes(int ntiles) { return size_t(ntiles) * 16 * 4; }
  __host__ __device__ static size_t ring_offset(int nw, int steps, int64_t G, int ntiles) {
    const size_t head = x_bytes(steps) + xsum_bytes(steps) + meta_bytes(G) + red_bytes(nw) + bias_bytes(ntiles);
    return (head + 255) / 256 * 256;
  }
  static size_t lds_bytes(int nw, int steps, int64_t G, int ntiles) {
    return ring_offset(nw, steps, G, ntiles) + size_t(nw) * R * NB * 2048;
  }
};

template <class Act, int NB, int R, int MMAX, int RM>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(1, 2)))
    decode_pline_kernel(const LinearArgs a, int ntiles_max) {
  using Geo = PLineGeom<NB, R, MMAX>;
  using Raw = typename Act::raw;
  constexpr int NM = 4;
  constexpr int NW = 8;      // waves per workgroup
  constexpr int D = R * NB;  // ring slots per wave
  static_assert(R == 2, "the wait counts below are written for two tiles ahead");

  extern __shared__ u32x4 lds[];
  uint8_t* const base = reinterpret_cast<uint8_t*>(lds);
  const int M = int(a.M);
  const int G = int(a.G);
  const int steps = int(a.K / 128);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;
  const int kq = lane >> 4;
  const bool asym = !a.symmetric;
  const int64_t tiles = (a.N + 15) / 16;
  const int64_t first = blockIdx.x;
  const int64_t stride = gridDim.x;
  const int ntiles = int((tiles - first + stride - 1) / stride);  // 1 .. ntiles_max (grid <= tiles)

  const int rp = Geo::row_pieces(steps);
  u32x4* const xl = lds;                                     // [MMAX][rp] arranged x pieces
  u32x4* const zero4 = xl + MMAX * rp;                       // 4 zero pieces
  float* const xsum = reinterpret_cast<float*>(zero4 + 4);   // [steps][16]
  float* const meta = xsum + steps * 16;                     // [2 buffers][s, z][G][16 rows]
  float* const red = meta + 2 * 2 * G * 16;                  // [2][NW][4][64]
  float* const bias_lds = red + 2 * NW * 256;                // [ntiles][16]
  uint8_t* const ring = base + Geo::ring_offset(NW, steps, G, ntiles_max) + size_t(wave) * D * 2048;

  // ---- activations and bias into registers ----
  const int x_pieces = M * steps * 16;
  const Raw* xg = static_cast<const Raw*>(a.x);
  constexpr int kXPer = MMAX > 4 ? 8 : 4;  // activation pieces per thread
  u32x4 xv[kXPer];  // the host checks x_pieces <= kXPer * 512
#pragma unroll
  for (int e = 0; e < kXPer; ++e) {
    int idx = tid + e * NW * 64;
    idx = idx < x_pieces ? idx : 0;
    const int m = idx / (steps * 16);
    const int c = idx - m * (steps * 16);
    xv[e] = *reinterpret_cast<const u32x4*>(xg + m * a.ldx + (c >> 4) * 128 + 8 * (c & 15));
  }
  // Bias of feature (tile j, c) for tid = 16 * j + c (the host checks 16 * ntiles_max <= 512),
  // through a buffer resource so that a missing bias or a feature past N reads zero, unbranched.
  const auto br = make_rsrc(a.bias ? a.bias : a.x, a.bias ? uint32_t(a.N * sizeof(Raw)) : 0u);
  const int64_t bn = (first + int64_t(tid >> 4) * stride) * 16 + (tid & 15);
  static_assert(sizeof(Raw) == 2, "16-bit activations");
  const uint16_t braw = __builtin_amdgcn_raw_buffer_load_b16(
      br, int(tid < 16 * ntiles && bn < a.N ? uint32_t(bn) * 2u : 0x7FFFFFF0u), 0, kLoadPolicy);
  __builtin_amdgcn_sched_barrier(0);

  // ---- direct-to-LDS loads: a tile's metadata (MW 4-byte loads per wave) and code blocks ----
  const uint32_t meta_total = uint32_t(a.N * a.G * 4);
  const auto ms = make_rsrc(a.scales, meta_total);
  const auto mz = make_rsrc(asym ? a.zeros : a.scales, meta_total);
  // Metadata loads per wave and tile: 2 arrays x G/4 loads of 64 floats over 8 waves, G / 16 = NB
  // (default cache policy: each load takes 16 bytes of 16 rows, the other loads of the tile the
  // rest of those lines)
  // (the host checks G == 16 * NB). Load q of this wave covers array p / (G/4), 64-float piece
  // p % (G/4), p = wave * NB + q; lane l takes row l % 16 and group l / 16 + 4 * piece, which
  // lands at [group][row] in LDS.
  const uint32_t meta_lane_off = uint32_t(col) * uint32_t(G) * 4 + uint32_t(kq) * 4;
  auto issue_meta = [&](int j) {
    const int64_t tile = first + int64_t(j) * stride;
    float* dstbase = meta + (j & 1) * 2 * G * 16;
    // The tile's offset goes in the per-lane offset, which the buffer range check covers (the
    // scalar offset is not checked): rows past N then read zeros instead of past the tensors.
    const uint32_t to = uint32_t(tile * 16 * a.G * 4);
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const int p = wave * NB + q;
      const int arr = p / (G / 4);
      const int piece = p - arr * (G / 4);
      float* dst = dstbase + arr * G * 16 + piece * 64;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(arr ? mz : ms, (__attribute__((address_space(3))) void*)dst, 4,
                                               to + meta_lane_off + uint32_t(piece) * 16, 0, 0, kLoadPolicy);
    }
  };
  const auto wq = make_rsrc(a.qw, uint32_t(a.N * a.ldq));
  const int r8 = lane >> 3;
  const uint32_t chunk_off = uint32_t((lane & 7) ^ r8) * 16;
  const int block0 = wave * NB;
  // Block ib of the j-th tile of this workgroup goes to slot (j % R) * NB + ib. Tiles past the
  // workgroup's list (only when it holds fewer than R) read the last row, and are never used.
  auto issue = [&](int j, int ib) {
    const int64_t tile = first + int64_t(j) * stride;
    uint32_t qo[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      int64_t n = tile * 16 + 8 * h + r8;
      n = n < a.N ? n : a.N - 1;  // rows past N repeat row N-1; their sums are never stored
      qo[h] = uint32_t(n * a.ldq) + chunk_off;
    }
    uint8_t* dst = ring + ((j % R) * NB + ib) * 2048;
    const uint32_t so = uint32_t(block0 + ib) * 128;
    load_lds16(wq, dst, qo[0], so);
    load_lds16(wq, dst + 1024, qo[1], so);
  };
  issue_meta(0);
#pragma unroll
  for (int j = 0; j < R; ++j)
#pragma unroll
    for (int ib = 0; ib < NB; ++ib) issue(j, ib);
  __builtin_amdgcn_sched_barrier(0);

  // ---- stage the activations (arranged) with per-step sums, and the bias ----
  for (int i = tid; i < steps * 16; i += NW * 64)
    if ((i & 15) >= M) xsum[i] = 0.0f;
  if (tid < 4) zero4[tid] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int e = 0; e < kXPer; ++e) {
    const int idx = tid + e * NW * 64;
    const int m = idx / (steps * 16);
    const int c = idx - m * (steps * 16);
    const uint32_t w4[4] = {xv[e].x, xv[e].y, xv[e].z, xv[e].w};
    float sum = 0.0f;
#pragma unroll
    for (int h = 0; h < 4; ++h) sum += Act::load(Raw(w4[h] & 0xFFFFu)) + Act::load(Raw(w4[h] >> 16));
    // The 16 pieces of one step and row sit in 16 consecutive lanes.
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) sum += __shfl_xor(sum, off, 64);
    if (idx < x_pieces) {
      xl[m * rp + c] = arrange<Act, kNibble>(xv[e]);
      if ((c & 15) == 0) xsum[(c >> 4) * 16 + m] = sum;
    }
  }
  if (tid < 16 * ntiles) bias_lds[tid] = Act::load(Raw(braw));
  wait_vmcnt<2 * D>();  // this wave's metadata loads of tile 0 (the code blocks may still fly)
  wait_lgkmcnt0();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // ---- per lane, constant over tiles ----
  const NibbleConsts nib = NibbleConsts::make<Act>(uint32_t(a.ldq) & 0u);
  const float z_shift = Act::kNibbleOffset;
  const float z_const = a.zero_const + z_shift;
  const int step0 = 2 * block0;
  const u32x4* const xrow = col < M ? xl + col * rp + step0 * 16 + kq * NM : zero4;
  const int xstep = col < M ? 16 : 0;
  uint32_t rd_off[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
    rd_off[h] = uint32_t((col >> 3) * 1024 + ((col & 7) * 8 + ((4 * h + kq) ^ (col & 7))) * 16);
  Raw* y = static_cast<Raw*>(a.y);

  for (int j = 0; j < ntiles; ++j) {
    const int64_t tile = first + int64_t(j) * stride;
    const int buf = j & 1;
    const bool more = j + 1 < ntiles;   // load the next tile's metadata
    const bool ahead = j + R < ntiles;  // refill with the blocks of tile j + R
    // Loads issued after block ib of this tile, while tiles are still loaded ahead: the D - 1
    // blocks behind it in the ring and the metadata of the tiles j + 2 - R .. j + 1 that exist
    // (tile 0's was loaded before any block).
    const int phase = !ahead ? 0 : (j == 0 ? 1 : 2);
    if (more) issue_meta(j + 1);
    const float* sg = meta + buf * 2 * G * 16 + step0 * 16 + col;  // [group][row]
    const float* zg = sg + G * 16;
    f32x4 tot = {0.f, 0.f, 0.f, 0.f};
    const uint8_t* slots = ring + (j % R) * NB * 2048;
    static_for<NB>([&](auto IB) {
      constexpr int ib = decltype(IB)::value;
      if (phase == 2) {
        wait_vmcnt<2 * (D - 1) + R * NB>();  // R tiles of metadata, NB loads per wave each
      } else if (phase == 1) {
        wait_vmcnt<2 * (D - 1) + NB>();      // tile 0: only tile 1's metadata came after its blocks
      } else {
        wait_vmcnt<0>();
      }
      const uint8_t* blk = slots + ib * 2048;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int i = 2 * ib + h;
        const u32x4 w = *reinterpret_cast<const u32x4*>(blk + rd_off[h]);
        u32x4 xa[NM];
#pragma unroll
        for (int jj = 0; jj < NM; ++jj) xa[jj] = xrow[i * xstep + jj];
        float xs[RM];
        if constexpr (RM == 4) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(xsum + (step0 + i) * 16 + 4 * kq);
#pragma unroll
          for (int r = 0; r < 4; ++r) xs[r] = v[r];
        } else {
          xs[0] = xsum[(step0 + i) * 16 + 4 * kq];
        }
        const float sc = sg[i * 16];
        const float zc = asym ? zg[i * 16] + z_shift : z_const;
        const uint32_t words[4] = {w.x, w.y, w.z, w.w};
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jj = 0; jj < NM; ++jj) acc = Mfma16<Act>::run(xa[jj], nib.operand(words[jj]), acc);
#pragma unroll
        for (int r = 0; r < RM; ++r) tot[r] = __builtin_fmaf(sc, __builtin_fmaf(-zc, xs[r], acc[r]), tot[r]);
      }
      if (ahead) {
        wait_lgkmcnt0();  // the slot's reads are done before the load overwrites it
        issue(j + R, ib);
      }
    });
    float* rb = red + buf * NW * 256;
#pragma unroll
    for (int r = 0; r < RM; ++r) rb[(wave * 4 + r) * 64 + lane] = tot[r];
    // This wave's metadata loads of tile j + 1 have landed before the barrier publishes them.
    if (ahead) {
      wait_vmcnt<2 * NB>();
    } else {
      wait_vmcnt<0>();
    }
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // Fixed-order sum over the waves (the K runs) of this tile's outputs.
    if (tid < 16 * M) {
      const int m = tid >> 4;
      const int c = tid & 15;
      const int src_lane = c + 16 * (m >> 2);
      const int r = m & 3;
      float v = 0.0f;
#pragma unroll
      for (int w2 = 0; w2 < NW; ++w2) v += rb[(w2 * 4 + r) * 64 + src_lane];
      v += bias_lds[j * 16 + c];
      const int64_t nn = tile * 16 + c;
      if (a.epilogue == kEpiSwiglu) {
        // Gate rows 8p .. 8p+3 and up rows 8p+4 .. 8p+7 sit four lanes apart (N % 8 == 0).
        const float up = __shfl_xor(v, 4, 64);
        if ((c & 4) == 0 && nn < a.N) y[m * a.ldy + (nn >> 3) * 4 + (c & 3)] = Act::store(swiglu<Act>(v, up));
      } else if (nn < a.N) {
        put_y<Act>(a, m * a.ldy + nn, v);
      }
    }
  }
}


// ---- multi-tile kernel (M <= 64, 2/4-bit codes, group a multiple of 128) ---------------------
//
// One workgroup owns NT tiles of 16 output features and all of K; its NW waves split K into
// contiguous ranges of whole 128-code steps, and their partial sums meet in LDS at the end in
// a fixed wave order. Lane (col, kq) = (lane % 16, lane / 16), per step of 128 codes:
// * codes: 16 bytes of row n0 + 16t + col at byte 64*step + 16*kq, for each tile t, i.e. codes
//   k = 32kq .. 32kq + 31 of the step; MFMA j (of four) takes the 8 codes of word j. One 16-byte
//   load per lane streams 16 rows x 64 bytes per tile -- half cache lines, fully used;
// * activations: the A operand of MFMA j for token row 16mb + col is then x[32kq + 8j ..+ 8] of
//   the step -- 64 contiguous bytes per lane and step, read with four 16-byte loads from L2
//   (the whole x[M, K] is a few hundred KB and stays there) straight into the MFMA layout. A
//   token block is shared by all NT tiles, so a larger NT cuts the activation traffic per code;
// * scales and zeros of the workgroup's 16*NT rows are staged in LDS once, with coalesced
//   16-byte loads (per-lane loads of a scale per row and step would touch as many cache lines
//   as the codes themselves).
// Codes and activations stream through a register ring of D steps: each slot is refilled with
// the step D ahead as soon as it has been consumed, unconditionally (past the end: the last
// step again), so the loads form one static sequence under the in-order completion counter.
// Arithmetic as in the kernels above: OFF + q operands (one v_and_or_b32 per code pair), one
// MFMA per token block against a ones operand for sum_k x_k, and per step and tile
//     tot += s * (sum_k (OFF + q_k) x_k - (OFF + z) * sum_k x_k).
constexpr int kMtMetaPer = 2;  // 16-byte metadata pieces per thread of the multi-tile kernel

// REFILL = false: every wave's whole range is in the ring at once (ns == D, checked on the
// host), so all loads are issued up front and none is repeated past the end.
// GS = 2: groups of 64 codes, two per step. As in the one-shot kernel, the lane's code words are
// transposed across the wave's four 16-lane rows so that MFMA e covers codes 32e .. 32e + 31 of
// the step, within group 2 step + e / 2; lane (col, kq) then loads the activations of codes
// 32e + 8kq (16 bytes at 64e + 16kq), and each group keeps its own sums and scale.
template <class Act, int NT, int MB, int D, int NW, int WPE, bool REFILL = true, int GS = 1>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
    decode_mt_kernel(const LinearArgs a, int ns, uint32_t group_magic) {
  static_assert(GS == 1 || GS == 2, "one or two groups per step");
  using Raw = typename Act::raw;
  extern __shared__ u32x4 lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;
  const int kq = lane >> 4;
  const int64_t n0 = int64_t(blockIdx.x) * (16 * NT);
  const bool asym = !a.symmetric;
  const int G = int(a.G);
  // LDS metadata: one (scale, OFF + zero) pair per row and group; rows of G + 2 pairs keep
  // 16-byte alignment and put the 16 rows a k-quarter reads on distinct banks.
  const int mstride = G + 2;
  f32x2* const sz_lds = reinterpret_cast<f32x2*>(lds);

  // ---- issue the loads: the workgroup's scales and zeros (rows n0 .. n0 + 16NT - 1, all G
  //      groups, one contiguous run of the [N, G] tensors), then the first D ring slots; only
  //      then wait for the metadata and stage it in LDS ----
  const uint32_t meta_bytes = uint32_t(a.N * a.G * 4);
  const auto ms = make_rsrc(a.scales, meta_bytes);
  const auto mz = make_rsrc(asym ? a.zeros : a.scales, meta_bytes);
  const int pieces = 16 * NT * G / 4;  // G % 4 == 0; at most kMtMetaPer per thread (host check)
  const uint32_t mbase = uint32_t(n0 * a.G * 4);
  u32x4 sv[kMtMetaPer], zv[kMtMetaPer];
#pragma unroll
  for (int e = 0; e < kMtMetaPer; ++e) {
    const int p = tid + e * NW * 64;
    const uint32_t off = mbase + uint32_t(p < pieces ? p : 0) * 16;  // past the tensors: zeros
    sv[e] = buf_load16(ms, off, 0);
    zv[e] = buf_load16(mz, off, 0);
  }

  const auto wq = make_rsrc(a.qw, uint32_t(a.N * a.ldq));
  uint32_t qoff[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int64_t n = n0 + 16 * t + col;
    n = n < a.N ? n : a.N - 1;  // rows past N repeat row N-1; their sums are never stored
    qoff[t] = uint32_t(n * a.ldq + 16 * kq);
  }
  const uint32_t xbytes = uint32_t(a.M * a.ldx * 2);
  const auto xr = make_rsrc(a.x, xbytes);
  uint32_t xoff[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int64_t m = 16 * mb + col;
    // Token rows past M read past the end of x: the buffer returns zeros.
    xoff[mb] = m < a.M ? uint32_t(m * a.ldx * 2 + (GS == 1 ? 64 : 16) * kq) : xbytes;
  }
  const int s_begin = wave * ns;

  u32x4 cw[D][NT];
  u32x4 cx[D][MB][4];
  auto load = [&](int slot, int i) {
    const int step = s_begin + (i < ns ? i : ns - 1);
#pragma unroll
    for (int t = 0; t < NT; ++t) cw[slot][t] = buf_load16(wq, qoff[t], uint32_t(step) * 64);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        cx[slot][mb][j] = buf_load16(xr, xoff[mb] + (GS == 1 ? 16 : 64) * j, uint32_t(step) * 256);
  };
#pragma unroll
  for (int r = 0; r < D; ++r) load(r, r);

  const float z_shift = Act::kNibbleOffset;
  const float z_const = a.zero_const + z_shift;
#pragma unroll
  for (int e = 0; e < kMtMetaPer; ++e) {
    const int p = tid + e * NW * 64;
    if (p < pieces) {
      const int row = (p * 4) / G;
      const int g = p * 4 - row * G;
      const f32x4 sf = __builtin_bit_cast(f32x4, sv[e]);
      const f32x4 zf = __builtin_bit_cast(f32x4, zv[e]);
      // Symmetric codes use the constant offset, so the arithmetic below never branches.
      f32x4 lo, hi;
      lo[0] = sf[0]; lo[1] = asym ? zf[0] + z_shift : z_const;
      lo[2] = sf[1]; lo[3] = asym ? zf[1] + z_shift : z_const;
      hi[0] = sf[2]; hi[1] = asym ? zf[2] + z_shift : z_const;
      hi[2] = sf[3]; hi[3] = asym ? zf[3] + z_shift : z_const;
      *reinterpret_cast<f32x4*>(sz_lds + row * mstride + g) = lo;
      *reinterpret_cast<f32x4*>(sz_lds + row * mstride + g + 2) = hi;
    }
  }
  __syncthreads();  // metadata staged

  const NibbleConsts nib = NibbleConsts::make<Act>(uint32_t(a.ldq) & 0u);
  const u32x4 ones = {Act::kOne2, Act::kOne2, Act::kOne2, Act::kOne2};
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};

  f32x4 tot[NT][MB];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) tot[t][mb] = zero4;

  auto compute_two_groups = [&](int slot, int step) {
    f32x2 sz[NT][2];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h) sz[t][h] = sz_lds[(16 * t + col) * mstride + 2 * step + h];
    u32x4 xa[MB][4];
    f32x4 xs[MB][2];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) xa[mb][j] = arrange<Act, kNibble>(cx[slot][mb][j]);
#pragma unroll
      for (int h = 0; h < 2; ++h)
        xs[mb][h] = Mfma16<Act>::run(xa[mb][2 * h + 1], ones, Mfma16<Act>::run(xa[mb][2 * h], ones, zero4));
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const u32x4 q = cw[slot][t];
      // T[e] in row kq = word kq of row e: codes 32e + 8kq .. + 8 of the step.
      const auto p02 = __builtin_amdgcn_permlane32_swap(q.x, q.z, false, false);
      const auto p13 = __builtin_amdgcn_permlane32_swap(q.y, q.w, false, false);
      const auto r01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
      const auto r23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
      const u32x4 b[4] = {nib.operand(r01[0]), nib.operand(r01[1]), nib.operand(r23[0]), nib.operand(r23[1])};
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const f32x4 acc =
              Mfma16<Act>::run(xa[mb][2 * h + 1], b[2 * h + 1], Mfma16<Act>::run(xa[mb][2 * h], b[2 * h], zero4));
#pragma unroll
          for (int r = 0; r < 4; ++r)
            tot[t][mb][r] = __builtin_fmaf(sz[t][h][0], __builtin_fmaf(-sz[t][h][1], xs[mb][h][r], acc[r]),
                                           tot[t][mb][r]);
        }
    }
  };
  auto compute = [&](int slot, int i) {
    const int step = s_begin + i;
    if constexpr (GS == 2) {
      compute_two_groups(slot, step);
      return;
    }
    const int g = int(div_small(uint32_t(step), group_magic));
    f32x2 sz[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) sz[t] = sz_lds[(16 * t + col) * mstride + g];
    u32x4 xa[MB][4];
    f32x4 xs[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) xa[mb][j] = arrange<Act, kNibble>(cx[slot][mb][j]);
      xs[mb] = Mfma16<Act>::run(xa[mb][0], ones, zero4);
#pragma unroll
      for (int j = 1; j < 4; ++j) xs[mb] = Mfma16<Act>::run(xa[mb][j], ones, xs[mb]);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float sc = sz[t][0];
      const float zc = sz[t][1];
      const u32x4 q = cw[slot][t];
      const u32x4 b[4] = {nib.operand(q.x), nib.operand(q.y), nib.operand(q.z), nib.operand(q.w)};
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        f32x4 acc = Mfma16<Act>::run(xa[mb][0], b[0], zero4);
#pragma unroll
        for (int j = 1; j < 4; ++j) acc = Mfma16<Act>::run(xa[mb][j], b[j], acc);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          tot[t][mb][r] = __builtin_fmaf(sc, __builtin_fmaf(-zc, xs[mb][r], acc[r]), tot[t][mb][r]);
      }
    }
  };

  // D steps at a time, so that every ring slot index is a constant. The refills are
  // unconditional, so the loads form one static sequence whatever ns is; only the arithmetic
  // of the steps past the end is skipped. (A second, tail copy of the loop body would give
  // the register allocator two shapes of the ring to reconcile, which it does by spilling.)
  for (int i0 = 0; i0 < ns; i0 += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      if (i0 + u < ns) compute(u, i0 + u);
      if constexpr (REFILL) load(u, i0 + u + D);
    }
  }

  // ---- fixed-order reduction over the waves: red[wave][t][mb][r][lane] ----
  __syncthreads();  // every wave is done with the metadata
  float* red = reinterpret_cast<float*>(lds);
  constexpr int kElems = NT * MB * 4 * 64;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave * kElems + ((t * MB + mb) * 4 + r) * 64 + lane] = tot[t][mb][r];
  __syncthreads();
  const Raw* bias = static_cast<const Raw*>(a.bias);
  Raw* y = static_cast<Raw*>(a.y);
  for (int e = tid; e < kElems; e += NW * 64) {
    const int ln = e & 63;
    const int r = (e >> 6) & 3;
    const int tm = e >> 8;
    const int t = tm / MB;
    const int mb = tm - t * MB;
    const int64_t m = 16 * mb + 4 * (ln >> 4) + r;
    const int64_t n = n0 + 16 * t + (ln & 15);
    if (m < a.M && n < a.N) {
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) v += red[w * kElems + e];
      if (bias) v += Act::load(bias[n]);
      if (a.epilogue == kEpiSwiglu) {
        // Gate rows 8p .. 8p+3 and up rows 8p+4 .. 8p+7 sit four lanes apart (N % 8 == 0).
        const float up = __shfl_xor(v, 4, 64);
        if ((n & 4) == 0) y[m * a.ldy + (n >> 3) * 4 + (n & 3)] = Act::store(swiglu<Act>(v, up));
      } else {
        put_y<Act>(a, m * a.ldy + n, v);
      }
    }
  }
}

// ---- N-split kernel (5..32 tokens, many tiles) -------------------------------------------------
//
// One workgroup owns NW * NT tiles of 16 output features, NT per wave, and all of K: no
// reduction across waves. Each wave streams its tiles' codes through a register ring of R * C
// steps.
// The activations of C steps at a time are fetched once per workgroup, arranged into MFMA
// operand order, summed per token (the zero-point term: one MFMA chain against ones per step
// and token block, instead of one per wave) and staged in LDS, double-buffered with one barrier
// per C steps. Piece ((mb * 4 + kq) * 4 + j) * 16 + col of a step holds x[16 mb + col][32 kq +
// 8 j .. + 8], which lane (col, kq) of every wave reads as fragment j. The staging waves hold
// whole token blocks: wave w fetches pieces (kPer * w + e) * 64 + lane, e < kPer, kPer a
// multiple of 4, so pieces e = 4p .. 4p+3 are the four k-quarters of one (step, token block)
// and lane j * 16 + col of each is row col, k-slice j of an MFMA operand. Arithmetic as in the
// multi-tile kernel.
//
// With `partials`, workgroup (x, y) covers steps [y * split_steps, (y + 1) * split_steps) only,
// stages the metadata of that slice's groups and writes its fp32 sums, without bias or
// activation, to partials[y][m][n] for the fixed-order reduction kernel.
template <class Act, int MB, int NT, int NW, int C, int R>
__global__ void __launch_bounds__(NW * 64)
    decode_nx_kernel(const LinearArgs a, uint32_t group_magic, int split_steps, float* partials) {
  using Raw = typename Act::raw;
  constexpr int kStepPieces = MB * 256;             // 16-byte activation pieces per step
  constexpr int kChunk = C * kStepPieces;           // pieces per chunk
  constexpr int kPer = kChunk / (NW * 64);          // pieces per thread per chunk
  static_assert(kPer * NW * 64 == kChunk && kPer % 4 == 0, "whole token blocks per wave");
  extern __shared__ u32x4 lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;
  const int kq = lane >> 4;
  const int64_t n0 = int64_t(blockIdx.x) * (16 * NT * NW);
  const bool asym = !a.symmetric;
  const int G = int(a.G);
  const int s0 = int(blockIdx.y) * split_steps;  // this workgroup's K slice: steps s0 .. s_end - 1
  const int s_end = s0 + split_steps;
  // Groups g0 .. g0 + gs - 1 of the slice; rows of gs + 2 pairs in LDS.
  const int g0 = partials ? int(div_small(uint32_t(s0), group_magic)) : 0;
  const int gs = partials ? int(div_small(uint32_t(s_end - 1), group_magic)) + 1 - g0 : G;
  const int mstride = gs + 2;
  f32x2* const sz_lds = reinterpret_cast<f32x2*>(lds);
  u32x4* const xbuf = lds + (16 * NT * NW * mstride * 8 + 15) / 16;  // [2][kChunk] pieces
  float* const xs_lds = reinterpret_cast<float*>(xbuf + 2 * kChunk);  // [2][C][MB][16] sums

  // ---- activations: this thread's pieces of a chunk ----
  const uint32_t xbytes = uint32_t(a.M * a.ldx * 2);
  const auto xr = make_rsrc(a.x, xbytes);
  uint32_t xoff[kPer];
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int q = ((kPer * wave + e) * 64 + lane) % kStepPieces;
    const int64_t row = 16 * (q >> 8) + (q & 15);
    // Token rows past M read past the end of x: the buffer returns zeros.
    xoff[e] = row < a.M ? uint32_t(row * a.ldx * 2 + 64 * ((q >> 6) & 3) + 16 * ((q >> 4) & 3)) : xbytes;
  }
  u32x4 xreg[kPer];
  auto load_x = [&](int chunk) {
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      int step = s0 + chunk * C + ((kPer * wave + e) * 64) / kStepPieces;
      step = step < s_end ? step : s_end - 1;
      xreg[e] = buf_load16(xr, xoff[e], uint32_t(step) * 256);
    }
  };
  const u32x4 ones = {Act::kOne2, Act::kOne2, Act::kOne2, Act::kOne2};
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  auto store_x = [&](int buf) {
    u32x4* dst = xbuf + buf * kChunk;
#pragma unroll
    for (int p = 0; p < kPer / 4; ++p) {
      f32x4 sum = zero4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = 4 * p + i;
        const u32x4 v = arrange<Act, kNibble>(xreg[e]);
        dst[(kPer * wave + e) * 64 + lane] = v;
        sum = Mfma16<Act>::run(v, ones, sum);
      }
      // Lane (c, r4) holds the sums of tokens 4 r4 .. 4 r4 + 3 of this (step, token block),
      // whose index within the chunk is (kPer * wave + 4 p) / 4.
      if (col == 0)
        *reinterpret_cast<f32x4*>(xs_lds + (buf * C * MB + (kPer * wave + 4 * p) / 4) * 16 + 4 * kq) = sum;
    }
  };

  // ---- the wave's codes: a ring of R * C steps over its NT tiles ----
  const auto wq = make_rsrc(a.qw, uint32_t(a.N * a.ldq));
  uint32_t qoff[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int64_t n = n0 + 16 * (wave * NT + t) + col;
    n = n < a.N ? n : a.N - 1;  // rows past N repeat row N-1; their sums are never stored
    qoff[t] = uint32_t(n * a.ldq + 16 * kq);
  }
  u32x4 cw[R * C][NT];
  auto load_codes = [&](int slot, int step) {
    const uint32_t so = uint32_t(step < s_end ? step : s_end - 1) * 64;
#pragma unroll
    for (int t = 0; t < NT; ++t) cw[slot][t] = buf_load16(wq, qoff[t], so);
  };

  // ---- prologue: loads of chunk 0 and the first R * C steps of codes, then the metadata of rows
  //      n0 .. n0 + 16 NT NW - 1 (one contiguous run of the [N, G] tensors) into LDS ----
  load_x(0);
#pragma unroll
  for (int u = 0; u < R * C; ++u) load_codes(u, s0 + u);
  const uint32_t meta_bytes = uint32_t(a.N * a.G * 4);
  const auto ms = make_rsrc(a.scales, meta_bytes);
  const auto mz = make_rsrc(asym ? a.zeros : a.scales, meta_bytes);
  const int pieces = 16 * NT * NW * G / 4;  // G % 4 == 0 (host check)
  const uint32_t mbase = uint32_t(n0 * a.G * 4);
  const float z_shift = Act::kNibbleOffset;
  const float z_const = a.zero_const + z_shift;
  if (partials) {
    // The slice's groups: a run of gs floats per row, not 16-byte aligned in general. Four
    // elements per thread are loaded before any is stored, so their round trips overlap.
    constexpr int kBatch = 4;
    const int total = 16 * NT * NW * gs;
    for (int i0 = tid; i0 < total; i0 += kBatch * NW * 64) {
      float sc[kBatch], zr[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int i = i0 + u * NW * 64;
        const int row = i / gs;
        const int gg = i - row * gs;
        // Rows past N, and elements past the slice's (a repeat of element 0), read past the
        // end of the tensors or in bounds; only elements of the slice are stored.
        const uint32_t off = i < total ? uint32_t(((n0 + row) * a.G + g0 + gg) * 4) : 0u;
        sc[u] = buf_load_f32(ms, off, 0);
        zr[u] = buf_load_f32(mz, off, 0);
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int i = i0 + u * NW * 64;
        if (i < total) {
          const int row = i / gs;
          sz_lds[row * mstride + (i - row * gs)] = f32x2{sc[u], asym ? zr[u] + z_shift : z_const};
        }
      }
    }
  }
  for (int p = partials ? pieces : tid; p < pieces; p += NW * 64) {
    const uint32_t off = mbase + uint32_t(p) * 16;  // rows past N: past the tensors, zeros
    const f32x4 sf = __builtin_bit_cast(f32x4, buf_load16(ms, off, 0));
    const f32x4 zf = __builtin_bit_cast(f32x4, buf_load16(mz, off, 0));
    const int row = (p * 4) / G;
    const int g = p * 4 - row * G;
    // Symmetric codes use the constant offset, so the arithmetic below never branches.
    f32x4 lo, hi;
    lo[0] = sf[0]; lo[1] = asym ? zf[0] + z_shift : z_const;
    lo[2] = sf[1]; lo[3] = asym ? zf[1] + z_shift : z_const;
    hi[0] = sf[2]; hi[1] = asym ? zf[2] + z_shift : z_const;
    hi[2] = sf[3]; hi[3] = asym ? zf[3] + z_shift : z_const;
    *reinterpret_cast<f32x4*>(sz_lds + row * mstride + g) = lo;
    *reinterpret_cast<f32x4*>(sz_lds + row * mstride + g + 2) = hi;
  }
  store_x(0);
  __syncthreads();

  const NibbleConsts nib = NibbleConsts::make<Act>(uint32_t(a.ldq) & 0u);
  f32x4 tot[NT][MB];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) tot[t][mb] = zero4;
  const f32x2* const sz_row = sz_lds + (16 * wave * NT + col) * mstride;

  // Chunk c reads buffer c % 2 while the registers fetch chunk c + 1 (the last chunk again at
  // the end, so that the loads keep one static order); they go to the other buffer, last read
  // during chunk c - 1, which the barrier at the end of chunk c - 1 has released. R chunks at a
  // time, so that every ring slot index is a constant.
  const int chunks = split_steps / C;  // split_steps % (R * C) == 0 (host check)
  for (int c0 = 0; c0 < chunks; c0 += R)
#pragma unroll
  for (int rr = 0; rr < R; ++rr) {
    const int c = c0 + rr;
    load_x(c + 1 < chunks ? c + 1 : c);
    const u32x4* xb = xbuf + (c & 1) * kChunk;
    const float* xsb = xs_lds + (c & 1) * (C * MB * 16);
#pragma unroll
    for (int u = 0; u < C; ++u) {
      const int step = s0 + c * C + u;
      const int g = int(div_small(uint32_t(step), group_magic)) - g0;
      u32x4 xa[MB][4];
      f32x4 xs[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int j = 0; j < 4; ++j) xa[mb][j] = xb[u * kStepPieces + ((mb * 4 + kq) * 4 + j) * 16 + col];
        xs[mb] = *reinterpret_cast<const f32x4*>(xsb + (u * MB + mb) * 16 + 4 * kq);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const f32x2 sz = sz_row[16 * t * mstride + g];
        const u32x4 q = cw[rr * C + u][t];
        const u32x4 b[4] = {nib.operand(q.x), nib.operand(q.y), nib.operand(q.z), nib.operand(q.w)};
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          f32x4 acc = Mfma16<Act>::run(xa[mb][0], b[0], zero4);
#pragma unroll
          for (int j = 1; j < 4; ++j) acc = Mfma16<Act>::run(xa[mb][j], b[j], acc);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            tot[t][mb][r] = __builtin_fmaf(sz[0], __builtin_fmaf(-sz[1], xs[mb][r], acc[r]), tot[t][mb][r]);
        }
      }
      load_codes(rr * C + u, step + R * C);
    }
    store_x((c + 1) & 1);
    __syncthreads();
  }

  // ---- lane (col, kq) holds tokens 16 mb + 4 kq + r of feature n0 + 16 (wave NT + t) + col ----
  if (partials) {
    float* part = partials + size_t(blockIdx.y) * size_t(a.M) * size_t(a.N);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int64_t nn = n0 + 16 * (wave * NT + t) + col;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t m = 16 * mb + 4 * kq + r;
          if (m < a.M && nn < a.N) part[m * a.N + nn] = tot[t][mb][r];
        }
    }
    return;
  }
  const Raw* bias = static_cast<const Raw*>(a.bias);
  Raw* y = static_cast<Raw*>(a.y);
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int64_t nn = n0 + 16 * (wave * NT + t) + col;
    const float b0 = (bias && nn < a.N) ? Act::load(bias[nn]) : 0.0f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = 16 * mb + 4 * kq + r;
        const float v = tot[t][mb][r] + b0;
        if (a.epilogue == kEpiSwiglu) {
          // Gate rows 8p .. 8p+3 and up rows 8p+4 .. 8p+7 sit four lanes apart (N % 8 == 0).
          const float up = __shfl_xor(v, 4, 64);
          if (m < a.M && nn < a.N && (nn & 4) == 0)
            y[m * a.ldy + (nn >> 3) * 4 + (nn & 3)] = Act::store(swiglu<Act>(v, up));
        } else if (m < a.M && nn < a.N) {
          put_y<Act>(a, m * a.ldy + nn, v);
        }
      }
  }
}

// ---- activations in whole lines -------------------------------------------------------------
//
// The decode kernels' MFMA layout gives lane (col, kq) the activations x[row col][32 kq + 8 j ..]
// of a 128-code step as fragment j: one 16-byte load per j puts 16 rows x 4 pieces spaced 64
// bytes apart in flight, half of every line it touches, and the four loads of a step touch the
// same 32 lines four times over. Broadcast to every CU, as the decode grids need it, that L2
// traffic is what costs: at 32 tokens over K = 4096 (256 KB per CU) the fragment-shaped loads
// took ~6 us of an o projection's 10.6 us. Instead each block of 16 token rows x one step
// (16 x 256 bytes) comes in as four loads of 4 rows x 256 bytes -- whole lines -- and goes
// through a per-wave LDS tile (rows padded to kXTileRow bytes, so the column reads below hit
// 16 distinct bank groups) into the MFMA layout. Token rows past M read zeros.
constexpr int kXTileRow = 272;
constexpr int kXTileBytes = 16 * kXTileRow;

// Raw loads of steps [step0, step0 + NS) of token blocks 0 .. MB - 1: piece [i][mb][h] holds
// row 16 mb + 4 h + lane / 16, bytes 16 (lane % 16) of the step.
template <int NS, int MB>
__device__ __forceinline__ void load_x_lines(u32x4 (&raw)[NS][MB][4], const LinearArgs& a, int64_t step0) {
  const uint32_t xbytes = uint32_t(a.M * a.ldx * 2);
  const auto xr = make_rsrc(a.x, xbytes);
  const int lane = threadIdx.x & 63;
  // Issued step by step, so the first step's pieces land first.
#pragma unroll
  for (int i = 0; i < NS; ++i)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int64_t m = 16 * mb + 4 * h + (lane >> 4);
        const uint32_t row = m < a.M ? uint32_t((m * a.ldx + step0 * 128) * 2 + 16 * (lane & 15)) : xbytes;
        raw[i][mb][h] = buf_load16(xr, row, uint32_t(i) * 256);
      }
}

// The same pieces rearranged through the wave's LDS tile into MFMA fragments: frag[i][mb][j] =
// x[16 mb + col][128 (step0 + i) + 32 kq + 8 j .. + 8] for lane (col, kq), or (TR, the order of
// transposed code words) x[...][128 (step0 + i) + 32 j + 8 kq .. + 8]. In place.
template <int NS, int MB, bool TR = false>
__device__ __forceinline__ void lines_to_fragments(u32x4 (&v)[NS][MB][4], uint8_t* tile) {
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int kq = lane >> 4;
#pragma unroll
  for (int i = 0; i < NS; ++i)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      wait_lgkmcnt0();  // the previous block's reads are done before its tile is overwritten
#pragma unroll
      for (int h = 0; h < 4; ++h)
        *reinterpret_cast<u32x4*>(tile + (4 * h + kq) * kXTileRow + 16 * col) = v[i][mb][h];
      wait_lgkmcnt0();
#pragma unroll
      for (int j = 0; j < 4; ++j)
        v[i][mb][j] = *reinterpret_cast<const u32x4*>(tile + col * kXTileRow + (TR ? 64 * j + 16 * kq : 64 * kq + 16 * j));
    }
  wait_lgkmcnt0();
}

// ---- resident-activation kernel (5..32 tokens, K = 4096, group 128) ----------------------------
//
// One workgroup owns TPW consecutive tiles of 16 output features and all of K. Wave w owns the
// K range of steps 4 w .. 4 w + 3 (512 codes) of every tile: its activations for that range
// (4 steps x MB token blocks, 32 / 64 VGPRs per block pair) come in once, in whole lines, and
// stay in registers while the wave streams the codes of the workgroup's tiles, 16 rows x 64
// bytes per step, through a ring of kKrRing loads. Per tile the wave adds its four
// steps, s * (sum (OFF + q) x - (OFF + z) sum x) per step as in the other decode kernels, and
// leaves the sums in LDS; after one barrier the workgroup adds the eight waves' sums in wave
// order, then bias and epilogue. No K split across workgroups, so no partial sums in memory and
// no second launch. With TPW = 7, gate_up's 1792 tiles fill 256 workgroups, one per CU.
constexpr int kKrWaves = 8;
constexpr int kKrSteps = 4;  // 128-code steps per wave: K = 4096
constexpr int kKrRing = 8;   // code loads in flight per wave
constexpr int kKrGrid = 256;

template <int TPW, int MB>
struct KrGeom {
  static constexpr size_t red_bytes = size_t(TPW) * kKrWaves * MB * 64 * 16;
  static constexpr size_t xt_bytes = size_t(kKrWaves) * kXTileBytes;
  static constexpr size_t lds_bytes() { return red_bytes + xt_bytes; }
};

template <class Act, int TPW, int MB>
__global__ void __launch_bounds__(kKrWaves * 64) decode_kr_kernel(const LinearArgs a) {
  using Geo = KrGeom<TPW, MB>;
  using Raw = typename Act::raw;
  constexpr int NW = kKrWaves;
  constexpr int SPW = kKrSteps;
  constexpr int D = kKrRing;
  constexpr int NIT = TPW * SPW;  // (tile, step) items per wave
  extern __shared__ u32x4 lds[];
  uint8_t* const base = reinterpret_cast<uint8_t*>(lds);
  f32x4* const red = reinterpret_cast<f32x4*>(base);  // [TPW][NW][MB][64]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;
  const int kq = lane >> 4;
  const bool asym = !a.symmetric;
  const int64_t tile0 = int64_t(blockIdx.x) * TPW;
  const int s0 = SPW * w;

  // ---- activations of the wave's K range, then the first codes and metadata ----
  u32x4 xa[SPW][MB][4];
  load_x_lines<SPW, MB>(xa, a, s0);
  __builtin_amdgcn_sched_barrier(0);
  const auto wq = make_rsrc(a.qw, uint32_t(a.N * a.ldq));
  const uint32_t meta_total = uint32_t(a.N * a.G * 4);
  const auto ms = make_rsrc(a.scales, meta_total);
  const auto mz = make_rsrc(asym ? a.zeros : a.scales, meta_total);
  // Item i = (tile t, step s): row 16 (tile0 + t) + col, bytes 64 (s0 + s) + 16 kq. Rows past N
  // repeat row N - 1; their sums are never stored.
  auto row_of = [&](int t) {
    const int64_t n = (tile0 + t) * 16 + col;
    return n < a.N ? n : a.N - 1;
  };
  // Non-temporal for one or two tiles per workgroup; with four or more (gate_up's 7) the
  // default policy streams faster (gate_up at 8 tokens: 17.7 -> 16.4 us), as the two 64-byte
  // halves of each line are requested by the same wave one item apart.
  constexpr int kCodePolicy = TPW >= 4 ? kLoadPolicy : kStreamPolicy;
  auto code = [&](int i) {
    return __builtin_amdgcn_raw_buffer_load_b128(
        wq, int(uint32_t(row_of(i / SPW) * a.ldq) + 64 * (s0 + i % SPW) + 16 * kq), 0, kCodePolicy);
  };
  // Scales and zeros of a tile row for the wave's four groups: one 16-byte load each (G % 4 == 0).
  auto meta = [&](const __amdgpu_buffer_rsrc_t& r, int t) {
    return __builtin_bit_cast(f32x4, buf_load16(r, uint32_t((row_of(t) * a.G + s0) * 4), 0));
  };
  f32x4 msc[2], mzc[2];
  msc[0] = meta(ms, 0);
  mzc[0] = meta(mz, 0);
  u32x4 ring[D];
#pragma unroll
  for (int i = 0; i < D; ++i) ring[i] = code(i < NIT ? i : NIT - 1);
  __builtin_amdgcn_sched_barrier(0);

  // ---- activations into MFMA operand order, with their per-step sums ----
  lines_to_fragments<SPW, MB>(xa, base + Geo::red_bytes + size_t(w) * kXTileBytes);
  const u32x4 ones = {Act::kOne2, Act::kOne2, Act::kOne2, Act::kOne2};
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  // xsum[s][mb][r]: sum of the step's activations of token 16 mb + 4 kq + r -- the product with
  // a matrix of ones puts it in every column, so each lane holds the four it scales.
  f32x4 xsum[SPW][MB];
#pragma unroll
  for (int s = 0; s < SPW; ++s)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      xsum[s][mb] = zero4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xa[s][mb][j] = arrange<Act, kNibble>(xa[s][mb][j]);
        xsum[s][mb] = Mfma16<Act>::run(xa[s][mb][j], ones, xsum[s][mb]);
      }
    }

  // ---- stream the tiles ----
  const NibbleConsts nib = NibbleConsts::make<Act>(uint32_t(a.ldq) & 0u);
  const float z_shift = Act::kNibbleOffset;
  const float z_const = a.zero_const + z_shift;
  f32x4 tot[MB];
#pragma unroll
  for (int i = 0; i < NIT; ++i) {
    const int t = i / SPW;
    const int s = i % SPW;
    if (s == 0) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) tot[mb] = zero4;
      if (t + 1 < TPW) {
        msc[(t + 1) & 1] = meta(ms, t + 1);
        mzc[(t + 1) & 1] = meta(mz, t + 1);
      }
    }
    const u32x4 q = ring[i % D];
    if (i + D < NIT) ring[i % D] = code(i + D);
    const float sc = msc[t & 1][s];
    const float zc = asym ? mzc[t & 1][s] + z_shift : z_const;
    const u32x4 b[4] = {nib.operand(q.x), nib.operand(q.y), nib.operand(q.z), nib.operand(q.w)};
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      f32x4 acc = Mfma16<Act>::run(xa[s][mb][0], b[0], zero4);
#pragma unroll
      for (int j = 1; j < 4; ++j) acc = Mfma16<Act>::run(xa[s][mb][j], b[j], acc);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        tot[mb][r] = __builtin_fmaf(sc, __builtin_fmaf(-zc, xsum[s][mb][r], acc[r]), tot[mb][r]);
    }
    if (s == SPW - 1) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) red[((t * NW + w) * MB + mb) * 64 + lane] = tot[mb];
    }
  }
  __syncthreads();

  // ---- fixed-order sum over the waves (the K ranges); lane (col, kq) of a tile / token block
  //      holds tokens 16 mb + 4 kq + r of feature 16 tile + col ----
  const Raw* bias = static_cast<const Raw*>(a.bias);
  Raw* y = static_cast<Raw*>(a.y);
  for (int e = tid; e < TPW * MB * 64; e += NW * 64) {
    const int ln = e & 63;
    const int mb = (e >> 6) % MB;
    const int t = (e >> 6) / MB;
    const int c = ln & 15;
    const int64_t n = (tile0 + t) * 16 + c;
    if (n >= a.N) continue;
    if (a.epilogue == kEpiSwiglu && (c & 4)) continue;  // the gate lane computes the pair
    f32x4 v = red[((t * NW) * MB + mb) * 64 + ln];
    f32x4 u = {0.f, 0.f, 0.f, 0.f};
    if (a.epilogue == kEpiSwiglu) u = red[((t * NW) * MB + mb) * 64 + ln + 4];
#pragma unroll
    for (int w2 = 1; w2 < NW; ++w2) {
      v += red[((t * NW + w2) * MB + mb) * 64 + ln];
      if (a.epilogue == kEpiSwiglu) u += red[((t * NW + w2) * MB + mb) * 64 + ln + 4];
    }
    const float bv = bias ? Act::load(bias[n]) : 0.0f;
    const float bu = (bias && a.epilogue == kEpiSwiglu) ? Act::load(bias[n + 4]) : 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t m = 16 * mb + 4 * (ln >> 4) + r;
      if (m >= a.M) continue;
      if (a.epilogue == kEpiSwiglu) {
        // Gate rows 8p .. 8p+3 and up rows 8p+4 .. 8p+7 (N % 8 == 0).
        y[m * a.ldy + (n >> 3) * 4 + (n & 3)] = Act::store(swiglu<Act>(v[r] + bv, u[r] + bu));
      } else {
        put_y<Act>(a, m * a.ldy + n, v[r] + bv);
      }
    }
  }
}

// ---- K-sliced persistent kernel (5..64 tokens, group a multiple of 128) -----------------------
//
// For grids of a few hundred tiles of 16 output features (qkv, o, down) a workgroup per tile
// reads the whole activation matrix for 16 rows of codes: at 32 tokens over K = 4096 that is
// 256 KB of activations against 32 KB of codes, and the kernels that split K over the waves of
// such a workgroup spend most of their time bringing activations in. Here the activations are
// brought in once per workgroup and reused over many tiles.
//
// Workgroup (s, p) of an S x P grid owns the K slice of blocks s * NW .. s * NW + NW - 1 (256
// codes each) and the tiles p, p + P, p + 2P, ...; wave w owns block b = s * NW + w of each of
// those tiles. The wave's activations (2 steps x MB token blocks, in MFMA operand order as in
// the multi-tile kernel, with their per-step sums) are loaded once into registers. The codes of
// a block come in whole cache lines (two direct-to-LDS loads of 8 rows x 128 bytes, swizzled as
// in the line-streaming kernel), together with the scales and zeros of its two steps (two
// 4-byte direct-to-LDS loads), into a per-wave ring of R tiles; a slot is refilled with the tile
// R further on as soon as it has been read. Every load inside the tile loop goes to LDS, four
// per tile and wave in one fixed order, so the waits are static counts of the loads issued
// after a tile's. Per tile the waves' sums meet in LDS (double-buffered, one barrier per tile)
// and are added in wave order; with S > 1 they go to partials[s][m][n] for the fixed-order
// reduction kernel, otherwise to y with bias and epilogue.
//
// Measured on MI355X (down, K = 14336, at 8 tokens): the workgroups' activations are in after
// ~1.8 us, the first tile completes at ~4.3 us (the first R tiles of every workgroup arrive as
// one burst) and the others every ~0.8 us, i.e. ~5.2 TB/s of codes in the steady state. Two
// other ways of bringing in the scales and zeros measured slower: staging those of all the
// workgroup's tiles once, along whole rows, behind a barrier (+0.4 us), and each wave loading
// its own for all its tiles ahead of the codes (+2.4 us). Deeper rings were slower too (R = 4:
// +1 us, R = 6: +2.6 us), as they lengthen the initial burst.
template <int NW, int R, int MB>
struct KsGeom {
  static constexpr int kCodeBytes = 2048;          // 16 rows x 128 bytes
  static constexpr int kSlot = kCodeBytes + 512;   // + scales and zeros: 64 floats each
  static constexpr size_t ring_bytes() { return size_t(NW) * R * kSlot; }
  static constexpr size_t red_bytes() { return size_t(2) * NW * MB * 4 * 64 * 4; }
  static constexpr size_t xt_bytes() { return size_t(NW) * kXTileBytes; }
  static constexpr size_t lds_bytes() { return ring_bytes() + red_bytes() + xt_bytes(); }
};

// FMT = kByte: 8-bit codes; a block of 128 bytes per row is one 128-code step (a slice of NW
// blocks covers 1024 codes), lane (col, kq) reads chunks 2kq and 2kq + 1 of its row, and the
// byte operands, flipped signs and zero-point offset are the one-shot kernel's.
// GS = 2: nibble codes in groups of 64, four groups per block. The lane's code words are
// transposed across the wave's rows as in the one-shot kernel (MFMA e covers codes 32e .. 32e +
// 31 of the step, inside group e / 2), the activation fragments are read in that order, and
// each group keeps its own sums and scale; lane l loads the metadata of row l % 16 of group
// l / 16 of the block.
template <class Act, int NW, int R, int MB, int FMT = kNibble, int GS = 1>
__global__ void __launch_bounds__(NW * 64)
    decode_ks_kernel(const LinearArgs a, int per_slice, uint32_t group_magic, float* partials) {
  static_assert(GS == 1 || (GS == 2 && FMT == kNibble), "groups of 64: nibble codes");
  constexpr int SPB = FMT == kNibble ? 2 : 1;  // 128-code steps per block
  using Geo = KsGeom<NW, R, MB>;
  using Raw = typename Act::raw;
  constexpr int kLoadsPerTile = 4;
  extern __shared__ u32x4 lds[];
  uint8_t* const base = reinterpret_cast<uint8_t*>(lds);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;
  const int kq = lane >> 4;
  const bool asym = !a.symmetric;
  const int slice = int(blockIdx.x) / per_slice;
  const int first = int(blockIdx.x) - slice * per_slice;
  const int64_t tiles = (a.N + 15) / 16;
  if (first >= tiles) return;  // the host sizes the grid so that this does not happen
  const int ntiles = int((tiles - first + per_slice - 1) / per_slice);
  const int blk = slice * NW + wave;  // this wave's block of 128 bytes per row
  uint8_t* const ring = base + size_t(wave) * R * Geo::kSlot;
  float* const red = reinterpret_cast<float*>(base + Geo::ring_bytes());

  // ---- the wave's activations, in whole lines: steps 2 b and 2 b + 1 of every token block ----
  u32x4 xa[SPB][MB][4];
  load_x_lines<SPB, MB>(xa, a, int64_t(blk) * SPB);
  __builtin_amdgcn_sched_barrier(0);

  // ---- direct-to-LDS loads of tile j's block into slot j % R ----
  const uint32_t meta_total = uint32_t(a.N * a.G * 4);
  const auto ms = make_rsrc(a.scales, meta_total);
  const auto mz = make_rsrc(asym ? a.zeros : a.scales, meta_total);
  // Metadata: lane l loads row l % 16 of step (l / 16) % 2 of the block (lanes 32..63 repeat
  // lanes 0..31), landing at float l of the slot's scale (zero) area.
  const uint32_t mgroup = GS == 2 ? uint32_t(4 * blk + (lane >> 4))
                                  : div_small(uint32_t(SPB * blk + (SPB == 2 ? (lane >> 4) & 1 : 0)), group_magic);
  const uint32_t meta_lane = (uint32_t(lane & 15) * uint32_t(a.G) + mgroup) * 4;
  const auto wq = make_rsrc(a.qw, uint32_t(a.N * a.ldq));
  const int r8 = lane >> 3;
  const uint32_t chunk_off = uint32_t((lane & 7) ^ r8) * 16;
  const uint32_t code_so = uint32_t(blk) * 128;
  auto issue = [&](int j) {
    const int64_t tile = first + int64_t(j) * per_slice;
    uint8_t* slot = ring + (j % R) * Geo::kSlot;
    // Rows past N: the metadata offset (per lane, so the buffer range check covers it; the
    // scalar offset is not checked) lies past the tensors and reads zeros; the codes repeat
    // row N - 1.
    const uint32_t mo = uint32_t(tile * 16 * a.G * 4) + meta_lane;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ms, (__attribute__((address_space(3))) void*)(slot + Geo::kCodeBytes),
                                             4, mo, 0, 0, kLoadPolicy);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(mz, (__attribute__((address_space(3))) void*)(slot + Geo::kCodeBytes + 256),
                                             4, mo, 0, 0, kLoadPolicy);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      int64_t n = tile * 16 + 8 * h + r8;
      n = n < a.N ? n : a.N - 1;
      load_lds16(wq, slot + 1024 * h, uint32_t(n * a.ldq) + chunk_off, code_so);
    }
  };
  // The first R tiles (the last one again where the list is shorter: those slots are never read).
#pragma unroll
  for (int j = 0; j < R; ++j) issue(j < ntiles ? j : ntiles - 1);
  __builtin_amdgcn_sched_barrier(0);

  // ---- activations into operand order (lane (col, kq), step i, token block mb, MFMA j takes
  //      x[16 mb + col][256 b + 128 i + 32 kq + 8 j .. + 8]), and their per-step sums (one MFMA
  //      chain against ones) ----
  lines_to_fragments<SPB, MB, GS == 2>(xa, base + Geo::ring_bytes() + Geo::red_bytes() + size_t(wave) * kXTileBytes);
  const u32x4 ones = {Act::kOne2, Act::kOne2, Act::kOne2, Act::kOne2};
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  // Per (step, group of the step, token block): the activation sums (with one group per step,
  // entry [i][0] holds the whole step's).
  f32x4 xs[SPB][GS][MB];
#pragma unroll
  for (int i = 0; i < SPB; ++i)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) xa[i][mb][j] = arrange<Act, FMT>(xa[i][mb][j]);
#pragma unroll
      for (int h = 0; h < GS; ++h) {
        constexpr int kPer = 4 / GS;
        xs[i][h][mb] = Mfma16<Act>::run(xa[i][mb][kPer * h], ones, zero4);
#pragma unroll
        for (int j = 1; j < kPer; ++j) xs[i][h][mb] = Mfma16<Act>::run(xa[i][mb][kPer * h + j], ones, xs[i][h][mb]);
      }
    }

  const NibbleConsts nib = NibbleConsts::make<Act>(uint32_t(a.ldq) & 0u);
  const bool flipped = FMT == kByte && a.signed_codes;
  const uint32_t flip = flipped ? 0x80808080u : 0u;
  const float z_shift = Codes<Act, FMT>::kOffset + (flipped ? 128.0f : 0.0f);
  const float z_const = a.zero_const + z_shift;
  // Byte offset, within a block, of chunk 4i + kq of row col (nibbles: step i of the block), or
  // of chunk 2kq + i (bytes: half i of the lane's 32 codes of the block's one step).
  uint32_t rd_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int chunk = FMT == kNibble ? 4 * i + kq : 2 * kq + i;
    rd_off[i] = uint32_t((col >> 3) * 1024 + ((col & 7) * 8 + (chunk ^ (col & 7))) * 16);
  }
  const Raw* bias = static_cast<const Raw*>(a.bias);
  Raw* y = static_cast<Raw*>(a.y);
  const int M = int(a.M);

  for (int j = 0; j < ntiles; ++j) {
    const int64_t tile = first + int64_t(j) * per_slice;
    // Tile j's loads are done once at most those of the tiles after it that were issued, up to
    // R - 1 of them, are outstanding.
    const int after = ntiles - 1 - j < R - 1 ? ntiles - 1 - j : R - 1;
    static_for<R>([&](auto K) {
      if (after == decltype(K)::value) wait_vmcnt<kLoadsPerTile * decltype(K)::value>();
    });
    const uint8_t* slot = ring + (j % R) * Geo::kSlot;
    const float* sm = reinterpret_cast<const float*>(slot + Geo::kCodeBytes);
    f32x4 tot[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) tot[mb] = zero4;
#pragma unroll
    for (int i = 0; i < SPB; ++i) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(slot + rd_off[i]);
      if constexpr (GS == 2) {
        // T[e] in row kq = word kq of row e: codes 32e + 8kq .. + 8 of the step.
        const auto p02 = __builtin_amdgcn_permlane32_swap(w.x, w.z, false, false);
        const auto p13 = __builtin_amdgcn_permlane32_swap(w.y, w.w, false, false);
        const auto r01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
        const auto r23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
        const u32x4 b[4] = {nib.operand(r01[0]), nib.operand(r01[1]), nib.operand(r23[0]), nib.operand(r23[1])};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float sc = sm[16 * (2 * i + h) + col];
          const float zc = asym ? sm[64 + 16 * (2 * i + h) + col] + z_shift : z_const;
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            const f32x4 acc = Mfma16<Act>::run(xa[i][mb][2 * h + 1], b[2 * h + 1],
                                               Mfma16<Act>::run(xa[i][mb][2 * h], b[2 * h], zero4));
#pragma unroll
            for (int r = 0; r < 4; ++r)
              tot[mb][r] = __builtin_fmaf(sc, __builtin_fmaf(-zc, xs[i][h][mb][r], acc[r]), tot[mb][r]);
          }
        }
        continue;
      }
      const float sc = sm[16 * i + col];
      const float zc = asym ? sm[64 + 16 * i + col] + z_shift : z_const;
      u32x4 b[4];
      if constexpr (FMT == kNibble) {
        b[0] = nib.operand(w.x);
        b[1] = nib.operand(w.y);
        b[2] = nib.operand(w.z);
        b[3] = nib.operand(w.w);
      } else {
        const u32x4 w2 = *reinterpret_cast<const u32x4*>(slot + rd_off[1]);
        const uint32_t words[8] = {w.x, w.y, w.z, w.w, w2.x, w2.y, w2.z, w2.w};
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) b[jj] = Codes<Act, kByte>::operand(words, jj, flip);
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        f32x4 acc = Mfma16<Act>::run(xa[i][mb][0], b[0], zero4);
#pragma unroll
        for (int jj = 1; jj < 4; ++jj) acc = Mfma16<Act>::run(xa[i][mb][jj], b[jj], acc);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          tot[mb][r] = __builtin_fmaf(sc, __builtin_fmaf(-zc, xs[i][0][mb][r], acc[r]), tot[mb][r]);
      }
    }
    if (j + R < ntiles) {
      wait_lgkmcnt0();  // the slot's reads are done before the loads overwrite it
      issue(j + R);
    }
    // ---- red[buf][wave][mb][r][lane]; one barrier, then the sum over the waves in order ----
    float* rb = red + (j & 1) * (NW * MB * 256);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) rb[((wave * MB + mb) * 4 + r) * 64 + lane] = tot[mb][r];
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    for (int e = tid; e < 16 * M; e += NW * 64) {
      const int m = e >> 4;
      const int c = e & 15;
      const int src = ((m >> 4) * 4 + (m & 3)) * 64 + c + 16 * ((m >> 2) & 3);
      float v = 0.0f;
#pragma unroll
      for (int w2 = 0; w2 < NW; ++w2) v += rb[w2 * MB * 256 + src];
      const int64_t n = tile * 16 + c;
      if (partials) {
        if (n < a.N) partials[(int64_t(slice) * a.M + m) * a.N + n] = v;
      } else {
        if (bias && n < a.N) v += Act::load(bias[n]);
        if (a.epilogue == kEpiSwiglu) {
          // Gate rows 8p .. 8p+3 and up rows 8p+4 .. 8p+7 sit four lanes apart (N % 8 == 0).
          const float up = __shfl_xor(v, 4, 64);
          if (n < a.N && (c & 4) == 0) y[m * a.ldy + (n >> 3) * 4 + (c & 3)] = Act::store(swiglu<Act>(v, up));
        } else if (n < a.N) {
          put_y<Act>(a, m * a.ldy + n, v);
        }
      }
    }
  }
}

// Fewest tokens for which the N-split kernel beats the multi-tile one on large grids.
constexpr int64_t kNxMinTokens = 5;

template <int MB, int NT, int NW, int C>
constexpr size_t nx_lds_bytes(int64_t G) {
  return size_t((16 * NT * NW * (G + 2) * 8 + 15) / 16) * 16 + size_t(2) * C * MB * 256 * 16 +
         size_t(2) * C * MB * 16 * 4;
}

// splits > 1: K in `splits` equal slices, fp32 partial sums into a.workspace (splits * M * N
// floats), then the reduction kernel.
template <class Act, int MB, int NT, int NW, int C, int R>
hipError_t launch_nx_cfg(const LinearArgs& a, uint32_t magic, hipStream_t stream, int splits = 1) {
  const int64_t steps = a.K / 128;
  if (splits < 1 || steps % splits != 0) return hipErrorInvalidValue;
  const int64_t split_steps = steps / splits;
  if (a.M > 16 * MB || split_steps % (R * C) != 0 || split_steps < R * C) return hipErrorInvalidValue;
  float* partials = nullptr;
  int64_t gs = a.G;
  if (splits > 1) {
    if (!a.workspace || a.workspace_bytes < size_t(splits) * a.M * a.N * 4) return hipErrorInvalidValue;
    partials = static_cast<float*>(a.workspace);
    const int64_t per_group = a.group / 128;
    gs = std::min<int64_t>(a.G, (split_steps + per_group - 1) / per_group + 1);
  }
  const size_t lds = nx_lds_bytes<MB, NT, NW, C>(gs);
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  auto kern = decode_nx_kernel<Act, MB, NT, NW, C, R>;
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return e;
  }
  const int64_t blocks = ((a.N + 15) / 16 + NT * NW - 1) / (NT * NW);
  hipLaunchKernelGGL(kern, dim3(unsigned(blocks), unsigned(splits)), dim3(NW * 64), lds, stream, a, magic,
                     int(split_steps), partials);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  return launch_splitk_reduce(a, partials, splits, stream);
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


template <class Act, int FMT, int NTT, int Q, int NW>
hipError_t launch_stream_cfg(const LinearArgs& a, int steps, uint32_t magic, hipStream_t stream) {
  const int64_t tiles = (a.N + 15) / 16;
  const int64_t blocks = (tiles + NTT - 1) / NTT;
  const size_t stage = StreamGeom<FMT>::lds_bytes(a.M, steps, a.G, NTT);
  const size_t red = size_t(NW) * NTT * a.M * 16 * sizeof(float);
  const size_t lds = stage > red ? stage : red;
  if (a.M == 1) {
    hipLaunchKernelGGL((decode_stream_kernel<Act, FMT, NTT, Q, NW, 1>), dim3(unsigned(blocks)),
                       dim3(NW * 64), lds, stream, a, steps, magic);
  } else {
    hipLaunchKernelGGL((decode_stream_kernel<Act, FMT, NTT, Q, NW, 4>), dim3(unsigned(blocks)),
                       dim3(NW * 64), lds, stream, a, steps, magic);
  }
  return hipGetLastError();
}

// Tiles per workgroup: two when there are enough tiles for every CU to take several.
inline int stream_ntt(const LinearArgs& a) { return (a.N + 15) / 16 >= 4 * 256 ? 2 : 1; }

template <class Act, int FMT, int NW>
hipError_t launch_stream_nw(const LinearArgs& a, int steps, int q, uint32_t magic, hipStream_t stream) {
  if (stream_ntt(a) == 2) return launch_stream_cfg<Act, FMT, 2, 2, NW>(a, steps, magic, stream);
  if (q == 4) return launch_stream_cfg<Act, FMT, 1, 4, NW>(a, steps, magic, stream);
  return launch_stream_cfg<Act, FMT, 1, 2, NW>(a, steps, magic, stream);
}

template <class Act, int FMT>
hipError_t launch_stream(const LinearArgs& a, int nw, int steps, int q, uint32_t magic,
                         hipStream_t stream) {
  if (nw == 8) return launch_stream_nw<Act, FMT, 8>(a, steps, q, magic, stream);
  return launch_stream_nw<Act, FMT, 4>(a, steps, q, magic, stream);
}

template <class Act, int C, int MMAX, int RM, int GS, bool F32X = false, int FMT = kNibble>
hipError_t launch_oneshot_cfg(const LinearArgs& a, int nw, hipStream_t stream) {
  const size_t lds = OneShotGeom<C, MMAX>::lds_bytes(nw, a.G);
  auto kernel = decode_oneshot_kernel<Act, C, MMAX, RM, false, GS, F32X, FMT>;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kernel, dim3(unsigned((a.N + 15) / 16)), dim3(unsigned(nw * 64)), lds, stream, a);
  return hipGetLastError();
}

template <class Act, int GS, int FMT = kNibble>
hipError_t launch_oneshot(const LinearArgs& a, int c, int nw, hipStream_t stream) {
  // (Two groups per step, or byte codes: no sixteen-step chunks, and no eight-step chunks at
  // 3-4 rows; see try_oneshot.)
  constexpr bool kLong = GS == 1 && FMT == kNibble;
  if (a.M == 1) {
    if constexpr (kLong) {
      if (c == 16) return launch_oneshot_cfg<Act, 16, 1, 1, GS, false, FMT>(a, nw, stream);
    }
    if (c == 8) return launch_oneshot_cfg<Act, 8, 1, 1, GS, false, FMT>(a, nw, stream);
    return launch_oneshot_cfg<Act, 4, 1, 1, GS, false, FMT>(a, nw, stream);
  }
  if (a.M > 4) return launch_oneshot_cfg<Act, 4, 8, 4, GS, false, FMT>(a, nw, stream);
  // Two tokens: half the activation loads and accumulator rows of the four-token form; measured
  // on MI355X, qkv 7.09 -> 6.75 us, o 5.49 -> 5.34, down 12.67 -> 11.65, gate_up level.
  if (a.M == 2) {
    if (c == 8) return launch_oneshot_cfg<Act, 8, 2, 2, GS, false, FMT>(a, nw, stream);
    return launch_oneshot_cfg<Act, 4, 2, 2, GS, false, FMT>(a, nw, stream);
  }
  if constexpr (kLong) {
    if (c == 8) return launch_oneshot_cfg<Act, 8, 4, 4, GS, false, FMT>(a, nw, stream);
  }
  return launch_oneshot_cfg<Act, 4, 4, 4, GS, false, FMT>(a, nw, stream);
}

// M <= 8, 2/4-bit codes in groups of 128 or 64, or 8-bit codes in groups of 128: the one-shot
// kernel (5-8 tokens in 4-step chunks only).
bool try_oneshot(const LinearArgs& a, hipStream_t stream, hipError_t* err) {
  const bool bytes = a.fmt == kByte;
  if (a.M > 8 || a.K % 128 != 0 || a.G % 4 != 0) return false;
  if (bytes ? a.group != 128 : (a.group != 128 && a.group != 64)) return false;
  if (a.epilogue == kEpiSwiglu && a.N % 8 != 0) return false;
  if (a.ldq % 16 != 0 || reinterpret_cast<uintptr_t>(a.qw) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(a.x) % 16 != 0 || a.ldx % 8 != 0) return false;
  if (a.N * a.ldq >= (int64_t(1) << 31) || a.N * a.G * 4 >= (int64_t(1) << 31)) return false;
  const int64_t tiles = (a.N + 15) / 16;
  if (tiles > 0x7FFFFFFF) return false;
  const int64_t steps = a.K / 128;
  // Chunk length: the shortest that keeps a tile within 16 waves. Short chunks spread the
  // per-wave compute over more waves, which finish as their data lands; on MI355X 4-step chunks
  // beat 8 and 16 on every Llama-3-8B projection where they fit.
  int chosen = 0;
  for (int c : {4, 8, 16}) {
    if (c == 16 && a.M > 1) continue;
    if (a.M > 4 && c != 4) continue;  // eight-row slices of longer chunks overflow the LDS
    if (steps % c != 0 || steps / c > 16) continue;
    chosen = c;
    break;
  }
  if (chosen == 0) return false;
  // Groups of 64 or byte codes with eight-step chunks at three or four rows, or sixteen-step
  // chunks, exceed the 128 VGPRs of a wave here (other kernels take those shapes).
  if ((a.group == 64 || bytes) && (chosen == 16 || (chosen == 8 && a.M > 2))) return false;
  const int nw = int(steps / chosen);
  if (16 * a.G / 4 > int64_t(nw) * 64) return false;  // one scale piece per thread
  if (16 * a.M > int64_t(nw) * 64) return false;      // one thread per output of the tile
  if (bytes)
    *err = a.act == kDtBf16 ? launch_oneshot<ActBf16, 1, kByte>(a, chosen, nw, stream)
                            : launch_oneshot<ActF16, 1, kByte>(a, chosen, nw, stream);
  else if (a.group == 64)
    *err = a.act == kDtBf16 ? launch_oneshot<ActBf16, 2>(a, chosen, nw, stream)
                            : launch_oneshot<ActF16, 2>(a, chosen, nw, stream);
  else
    *err = a.act == kDtBf16 ? launch_oneshot<ActBf16, 1>(a, chosen, nw, stream)
                            : launch_oneshot<ActF16, 1>(a, chosen, nw, stream);
  return true;
}

// fp32 activations of one or two tokens, as three bf16 pieces each (three or six rows), on the
// one-shot kernel with the split and the pieces' sum inside it: 4-step chunks (8 for one token
// on rows longer than 16 four-step chunks, groups of 128), groups of 64 or 128, 2/4-bit codes;
// y and bias fp32.
bool try_oneshot_f32(const LinearArgs& a, hipStream_t stream, hipError_t* err) {
  if (a.act != kDtF32 || a.fmt != kNibble || a.M < 1 || a.M > 2 || a.epilogue != kEpiNone) return false;
  if ((a.group != 128 && a.group != 64) || a.K % 128 != 0 || a.G % 4 != 0) return false;
  if (a.ldq % 16 != 0 || reinterpret_cast<uintptr_t>(a.qw) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(a.x) % 16 != 0 || a.ldx % 4 != 0) return false;
  if (a.N * a.ldq >= (int64_t(1) << 31) || a.N * a.G * 4 >= (int64_t(1) << 31)) return false;
  const int64_t tiles = (a.N + 15) / 16;
  if (tiles > 0x7FFFFFFF) return false;
  // Two tokens (six piece rows) over 1024 tiles or more, groups of 128: the split into pieces
  // and the decode kernels lead (gate_up: 24.4 us here against 21.9; with groups of 64 this form
  // leads, 26.3 against 28.3).
  if (a.M == 2 && tiles >= 1024 && a.group != 64) return false;
  const int64_t steps = a.K / 128;
  if (steps % 4 != 0) return false;
  // Rows longer than 16 chunks of four steps (down, K 14336 at one token): eight-step chunks of
  // the three piece rows, one token in groups of 128 only (with groups of 64 the form spills).
  const bool eight = a.M == 1 && a.group == 128 && steps % 8 == 0 && steps / 8 <= 16;
  const int c = steps / 4 <= 16 ? 4 : eight ? 8 : 0;
  if (c == 0) return false;
  const int nw = int(steps / c);
  if (16 * a.G / 4 > int64_t(nw) * 64) return false;  // one scale piece per thread
  if (c == 8)
    *err = launch_oneshot_cfg<ActBf16, 8, 3, 3, 1, true>(a, nw, stream);
  else if (a.M == 1)  // three piece rows: 92 / 62 VGPRs against 104 / 67 for four-row slices
    *err = a.group == 64 ? launch_oneshot_cfg<ActBf16, 4, 3, 3, 2, true>(a, nw, stream)
                         : launch_oneshot_cfg<ActBf16, 4, 3, 3, 1, true>(a, nw, stream);
  else
    *err = a.group == 64 ? launch_oneshot_cfg<ActBf16, 4, 8, 4, 2, true>(a, nw, stream)
                         : launch_oneshot_cfg<ActBf16, 4, 8, 4, 1, true>(a, nw, stream);
  return true;
}

template <class Act, int NB, int D, int MMAX, int RM, int FMT, int GS>
hipError_t launch_line_cfg(const LinearArgs& a, int nw, hipStream_t stream) {
  const size_t lds = LineGeom<NB, D, MMAX, FMT == kNibble ? 2 : 1>::lds_bytes(nw, a.G);
  auto kernel = decode_line_kernel<Act, NB, D, MMAX, RM, FMT, GS>;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kernel, dim3(unsigned((a.N + 15) / 16)), dim3(unsigned(nw * 64)), lds, stream, a);
  return hipGetLastError();
}

// One token only (try_line): the four-row forms would spill and are not instantiated.
template <class Act, int NB, int D, int FMT, int GS>
hipError_t launch_line_m(const LinearArgs& a, int nw, hipStream_t stream) {
  if (a.M != 1) return hipErrorInvalidValue;
  return launch_line_cfg<Act, NB, D, 1, 1, FMT, GS>(a, nw, stream);
}

template <class Act, int FMT, int GS = 1>
hipError_t launch_line(const LinearArgs& a, int nb, int d, int nw, hipStream_t stream) {
  if (nb == 2) return launch_line_m<Act, 2, 2, FMT, GS>(a, nw, stream);
  if (nb == 4)
    return d == 4 ? launch_line_m<Act, 4, 4, FMT, GS>(a, nw, stream) : launch_line_m<Act, 4, 2, FMT, GS>(a, nw, stream);
  return d == 4 ? launch_line_m<Act, 8, 4, FMT, GS>(a, nw, stream) : launch_line_m<Act, 8, 2, FMT, GS>(a, nw, stream);
}

// One token, 2/4-bit codes in groups of 128 or 64 or 8-bit codes in groups of 128, rows of at
// least 8192 codes: the line-streaming kernel. Measured on MI355X at one token: down (K 14336)
// 11.4 -> 9.2 us against the one-shot kernel; on K = 4096 the two are within 2 %, and at 2-4
// tokens the one-shot kernel leads.
bool try_line(const LinearArgs& a, hipStream_t stream, hipError_t* err) {
  if (a.M != 1 || a.K < 8192) return false;
  const bool bytes = a.fmt == kByte;
  const bool g64 = !bytes && a.group == 64;
  const int64_t block_k = bytes ? 128 : 256;  // codes per block of 128 bytes per row
  if ((a.group != 128 && !g64) || a.K % block_k != 0 || a.G % 4 != 0) return false;
  if (a.epilogue == kEpiSwiglu && a.N % 8 != 0) return false;
  if (a.ldq % 16 != 0 || reinterpret_cast<uintptr_t>(a.qw) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(a.x) % 16 != 0 || a.ldx % 8 != 0) return false;
  if (a.N * a.ldq >= (int64_t(1) << 31) || a.N * a.G * 4 >= (int64_t(1) << 31)) return false;
  if ((a.N + 15) / 16 > 0x7FFFFFFF) return false;
  const int64_t blocks = a.K / block_k;
  // Blocks per wave: the fewest that keep a tile within 16 waves (short runs spread the
  // per-wave arithmetic over more waves, which finish as their data lands).
  int nb = 0;
  for (int c : {2, 4, 8}) {
    if (c == 8 && a.M > 1) continue;
    if (blocks % c != 0 || blocks / c > 16) continue;
    nb = c;
    break;
  }
  if (nb == 0) return false;
  const int nw = int(blocks / nb);
  if (16 * a.G / 4 > int64_t(nw) * 64) return false;  // one scale piece per thread
  // Ring depth: every block of the wave up front when LDS allows, else two.
  auto lds_geo = [&](auto geo_nb, auto geo_d) -> size_t {
    constexpr int kNb = decltype(geo_nb)::value, kD = decltype(geo_d)::value;
    return bytes ? LineGeom<kNb, kD, 1, 1>::lds_bytes(nw, a.G) : LineGeom<kNb, kD, 1, 2>::lds_bytes(nw, a.G);
  };
  using I2 = std::integral_constant<int, 2>;
  using I4 = std::integral_constant<int, 4>;
  using I8 = std::integral_constant<int, 8>;
  auto lds_for = [&](int d) -> size_t {
    if (nb == 2) return lds_geo(I2{}, I2{});
    if (nb == 4) return d == 4 ? lds_geo(I4{}, I4{}) : lds_geo(I4{}, I2{});
    return d == 4 ? lds_geo(I8{}, I4{}) : lds_geo(I8{}, I2{});
  };
  int d = nb == 2 ? 2 : 4;
  if (lds_for(d) > 96 * 1024) d = 2;
  if (lds_for(d) > 160 * 1024) return false;
  if (bytes)
    *err = a.act == kDtBf16 ? launch_line<ActBf16, kByte>(a, nb, d, nw, stream)
                            : launch_line<ActF16, kByte>(a, nb, d, nw, stream);
  else if (g64)
    *err = a.act == kDtBf16 ? launch_line<ActBf16, kNibble, 2>(a, nb, d, nw, stream)
                            : launch_line<ActF16, kNibble, 2>(a, nb, d, nw, stream);
  else
    *err = a.act == kDtBf16 ? launch_line<ActBf16, kNibble>(a, nb, d, nw, stream)
                            : launch_line<ActF16, kNibble>(a, nb, d, nw, stream);
  return true;
}

// Tiles of code blocks each wave keeps in flight ahead of the one it computes.
constexpr int kPlineAhead = 2;
// Workgroups of the persistent kernel: one per CU of the MI355X.
constexpr int kPlineGrid = 256;

template <int NB, int MMAX>
size_t pline_lds(int steps, int64_t G, int ntiles) {
  return PLineGeom<NB, kPlineAhead, MMAX>::lds_bytes(8, steps, G, ntiles);
}

template <class Act, int NB, int MMAX, int RM>
hipError_t launch_pline_cfg(const LinearArgs& a, int grid, int ntiles, hipStream_t stream) {
  const size_t lds = pline_lds<NB, MMAX>(int(a.K / 128), a.G, ntiles);
  auto kernel = decode_pline_kernel<Act, NB, kPlineAhead, MMAX, RM>;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kernel, dim3(unsigned(grid)), dim3(512), lds, stream, a, ntiles);
  return hipGetLastError();
}

template <class Act, int NB>
hipError_t launch_pline_nb(const LinearArgs& a, int grid, int ntiles, hipStream_t stream) {
  if (a.M == 1) return launch_pline_cfg<Act, NB, 1, 1>(a, grid, ntiles, stream);
  if (a.M <= 4) return launch_pline_cfg<Act, NB, 4, 4>(a, grid, ntiles, stream);
  return launch_pline_cfg<Act, NB, 8, 4>(a, grid, ntiles, stream);
}

// 2 <= M <= 8, 2/4-bit codes, group 128, at least four tiles of 16 features per CU: the persistent
// line-streaming kernel (8 waves per workgroup, K = 4096 or 8192).
bool try_pline(const LinearArgs& a, hipStream_t stream, hipError_t* err) {
  // Measured on MI355X (gate_up, N 28672): at one token the one-shot kernel stays ahead (13.4
  // against 15.5 us); at 2-4 tokens this kernel leads it (15.5-16.2 against 17.8 us), and at
  // 5-8 tokens the N-split kernel (17.5-17.9 against 18.0-18.6 us).
  if (a.fmt != kNibble || a.M < 2 || a.M > 8 || a.group != 128 || a.K % 256 != 0) return false;
  if (a.epilogue == kEpiSwiglu && a.N % 8 != 0) return false;
  if (a.ldq % 16 != 0 || reinterpret_cast<uintptr_t>(a.qw) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(a.x) % 16 != 0 || a.ldx % 8 != 0) return false;
  if (a.N * a.ldq >= (int64_t(1) << 31) || a.N * a.G * 4 >= (int64_t(1) << 31)) return false;
  const int64_t tiles = (a.N + 15) / 16;
  if (tiles < 4 * kPlineGrid) return false;
  const int64_t blocks = a.K / 256;
  if (blocks % 8 != 0) return false;
  const int nb = int(blocks / 8);
  if (nb != 2 && nb != 4) return false;
  const int steps = int(a.K / 128);
  if (a.G != 16 * nb) return false;                 // metadata: G / 16 = NB loads per wave and tile
  if (a.M * steps * 16 > (a.M > 4 ? 8 : 4) * 512) return false;  // activations: 4 (8) pieces per thread
  const int grid = kPlineGrid;
  const int64_t ntiles = (tiles + grid - 1) / grid;
  if (16 * ntiles > 512) return false;              // bias: one value per thread
  const int mmax = a.M == 1 ? 1 : a.M <= 4 ? 4 : 8;
  const size_t lds = mmax == 1 ? (nb == 2 ? pline_lds<2, 1>(steps, a.G, int(ntiles)) : pline_lds<4, 1>(steps, a.G, int(ntiles)))
                   : mmax == 4 ? (nb == 2 ? pline_lds<2, 4>(steps, a.G, int(ntiles)) : pline_lds<4, 4>(steps, a.G, int(ntiles)))
                               : (nb == 2 ? pline_lds<2, 8>(steps, a.G, int(ntiles)) : pline_lds<4, 8>(steps, a.G, int(ntiles)));
  if (lds > 160 * 1024) return false;
  if (a.act == kDtBf16)
    *err = nb == 2 ? launch_pline_nb<ActBf16, 2>(a, grid, int(ntiles), stream)
                   : launch_pline_nb<ActBf16, 4>(a, grid, int(ntiles), stream);
  else
    *err = nb == 2 ? launch_pline_nb<ActF16, 2>(a, grid, int(ntiles), stream)
                   : launch_pline_nb<ActF16, 4>(a, grid, int(ntiles), stream);
  return true;
}

// Small M: the streaming kernel, when the step geometry fits and x[M, K] fits in LDS.
bool try_stream(const LinearArgs& a, hipStream_t stream, hipError_t* err) {
  if (a.M > 16 || a.epilogue != kEpiNone) return false;
  const int step_k = a.fmt == kNibble ? 128 : 64;
  if (a.group % step_k != 0 || a.K % step_k != 0 || a.ldq % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(a.qw) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(a.x) % 16 != 0 || a.ldx % 8 != 0) return false;
  const int64_t steps = a.K / step_k;
  if (steps >= 65536 || (a.N + 15) / 16 > 0x7FFFFFFF) return false;
  // 32-bit buffer offsets.
  if (a.N * a.ldq >= (int64_t(1) << 31) || a.N * a.G * 4 >= (int64_t(1) << 31)) return false;
  const int ntt = stream_ntt(a);
  const size_t lds = a.fmt == kNibble ? StreamGeom<kNibble>::lds_bytes(a.M, steps, a.G, ntt)
                                      : StreamGeom<kByte>::lds_bytes(a.M, steps, a.G, ntt);
  if (lds > kStreamLds) return false;
  // Waves per workgroup: 4, or 8 when the staged activations need the extra threads (they
  // are loaded in one batch of kStageBatch 16-byte pieces per thread). Several workgroups
  // share a CU.
  const int64_t pieces = a.M * a.K / 8;
  const int64_t meta_pieces = (int64_t(ntt) * 16 * a.G + 3) / 4;
  int nw = 0;
  for (int cand : {4, 8}) {
    if (steps % cand == 0 && pieces <= int64_t(kStageBatch) * cand * 64 &&
        meta_pieces <= int64_t(kMetaBatch) * cand * 64) {
      nw = cand;
      break;
    }
  }
  if (nw == 0) return false;
  // Ring depth: Q steps per wave ahead (4 or 2, dividing the wave's step count).
  const int64_t my_steps = steps / nw;
  const int q = my_steps % 4 == 0 ? 4 : (my_steps % 2 == 0 ? 2 : 0);
  if (q == 0) return false;
  const uint32_t per_group = uint32_t(a.group / step_k);
  const uint32_t magic = per_group == 1 ? 0u
      : uint32_t((uint64_t(1) << 32) / per_group + ((uint64_t(1) << 32) % per_group != 0));
  if (a.act == kDtBf16) {
    *err = a.fmt == kNibble ? launch_stream<ActBf16, kNibble>(a, nw, int(steps), q, magic, stream)
                            : launch_stream<ActBf16, kByte>(a, nw, int(steps), q, magic, stream);
  } else {
    *err = a.fmt == kNibble ? launch_stream<ActF16, kNibble>(a, nw, int(steps), q, magic, stream)
                            : launch_stream<ActF16, kByte>(a, nw, int(steps), q, magic, stream);
  }
  return true;
}


// ---- multi-tile kernel dispatch ----

struct MtConfig {
  int nt, mb, d, nw;
  bool refill = true;  // false: each wave's whole range is loaded up front (steps == d * nw)
};

template <class Act, int NT, int MB, int D, int NW, int WPE, bool REFILL, int GS>
hipError_t launch_mt_cfg(const LinearArgs& a, int steps, uint32_t magic, hipStream_t stream) {
  if (!REFILL && steps != D * NW) return hipErrorInvalidValue;
  const int64_t blocks = (a.N + 16 * NT - 1) / (16 * NT);
  const size_t meta = size_t(16) * NT * (a.G + 2) * 8;
  const size_t red = size_t(NW) * NT * MB * 4 * 64 * 4;
  const size_t lds = meta > red ? meta : red;
  auto kern = decode_mt_kernel<Act, NT, MB, D, NW, WPE, REFILL, GS>;
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(unsigned(blocks)), dim3(NW * 64), lds, stream, a, steps / NW, magic);
  return hipGetLastError();
}

// The instantiated configurations; `pick_mt` chooses among them. GS: groups per step.
template <class Act, int GS>
hipError_t launch_mt(const LinearArgs& a, MtConfig c, int steps, uint32_t magic, hipStream_t stream) {
#define LLMOPT_MT(NT, MB, D, NW, WPE, R)                                                     \
  if (c.nt == NT && c.mb == MB && c.d == D && c.nw == NW && c.refill == R)                   \
    return launch_mt_cfg<Act, NT, MB, D, NW, WPE, R, GS>(a, steps, magic, stream);
  LLMOPT_MT(8, 1, 2, 8, 2, true)
  LLMOPT_MT(2, 1, 4, 8, 2, true)
  LLMOPT_MT(1, 1, 4, 8, 4, true)
  LLMOPT_MT(4, 2, 2, 4, 2, true)
  // Four token blocks with two groups per step would spill inside the main loop.
  if constexpr (GS == 1) {
    LLMOPT_MT(2, 4, 2, 8, 2, true)
  }
  LLMOPT_MT(2, 1, 2, 16, 2, false)
  LLMOPT_MT(1, 2, 4, 8, 2, false)
  LLMOPT_MT(2, 2, 2, 2, 2, true)
#undef LLMOPT_MT
  return hipErrorInvalidValue;
}

// Configuration by token blocks MB = ceil(M / 16) (3 -> 4) and output tiles, as measured on
// MI355X over the Llama-3-8B projections: more feature tiles per workgroup share each
// activation load across more rows, fewer give the grid more workgroups.
// Returns nt = 0 when an older kernel is faster (M <= 16 with long rows: the streaming kernel).
MtConfig pick_mt(const LinearArgs& a, int64_t steps) {
  const int64_t tiles = (a.N + 15) / 16;
  if (a.M <= 16) {
    if (steps > 64) return MtConfig{0, 1, 0, 0};
    if (tiles >= 1024) return MtConfig{8, 1, 2, 8};
    // 32 steps (K = 4096): 16 waves of two steps each, all loaded up front (qkv 12.6 -> 10.2 us
    // at M = 8, 16.2 -> 12.5 us at M = 16; o 14.4 -> 12.2 us at M = 16).
    if (steps == 32) return MtConfig{2, 1, 2, 16, false};
    if (tiles >= 384) return MtConfig{2, 1, 4, 8};
    return MtConfig{1, 1, 4, 8};
  }
  if (a.M <= 32) {
    // 32 steps over at most 256 tiles (o): one tile per workgroup, 8 waves of four steps each,
    // all loaded up front (M = 24 / 32: 15.9 / 17.6 -> 11.1 / 12.4 us); larger grids keep the
    // four-tile workgroups, which share each activation load over four tiles.
    if (steps == 32 && tiles <= 256) return MtConfig{1, 2, 4, 8, false};
    // Up to 512 tiles (qkv): two tiles per wave, two waves of 16 steps (M = 24 / 32: 16.2 /
    // 17.7 -> 13.2 / 14.3 us).
    if (steps == 32 && tiles <= 512) return MtConfig{2, 2, 2, 2};
    return MtConfig{4, 2, 2, 4};
  }
  return MtConfig{2, 4, 2, 8};
}

// 5 .. 32 tokens over at least 1024 output tiles (gate_up): the N-split kernel, eight waves of
// one tile each per workgroup, activations shared through LDS (gate_up at M = 8 / 16 / 24 / 32:
// 22.1 / 24.6 / 30.6 / 33.9 -> 17.9 / 19.3 / 21.5 / 22.6 us). Smaller grids keep the multi-tile
// kernel: eight tiles per workgroup leave too few workgroups to fill the chip.
//
// Smaller grids with long rows (down: K 14336), given a workspace, from 12 tokens: the same
// kernel over K slices, enough of them for 256 workgroups, then the fixed-order reduction of
// the slices' fp32 sums (down at M = 16 / 24 / 32: 27.3 / 34.4 / 34.3 -> 24.0 / 25.7 / 26.8 us,
// the last two against the split-K GEMM). With K = 4096 (qkv, o) the slices are too short to
// pay for the partial sums and the second launch (M = 32: 14.3 / 12.3 -> 20.8 / 13.7 us).
int nx_splits(int64_t M, int64_t N, int64_t steps) {
  if (M < 12 || M > 32 || N % 8 != 0 || steps < 64) return 0;
  const int64_t tiles = (N + 15) / 16;
  if (tiles >= 1024) return 0;
  const int64_t chunks = steps / (M <= 16 ? 8 : 4);
  if (chunks * (M <= 16 ? 8 : 4) != steps) return 0;
  const int64_t wgs = (tiles + 7) / 8;
  for (int64_t s = 2; s <= chunks; ++s)
    if (chunks % s == 0 && wgs * s >= 256) return int(s);
  return 0;
}

template <class Act>
bool try_nx(const LinearArgs& a, int64_t steps, uint32_t magic, hipStream_t stream, hipError_t* err) {
  const int splits = nx_splits(a.M, a.N, steps);
  if (splits > 0) {
    if (!a.workspace || a.workspace_bytes < size_t(splits) * a.M * a.N * 4 ||
        reinterpret_cast<uintptr_t>(a.workspace) % 16 != 0)
      return false;
    *err = a.M <= 16 ? launch_nx_cfg<Act, 1, 1, 8, 8, 1>(a, magic, stream, splits)
                     : launch_nx_cfg<Act, 2, 1, 8, 4, 1>(a, magic, stream, splits);
    return true;
  }
  if (a.M < kNxMinTokens || a.M > 64 || (a.N + 15) / 16 < 1024) return false;
  if (a.M > 32) {
    if (steps % 2 != 0 || nx_lds_bytes<4, 1, 8, 2>(a.G) > 160 * 1024) return false;
    *err = launch_nx_cfg<Act, 4, 1, 8, 2, 1>(a, magic, stream);
    return true;
  }
  if (a.M <= 16) {
    if (steps % 8 != 0 || nx_lds_bytes<1, 1, 8, 8>(a.G) > 160 * 1024) return false;
    *err = launch_nx_cfg<Act, 1, 1, 8, 8, 1>(a, magic, stream);
  } else {
    if (steps % 4 != 0 || nx_lds_bytes<2, 1, 8, 4>(a.G) > 160 * 1024) return false;
    *err = launch_nx_cfg<Act, 2, 1, 8, 4, 1>(a, magic, stream);
  }
  return true;
}

// ---- K-sliced persistent kernel dispatch ----

constexpr int kKsWaves = 8;   // waves per workgroup: a K slice of 8 blocks, 2048 codes
constexpr int kKsAhead = 3;   // tiles each wave keeps in flight
constexpr int kKsGrid = 256;  // workgroups: one per CU

struct KsPlan {
  int slices = 0;     // 0: the kernel does not take the shape
  int per_slice = 0;  // workgroups per slice
};

// Token counts and grids where the kernel leads (measured on MI355X against the multi-tile,
// one-shot and streaming kernels over the Llama-3-8B projections): long rows (K >= 8192) from 5
// tokens (down at 8 / 16 / 32 tokens: 21.2 / 22.4 / 25.3 -> 14.1 / 15.2 / 19.8 us), K = 4096
// from 17 (qkv at 24 / 32: 13.2 / 14.4 -> 12.1 / 13.0 us; o: 11.1 / 12.3 -> 10.8 / 11.7 us;
// at 5-32 tokens over K = 4096 the resident-activation kernel, tried first, leads in turn);
// below those the activations are small enough for the per-tile kernels. Up to 64 tokens (four
// token blocks). Grids of 1024 tiles or more (gate_up) are faster on the N-split kernel
// (gate_up at 32 tokens: 24.6 against 28 us). 8 waves, slices of 2048 codes; 16 waves with K =
// 4096 in one slice and no reduction kernel measured no faster at 2..16 tokens (qkv at 8
// tokens: 9.3 against 9.1 us).
KsPlan plan_ks(int64_t M, int64_t N, int64_t K, int64_t group, int bits) {
  KsPlan p;
  if (bits != 2 && bits != 4 && bits != 8) return p;
  // Byte codes: no resident-activation, N-split or multi-tile form takes them, so the kernel
  // serves them from fewer tokens and on any grid (the streaming and skinny kernels are the
  // alternative: down at 3-4 tokens 27 us there).
  // Groups of 64 (nibble codes): the multi-tile kernel takes 9-32 tokens, the skinny one 33-64;
  // here from 9 tokens (3 on rows of K >= 8192: down at 3-4 tokens 15.0-16.0 -> 14.7-14.8 us,
  // and the fp32 path's three piece rows of one token) up to 48 (three token blocks; four
  // would spill) and on any grid as well.
  const bool bytes = bits == 8;
  const bool g64 = group == 64 && !bytes;
  const bool wide = bytes || g64;  // no resident-activation or N-split form
  const int64_t min_m = K >= 8192 ? (bytes || g64 ? 3 : 5) : (wide ? 9 : 17);
  if (M > (g64 ? 48 : 64) || M < min_m || (group % 128 != 0 && !g64)) return p;
  const int64_t tiles = (N + 15) / 16;
  if ((tiles >= 1024 && !wide) || tiles < 1) return p;
  const int64_t block_k = bits == 8 ? 128 : 256;  // codes per block of 128 bytes per row
  if (K % (block_k * kKsWaves) != 0) return p;
  const int64_t slices = K / (block_k * kKsWaves);
  if (slices > kKsGrid) return p;
  p.slices = int(slices);
  p.per_slice = int(std::min<int64_t>(tiles, std::max<int64_t>(1, kKsGrid / slices)));
  return p;
}

size_t ks_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group, int bits) {
  const KsPlan p = plan_ks(M, N, K, group, bits);
  return p.slices > 1 ? size_t(p.slices) * size_t(M) * size_t(N) * 4 : 0;
}

template <class Act, int MB, int FMT, int GS>
hipError_t launch_ks_cfg(const LinearArgs& a, const KsPlan& p, uint32_t magic, hipStream_t stream) {
  using Geo = KsGeom<kKsWaves, kKsAhead, MB>;
  static_assert(Geo::lds_bytes() <= 160 * 1024, "LDS of one CU");
  auto kern = decode_ks_kernel<Act, kKsWaves, kKsAhead, MB, FMT, GS>;
  const size_t lds = Geo::lds_bytes();
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return e;
  }
  float* partials = p.slices > 1 ? static_cast<float*>(a.workspace) : nullptr;
  hipLaunchKernelGGL(kern, dim3(unsigned(p.slices * p.per_slice)), dim3(kKsWaves * 64), lds, stream, a,
                     p.per_slice, magic, partials);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.slices == 1) return e;
  if (a.defer_reduce && a.deferred_planes && a.epilogue == kEpiNone) {
    *a.deferred_planes = p.slices;  // the caller's consumer adds the slices up
    return hipSuccess;
  }
  return launch_splitk_reduce(a, partials, p.slices, stream);
}

template <class Act, int FMT, int GS = 1>
hipError_t launch_ks_mb(const LinearArgs& a, const KsPlan& p, uint32_t magic, hipStream_t stream) {
  if (a.M <= 16) return launch_ks_cfg<Act, 1, FMT, GS>(a, p, magic, stream);
  if (a.M <= 32) return launch_ks_cfg<Act, 2, FMT, GS>(a, p, magic, stream);
  // Two groups per step: three token blocks (240 VGPRs); four would spill (plan_ks stops
  // groups of 64 at 48).
  if constexpr (GS == 1) return launch_ks_cfg<Act, 4, FMT, GS>(a, p, magic, stream);
  if (a.M <= 48) return launch_ks_cfg<Act, 3, FMT, GS>(a, p, magic, stream);
  return hipErrorInvalidValue;
}

bool try_ks(const LinearArgs& a, hipStream_t stream, hipError_t* err) {
  const KsPlan p = plan_ks(a.M, a.N, a.K, a.group, a.bits);
  if (p.slices == 0) return false;
  if (a.epilogue == kEpiSwiglu && a.N % 8 != 0) return false;
  if (a.ldq % 16 != 0 || reinterpret_cast<uintptr_t>(a.qw) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(a.x) % 16 != 0 || a.ldx % 8 != 0) return false;
  if (a.N * a.ldq >= (int64_t(1) << 31) || a.N * a.G * 4 >= (int64_t(1) << 31)) return false;
  if (a.M * a.ldx * 2 >= (int64_t(1) << 31)) return false;
  if (p.slices > 1) {
    const size_t need = size_t(p.slices) * size_t(a.M) * size_t(a.N) * 4;
    if (!a.workspace || a.workspace_bytes < need || reinterpret_cast<uintptr_t>(a.workspace) % 16 != 0)
      return false;
  }
  const uint32_t per_group = a.group == 64 ? 1u : uint32_t(a.group / 128);
  const uint32_t magic = per_group == 1 ? 0u
      : uint32_t((uint64_t(1) << 32) / per_group + ((uint64_t(1) << 32) % per_group != 0));
  if (a.fmt == kByte)
    *err = a.act == kDtBf16 ? launch_ks_mb<ActBf16, kByte>(a, p, magic, stream)
                            : launch_ks_mb<ActF16, kByte>(a, p, magic, stream);
  else if (a.group == 64)
    *err = a.act == kDtBf16 ? launch_ks_mb<ActBf16, kNibble, 2>(a, p, magic, stream)
                            : launch_ks_mb<ActF16, kNibble, 2>(a, p, magic, stream);
  else
    *err = a.act == kDtBf16 ? launch_ks_mb<ActBf16, kNibble>(a, p, magic, stream)
                            : launch_ks_mb<ActF16, kNibble>(a, p, magic, stream);
  return true;
}

// ---- resident-activation kernel dispatch ----

template <class Act, int TPW, int MB>
hipError_t launch_kr_cfg(const LinearArgs& a, int grid, hipStream_t stream) {
  using Geo = KrGeom<TPW, MB>;
  static_assert(Geo::lds_bytes() <= 160 * 1024, "LDS of one CU");
  auto kern = decode_kr_kernel<Act, TPW, MB>;
  const size_t lds = Geo::lds_bytes();
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(unsigned(grid)), dim3(kKrWaves * 64), lds, stream, a);
  return hipGetLastError();
}

template <class Act, int MB>
hipError_t launch_kr_mb(const LinearArgs& a, int tpw, int grid, hipStream_t stream) {
  if (tpw == 1) return launch_kr_cfg<Act, 1, MB>(a, grid, stream);
  if (tpw == 2) return launch_kr_cfg<Act, 2, MB>(a, grid, stream);
  if (tpw == 4) return launch_kr_cfg<Act, 4, MB>(a, grid, stream);
  return launch_kr_cfg<Act, 7, MB>(a, grid, stream);
}

// Tiles per workgroup of the resident-activation kernel: the fewest of {1, 2, 4, 7} that cover
// the tiles with at most one workgroup per CU; 0 when even 7 do not.
int kr_tiles_per_wg(int64_t tiles) {
  for (int t : {1, 2, 4, 7})
    if (tiles <= int64_t(t) * kKrGrid) return t;
  return 0;
}

// The shapes the resident-activation kernel takes (alignment aside): 5..32 tokens (9..32 on
// grids of at most 512 tiles), K = 4096, 2/4-bit codes in groups of 128, at most 7 tiles per
// workgroup over 256 workgroups.
bool kr_shape(int64_t M, int64_t N, int64_t K, int64_t group, int bits) {
  if ((bits != 2 && bits != 4) || group != 128 || K != 4096) return false;
  // At 5-8 tokens, grids of up to 512 tiles (one or two per workgroup here) go to the one-shot
  // kernel's eight-row form instead: measured on MI355X, o 6.1 -> 5.3 us at 5-6 tokens and
  // 6.2 -> 5.6 at 8, qkv 7.7 -> 7.2-7.7; gate_up (1792 tiles) is 7-12 % faster here.
  if (M <= 8 && (N + 15) / 16 <= 512) return false;
  return M >= 5 && M <= 32 && N >= 1 && kr_tiles_per_wg((N + 15) / 16) > 0;
}

// 5..32 tokens, K = 4096, 2/4-bit codes, group 128: the resident-activation kernel.
bool try_kr(const LinearArgs& a, hipStream_t stream, hipError_t* err) {
  if (a.fmt != kNibble || a.G != 32 || !kr_shape(a.M, a.N, a.K, a.group, a.bits)) return false;
  if (a.epilogue == kEpiSwiglu && a.N % 8 != 0) return false;
  if (a.ldq % 16 != 0 || reinterpret_cast<uintptr_t>(a.qw) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(a.x) % 16 != 0 || a.ldx % 8 != 0) return false;
  if (a.N * a.ldq >= (int64_t(1) << 31) || a.N * a.G * 4 >= (int64_t(1) << 31)) return false;
  if (a.M * a.ldx * 2 >= (int64_t(1) << 31)) return false;
  const int64_t tiles = (a.N + 15) / 16;
  const int tpw = kr_tiles_per_wg(tiles);
  if (tpw == 0) return false;
  const int grid = int((tiles + tpw - 1) / tpw);
  if (a.M <= 16)
    *err = a.act == kDtBf16 ? launch_kr_mb<ActBf16, 1>(a, tpw, grid, stream) : launch_kr_mb<ActF16, 1>(a, tpw, grid, stream);
  else
    *err = a.act == kDtBf16 ? launch_kr_mb<ActBf16, 2>(a, tpw, grid, stream) : launch_kr_mb<ActF16, 2>(a, tpw, grid, stream);
  return true;
}

// M <= 64, 2/4-bit codes, groups of 64 or a multiple of 128 codes: the multi-tile kernel.
bool try_mt(const LinearArgs& a, hipStream_t stream, hipError_t* err) {
  if (a.fmt != kNibble || a.M < 1 || a.M > 64) return false;
  if (a.epilogue == kEpiSwiglu && a.N % 8 != 0) return false;
  const bool g64 = a.group == 64;
  if ((a.group % 128 != 0 && !g64) || a.K % 128 != 0 || a.G % 4 != 0) return false;
  if (a.ldq % 16 != 0 || reinterpret_cast<uintptr_t>(a.qw) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(a.x) % 16 != 0 || a.ldx % 8 != 0) return false;
  if (a.N * a.ldq >= (int64_t(1) << 31) || a.N * a.G * 4 >= (int64_t(1) << 31)) return false;
  if (a.M * a.ldx * 2 >= (int64_t(1) << 31) || a.K * 2 >= (int64_t(1) << 31)) return false;
  if ((a.N + 15) / 16 > 0x7FFFFFFF) return false;
  const int64_t steps = a.K / 128;
  const uint32_t per_group = g64 ? 1u : uint32_t(a.group / 128);
  const uint32_t magic = per_group == 1 ? 0u
      : uint32_t((uint64_t(1) << 32) / per_group + ((uint64_t(1) << 32) % per_group != 0));
  if (!g64 && (a.act == kDtBf16 ? try_nx<ActBf16>(a, steps, magic, stream, err)
                                : try_nx<ActF16>(a, steps, magic, stream, err)))
    return true;
  // The metadata block of the workgroup must fit in LDS, and its loads in two per thread.
  auto fits = [&](const MtConfig& c) {
    if (c.nt == 0 || steps % c.nw != 0 || (!c.refill && steps != int64_t(c.d) * c.nw)) return false;
    if (size_t(16) * c.nt * (a.G + 2) * 8 > 160 * 1024) return false;
    return int64_t(16) * c.nt * a.G / 4 <= int64_t(kMtMetaPer) * c.nw * 64;
  };
  MtConfig c = pick_mt(a, steps);
  if (g64 && !fits(c)) {
    // Groups of 64 have twice the metadata per row, and no streaming kernel takes them: the
    // configurations of the same token blocks with fewer tiles per workgroup, in turn.
    const MtConfig alt[] = {MtConfig{2, 1, 4, 8}, MtConfig{1, 1, 4, 8}, MtConfig{1, 2, 4, 8, false}};
    const int mb = a.M <= 16 ? 1 : a.M <= 32 ? 2 : 4;
    c = MtConfig{0, mb, 0, 0};
    for (const MtConfig& t : alt)
      if (t.mb == mb && fits(t)) {
        c = t;
        break;
      }
  }
  if (!fits(c) || (g64 && c.mb > 2)) return false;  // 33-64 tokens in groups of 64: the skinny kernel
  if (g64)
    *err = a.act == kDtBf16 ? launch_mt<ActBf16, 2>(a, c, int(steps), magic, stream)
                            : launch_mt<ActF16, 2>(a, c, int(steps), magic, stream);
  else
    *err = a.act == kDtBf16 ? launch_mt<ActBf16, 1>(a, c, int(steps), magic, stream)
                            : launch_mt<ActF16, 1>(a, c, int(steps), magic, stream);
  return true;
}

hipError_t launch_skinny(const LinearArgs& a, hipStream_t stream, bool* fits) {
  *fits = false;
  if (a.act != kDtBf16 && a.act != kDtF16) return hipSuccess;
  if (a.epilogue != kEpiNone) return hipSuccess;
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


}  // namespace

hipError_t launch_linear_oneshot_f32(const LinearArgs& a, hipStream_t stream, bool* fits) {
  hipError_t err = hipSuccess;
  *fits = try_oneshot_f32(a, stream, &err);
  return err;
}

bool ks_takes(int64_t M, int64_t N, int64_t K, int64_t group, int bits) {
  return plan_ks(M, N, K, group, bits).slices > 0;
}

bool nx_takes_wide(int64_t M, int64_t N, int64_t K, int64_t group, int bits) {
  // try_nx's 33-64-token form, reached through try_mt (its shape conditions; alignments are
  // checked at launch, and a refusal there falls back to the GEMM).
  if (bits != 2 && bits != 4) return false;
  if (M <= 32 || M > 64 || (N + 15) / 16 < 1024) return false;
  if (group % 128 != 0 || K % 128 != 0 || (K / group) % 4 != 0) return false;
  return (K / 128) % 2 == 0 && nx_lds_bytes<4, 1, 8, 2>(K / group) <= 160 * 1024;
}

size_t decode_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group, int bits) {
  // The split of the kernel the decode path tries first: none for the resident-activation
  // kernel, else the K-sliced kernel's (nibble or byte codes), else the N-split kernel's over K
  // slices.
  if (bits == 8) return ks_takes(M, N, K, group, bits) ? ks_workspace_bytes(M, N, K, group, bits) : 0;
  if (bits != 2 && bits != 4) return 0;
  if (kr_shape(M, N, K, group, bits)) return 0;
  if (ks_takes(M, N, K, group, bits)) return ks_workspace_bytes(M, N, K, group, bits);
  if (group % 128 != 0 || K % 128 != 0 || (K / group) % 4 != 0) return 0;
  const int splits = nx_splits(M, N, K / 128);
  return splits > 0 ? size_t(splits) * size_t(M) * size_t(N) * 4 : 0;
}

hipError_t launch_linear_decode(const LinearArgs& a, hipStream_t stream, bool* fits) {
  *fits = false;
  if (a.act != kDtBf16 && a.act != kDtF16) return hipSuccess;
  if (a.M < 1 || a.M > 64) return hipSuccess;
  hipError_t err = hipSuccess;
  if (try_kr(a, stream, &err) || try_pline(a, stream, &err) || try_line(a, stream, &err) || try_ks(a, stream, &err) ||
      try_oneshot(a, stream, &err) || try_mt(a, stream, &err) || try_stream(a, stream, &err)) {
    *fits = true;
    return err;
  }
  return launch_skinny(a, stream, fits);
}

}  // namespace llmopt
