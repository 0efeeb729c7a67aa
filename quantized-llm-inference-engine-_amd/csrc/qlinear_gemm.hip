// Prefill-regime quantized linear: an MFMA GEMM whose weight operand never touches LDS.
//
// Replaces QuantLinear.forward (src/llmopt/quantization/quant_linear.py:93-113) for long
// batches: y = x @ dequant(qweight)^T + bias, where the reference first expands the whole
// weight to a dense compute-dtype matrix (quantizers.py:204-239) and then calls F.linear.
//
// The kernel computes the transposed tile D = W x^T with v_mfma_f32_32x32x16_{bf16,f16}: the
// A operand of that instruction gives lane l row l % 32 and eight consecutive k of half l / 32,
// which is exactly one 32-bit word of packed 4-bit codes. Each wave therefore loads its own
// weight rows straight from HBM (one 16-byte load per 32-row tile per 64-wide k stage),
// dequantizes them in registers to the reference's values -- fp32 (q - z) * s rounded once,
// then a round-to-nearest-even cast -- and feeds them to the MFMAs. Only
// the activations go through LDS, so an MFMA costs half a kilobyte of LDS reads instead of a
// kilobyte (LDS reads and MFMAs compete on this part), and no weight is dequantized twice.
//
// Layout. A workgroup owns 256 output features x (32 * TT) tokens; its four waves (one per
// SIMD) each take 64 features and every token, i.e. 2 x TT accumulator tiles of 32 x 32.
// Within a 64-wide stage, lane half h owns codes k = 32h .. 32h + 31 (bytes 16h .. 16h + 15 of
// the row's 32-byte stage slice) and feeds codes 8s .. 8s + 7 of those to k-slice s; the
// activation fragment of k-slice s, half h is then the 16-byte chunk 4h + s of the token's
// 64-element stage row. The MFMA sums over all 16 k of a slice, so this relabelling of k is
// free; A and B only have to agree on it.
//
// Pipeline, per 64-wide stage kt (stages are walked four at a time, so every ring slot and
// LDS buffer index below is a compile-time constant):
//   * the activations of stage kt + 2, loaded into registers during stage kt - 1, are stored
//     to LDS buffer (kt + 2) % 4, swizzled so that 32 consecutive token rows of one 16-byte
//     chunk hit distinct banks;
//   * four k-slices of 2 x TT MFMAs read activation fragments from buffer kt % 4 and weight
//     fragments dequantized from a four-stage register ring of packed codes; every k-slice
//     prepares the fragments of the next one, the last k-slice those of stage kt + 1, whose
//     buffer is already complete -- so no MFMA waits on LDS and the barrier costs no refill;
//   * in k-slice 2 the activation loads of stage kt + 3 are issued; at the end of the stage
//     the packed codes of stage kt + 4 and, once per group (every one or two stages), the
//     scales and zeros, then one barrier.
// Scales and zeros are loaded per lane (each lane owns one weight row of a tile); loading them
// once per group instead of once per stage matters: each such load touches 32 cache lines.
#include "qcommon.hpp"
#include "qkernels.hpp"

namespace llmopt {
namespace {

constexpr int kBN = 256;  // output features per workgroup (4 waves x 64)
constexpr int kBK = 64;   // K per stage
constexpr int kThreads = 256;
constexpr int kRing = 4;   // stages of packed codes in flight (= LDS activation buffers)
constexpr int kGroupM = 4;  // token tiles per sweep over the feature tiles

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned char uc4 __attribute__((ext_vector_type(4)));

template <class Act>
struct Mfma32x;
template <>
struct Mfma32x<ActBf16> {
  __device__ static f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // Two fp32 values -> two bf16 (round to nearest even) with one v_cvt_pk_bf16_f32.
  __device__ static uint32_t pack(float lo, float hi) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
  }
};
template <>
struct Mfma32x<ActF16> {
  __device__ static f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static uint32_t pack(float lo, float hi) {
    return uint32_t(f32_to_f16_rne(lo)) | (uint32_t(f32_to_f16_rne(hi)) << 16);
  }
};

// Byte offset (within a [rows][64] buffer of 16-bit values) of 16-byte chunk `c` of row `r`.
// A row is half of the 64 banks; XOR-ing the chunk with (r / 2) % 8 gives 16 consecutive rows
// 16 distinct 4-bank groups, so the 16 lanes that a 16-byte LDS access serves together never
// collide, both for the fragment reads (consecutive rows, one chunk) and for the stores
// (8 rows, all chunks).
__device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

// Per (row, group) constants of the biased dequantization below. For an integer zero point z
// with 16 - z in [0, 240] and |s| < 2^120, adding b = 16 - z to every code byte (no carry
// crosses a byte: q + b <= 255) gives f = q + 16 - z exactly, and fma(f, s, -16 s) rounds the
// exact value (q - z) s once, as the reference's (q - z) * s does (16 s is exact). Any other
// (s, z) -- fractional or out-of-range zero points, huge or non-finite scales, none of which
// the quantizers produce -- takes b = 0 and fma(q, s, -z s), within an ulp of the reference.
struct BiasedMeta {
  uint32_t bias;  // b replicated into the four bytes
  float c;        // -16 s, or -z s
};
__device__ __forceinline__ BiasedMeta biased_meta(float z, float s) {
  const bool exact = z == __builtin_rintf(z) && z >= -224.0f && z <= 16.0f && __builtin_fabsf(s) < 0x1p120f;
  BiasedMeta m;
  m.bias = exact ? uint32_t(16 - int(z)) * 0x01010101u : 0u;
  m.c = exact ? -16.0f * s : -(z * s);
  return m;
}

// Eight packed codes (one 32-bit word) -> the A fragment of one k-slice with the biased
// arithmetic above: per 8 codes two masks, a shift, two byte-wise adds, 8 conversions, 8 fmas
// and 4 packs (3.1 VALU per code against 3.9 for a subtraction and a multiplication each).
template <class Act>
__device__ __forceinline__ u32x4 dequant8_biased(uint32_t word, uint32_t nib_mask, BiasedMeta m, float s) {
  const uc4 lo = __builtin_bit_cast(uc4, (word & nib_mask) + m.bias);         // codes 0, 2, 4, 6
  const uc4 hi = __builtin_bit_cast(uc4, ((word >> 4) & nib_mask) + m.bias);  // codes 1, 3, 5, 7
  u32x4 out;
  out.x = Mfma32x<Act>::pack(__builtin_fmaf(float(lo.x), s, m.c), __builtin_fmaf(float(hi.x), s, m.c));
  out.y = Mfma32x<Act>::pack(__builtin_fmaf(float(lo.y), s, m.c), __builtin_fmaf(float(hi.y), s, m.c));
  out.z = Mfma32x<Act>::pack(__builtin_fmaf(float(lo.z), s, m.c), __builtin_fmaf(float(hi.z), s, m.c));
  out.w = Mfma32x<Act>::pack(__builtin_fmaf(float(lo.w), s, m.c), __builtin_fmaf(float(hi.w), s, m.c));
  return out;
}

// Eight byte codes (two 32-bit words) -> the A fragment of one k-slice. Signed 8-bit codes
// arrive with their sign bit flipped (q + 128) and the offset folded into z, which is exact.
template <class Act>
__device__ __forceinline__ u32x4 dequant8_bytes(uint32_t w0, uint32_t w1, float z, float s) {
  const uc4 b0 = __builtin_bit_cast(uc4, w0);
  const uc4 b1 = __builtin_bit_cast(uc4, w1);
  u32x4 out;
  out.x = Mfma32x<Act>::pack(dequant_exact(float(b0.x), z, s), dequant_exact(float(b0.y), z, s));
  out.y = Mfma32x<Act>::pack(dequant_exact(float(b0.z), z, s), dequant_exact(float(b0.w), z, s));
  out.z = Mfma32x<Act>::pack(dequant_exact(float(b1.x), z, s), dequant_exact(float(b1.y), z, s));
  out.w = Mfma32x<Act>::pack(dequant_exact(float(b1.z), z, s), dequant_exact(float(b1.w), z, s));
  return out;
}

// EPI is the output epilogue (kEpiNone or kEpiSwiglu), a template parameter so that the plain
// kernel's register allocation is not shaped by the fused activation's extra live values.
// FMT is the code storage: kNibble (two codes per byte, widths 1-7) or kByte (8-bit codes).
template <class Act, int TT, int GP, bool SPLIT, int EPI, int FMT>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
    qlinear_gemm_kernel(const LinearArgs a, int tiles_m, int tiles_n, uint32_t group_magic,
                        int splits, float* partials) {
  constexpr int kCB = FMT == kNibble ? 1 : 2;  // 16-byte code loads per tile and stage
  using Raw = typename Act::raw;
  constexpr int kBM = 32 * TT;          // tokens per workgroup
  constexpr int kXStage = kBM * kBK * 2;  // bytes of one activation stage
  constexpr int kXPer = kBM * 8 / kThreads;  // 16-byte activation chunks per thread per stage
  // Four activation stage buffers as separate arrays, so that the compiler can see that the
  // stores of stage kt + 2 and the fragment reads of stages kt and kt + 1 never alias.
  __shared__ __attribute__((aligned(16))) uint8_t xs0[kXStage];
  __shared__ __attribute__((aligned(16))) uint8_t xs1[kXStage];
  __shared__ __attribute__((aligned(16))) uint8_t xs2[kXStage];
  __shared__ __attribute__((aligned(16))) uint8_t xs3[kXStage];
  auto xbuf = [&](int i) -> uint8_t* { return i == 0 ? xs0 : i == 1 ? xs1 : i == 2 ? xs2 : xs3; };

  // ---- tile order: even split over the XCDs; K splits outermost, then kGroupM token-tiles
  //      per sweep over the feature tiles ----
  int bid = blockIdx.x;
  const int nblk = gridDim.x;
  if (nblk % 8 == 0) bid = (bid % 8) * (nblk / 8) + bid / 8;
  const int ntiles = tiles_m * tiles_n;
  const int split = bid / ntiles;
  const int tile = bid - split * ntiles;
  const int per_group = kGroupM * tiles_n;
  const int first_m = (tile / per_group) * kGroupM;
  const int rows_in_group = min(tiles_m - first_m, kGroupM);
  const int tm = first_m + (tile % per_group) % rows_in_group;
  const int tn = (tile % per_group) / rows_in_group;
  const int64_t m0 = int64_t(tm) * kBM;
  const int64_t n0 = int64_t(tn) * kBN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;  // 0..3: 64 features each
  const int frow = lane & 31;
  const int half = lane >> 5;

  // ---- weight rows of this lane: n0 + 64 wave + 32 i + frow, bytes 16 half .. of a stage ----
  const auto wq = make_rsrc(a.qw, uint32_t(a.N * a.ldq));
  const bool asym = !a.symmetric;
  const uint32_t meta_bytes = uint32_t(a.N * a.G * 4);
  const auto ms = make_rsrc(a.scales, meta_bytes);
  const auto mz = make_rsrc(asym ? a.zeros : a.scales, meta_bytes);
  uint32_t wq_off[2], meta_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    int64_t n = n0 + 64 * wave + 32 * i + frow;
    n = n < a.N ? n : a.N - 1;  // rows past N repeat row N-1; their outputs are never stored
    wq_off[i] = uint32_t(n * a.ldq + half * 16 * kCB);
    meta_off[i] = uint32_t(n * a.G * 4);
  }
  const float z_const = a.zero_const;
  // This workgroup's stages: split `split` of the K range, cut at whole metadata periods so
  // that a period never straddles two splits.
  const int units = int(a.K / kBK) / GP;
  const int kt_base = (split * units / splits) * GP;
  const int ktiles = ((split + 1) * units / splits) * GP - kt_base;

  // Packed codes: ring slot u holds stage kt0 + u. Scales and zeros are loaded once per GP
  // stages (GP = 2 when a group spans a multiple of two stages, else 1) into meta slot u / GP.
  // GP stops at 2: the first k-slice of stage kt + 1 is dequantized during stage kt, so a meta
  // slot must be refilled a stage before its first use, which needs at least two slots.
  static_assert(GP == 1 || GP == 2, "metadata period of one or two stages");
  u32x4 wring[kRing][2][kCB];
  float sring[kRing][2], zring[kRing][2];
  // Nibble codes: the biased-dequantization constants of each meta slot, derived from its
  // loaded scale and zero point once per slot, a stage or more after the loads were issued.
  BiasedMeta bring[kRing][2];
  auto load_codes = [&](int slot, int kt) {
    const int ktc = kt_base + (kt < ktiles ? kt : ktiles - 1);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int c = 0; c < kCB; ++c) wring[slot][i][c] = buf_load16(wq, wq_off[i] + 16 * c, uint32_t(ktc) * 32 * kCB);
  };
  auto load_meta = [&](int slot, int kt) {
    const int ktc = kt_base + (kt < ktiles ? kt : ktiles - 1);
    // The group index can differ between the two halves of a wave (group 32), so it goes in
    // the per-lane offset; a lane-varying scalar offset would turn each load into a loop.
    const uint32_t g4 = div_small(uint32_t(ktc * kBK + half * 32), group_magic) * 4;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      sring[slot][i] = buf_load_f32(ms, meta_off[i] + g4, 0);
      zring[slot][i] = buf_load_f32(mz, meta_off[i] + g4, 0);
    }
  };

  // ---- activations: chunk e = tid + 256 i -> token row tid / 8 + 32 i, chunk tid % 8 ----
  // The swizzle depends on row / 2 mod 8, which + 32 i leaves alone, so the LDS destinations
  // are one offset plus constants.
  const auto xr = make_rsrc(a.x, uint32_t(a.M * a.ldx * 2));
  uint32_t xoff[kXPer];
#pragma unroll
  for (int i = 0; i < kXPer; ++i) {
    int64_t m = m0 + (tid >> 3) + 32 * i;
    m = m < a.M ? m : a.M - 1;  // rows past M repeat row M-1; their outputs are never stored
    xoff[i] = uint32_t((m * a.ldx + 8 * (tid & 7)) * 2);
  }
  const int xdst = swz(tid >> 3, tid & 7);
  u32x4 xreg[kXPer];
  auto load_x = [&](int kt) {
    const int ktc = kt_base + (kt < ktiles ? kt : ktiles - 1);
#pragma unroll
    for (int i = 0; i < kXPer; ++i) xreg[i] = buf_load16(xr, xoff[i], uint32_t(ktc) * (kBK * 2));
  };
  auto stash_x = [&](uint8_t* buf) {
#pragma unroll
    for (int i = 0; i < kXPer; ++i) *reinterpret_cast<u32x4*>(buf + xdst + 32 * 128 * i) = xreg[i];
  };

  const uint32_t nib_mask = 0x0F0F0F0Fu | uint32_t(uint64_t(a.ldq) >> 48);
  const bool flipped = FMT == kByte && a.signed_codes;
  const uint32_t flip = flipped ? 0x80808080u : 0u;
  const float z_flip = flipped ? 128.0f : 0.0f;

  // ---- prologue: activations of stages 0 and 1 in LDS, stage 2 in registers, codes and
  //      metadata of stages 0 .. 3 in flight, fragments of stage 0, k-slice 0 ready ----
  load_x(0);
  stash_x(xs0);
  load_x(1);
  stash_x(xs1);
  load_x(2);
#pragma unroll
  for (int r = 0; r < kRing; ++r) load_codes(r, r);
#pragma unroll
  for (int r = 0; r < kRing / GP; ++r) load_meta(r, r * GP);
  __syncthreads();

  f32x16 acc[2][TT];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < TT; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  auto read_b = [&](const uint8_t* buf, int ks, u32x4* bf) {
#pragma unroll
    for (int j = 0; j < TT; ++j)
      bf[j] = *reinterpret_cast<const u32x4*>(buf + swz(32 * j + frow, 4 * half + ks));
  };
  auto word = [](const u32x4& q, int w) { return w == 0 ? q.x : w == 1 ? q.y : w == 2 ? q.z : q.w; };
  auto prep_meta = [&](int slot) {
    if constexpr (FMT == kNibble) {
#pragma unroll
      for (int i = 0; i < 2; ++i) bring[slot][i] = biased_meta(asym ? zring[slot][i] : z_const, sring[slot][i]);
    }
  };
  auto dequant_a = [&](int u, int ks, u32x4* af) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if constexpr (FMT == kNibble) {
        af[i] = dequant8_biased<Act>(word(wring[u][i][0], ks), nib_mask, bring[u / GP][i], sring[u / GP][i]);
      } else {
        // Codes 8ks .. 8ks + 7 of the lane's 32: words 2ks and 2ks + 1 of its 32 bytes.
        const float z = (asym ? zring[u / GP][i] : z_const) + z_flip;
        const u32x4 q = wring[u][i][ks >> 1];
        af[i] = dequant8_bytes<Act>(word(q, (2 * ks) & 3) ^ flip, word(q, (2 * ks + 1) & 3) ^ flip, z,
                                    sring[u / GP][i]);
      }
    }
  };
  u32x4 af[2], bf[TT];
  read_b(xs0, 0, bf);
  prep_meta(0);
  dequant_a(0, 0, af);

  // Stage kt uses LDS buffer kt % 4 and ring slot kt % 4; stages are walked four at a time so
  // that both are constants. The main loop has no conditional stage: a loop-back path that
  // skipped stages would make the compiler wait for every load in flight at the top of the
  // loop. Each k-slice prepares the fragments of the next one (the last k-slice those of the
  // next stage, whose activations were stored a stage earlier), so no MFMA waits for LDS.
  // Buffer (kt + 2) % 4, stored during stage kt, was last read during stage kt - 2 (and its
  // first fragments during kt - 3): the barrier that ends stage kt - 1 orders the two.
  static_assert(kRing == 4, "the stage loop assumes a four-deep ring");
  auto stage = [&](const int u, const int kt) {
    const uint8_t* cur = xbuf(u);
    const uint8_t* nxt = xbuf((u + 1) % 4);
    // The next stage opens meta slot ((u + 1) % 4) / GP: its loads were issued at the end of
    // stage kt + 1 - GP or earlier, and the slot's previous stages were dequantized by now.
    if (((u + 1) % 4) % GP == 0) prep_meta(((u + 1) % 4) / GP);
    stash_x(xbuf((u + 2) % 4));  // stage kt + 2 (past the end: a clamped stage nobody reads)
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      // The activation registers were stored to LDS during k-slices 0 and 1; refill them here,
      // so that at the next stage's stores only the later code loads are still in flight.
      if (ks == 2) load_x(kt + 3);
      u32x4 an[2], bn[TT];
      if (ks < kBK / 16 - 1) {
        read_b(cur, ks + 1, bn);
        dequant_a(u, ks + 1, an);
      } else {
        read_b(nxt, 0, bn);
        dequant_a((u + 1) % 4, 0, an);
      }
#pragma unroll
      for (int j = 0; j < TT; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i) acc[i][j] = Mfma32x<Act>::run(af[i], bf[j], acc[i][j]);
      // Per pair of MFMAs: eight dequantization VALU ops and one fragment read; the
      // activation stores go with the first two k-slices.
#pragma unroll
      for (int p = 0; p < TT; ++p) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        if (ks < 2 && (p & 1)) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS store
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < TT; ++j) bf[j] = bn[j];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = an[i];
    }
    load_codes(u, kt + kRing);
    // Meta slot u / GP was last read for stage kt (its last k-slices were dequantized above).
    if (u % GP == GP - 1) load_meta(u / GP, kt + 1 + kRing - GP);
    __syncthreads();
  };
  int kt0 = 0;
  for (; kt0 + kRing <= ktiles; kt0 += kRing) {
#pragma unroll
    for (int u = 0; u < kRing; ++u) stage(u, kt0 + u);
  }
#pragma unroll
  for (int u = 0; u < kRing - 1; ++u)
    if (kt0 + u < ktiles) stage(u, kt0 + u);

  // ---- epilogue: lane holds token m = lane % 32 of each 32x32 tile and features
  //      8q + 4(lane/32) + r, r < 4 -> one 8-byte store per q ----
  const Raw* bias = static_cast<const Raw*>(a.bias);
  Raw* y = static_cast<Raw*>(a.y);
  const bool vec = (a.ldy % 4 == 0) && (reinterpret_cast<uintptr_t>(a.y) % 8 == 0);
#pragma unroll
  for (int j = 0; j < TT; ++j) {
    const int64_t m = m0 + 32 * j + frow;
    if (m >= a.M) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t n = n0 + 64 * wave + 32 * i + 8 * q + 4 * half;
        if (SPLIT) {
          // Split K: fp32 partial sums into partials[split][m][n]; the reduction kernel that
          // follows on the stream adds the splits in order and applies the bias.
          float* dst = partials + (size_t(split) * a.M + m) * a.N + n;
          if (n + 3 < a.N && a.N % 4 == 0) {
            *reinterpret_cast<f32x4*>(dst) =
                f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (n + r < a.N) dst[r] = acc[i][j][4 * q + r];
          }
          continue;
        }
        const f32x4 t = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          v[r] = t[r];
          if (bias && n + r < a.N) v[r] += Act::load(bias[n + r]);
        }
        if (EPI == kEpiSwiglu) {
          // Rounded gate / up values go to this wave's LDS tile [token][64 fused rows]; the
          // activation is applied below.
          Raw* tile = reinterpret_cast<Raw*>(xbuf(wave)) + (32 * j + frow) * 64 + 32 * i + 8 * q + 4 * half;
          u32x2 pk;
          pk.x = uint32_t(Act::store(v[0])) | (uint32_t(Act::store(v[1])) << 16);
          pk.y = uint32_t(Act::store(v[2])) | (uint32_t(Act::store(v[3])) << 16);
          *reinterpret_cast<u32x2*>(tile) = pk;
          continue;
        }
        Raw* dst = y + m * a.ldy + n;
        if (vec && n + 3 < a.N) {
          u32x2 pk;
          pk.x = uint32_t(Act::store(v[0])) | (uint32_t(Act::store(v[1])) << 16);
          pk.y = uint32_t(Act::store(v[2])) | (uint32_t(Act::store(v[3])) << 16);
          *reinterpret_cast<u32x2*>(dst) = pk;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < a.N) dst[r] = Act::store(v[r]);
        }
      }
    }
  }

  if (EPI == kEpiSwiglu) {
    // Each wave owns 64 fused rows = 8 gate/up blocks = 32 output features of 32 * TT tokens.
    // A lane takes one block: output features 4q .. 4q + 3 of one token, whose gate and up
    // values are two 8-byte runs of the tile row (fused rows 8q .. 8q + 3 and 8q + 4 .. 8q + 7),
    // and stores the four results at once; eight lanes cover a token's 64-byte run.
    const Raw* tile = reinterpret_cast<const Raw*>(xbuf(wave));
    const int64_t out0 = (n0 + 64 * wave) / 2;
    for (int e = lane; e < 32 * TT * 8; e += 64) {
      const int t = e >> 3;
      const int q = e & 7;
      const int64_t m = m0 + t;
      const int64_t f = out0 + 4 * q;
      // N % 8 == 0: a block is either wholly inside the output or wholly past it.
      if (m >= a.M || 2 * f >= a.N) continue;
      const u32x2 gw = *reinterpret_cast<const u32x2*>(tile + t * 64 + 8 * q);
      const u32x2 uw = *reinterpret_cast<const u32x2*>(tile + t * 64 + 8 * q + 4);
      const uint32_t gs[4] = {gw.x & 0xFFFFu, gw.x >> 16, gw.y & 0xFFFFu, gw.y >> 16};
      const uint32_t us[4] = {uw.x & 0xFFFFu, uw.x >> 16, uw.y & 0xFFFFu, uw.y >> 16};
      Raw out[4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        out[r] = Act::store(swiglu<Act>(Act::load(Raw(gs[r])), Act::load(Raw(us[r]))));
      Raw* dst = y + m * a.ldy + f;
      if (vec) {
        u32x2 pk;
        pk.x = uint32_t(out[0]) | (uint32_t(out[1]) << 16);
        pk.y = uint32_t(out[2]) | (uint32_t(out[3]) << 16);
        *reinterpret_cast<u32x2*>(dst) = pk;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[r] = out[r];
      }
    }
  }
}

// Threads per workgroup of the reduction kernel: small workgroups spread a few thousand threads
// over every CU.
constexpr int kReduceThreads = 64;
// Splits whose partial sums a thread loads before adding any of them: the loads of a batch are
// in flight together instead of one round trip per split (down at 16 tokens, 14 splits: 5.4 us
// for the reduction with one load at a time).
constexpr int kReduceBatch = 8;

// y[m, n] = bias[n] + sum over splits, in split order, of partials[split][m][n]: four columns
// per thread. Deterministic: the order of the additions never depends on timing.
template <class Act>
__global__ void __launch_bounds__(kReduceThreads) splitk_reduce_kernel(const LinearArgs a, const float* partials, int splits) {
  using Raw = typename Act::raw;
  if (a.epilogue == kEpiSwiglu) {
    // One thread per output feature group of four: fused columns 8p .. 8p+7 (N % 8 == 0).
    const int64_t p8 = a.N / 8;
    const int64_t e = int64_t(blockIdx.x) * kReduceThreads + threadIdx.x;
    if (e >= a.M * p8) return;
    const int64_t m = e / p8;
    const int64_t n = (e - m * p8) * 8;
    const size_t plane = size_t(a.M) * a.N;
    const float* p = partials + size_t(m) * a.N + n;
    float g[4], u[4];
    for (int s0 = 0; s0 < splits; s0 += kReduceBatch) {
      f32x4 tg[kReduceBatch], tu[kReduceBatch];
#pragma unroll
      for (int i = 0; i < kReduceBatch; ++i) {
        if (s0 + i < splits) {
          tg[i] = *reinterpret_cast<const f32x4*>(p + size_t(s0 + i) * plane);
          tu[i] = *reinterpret_cast<const f32x4*>(p + size_t(s0 + i) * plane + 4);
        }
      }
#pragma unroll
      for (int i = 0; i < kReduceBatch; ++i) {
        if (s0 + i < splits) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            g[r] = s0 + i == 0 ? tg[i][r] : g[r] + tg[i][r];
            u[r] = s0 + i == 0 ? tu[i][r] : u[r] + tu[i][r];
          }
        }
      }
    }
    const Raw* bias = static_cast<const Raw*>(a.bias);
    Raw* y = static_cast<Raw*>(a.y) + m * a.ldy + n / 2;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float gb = bias ? g[r] + Act::load(bias[n + r]) : g[r];
      const float ub = bias ? u[r] + Act::load(bias[n + 4 + r]) : u[r];
      y[r] = Act::store(swiglu<Act>(gb, ub));
    }
    return;
  }
  const int64_t n4 = (a.N + 3) / 4;
  const int64_t e = int64_t(blockIdx.x) * kReduceThreads + threadIdx.x;
  if (e >= a.M * n4) return;
  const int64_t m = e / n4;
  const int64_t n = (e - m * n4) * 4;
  const size_t plane = size_t(a.M) * a.N;
  const Raw* bias = static_cast<const Raw*>(a.bias);
  const float* p = partials + size_t(m) * a.N + n;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (n + 3 < a.N && a.N % 4 == 0) {
    for (int s0 = 0; s0 < splits; s0 += kReduceBatch) {
      f32x4 t[kReduceBatch];
#pragma unroll
      for (int i = 0; i < kReduceBatch; ++i)
        if (s0 + i < splits) t[i] = *reinterpret_cast<const f32x4*>(p + size_t(s0 + i) * plane);
#pragma unroll
      for (int i = 0; i < kReduceBatch; ++i) {
        if (s0 + i < splits) {
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = s0 + i == 0 ? t[i][r] : v[r] + t[i][r];
        }
      }
    }
  } else {
    for (int s = 0; s < splits; ++s)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n + r < a.N) v[r] = s == 0 ? p[s * plane + r] : v[r] + p[s * plane + r];
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (n + r >= a.N) break;
    float o = v[r];
    if (bias) o += Act::load(bias[n + r]);
    put_y<Act>(a, m * a.ldy + n + r, o);
  }
}

// ---- launch plan: token-tile height (32 * TT) and K splits ----------------------------------
//
// A 256 x 256 tile is the most efficient per MFMA, but a short or narrow GEMM gives too few of
// them for 256 CUs (one workgroup per CU). Smaller token tiles raise the workgroup count at a
// higher dequantization cost per MFMA; K splits raise it at the cost of storing and re-reading
// fp32 partial sums that a second kernel adds up. The plan minimizes a simple time model:
// rounds of 256 workgroups x stages per workgroup x time per stage, plus the partial-sum
// traffic of a split, with per-stage times measured on MI355X.
struct GemmPlan {
  int tt = 0;      // 0: the GEMM does not take these sizes
  int splits = 1;
  int64_t tiles_m = 0, tiles_n = 0;
  size_t partial_bytes = 0;
  size_t workspace() const { return splits > 1 ? partial_bytes : 0; }
};

GemmPlan plan_gemm(int64_t M, int64_t N, int64_t K, int64_t group, int fmt) {
  GemmPlan best;
  if (M < 1 || N < 1 || K % kBK != 0 || group % 32 != 0) return best;
  const int gp = group % 128 == 0 ? 2 : 1;
  const int64_t units = K / kBK / gp;
  const double stage_us[9] = {0, 0, 0.95, 0, 1.35, 0, 0, 0, 2.1};
  double best_t = 1e30;
  for (int tt : {8, 4, 2}) {
    if (fmt == kByte && tt == 8) continue;  // the byte-code ring does not fit the 256-token tile
    const int64_t tm = (M + 32 * tt - 1) / (32 * tt);
    const int64_t tn = (N + kBN - 1) / kBN;
    if (tm * tn > 0x7FFFFFFF / 8) continue;
    for (int sp = 1; sp <= 8; ++sp) {
      if (sp > units || (tt == 8 && sp > 1)) break;  // the 256-token tile never splits
      const int64_t wgs = tm * tn * sp;
      const int64_t rounds = (wgs + 255) / 256;
      const double stages = double((units + sp - 1) / sp * gp);
      // Split: write and re-read sp fp32 planes of M x N at ~4 TB/s, plus one more launch.
      const double red = sp > 1 ? 2.0 * sp * double(M) * double(N) * 4.0 / 4e6 + 3.0 : 0.0;
      const double t = double(rounds) * stages * stage_us[tt] + red;
      if (t < best_t * 0.97) {
        best_t = t;
        best.tt = tt;
        best.splits = sp;
        best.tiles_m = tm;
        best.tiles_n = tn;
      }
    }
  }
  if (best.tt) {
    best.partial_bytes = size_t(best.splits) * size_t(M) * size_t(N) * 4;
  }
  return best;
}

template <class Act, int TT, int FMT>
void launch_tt(const LinearArgs& a, const GemmPlan& plan, int splits, hipStream_t stream, uint32_t magic) {
  float* partials = splits > 1 ? static_cast<float*>(a.workspace) : nullptr;
  const int ntiles = int(plan.tiles_m * plan.tiles_n);
  const dim3 grid(unsigned(ntiles * splits)), block(kThreads);
  // The split epilogue is a separate instantiation: its extra live values would push the
  // 256-token tile's main loop into spills. (Split results get the activation, if any, from
  // the reduction kernel.)
  constexpr bool kCanSplit = TT < 8;
  const int tm = int(plan.tiles_m), tn = int(plan.tiles_n);
  const bool gp2 = a.group % 128 == 0;
  if (kCanSplit && splits > 1) {
    if (gp2)
      hipLaunchKernelGGL((qlinear_gemm_kernel<Act, TT, 2, kCanSplit, kEpiNone, FMT>), grid, block, 0, stream, a, tm,
                         tn, magic, splits, partials);
    else
      hipLaunchKernelGGL((qlinear_gemm_kernel<Act, TT, 1, kCanSplit, kEpiNone, FMT>), grid, block, 0, stream, a, tm,
                         tn, magic, splits, partials);
    const int64_t threads = a.epilogue == kEpiSwiglu ? a.M * (a.N / 8) : a.M * ((a.N + 3) / 4);
    hipLaunchKernelGGL(splitk_reduce_kernel<Act>, dim3(unsigned((threads + kReduceThreads - 1) / kReduceThreads)),
                       dim3(kReduceThreads), 0, stream, a, partials, splits);
  } else if (a.epilogue == kEpiSwiglu) {
    if (gp2)
      hipLaunchKernelGGL((qlinear_gemm_kernel<Act, TT, 2, false, kEpiSwiglu, FMT>), grid, block, 0, stream, a, tm, tn,
                         magic, 1, partials);
    else
      hipLaunchKernelGGL((qlinear_gemm_kernel<Act, TT, 1, false, kEpiSwiglu, FMT>), grid, block, 0, stream, a, tm, tn,
                         magic, 1, partials);
  } else {
    if (gp2)
      hipLaunchKernelGGL((qlinear_gemm_kernel<Act, TT, 2, false, kEpiNone, FMT>), grid, block, 0, stream, a, tm, tn,
                         magic, 1, partials);
    else
      hipLaunchKernelGGL((qlinear_gemm_kernel<Act, TT, 1, false, kEpiNone, FMT>), grid, block, 0, stream, a, tm, tn,
                         magic, 1, partials);
  }
}

template <class Act>
void launch_act(const LinearArgs& a, const GemmPlan& plan, int splits, hipStream_t stream, uint32_t magic) {
  if (a.fmt == kByte) {  // byte codes: two code loads per tile and stage; tiles of up to 128 tokens
    if (plan.tt == 4) launch_tt<Act, 4, kByte>(a, plan, splits, stream, magic);
    else launch_tt<Act, 2, kByte>(a, plan, splits, stream, magic);
    return;
  }
  if (plan.tt == 8) launch_tt<Act, 8, kNibble>(a, plan, splits, stream, magic);
  else if (plan.tt == 4) launch_tt<Act, 4, kNibble>(a, plan, splits, stream, magic);
  else launch_tt<Act, 2, kNibble>(a, plan, splits, stream, magic);
}

}  // namespace

hipError_t launch_splitk_reduce(const LinearArgs& a, const float* partials, int splits, hipStream_t stream) {
  const int64_t threads = a.epilogue == kEpiSwiglu ? a.M * (a.N / 8) : a.M * ((a.N + 3) / 4);
  if (a.act == kDtBf16)
    hipLaunchKernelGGL(splitk_reduce_kernel<ActBf16>, dim3(unsigned((threads + kReduceThreads - 1) / kReduceThreads)),
                       dim3(kReduceThreads), 0, stream, a, partials, splits);
  else
    hipLaunchKernelGGL(splitk_reduce_kernel<ActF16>, dim3(unsigned((threads + kReduceThreads - 1) / kReduceThreads)),
                       dim3(kReduceThreads), 0, stream, a, partials, splits);
  return hipGetLastError();
}

size_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group, int fmt) {
  return plan_gemm(M, N, K, group, fmt).workspace();
}

hipError_t launch_linear_gemm(const LinearArgs& a, hipStream_t stream, bool* fits) {
  *fits = false;
  if (a.act != kDtBf16 && a.act != kDtF16) return hipSuccess;
  if (a.M < 1) return hipSuccess;
  // A lane's 32 codes of a stage lie in one group; 16-byte aligned rows and activations.
  if (a.K % kBK != 0 || a.K / kBK >= 65536 || a.group % 32 != 0) return hipSuccess;
  if (a.ldq % 16 != 0 || reinterpret_cast<uintptr_t>(a.qw) % 16 != 0) return hipSuccess;
  if (a.ldx % 8 != 0 || reinterpret_cast<uintptr_t>(a.x) % 16 != 0) return hipSuccess;
  if (a.N * a.ldq >= (int64_t(1) << 31) || a.N * a.G * 4 >= (int64_t(1) << 31)) return hipSuccess;
  if (a.M * a.ldx * 2 >= (int64_t(1) << 31)) return hipSuccess;
  if (a.epilogue == kEpiSwiglu && a.N % 8 != 0) return hipSuccess;
  const GemmPlan plan = plan_gemm(a.M, a.N, a.K, a.group, a.fmt);
  if (plan.tt == 0) return hipSuccess;
  // Without a large enough workspace the plan runs unsplit (same tiles, one workgroup per tile).
  int splits = plan.splits;
  if (splits > 1 && (a.workspace == nullptr || a.workspace_bytes < plan.workspace() ||
                     reinterpret_cast<uintptr_t>(a.workspace) % 16 != 0))
    splits = 1;
  const uint32_t g = uint32_t(a.group);
  const uint32_t magic =
      g == 1 ? 0u : uint32_t((uint64_t(1) << 32) / g + ((uint64_t(1) << 32) % g != 0));
  *fits = true;
  if (a.act == kDtBf16)
    launch_act<ActBf16>(a, plan, splits, stream, magic);
  else
    launch_act<ActF16>(a, plan, splits, stream, magic);
  return hipGetLastError();
}

}  // namespace llmopt
