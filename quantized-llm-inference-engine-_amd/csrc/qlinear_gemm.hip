// Prefill-regime quantized linear, second generation: a 256 x 256 MFMA GEMM whose packed
// weight tiles are dequantized into LDS while the previous tile is being multiplied.
//
// Replaces QuantLinear.forward (src/llmopt/quantization/quant_linear.py:93-113) for long
// batches: y = x @ dequant(qweight)^T + bias, where the reference first expands the whole
// weight to a dense compute-dtype matrix (quantizers.py:204-239) and then calls F.linear.
//
// Shape of the computation. The kernel computes the transposed tile D = W x^T, so that the
// MFMA output gives each lane four consecutive output features of one token (one 8-byte
// store). A workgroup owns 256 output features x 256 tokens and walks K in 64-wide stages.
// Eight waves (two per SIMD) split the tile 2 (features) x 4 (tokens); each wave owns
// 128 x 64 = 4 x 2 tiles of v_mfma_f32_32x32x16_{bf16,f16}.
//
// Pipeline, per stage kt:
//   * MFMAs on LDS buffer kt % 2 (weight rows as A, activation rows as B);
//   * meanwhile every thread dequantizes its 32 codes of stage kt + 1 -- exactly as the
//     reference does: fp32 (q - z) * s with one rounding, then a round-to-nearest-even cast --
//     and stores them, with the activations it loaded one stage earlier, into buffer
//     (kt + 1) % 2;
//   * then it issues the loads for later stages: activations of stage kt + 2 and packed codes
//     (plus scale and zero) of stage kt + 1 + kRing, kept in a small register ring so that HBM
//     latency is covered by kRing - 1 stages of MFMA work;
//   * one barrier per stage.
// LDS rows are 64 elements (128 bytes) with the 16-byte chunk index XOR-swizzled by the row, so
// the fragment reads of 32 consecutive rows spread over the banks.
// Workgroup ids are spread evenly over the 8 XCDs and walked in groups of 8 token-tiles per
// sweep over the feature tiles, so workgroups that run together share tiles in L2.
#include "qcommon.hpp"
#include "qkernels.hpp"

namespace llmopt {
namespace {

constexpr int kBM = 256;  // tokens per workgroup
constexpr int kBN = 256;  // output features per workgroup
constexpr int kBK = 64;   // K per stage
constexpr int kThreads = 512;
constexpr int kRing = 4;  // stages of packed codes in flight per thread (even: see the loop)
constexpr int kGroupM = 8;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

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

// Byte offset (within a [rows][64] bf16 buffer) of 16-byte chunk `c` of row `r`. A row is half
// of the 64 banks; XOR-ing the chunk with (r / 2) % 8 gives 16 consecutive rows 16 distinct
// 4-bank groups, so the 16 lanes that a 16-byte LDS access serves together never collide,
// both for the fragment reads (16 rows, one chunk) and for the stores (8 rows, two halves).
__device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }



template <class Act>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
    qlinear_gemm_kernel(const LinearArgs a, int tiles_m, int tiles_n, uint32_t group_magic) {
  using Raw = typename Act::raw;
  // Two LDS stage buffers as separate arrays: the compiler can then see that the stores of
  // stage kt + 1 and the fragment reads of stage kt never alias, and interleave them.
  // Each holds the dequantized weight tile [kBN][64] followed by the activation tile [kBM][64].
  constexpr int kStage = (kBN + kBM) * kBK * 2;
  __shared__ __attribute__((aligned(16))) uint8_t sbuf0[kStage];
  __shared__ __attribute__((aligned(16))) uint8_t sbuf1[kStage];

  // ---- tile order: even split over the XCDs, then kGroupM token-tiles per feature sweep ----
  int bid = blockIdx.x;
  const int nblk = gridDim.x;
  if (nblk % 8 == 0) bid = (bid % 8) * (nblk / 8) + bid / 8;
  const int per_group = kGroupM * tiles_n;
  const int first_m = (bid / per_group) * kGroupM;
  const int rows_in_group = min(tiles_m - first_m, kGroupM);
  const int tm = first_m + (bid % per_group) % rows_in_group;
  const int tn = (bid % per_group) / rows_in_group;
  const int64_t m0 = int64_t(tm) * kBM;
  const int64_t n0 = int64_t(tn) * kBN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wn = wave >> 2;  // 0..1: 128 features
  const int wm = wave & 3;   // 0..3: 64 tokens

  // ---- per-thread load assignments ----
  // Packed codes: row tid/2, 16 bytes (32 codes) at half tid%2 of the stage's 32 bytes.
  const int w_row = tid >> 1;
  const int w_half = tid & 1;
  int64_t wn_row = n0 + w_row;
  wn_row = wn_row < a.N ? wn_row : a.N - 1;
  const auto wq = make_rsrc(a.qw, uint32_t(a.N * a.ldq));
  const uint32_t wq_off = uint32_t(wn_row * a.ldq + w_half * 16);
  const bool asym = !a.symmetric;
  const uint32_t meta_bytes = uint32_t(a.N * a.G * 4);
  const auto ms = make_rsrc(a.scales, meta_bytes);
  const auto mz = make_rsrc(asym ? a.zeros : a.scales, meta_bytes);
  const uint32_t meta_off = uint32_t(wn_row * a.G * 4);
  const float z_const = a.zero_const;
  // Activations: 4 chunks of 16 bytes; chunk e = tid + 512 i -> row tid/8 + 64 i, chunk tid%8.
  // The swizzle depends on row/2 mod 8, which the + 64 i leaves alone, so the LDS
  // destinations are one offset plus constants.
  const auto xr = make_rsrc(a.x, uint32_t(a.M * a.ldx * 2));
  uint32_t xoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int64_t m = m0 + (tid >> 3) + 64 * i;
    m = m < a.M ? m : a.M - 1;  // rows past M repeat row M-1; their outputs are never stored
    xoff[i] = uint32_t((m * a.ldx + 8 * (tid & 7)) * 2);
  }
  const int xdst = kBN * 128 + swz(tid >> 3, tid & 7);

  u32x4 wring[kRing];
  float sring[kRing], zring[kRing];
  auto load_w = [&](int slot, int kt) {
    const int ktc = kt < (int)(a.K / kBK) ? kt : (int)(a.K / kBK) - 1;
    wring[slot] = buf_load16(wq, wq_off, uint32_t(ktc) * 32);
    // The group index differs between the two threads of a row (w_half), so it goes in the
    // per-lane offset; a lane-varying scalar offset would turn each load into a loop.
    const uint32_t g = div_small(uint32_t(ktc * kBK + w_half * 32), group_magic);
    sring[slot] = buf_load_f32(ms, meta_off + g * 4, 0);
    zring[slot] = buf_load_f32(mz, meta_off + g * 4, 0);
  };
  u32x4 xreg[4];
  auto load_x = [&](int kt) {
    const int ktc = kt < (int)(a.K / kBK) ? kt : (int)(a.K / kBK) - 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) xreg[i] = buf_load16(xr, xoff[i], uint32_t(ktc) * (kBK * 2));
  };
  // Dequantize ring slot -> 32 bf16/fp16 weights -> four 16-byte chunks of the W buffer, with
  // the reference's arithmetic: fp32 (q - z), then * s, each rounded once, then a round-to-
  // nearest-even cast (bit-exact for any zero point). The nibble mask comes from a kernel
  // argument (its extra bits are always zero), so the compiler cannot tell that only four bits
  // per byte survive and converts each code with one v_cvt_f32_ubyte{0..3}: 31 VALU per 8
  // codes, with nothing (such as an asm barrier) that would stop the scheduler from spreading
  // them between the MFMAs.
  const uint32_t nib_mask = 0x0F0F0F0Fu | uint32_t(uint64_t(a.ldq) >> 48);
  auto stash_w = [&](int slot, uint8_t* buf) {
    const float s = sring[slot];
    const float z = asym ? zring[slot] : z_const;
    const uint32_t words[4] = {wring[slot].x, wring[slot].y, wring[slot].z, wring[slot].w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t lo = words[d] & nib_mask;         // codes 0, 2, 4, 6 of this word
      const uint32_t hi = (words[d] >> 4) & nib_mask;  // codes 1, 3, 5, 7
      u32x4 out;
      out.x = Mfma32x<Act>::pack(dequant_exact(float(lo & 0xFFu), z, s),
                                 dequant_exact(float(hi & 0xFFu), z, s));
      out.y = Mfma32x<Act>::pack(dequant_exact(float((lo >> 8) & 0xFFu), z, s),
                                 dequant_exact(float((hi >> 8) & 0xFFu), z, s));
      out.z = Mfma32x<Act>::pack(dequant_exact(float((lo >> 16) & 0xFFu), z, s),
                                 dequant_exact(float((hi >> 16) & 0xFFu), z, s));
      out.w = Mfma32x<Act>::pack(dequant_exact(float(lo >> 24), z, s),
                                 dequant_exact(float(hi >> 24), z, s));
      *reinterpret_cast<u32x4*>(buf + swz(w_row, w_half * 4 + d)) = out;
    }
  };
  auto stash_x = [&](uint8_t* buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(buf + xdst + 64 * 128 * i) = xreg[i];
  };

  const int ktiles = int(a.K / kBK);
  // ---- prologue ----
#pragma unroll
  for (int r = 0; r < kRing; ++r) load_w(r, r);
  load_x(0);
  stash_w(0, sbuf0);
  stash_x(sbuf0);
  load_x(1);
  load_w(0, kRing);  // slot 0 is free again
  __syncthreads();

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int frag_row = lane & 31;
  const int frag_half = lane >> 5;
  // The ring slot holding stage kt + 1 is (kt + 1) % kRing; stages are walked kRing at a time
  // so that every slot index and the buffer parity are constants. The main loop has no
  // conditional stage: a loop-back path that skipped stages would make the compiler wait for
  // every load in flight at the top of the loop.
  auto stage = [&](const int u, const int kt) {
    // kt - u is a multiple of kRing (even), so kt & 1 == u & 1 is a compile-time constant.
    uint8_t* cur = (u & 1) ? sbuf1 : sbuf0;
    uint8_t* nxt = (u & 1) ? sbuf0 : sbuf1;
    const uint8_t* wb = cur;
    const uint8_t* xb = cur + kBN * 128;
    // Stage kt + 1 into the other buffer (the last stage re-stages the clamped last stage,
    // which nothing reads) -- independent of the MFMAs below, so the scheduler can
    // interleave the two.
    stash_w((u + 1) % kRing, nxt);
    stash_x(nxt);
#pragma unroll
    for (int s = 0; s < kBK / 16; ++s) {
      u32x4 af[4], bf[2];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const u32x4*>(wb + swz(wn * 128 + 32 * i + frag_row, 2 * s + frag_half));
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *reinterpret_cast<const u32x4*>(xb + swz(wm * 64 + 32 * j + frag_row, 2 * s + frag_half));
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = Mfma32x<Act>::run(af[i], bf[j], acc[i][j]);
    }
    // Issue order: the first k-slice's fragments, then per MFMA a few dequantization VALU
    // ops, spreading the fragment reads and the LDS stores of the next stage between them.
    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);  // 6 LDS reads
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS store
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // LDS reads
    }
    load_x(kt + 2);
    load_w((u + 1) % kRing, kt + 1 + kRing);
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
  for (int j = 0; j < 2; ++j) {
    const int64_t m = m0 + wm * 64 + 32 * j + (lane & 31);
    if (m >= a.M) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t n = n0 + wn * 128 + 32 * i + 8 * q + 4 * (lane >> 5);
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          v[r] = acc[i][j][4 * q + r];
          if (bias && n + r < a.N) v[r] += Act::load(bias[n + r]);
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
}

}  // namespace

hipError_t launch_linear_gemm(const LinearArgs& a, hipStream_t stream, bool* fits) {
  *fits = false;
  if (a.act != kDtBf16 && a.act != kDtF16) return hipSuccess;
  if (a.fmt != kNibble || a.M < 1) return hipSuccess;
  // A thread's 32 codes of a stage lie in one group; 16-byte aligned rows and activations.
  if (a.K % kBK != 0 || a.K / kBK >= 65536 || a.group % 32 != 0) return hipSuccess;
  if (a.ldq % 16 != 0 || reinterpret_cast<uintptr_t>(a.qw) % 16 != 0) return hipSuccess;
  if (a.ldx % 8 != 0 || reinterpret_cast<uintptr_t>(a.x) % 16 != 0) return hipSuccess;
  if (a.N * a.ldq >= (int64_t(1) << 31) || a.N * a.G * 4 >= (int64_t(1) << 31)) return hipSuccess;
  if (a.M * a.ldx * 2 >= (int64_t(1) << 31)) return hipSuccess;
  const int64_t tm = (a.M + kBM - 1) / kBM;
  const int64_t tn = (a.N + kBN - 1) / kBN;
  if (tm * tn > 0x7FFFFFFF) return hipSuccess;
  const uint32_t g = uint32_t(a.group);
  const uint32_t magic =
      g == 1 ? 0u : uint32_t((uint64_t(1) << 32) / g + ((uint64_t(1) << 32) % g != 0));
  *fits = true;
  if (a.act == kDtBf16) {
    hipLaunchKernelGGL(qlinear_gemm_kernel<ActBf16>, dim3(unsigned(tm * tn)), dim3(kThreads), 0,
                       stream, a, int(tm), int(tn), magic);
  } else {
    hipLaunchKernelGGL(qlinear_gemm_kernel<ActF16>, dim3(unsigned(tm * tn)), dim3(kThreads), 0,
                       stream, a, int(tm), int(tn), magic);
  }
  return hipGetLastError();
}

}  // namespace llmopt
