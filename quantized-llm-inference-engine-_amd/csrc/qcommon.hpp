// Shared device helpers for the gfx950 quantized-linear kernels.
//
// Storage formats (the reference layout, src/llmopt/quantization/quantizers.py:83-97):
//   kNibble : bits 2 and 4. uint8 [N, ldq]; column k in byte k>>1, even k in bits 0-3.
//   kByte   : bits 8. uint8 (asymmetric) or int8 (symmetric) [N, ldq], one code per byte.
// Group metadata: fp32 scales/zeros [N, G], G = K / group, row-major.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llmopt {

enum : int { kNibble = 0, kByte = 1 };
enum : int { kDtF32 = 0, kDtF16 = 1, kDtBf16 = 2 };

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// ---- scalar conversions ----------------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// fp32 -> bf16, round to nearest even; NaN becomes the canonical 0x7FC0 (torch's c10::BFloat16).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return float(__builtin_bit_cast(_Float16, h));
}

// fp32 -> fp16 with the hardware conversion (round to nearest even in the default mode).
// The empty asm pins `f` as a finished fp32 value: without it the backend folds a preceding
// fp32 multiply into v_fma_mixlo_f16, which rounds the exact product once to fp16 instead of
// rounding to fp32 first and then to fp16 as torch's `(q - z) * s` followed by `.to(fp16)`
// does (the two differ on about 0.2% of dequantized weights).
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  asm("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, _Float16(f));
}

// Activation element types. `raw` is the storage word; load/store convert through fp32.
struct ActF32 {
  using raw = float;
  static constexpr int id = kDtF32;
  __device__ static float load(raw v) { return v; }
  __device__ static raw store(float f) { return f; }
};
struct ActF16 {
  using raw = uint16_t;
  static constexpr int id = kDtF16;
  static constexpr uint32_t kOne2 = 0x3C003C00u;       // (1.0, 1.0)
  static constexpr uint32_t kNibbleMagic2 = 0x64006400u;  // 1024.0: OR-ing an int < 1024 gives 1024+q
  static constexpr float kNibbleOffset = 1024.0f;
  __device__ static float load(raw v) { return f16_to_f32(v); }
  __device__ static raw store(float f) { return f32_to_f16_rne(f); }
};
struct ActBf16 {
  using raw = uint16_t;
  static constexpr int id = kDtBf16;
  static constexpr uint32_t kOne2 = 0x3F803F80u;        // (1.0, 1.0)
  static constexpr uint32_t kNibbleMagic2 = 0x43004300u;  // 128.0: OR-ing an int < 128 gives 128+q
  static constexpr float kNibbleOffset = 128.0f;
  __device__ static float load(raw v) { return bf16_to_f32(v); }
  __device__ static raw store(float f) { return f32_to_bf16_rne(f); }
};

// The gated activation of the reference's MLP, silu(gate(x)) * up(x) (layers.py:44), with its
// roundings: gate and up are linear outputs in the compute dtype, silu runs in fp32 on the
// rounded gate and is rounded, and the product of the two rounded values is rounded by the
// caller's store. The exponential is the hardware one (a few fp32 ulps), which the rounding
// to bf16/fp16 that follows hides.
template <class Act>
__device__ __forceinline__ float swiglu(float g, float u) {
  const float gr = Act::load(Act::store(g));
  const float ur = Act::load(Act::store(u));
  const float s = Act::load(Act::store(gr / (1.0f + __expf(-gr))));
  return s * ur;
}

// ---- exact MFMA operands from packed nibbles ------------------------------------------------------
//
// A 4-bit code q becomes an exact bf16 (fp16) operand without float math: OR-ing it into the
// mantissa of 128.0 (1024.0) gives OFF + q. One 32-bit word of eight codes (k0 .. k7, low nibble
// first) yields four operand words holding the pairs (k0,k4) (k1,k5) (k2,k6) (k3,k7).
// The mask sits in a VGPR and the magic in an SGPR, so each pair is a single v_and_or_b32 (gfx9
// VOP3 takes no literal and one scalar operand): 7 VALU ops per 8 codes.
struct NibbleConsts {
  uint32_t mask;   // 0x000F000F, VGPR
  uint32_t magic;  // Act::kNibbleMagic2, SGPR
  template <class Act>
  __device__ static NibbleConsts make(uint32_t opaque_zero) {
    NibbleConsts c;
    c.mask = 0x000F000Fu | opaque_zero;
    c.magic = Act::kNibbleMagic2 | opaque_zero;
    asm("" : "+v"(c.mask));
    asm("" : "+s"(c.magic));
    return c;
  }
  __device__ u32x4 operand(uint32_t d) const {
    u32x4 r;
    r.x = (d & mask) | magic;
    r.y = ((d >> 4) & mask) | magic;
    r.z = ((d >> 8) & mask) | magic;
    r.w = ((d >> 12) & mask) | magic;
    return r;
  }
};

// Eight consecutive activations (x0..x7 in d) rearranged into the code order of the operand
// above (nibbles) or of the byte-code operands of the decode kernels.
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


// ---- code access -----------------------------------------------------------------------------

// Numeric value of code k of one weight row, exactly as the reference reads it:
// nibble storage -> (byte >> 4*(k&1)) & 0xF; uint8 -> 0..255; int8 -> -128..127.
__device__ __forceinline__ float code_value(const uint8_t* row, int64_t k, int fmt, int signed_codes) {
  if (fmt == kNibble) {
    const uint32_t b = row[k >> 1];
    return float((b >> ((k & 1) * 4)) & 0xFu);
  }
  const uint8_t b = row[k];
  return signed_codes ? float(int8_t(b)) : float(b);
}

// The reference's fp32 dequantization of one code: (q - z) * s with one rounding at each
// step, never contracted into an fma (the subtraction is exact for integer-valued z).
__device__ __forceinline__ float dequant_exact(float q, float z, float s) {
  const float d = __fsub_rn(q, z);
  return __fmul_rn(d, s);
}

// ---- buffer loads ---------------------------------------------------------------------------------
// A raw buffer resource over `bytes` bytes at `base` (gfx9 data format word). Loads take a
// per-lane 32-bit byte offset plus a wave-uniform one; addressing stays 32-bit, which keeps
// one VGPR per stream instead of a 64-bit pointer.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, int(bytes), 0x00020000);
}
// Loads use the default cache policy. Marking them volatile (bit 31 of the policy operand) would
// pin them in program order, but the backend then also makes them system-coherent (sc0 sc1),
// which cost 5-25% of the bandwidth of these streams on MI355X; the prefetch rings work without it.
constexpr int kLoadPolicy = 0;
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, int(voff), int(soff), kLoadPolicy);
}
// Packed codes read exactly once per launch go through LDS with non-temporal (nt) loads of
// whole 128-byte lines: measured on MI355X, a pure read of 56 MiB takes 9.8-10.0 us with
// nt loads that each cover 8 rows x 128 B, against 11.2 us with the default policy and 11.5 us
// when each load covers 16 rows x 64 B (half lines, which nt does not help).
constexpr int kStreamPolicy = 2;

// Direct-to-LDS load: lane l's 16 bytes at (voff + soff) land at lds + 16 * l. `lds` must be
// wave-uniform. The hardware counts it in vmcnt; nothing waits for it implicitly, so readers
// of that LDS call wait_vmcnt<> first.
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0,
                                           kStreamPolicy);
}

// Wait until at most N vector-memory loads of this wave are outstanding (loads complete in
// issue order). The memory clobber keeps LDS reads of direct-loaded data after the wait.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Wait for this wave's LDS reads and writes: before a direct load may overwrite LDS that was
// just read.
__device__ __forceinline__ void wait_lgkmcnt0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ float buf_load_f32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, int(voff), int(soff), kLoadPolicy));
}

// Fast exact division of small non-negative integers by a runtime divisor (< 2^16, dividend
// < 2^16): q = umulhi(c, ceil(2^32 / d)). A divisor of 1 is encoded as magic 0.
__device__ __forceinline__ uint32_t div_small(uint32_t c, uint32_t magic) {
  return magic ? __umulhi(c, magic) : c;
}

}  // namespace llmopt
