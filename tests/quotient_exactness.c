/* The quantizer's division-free quotient (csrc/quantize_rtn.hip, rint_quotients):
 *   r = RN(1/s), q0 = RN(w r), e = RN(w - s q0) (one fma), q1 = RN(q0 + e r) (one fma),
 * against the correctly rounded RN(w / s), for every fp32 s in [1, 2) (every significand),
 * every half-integer h = k + 0.5 with k < 256 (|w / s| stays below 256 for 2- to 8-bit codes),
 * and every w within 4 ulps of RN(s h): the only w for which rne(q1) could differ from
 * rne(w / s), since elsewhere both lie within an ulp of w / s and no half-integer is that
 * close. All steps scale exactly with s and w (same power of two) while the remainder stays
 * exactly representable: for every s from 2^-100 to 2^120 once |w / s| >= 1/4 (below that
 * both sides round to zero); the quantizers' smallest scale, 1e-8 / 127 (8-bit symmetric), is
 * inside that range. Prints the case count and the number of
 * cases where q1 != RN(w / s); exits 1 if any. argv[1] (optional): significand stride. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

int main(int argc, char** argv) {
  const uint32_t stride = argc > 1 ? (uint32_t)strtoul(argv[1], 0, 10) : 1u;
  long long cases = 0, wrong = 0, wrong_rint = 0;
#pragma omp parallel for reduction(+ : cases, wrong, wrong_rint) schedule(static)
  for (uint32_t m = 0; m < (1u << 23); m += stride) {
    const float s = from_bits(0x3F800000u | m);
    const float r = 1.0f / s;
    for (int k = 0; k < 256; ++k) {
      const uint32_t w0 = to_bits(s * ((float)k + 0.5f));
      for (int j = -4; j <= 4; ++j) {
        const float w = from_bits(w0 + (uint32_t)j);
        const float want = w / s;
        const float q0 = w * r;
        const float e = fmaf(-s, q0, w);
        const float q1 = fmaf(e, r, q0);
        cases++;
        wrong += q1 != want;
        wrong_rint += rintf(q1) != rintf(want);
      }
    }
  }
  printf("cases %lld wrong %lld wrong_rint %lld\n", cases, wrong, wrong_rint);
  return wrong != 0 || wrong_rint != 0;
}
