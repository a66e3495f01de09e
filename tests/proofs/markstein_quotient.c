/*
 * Exhaustive check of the quotient the rotate-quantize kernel uses (test infrastructure, CPU only).
 *
 * The kernel quantizes q = rint(RN(a / d)) where a is a bf16-precision value (at most 8 significant bits) and
 * d = sx * 2^n is any positive normal fp32. It computes RN(a / d) as
 *     inv = RN(1 / d)            (once per row, correctly rounded division)
 *     q0  = RN(a * inv)
 *     r   = fma(-q0, d, a)        (exact remainder)
 *     q1  = fma(r, inv, q0)
 * and this program checks q1 == RN(a / d) (bitwise) and rint(q1) == rint(a / d) for every fp32 significand of d in
 * [1, 2) and every 8-bit significand of a with |a / d| in [2^-6, 128] (both signs). Scaling a and d by the same or by
 * different powers of two scales every step exactly (no overflow or underflow in the kernel's range), so this covers
 * all normal inputs; for |a / d| < 2^-6 both sides round to zero, since |q1| stays within a few ulps of |a / d|.
 *
 * Build and run (all 2^23 divisor significands, ~27e9 quotients, ~30 s on 8 cores; result: 0 differ):
 *   gcc -O2 -mfma -ffp-contract=off -fopenmp markstein_quotient.c -o markstein -lm && ./markstein
 * `./markstein S` checks every S-th divisor significand only (the CPU test suite runs S = 64).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

int main(int argc, char** argv) {
  const uint32_t stride = argc > 1 ? (uint32_t)atoi(argv[1]) : 1u;
  long long bad_q = 0, bad_rint = 0, checked = 0;
#pragma omp parallel for reduction(+ : bad_q, bad_rint, checked) schedule(static, 4096)
  for (uint32_t dm = 0; dm < (1u << 23); dm += stride) {
    const float d = from_bits(0x3f800000u | dm); /* [1, 2) */
    const float inv = 1.0f / d;
    for (int e = -12; e <= 0; ++e) {
      for (uint32_t am = 128; am < 256; ++am) {
        for (int sgn = 0; sgn < 2; ++sgn) {
          float a = ldexpf((float)am, e);
          if (sgn) a = -a;
          const float exact = a / d;
          if (fabsf(exact) > 128.0f) continue;
          const float q0 = a * inv;
          const float r = fmaf(-q0, d, a);
          const float q1 = fmaf(r, inv, q0);
          checked++;
          if (bits_of(q1) != bits_of(exact)) bad_q++;
          if (rintf(q1) != rintf(exact)) bad_rint++;
        }
      }
    }
  }
  printf("checked %lld quotients: %lld differ from RN(a/d), %lld round to a different integer\n", checked, bad_q,
         bad_rint);
  return (bad_q || bad_rint) ? 1 : 0;
}
