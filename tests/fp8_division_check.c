/* Exhaustive check of the fp8 requantisation's division (CPU, test infrastructure).
 *
 * The shift kernel divides by the layer's K scale s with Markstein's correction:
 *   r = RN(1/s), q0 = RN(y*r), e = fma(-q0, s, y), q = fma(e, r, q0)
 * and needs q == RN(y/s).  For each scale given on the command line this walks every
 * fp32 y with 2^-12 <= |y/s| < 2^10, both signs, and counts the y where q differs from
 * the correctly rounded quotient.  Below 2^-12 every quotient encodes to a signed zero
 * in e4m3fn either way; above 2^10 no rotated fp8 value can reach.
 * Exit status 0 means no mismatch.  Build with contraction off:
 *   gcc -O2 -ffp-contract=off fp8_division_check.c -lm
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

static uint32_t to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  return u;
}

int main(int argc, char** argv) {
  long long total = 0, mismatches = 0;
  for (int i = 1; i < argc; ++i) {
    const float s = strtof(argv[i], NULL);
    const float r = 1.0f / s;
    const uint32_t first = to_bits(ldexpf(s, -12));
    const uint32_t last = to_bits(ldexpf(s, 10));
    long long bad = 0;
    static const uint32_t signs[2] = {0u, 0x80000000u};
    for (uint32_t u = first; u < last; ++u) {
      for (int k = 0; k < 2; ++k) {
        const float y = from_bits(u | signs[k]);
        const float q0 = y * r;
        const float q = fmaf(fmaf(-q0, s, y), r, q0);
        if (to_bits(q) != to_bits(y / s)) {
          if (bad < 3) printf("scale %a: y %a gives %a, want %a\n", s, y, q, y / s);
          ++bad;
        }
        ++total;
      }
    }
    printf("scale %.9g: %lld mismatches\n", s, bad);
    mismatches += bad;
  }
  printf("checked %lld quotients, %lld mismatches\n", total, mismatches);
  return mismatches != 0;
}
