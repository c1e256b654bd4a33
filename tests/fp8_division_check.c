/* Exhaustive check of the fp8 requantisation's division (CPU, test infrastructure).
 *
 * The shift kernel divides by the layer's K scale s (marathon_amd/csrc/fp8_e4m3.h) as
 *   r = RN(1/s), rz = 1/s rounded toward zero, rlo = RN(fma(-rz, s, 1) * rz)   (per layer)
 *   q0 = fma(y, rz, RN(y*rlo)), e = fma(q0, s, -y), q = fma(-e, r, q0)        (per element)
 * and needs q == RN(y/s): q0 is within one ulp of y/s, so Markstein's theorem makes q
 * correctly rounded.  This program checks that with the same operations: for each scale
 * given (as the hex bit pattern of the fp32 value) it walks every fp32 y with
 * 2^-12 <= |y/s| < 2^10, both signs, and counts the y where q differs from the
 * correctly rounded quotient.  Below 2^-12 every quotient encodes to a signed zero in
 * e4m3fn either way (the smallest nonzero code is 2^-9); at and above 2^10 every
 * quotient clamps to 448.  "random N" instead draws N (scale, y) pairs with scales over
 * 41 binades.  A leading "plain" argument checks q0 = RN(y*r) alone instead, a quotient
 * that is often one ulp off: the walk must find those.  Exit status 0 means no mismatch.
 * Build with contraction off:
 *   gcc -O2 -ffp-contract=off fp8_division_check.c -lm -lpthread
 */
#include <math.h>
#include <pthread.h>
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

typedef struct {
  float s, r, rz, rlo;
} Divisor;

static Divisor divisor(float s) {
  Divisor d;
  d.s = s;
  d.r = 1.0f / s;
  d.rz = fmaf(-d.r, s, 1.0f) < 0.0f ? from_bits(to_bits(d.r) - 1u) : d.r;
  d.rlo = fmaf(-d.rz, s, 1.0f) * d.rz;
  return d;
}

static int plain = 0;

static float quotient(float y, const Divisor* d) {
  if (plain) return y * d->r;
  const float q0 = fmaf(y, d->rz, y * d->rlo);
  return fmaf(-fmaf(q0, d->s, -y), d->r, q0);
}

static int quotient_ok(float y, const Divisor* d) {
  return to_bits(quotient(y, d)) == to_bits(y / d->s);
}

typedef struct {
  float s;
  uint32_t lo, hi;
  long long bad, total;
} Job;

static void* walk(void* arg) {
  Job* j = (Job*)arg;
  const Divisor d = divisor(j->s);
  for (uint32_t u = j->lo; u < j->hi; ++u) {
    if (!quotient_ok(from_bits(u), &d)) ++j->bad;
    if (!quotient_ok(from_bits(u | 0x80000000u), &d)) ++j->bad;
    j->total += 2;
  }
  return NULL;
}

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64(void) {
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 7;
  rng_state ^= rng_state << 17;
  return rng_state;
}

int main(int argc, char** argv) {
  long long total = 0, mismatches = 0;
  if (argc > 1 && strcmp(argv[1], "plain") == 0) {
    plain = 1;
    --argc;
    ++argv;
  }
  if (argc == 3 && strcmp(argv[1], "random") == 0) {
    const long long n = atoll(argv[2]);
    for (long long i = 0; i < n; ++i) {
      const uint64_t x = next_u64();
      const float s = from_bits((uint32_t)(x & 0x7FFFFF) | ((uint32_t)(107 + (x >> 23) % 41) << 23));
      const float q = from_bits((uint32_t)((x >> 32) & 0x7FFFFF) |
                                ((uint32_t)(115 + (x >> 55) % 22) << 23));
      const float y = q * s;
      if (!isfinite(y) || y == 0.0f) continue;
      const Divisor d = divisor(s);
      if (!quotient_ok(y, &d)) ++mismatches;
      ++total;
    }
    printf("checked %lld random quotients, %lld mismatches\n", total, mismatches);
    return mismatches != 0;
  }
  enum { kThreads = 8 };
  for (int i = 1; i < argc; ++i) {
    const float s = from_bits((uint32_t)strtoul(argv[i], NULL, 16));
    const uint32_t first = to_bits(ldexpf(s, -12));
    const uint32_t last = to_bits(ldexpf(s, 10));
    Job jobs[kThreads];
    pthread_t th[kThreads];
    const uint32_t step = (last - first + kThreads - 1) / kThreads;
    for (int t = 0; t < kThreads; ++t) {
      jobs[t].s = s;
      jobs[t].lo = first + step * (uint32_t)t < last ? first + step * (uint32_t)t : last;
      jobs[t].hi = jobs[t].lo + step < last ? jobs[t].lo + step : last;
      jobs[t].bad = jobs[t].total = 0;
      pthread_create(&th[t], NULL, walk, &jobs[t]);
    }
    long long bad = 0;
    for (int t = 0; t < kThreads; ++t) {
      pthread_join(th[t], NULL);
      bad += jobs[t].bad;
      total += jobs[t].total;
    }
    /* a zero quotient keeps the sign of y (-0 / s = -0) */
    const Divisor d = divisor(s);
    bad += to_bits(quotient(0.0f, &d)) != 0u;
    bad += to_bits(quotient(-0.0f, &d)) != 0x80000000u;
    total += 2;
    printf("scale %a: %lld mismatches\n", s, bad);
    mismatches += bad;
  }
  printf("checked %lld quotients, %lld mismatches\n", total, mismatches);
  return mismatches != 0;
}
