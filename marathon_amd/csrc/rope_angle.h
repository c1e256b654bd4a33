// rope_angle.h -- cos and sin of a rotation angle, one routine for the host and the device.
//
// A span's rotation tables hold, for frequency f, the cosine and sine of the fp32 angle
// fl32(delta * inv_freq[f]) (shift_kernels.py:73), each evaluated in double precision
// and rounded once to fp32.  The plan pass and the small path compute them on the
// device; the host computes them for the direct path and for rope_shift.  All of them
// call this function, built from IEEE double operations only (multiply, add, fused
// multiply-add, round to integer), with contraction off, so the host and the device
// produce the same bits by construction.
//
// Method.  The angle x is an fp32 value, so |x| < 2^31.  Reduction by pi/2 (Cody and
// Waite's method, with fused multiply-adds): k = rint(x * 2/pi); pi/2 is split into
// three doubles P1 + P2 + P3 (P1 = RN(pi/2), P2 = RN(pi/2 - P1), P3 = RN(pi/2 - P1 - P2),
// from a 200-digit expansion of pi; the rest is below 6e-50).  t = x - k*P1 is exact in
// one fma (it is a multiple of 2^-52 below 1 in magnitude); r = t - k*P2 - k*P3 is carried
// as hi + lo through an exact product error and Knuth's two-sum, so r is known to far
// better than double precision even where x lies close to a multiple of pi/2.  Then
// Taylor series of sin and cos on |r| <= pi/4 + tiny (odd terms to r^21, even terms to
// r^20; the first omitted term is below 2^-70 relative), evaluated by Horner's rule with
// fmas, the r^1 and r^0 terms added last, and lo folded in to first order:
//   sin(hi + lo) = hi + (hi * r2 * S(r2) + lo * (1 - r2/2))
//   cos(hi + lo) = 1 + (r2 * C(r2) - hi * lo)
// with the quadrant k mod 4 selecting and signing the two.  The coefficients are 1/n!
// rounded to double.  The double results are within about one double ulp of the exact
// values, so their fp32 roundings are the correctly rounded fp32 values except where an
// exact value lies within about 2^-28 of an fp32 rounding boundary, relatively; the tests
// compare them with float64 numpy over every delta in [-131072, 131072] and far beyond.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define MKV_HOST_DEVICE __host__ __device__
#else
#define MKV_HOST_DEVICE
#endif

namespace mkv_rope {

MKV_HOST_DEVICE inline void angle_cos_sin(int32_t delta, float inv_freq, float& c, float& s) {
  constexpr double kP1 = 0x1.921fb54442d18p+0;
  constexpr double kP2 = 0x1.1a62633145c07p-54;
  constexpr double kP3 = -0x1.f1976b7ed8fbcp-110;
  constexpr double kTwoOverPi = 0x1.45f306dc9c883p-1;
  // (-1)^k / (2k+1)!, k = 1..10, and (-1)^k / (2k)!, k = 1..10, rounded to double
  constexpr double kS[10] = {-0x1.5555555555555p-3, 0x1.1111111111111p-7,
                             -0x1.a01a01a01a01ap-13, 0x1.71de3a556c734p-19,
                             -0x1.ae64567f544e4p-26, 0x1.6124613a86d09p-33,
                             -0x1.ae7f3e733b81fp-41, 0x1.952c77030ad4ap-49,
                             -0x1.2f49b46814157p-57, 0x1.71b8ef6dcf572p-66};
  constexpr double kC[10] = {-0x1.0000000000000p-1, 0x1.5555555555555p-5,
                             -0x1.6c16c16c16c17p-10, 0x1.a01a01a01a01ap-16,
                             -0x1.27e4fb7789f5cp-22, 0x1.1eed8eff8d898p-29,
                             -0x1.93974a8c07c9dp-37, 0x1.ae7f3e733b81fp-45,
                             -0x1.6827863b97d97p-53, 0x1.e542ba4020225p-62};
  const float ang = static_cast<float>(delta) * inv_freq;  // fp32, rounded once
  const double x = static_cast<double>(ang);
  const double k = __builtin_rint(x * kTwoOverPi);
  const double t = __builtin_fma(-k, kP1, x);  // exact
  const double p = k * kP2;
  const double pe = __builtin_fma(k, kP2, -p);  // p + pe == k * P2 exactly
  const double hi = t - p;                      // two-sum: hi + err == t - p exactly
  const double bb = hi - t;
  const double err = (t - (hi - bb)) + (-p - bb);
  const double lo = err - pe - k * kP3;
  const double r2 = hi * hi;
  double ps = kS[9];
  double pc = kC[9];
  for (int i = 8; i >= 0; --i) {
    ps = __builtin_fma(ps, r2, kS[i]);
    pc = __builtin_fma(pc, r2, kC[i]);
  }
  const double sin_r = hi + __builtin_fma(hi, ps * r2, lo * (1.0 - 0.5 * r2));
  const double cos_r = 1.0 + (pc * r2 - hi * lo);
  double sv, cv;
  switch (static_cast<int>(static_cast<int64_t>(k) & 3)) {
    case 0: sv = sin_r; cv = cos_r; break;
    case 1: sv = cos_r; cv = -sin_r; break;
    case 2: sv = -sin_r; cv = -cos_r; break;
    default: sv = -cos_r; cv = sin_r; break;
  }
  c = static_cast<float>(cv);
  s = static_cast<float>(sv);
}

}  // namespace mkv_rope
