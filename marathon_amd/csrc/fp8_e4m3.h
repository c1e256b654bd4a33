// fp8 e4m3fn (OCP) codec for gfx950 device code: decode, requantise, encode.
//
// Shared by the shift kernel and the test library that checks it value by value.
// gfx950's v_cvt_pk_f32_fp8 decodes every code exactly; v_cvt_pk_fp8_f32 rounds to
// nearest even, and its NaN code is 0xFF where the format's canonical NaN is 0x7F, so
// callers rewrite NaN lanes to 0x7F.
//
// quant(): RN(y / s) for the layer's K scale s, with no division per element.  Once per
// layer (divisor()): r = RN(1/s) by an IEEE division; rz = 1/s rounded toward zero (r,
// or r's predecessor when 1 - r*s < 0); t = 1 - rz*s, exact in one fma (0 <= t < 2^-23
// and a multiple of ulp(rz) * ulp(s)); rlo = RN(t * rz).  Since 1/s = rz / (1 - t),
// rz + rlo is within 2^-45 of 1/s, relatively.  Per element, four VALU operations:
//   q0 = RN(y*rz + RN(y*rlo))   within 1/2 ulp + 2^-21 ulp of y/s, so within one ulp;
//   e  = RN(q0*s - y)            exact, q0 being within one ulp;
//   q  = RN(q0 - e*r)            = RN(y/s) by Markstein's theorem (r within half an ulp
//                                of 1/s and q0 within one ulp of y/s: P. Markstein, IBM
//                                J. Res. Dev. 34(1), 1990).
// The compiler's correctly rounded division takes about ten operations (measured 8%
// slower on the fp8 Qwen3-14B shift); one correction from q0 = RN(y*r) takes three, but
// that q0 can be 1.5 ulps off, outside the theorem (MKV_FP8_SPLIT_RCP=0 builds it).
// Conditions: 2^-90 <= s <= 2^100, so that nothing underflows or overflows for any
// quotient that can change an e4m3fn code (2^-12 <= |y/s| < 2^10): smaller quotients
// encode to a signed zero either way, larger ones clamp.  Signed zeros: rlo >= 0, so for
// y = +-0 both products in q0 are zeros of y's sign and q0 = y; then e = +0 and
// q = -0*r + q0 = q0.  Checked on the CPU besides (tests/fp8_division_check.c, the same
// operations): every fp32 y with 2^-12 <= |y/s| < 2^10 at every K scale of the fp8
// workloads and GPU tests, and 3e8 random (s, y) pairs over 41 binades of s.  The result
// is clamped to +-448 by one median-of-three; what it gives for a NaN does not matter,
// since callers that can see NaN inputs rewrite those bytes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mkv_fp8 {

typedef float f2 __attribute__((ext_vector_type(2)));

// Whether any byte of w is a NaN code (S.1111.111).
__device__ __forceinline__ bool has_nan_code(uint32_t w) {
  return (((w & 0x7F7F7F7Fu) + 0x01010101u) & 0x80808080u) != 0;
}

// The four codes of w, low byte first, as exact floats.
__device__ __forceinline__ void decode4(uint32_t w, float* out) {
  const f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
  const f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
  out[0] = lo[0];
  out[1] = lo[1];
  out[2] = hi[0];
  out[3] = hi[1];
}

// q clamped to +-448 (one v_med3_f32; a NaN q gives some value, which callers rewrite).
__device__ __forceinline__ float clamp448(float q) {
  return __builtin_amdgcn_fmed3f(q, -448.0f, 448.0f);
}

#ifndef MKV_FP8_SPLIT_RCP
#define MKV_FP8_SPLIT_RCP 1
#endif

// A layer's K scale and the reciprocals quant() divides with, made once per layer.
struct Divisor {
  float s;    // the K scale (positive, normal)
  float r;    // RN(1 / s)
  float rz;   // 1 / s rounded toward zero: r, or r's predecessor when r > 1 / s
  float rlo;  // RN((1 - rz * s) * rz) >= 0: rz + rlo = 1 / s within 2^-45 relative
};

// A wave-uniform float into a scalar register: the VALU operations take it as their one
// scalar operand, so it holds no vector register.
__device__ __forceinline__ float to_sgpr(float x) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}

// s must be wave-uniform.
__device__ __forceinline__ Divisor divisor(float s) {
  Divisor d;
  d.s = s;
  const float r = 1.0f / s;  // IEEE division: correctly rounded
  const float rz = __builtin_fmaf(-r, s, 1.0f) < 0.0f ? __uint_as_float(__float_as_uint(r) - 1u) : r;
  d.r = to_sgpr(r);
  d.rz = to_sgpr(rz);
  d.rlo = to_sgpr(__builtin_fmaf(-rz, s, 1.0f) * rz);
  return d;
}

// The divisor of scale 1 (no dequantisation), without a division.
__device__ __forceinline__ Divisor unit_divisor() { return Divisor{1.0f, 1.0f, 1.0f, 0.0f}; }

// clamp(RN(y / d.s)) for finite y.
__device__ __forceinline__ float quant(float y, const Divisor& d) {
#if MKV_FP8_SPLIT_RCP
  const float q0 = __builtin_fmaf(y, d.rz, y * d.rlo);
#else
  const float q0 = y * d.r;
#endif
  const float e = __builtin_fmaf(q0, d.s, -y);
  return clamp448(__builtin_fmaf(-e, d.r, q0));
}

// Four in-range floats to four codes (round to nearest even), low byte first.
__device__ __forceinline__ uint32_t encode4(const float* q) {
  int v = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
  v = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], v, true);
  return static_cast<uint32_t>(v);
}

// Byte b of w set to the canonical NaN code.
__device__ __forceinline__ uint32_t with_nan(uint32_t w, int b) {
  return (w & ~(0xFFu << (8 * b))) | (0x7Fu << (8 * b));
}

}  // namespace mkv_fp8
