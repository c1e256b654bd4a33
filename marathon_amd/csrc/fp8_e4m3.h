// fp8 e4m3fn (OCP) codec for gfx950 device code: decode, requantise, encode.
//
// Shared by the shift kernel and the test library that checks it value by value.
// gfx950's v_cvt_pk_f32_fp8 decodes every code exactly; v_cvt_pk_fp8_f32 rounds to
// nearest even, and its NaN code is 0xFF where the format's canonical NaN is 0x7F, so
// callers rewrite NaN lanes to 0x7F.
//
// quant(): y / scale through Markstein's correction, q0 = RN(y * r),
// e = RN(q0 * scale - y), q = RN(-e * r + q0) with r = RN(1 / scale): three VALU
// operations where the compiler's correctly rounded division takes about ten (measured
// 8% slower on the fp8 Qwen3-14B shift).  -e is the usual residual RN(y - q0 * scale)
// (rounding is symmetric), so q is Markstein's quotient, which his theorem makes the
// correctly rounded one whenever q0 is within one ulp of y / scale.  Checked
// exhaustively on the CPU: q equals RN(y / scale) for every fp32 y with
// 2^-12 <= |y / scale| < 2^10 (the quotients that can change an e4m3fn code) at every
// K scale of the fp8 workloads and GPU tests, and on 3e8 random pairs with scales over
// 41 binades; other scales are checked only by that random sample.  Smaller quotients
// encode to a signed zero either way, larger ones clamp.  Computing the residual with
// its sign flipped also keeps the sign of a zero quotient: y = -0 gives e = +0 and
// q = -0 + -0 = -0, y = +0 gives q = -0 + +0 = +0.  The result is clamped to +-448 by
// one median-of-three; what it gives for a NaN does not matter, since callers that can
// see NaN inputs rewrite those bytes.
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

// clamp(RN(y / scale)) for finite y; rcp must be RN(1 / scale).
__device__ __forceinline__ float quant(float y, float scale, float rcp) {
  const float q0 = y * rcp;
  const float e = __builtin_fmaf(q0, scale, -y);
  return clamp448(__builtin_fmaf(-e, rcp, q0));
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
