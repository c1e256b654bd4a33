// Test library (not product code): runs the shift kernel's fp8 e4m3fn codec
// (marathon_amd/csrc/fp8_e4m3.h) on arbitrary values, so the GPU tests can check the
// hardware conversions value by value against the oracle -- every midpoint, near
// midpoint, clamp and special value, which real shifts reach only by chance.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fp8_e4m3.h"

namespace {

// out[i] = code of y[i]: clamp(y) (quantize == 0) or clamp(RN(y / scale)) (quantize
// != 0), NaN -> 0x7F, exactly as the shift kernel encodes.  n is a multiple of 4.
__global__ void encode_kernel(const float* y, float scale, int quantize, uint32_t* out,
                              int64_t n4) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  const mkv_fp8::Divisor dv = mkv_fp8::divisor(scale);
  float q[4];
  for (int b = 0; b < 4; ++b) {
    const float v = y[4 * i + b];
    q[b] = quantize ? mkv_fp8::quant(v, dv) : mkv_fp8::clamp448(v);
  }
  uint32_t w = mkv_fp8::encode4(q);
  for (int b = 0; b < 4; ++b) {
    const float v = y[4 * i + b];
    if (v != v) w = mkv_fp8::with_nan(w, b);
  }
  out[i] = w;
}

__global__ void decode_kernel(const uint32_t* codes, float* out, int64_t n4) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  mkv_fp8::decode4(codes[i], out + 4 * i);
}

}  // namespace

extern "C" int fp8_probe_encode(const float* y, float scale, int quantize, uint32_t* out,
                                int64_t n, void* stream) {
  if (n % 4 != 0 || n < 0) return 1;
  const int64_t n4 = n / 4;
  if (n4 == 0) return 0;
  hipLaunchKernelGGL(encode_kernel, dim3(static_cast<unsigned>((n4 + 255) / 256)), dim3(256),
                     0, static_cast<hipStream_t>(stream), y, scale, quantize, out, n4);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

extern "C" int fp8_probe_decode(const uint32_t* codes, float* out, int64_t n, void* stream) {
  if (n % 4 != 0 || n < 0) return 1;
  const int64_t n4 = n / 4;
  if (n4 == 0) return 0;
  hipLaunchKernelGGL(decode_kernel, dim3(static_cast<unsigned>((n4 + 255) / 256)), dim3(256),
                     0, static_cast<hipStream_t>(stream), codes, out, n4);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
