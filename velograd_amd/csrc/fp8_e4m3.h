// fp32 -> fp8 E4M3 ("e4m3fn", OCP) encoding shared by the device kernels and a CPU check
// (tests/fp8_check.cpp, built by tests/test_fp8_codec.py).
//
// Format: bias 7, no infinities, S.1111.111 is NaN, largest finite value 448 = 1.75 * 2^8,
// smallest normal 2^-6, subnormals m * 2^-9 — the E4M3 the reference decodes at
// include/velograd/kernels.h:58-73.
#ifndef VELOGRAD_FP8_E4M3_H
#define VELOGRAD_FP8_E4M3_H

#include <stdint.h>

#ifndef VG_HOST_DEVICE
#define VG_HOST_DEVICE
#endif

namespace vg_fp8 {

constexpr float kE4M3Max = 448.0f;

// Round to nearest even, saturating: |f| > 448 (infinities included) gives +-448; NaN gives the
// NaN code with f's sign.  Integer steps plus one exact power-of-two product, so the result does
// not depend on the hardware's conversion instructions; written without branches (both the
// normal and the subnormal candidate are formed, then selected).
VG_HOST_DEVICE inline uint32_t e4m3_encode(float f) {
  const uint32_t bits = __builtin_bit_cast(uint32_t, f);
  const uint32_t abits = bits & 0x7fffffffu;
  const uint32_t a = abits < 0x43e00000u ? abits : 0x43e00000u;  // saturate at 448 = 1.75 * 2^8
  // normal (a >= 2^-6): keep 3 mantissa bits, round half to even over the 20 dropped bits (a
  // carry out of the mantissa moves to the next binade), then rebias the exponent 127 -> 7
  const uint32_t lsb = (a >> 20) & 1u;
  const uint32_t normal = ((a + 0x7ffffu + lsb) >> 20) - (120u << 3);
  // subnormal (a < 2^-6): multiples of 2^-9; a * 512 is exact and rint rounds half to even; a
  // result of 8 is 2^-6, whose code is 0x08 as well
  const uint32_t sub = (uint32_t)__builtin_rintf(__builtin_bit_cast(float, a) * 512.0f);
  uint32_t code = a < 0x3c800000u ? sub : normal;
  code = abits > 0x7f800000u ? 0x7fu : code;  // NaN
  return ((bits >> 24) & 0x80u) | code;
}

// The multiplier that maps a row onto the e4m3 range: 1 / scale with scale = amax / 448, or 1
// where scale is zero or below the smallest normal float (where 1 / scale could overflow).  A
// NaN scale gives NaN, so a row holding a NaN encodes as NaN throughout.
VG_HOST_DEVICE inline float inverse_scale(float scale) {
  return scale < 1.17549435e-38f ? 1.0f : 1.0f / scale;
}

// Code of y in a row whose inverse_scale is `inv`.
VG_HOST_DEVICE inline uint32_t quantize_e4m3(float y, float inv) { return e4m3_encode(y * inv); }

}  // namespace vg_fp8

#endif  // VELOGRAD_FP8_E4M3_H
