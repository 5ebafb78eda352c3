// CPU build of the device code's fp8 E4M3 and MX encoders (velograd_amd/csrc/fp8_e4m3.h,
// mx_formats.h) as a small shared library, loaded by tests/test_fp8_codec.py and
// tests/test_mx_codec.py and compared with the oracle's independent nearest-value encoders.
#include <stdint.h>

#include "fp8_e4m3.h"

extern "C" void vg_e4m3_encode_n(const float* in, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)vg_fp8::e4m3_encode(in[i]);
}

extern "C" void vg_e4m3_quantize_n(const float* in, float scale, uint8_t* out, int64_t n) {
  const float inv = vg_fp8::inverse_scale(scale);
  for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)vg_fp8::quantize_e4m3(in[i], inv);
}

// MX helpers (velograd_amd/csrc/mx_formats.h).
#include "mx_formats.h"

extern "C" void vg_e2m1_encode_n(const float* in, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)vg_mx::e2m1_encode(in[i]);
}

extern "C" void vg_mx_scale_n(const float* amax, int32_t emax, uint8_t* code, float* factor,
                              int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const uint32_t bits = __builtin_bit_cast(uint32_t, amax[i]) & 0x7fffffffu;
    code[i] = (uint8_t)vg_mx::scale_code(bits, emax);
    factor[i] = bits < 0x7f800000u ? vg_mx::inverse_scale(vg_mx::shared_exp(bits, emax)) : 0.0f;
  }
}
