// CPU build of the device code's fp8 E4M3 encoder (velograd_amd/csrc/fp8_e4m3.h) as a small
// shared library, loaded by tests/test_fp8_codec.py and compared with the oracle's independent
// nearest-value encoder.
#include <stdint.h>

#include "fp8_e4m3.h"

extern "C" void vg_e4m3_encode_n(const float* in, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)vg_fp8::e4m3_encode(in[i]);
}

extern "C" void vg_e4m3_quantize_n(const float* in, float scale, uint8_t* out, int64_t n) {
  const float inv = vg_fp8::inverse_scale(scale);
  for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)vg_fp8::quantize_e4m3(in[i], inv);
}
