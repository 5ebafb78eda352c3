// OCP Microscaling (MX) block formats shared by the device kernels and a CPU check
// (tests/fp8_check.cpp, built by tests/test_mx_codec.py): blocks of 32 consecutive elements
// share one E8M0 scale X = 2^s; the elements are fp8 E4M3 (MXFP8) or fp4 E2M1 (MXFP4) codes
// of v / X.  The reference enumerates both element formats (include/velograd/kernels.h:29-37)
// and decodes E2M1 through its table (kernels.h:47-51) with one scale per 32 elements and the
// even element in the low nibble (kernels.h:97-101, 339-347).
//
// Shared exponent (OCP MX v1.0): s = floor(log2(amax)) - emax_elem, emax_elem = 8 for E4M3
// (448 = 1.75 * 2^8) and 2 for E2M1 (6 = 1.5 * 2^2), clamped to E8M0's [-127, 127]; the scale
// code is s + 127.  An all-zero block takes code 0; a block whose amax is not finite takes the
// NaN code 0xFF and zero element codes.  Elements: round to nearest even, saturating.
#ifndef VELOGRAD_MX_FORMATS_H
#define VELOGRAD_MX_FORMATS_H

#include <stdint.h>

#ifndef VG_HOST_DEVICE
#define VG_HOST_DEVICE
#endif

namespace vg_mx {

constexpr int kBlock = 32;
constexpr int kEmaxE4M3 = 8;
constexpr int kEmaxE2M1 = 2;
constexpr uint32_t kScaleNaN = 0xffu;

// floor(log2(a)) for the bit pattern of a finite a > 0 (normal or subnormal), exactly.
VG_HOST_DEVICE inline int floor_log2_bits(uint32_t abits) {
  const int e = (int)(abits >> 23);
  if (e != 0) return e - 127;
  // subnormal: a = m * 2^-149 with 1 <= m < 2^23
  return (31 - __builtin_clz(abits)) - 149;
}

// Shared exponent s of a block from the bit pattern of its amax (sign cleared); the block's
// E8M0 scale code is s + 127 when amax is finite.
VG_HOST_DEVICE inline int shared_exp(uint32_t amax_bits, int emax) {
  if (amax_bits == 0) return -127;
  int s = floor_log2_bits(amax_bits) - emax;
  if (s < -127) s = -127;
  if (s > 127) s = 127;
  return s;
}

// E8M0 scale code of a block: 0xFF for a non-finite amax.
VG_HOST_DEVICE inline uint32_t scale_code(uint32_t amax_bits, int emax) {
  if (amax_bits >= 0x7f800000u) return kScaleNaN;
  return (uint32_t)(shared_exp(amax_bits, emax) + 127);
}

// 2^-s, the exact factor that maps a block onto its element range (2^127 .. 2^-127).
VG_HOST_DEVICE inline float inverse_scale(int s) {
  const int e = 127 - s;  // biased exponent of 2^-s
  if (e >= 1) return __builtin_bit_cast(float, (uint32_t)e << 23);
  return __builtin_bit_cast(float, 0x00400000u);  // e == 0: 2^-127, a subnormal
}

// fp32 -> E2M1 nibble (sign in bit 3), round to nearest even over {0, .5, 1, 1.5, 2, 3, 4, 6},
// saturating at 6.  Each comparison adds one step past a midpoint; at a midpoint the strict or
// non-strict comparison picks the even code.  NaN gives 0 (E2M1 has no NaN; blocks holding a
// NaN are marked by their scale).
VG_HOST_DEVICE inline uint32_t e2m1_encode(float v) {
  const uint32_t bits = __builtin_bit_cast(uint32_t, v);
  const float a = __builtin_bit_cast(float, bits & 0x7fffffffu);
  const uint32_t code = (uint32_t)(a > 0.25f) + (uint32_t)(a >= 0.75f) + (uint32_t)(a > 1.25f) +
                        (uint32_t)(a >= 1.75f) + (uint32_t)(a > 2.5f) + (uint32_t)(a >= 3.5f) +
                        (uint32_t)(a > 5.0f);
  return ((bits >> 28) & 0x8u) | code;
}

}  // namespace vg_mx

#endif  // VELOGRAD_MX_FORMATS_H
