// Shared by the library's translation units: element codecs, 16-byte global accesses, wave64
// reductions, and the host-side error state and device facts.  Everything lives in namespace
// `vg`; the error text is one thread-local buffer for the whole library (an inline variable).
#ifndef VELOGRAD_COMMON_H
#define VELOGRAD_COMMON_H

#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <atomic>

#include "velograd_kernels.h"

#ifndef VG_HOST_DEVICE
#define VG_HOST_DEVICE __host__ __device__
#endif
#include "launch_plan.h"

namespace vg {

using vg_plan::kWave;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------------------------------
// Element codecs: 16 bytes <-> fp32 registers.
// ------------------------------------------------------------------------------------------
template <int DT>
struct Codec;

template <>
struct Codec<VELOGRAD_DTYPE_F32> {
  static constexpr int kBytes = 4;
  static constexpr int kVec = 4;
  __device__ static inline void unpack(const u32x4 v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // Copy the element out first: hipcc 7.2 bit-casts an ext_vector element lvalue
      // (`__builtin_bit_cast(float, v[i])`) as element 0 whatever i is.
      const uint32_t u = v[i];
      f[i] = __builtin_bit_cast(float, u);
    }
  }
  __device__ static inline u32x4 pack(const float* f) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __builtin_bit_cast(uint32_t, f[i]);
    return v;
  }
  __device__ static inline float load1(const void* p, int64_t i) {
    return static_cast<const float*>(p)[i];
  }
  __device__ static inline void store1(void* p, int64_t i, float f) {
    static_cast<float*>(p)[i] = f;
  }
};

template <>
struct Codec<VELOGRAD_DTYPE_BF16> {
  static constexpr int kBytes = 2;
  static constexpr int kVec = 8;
  __device__ static inline void unpack(const u32x4 v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __builtin_bit_cast(float, v[i] << 16);
      f[2 * i + 1] = __builtin_bit_cast(float, v[i] & 0xffff0000u);
    }
  }
  __device__ static inline u32x4 pack(const float* f) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bf16x2 p = {(__bf16)f[2 * i], (__bf16)f[2 * i + 1]};  // v_cvt_pk_bf16_f32, RNE
      v[i] = __builtin_bit_cast(uint32_t, p);
    }
    return v;
  }
  __device__ static inline float load1(const void* p, int64_t i) {
    const uint32_t u = static_cast<const uint16_t*>(p)[i];
    return __builtin_bit_cast(float, u << 16);
  }
  __device__ static inline void store1(void* p, int64_t i, float f) {
    static_cast<__bf16*>(p)[i] = (__bf16)f;
  }
};

template <>
struct Codec<VELOGRAD_DTYPE_F16> {
  static constexpr int kBytes = 2;
  static constexpr int kVec = 8;
  __device__ static inline void unpack(const u32x4 v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t u = v[i];  // scalar copy: see the fp32 codec
      const f16x2 h = __builtin_bit_cast(f16x2, u);
      f[2 * i] = (float)h[0];
      f[2 * i + 1] = (float)h[1];
    }
  }
  __device__ static inline u32x4 pack(const float* f) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f16x2 p = {(_Float16)f[2 * i], (_Float16)f[2 * i + 1]};
      v[i] = __builtin_bit_cast(uint32_t, p);
    }
    return v;
  }
  __device__ static inline float load1(const void* p, int64_t i) {
    return (float)static_cast<const _Float16*>(p)[i];
  }
  __device__ static inline void store1(void* p, int64_t i, float f) {
    static_cast<_Float16*>(p)[i] = (_Float16)f;
  }
};

template <int DT>
__device__ inline u32x4 load16(const void* base, int64_t elem) {
  return *reinterpret_cast<const u32x4*>(static_cast<const char*>(base) +
                                         elem * Codec<DT>::kBytes);
}

template <int DT>
__device__ inline void store16(void* base, int64_t elem, const u32x4 v) {
  *reinterpret_cast<u32x4*>(static_cast<char*>(base) + elem * Codec<DT>::kBytes) = v;
}

// Streamed activations are touched once per launch: non-temporal loads and stores keep them from
// displacing reusable lines (weight, partial sums) in L2 and the MALL.  A stream-pattern probe
// with the fwd (2 reads + 2 writes) and bwd (2 reads + 1 write) shapes measured +8..12% from the
// non-temporal forms on MI355X.  Build with -DVG_STREAM_NT=0 to compare, or set the loads' and
// the stores' policy alone with VG_STREAM_NT_LOAD / VG_STREAM_NT_STORE.
#ifndef VG_STREAM_NT
#define VG_STREAM_NT 1
#endif
#ifndef VG_STREAM_NT_LOAD
#define VG_STREAM_NT_LOAD VG_STREAM_NT
#endif
#ifndef VG_STREAM_NT_STORE
#define VG_STREAM_NT_STORE VG_STREAM_NT
#endif

template <int DT>
__device__ inline u32x4 load16_stream(const void* base, int64_t elem) {
  const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const char*>(base) +
                                                  elem * Codec<DT>::kBytes);
#if VG_STREAM_NT_LOAD
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}

template <int DT>
__device__ inline void store16_stream(void* base, int64_t elem, const u32x4 v) {
  u32x4* p = reinterpret_cast<u32x4*>(static_cast<char*>(base) + elem * Codec<DT>::kBytes);
#if VG_STREAM_NT_STORE
  __builtin_nontemporal_store(v, p);
#else
  *p = v;
#endif
}

// Half a chunk (8 bytes) of a stream whose rows start on 8-byte boundaries only, with the same
// cache policy as the 16-byte forms.
template <int DT>
__device__ inline u32x2 load8_stream(const void* base, int64_t elem) {
  const u32x2* p = reinterpret_cast<const u32x2*>(static_cast<const char*>(base) +
                                                  elem * Codec<DT>::kBytes);
#if VG_STREAM_NT_LOAD
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}

template <int DT>
__device__ inline void store8_stream(void* base, int64_t elem, const u32x2 v) {
  u32x2* p = reinterpret_cast<u32x2*>(static_cast<char*>(base) + elem * Codec<DT>::kBytes);
#if VG_STREAM_NT_STORE
  __builtin_nontemporal_store(v, p);
#else
  *p = v;
#endif
}

// ------------------------------------------------------------------------------------------
// Reductions.
// ------------------------------------------------------------------------------------------
template <int CTRL>
__device__ inline float dpp_move(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// cos and sin of |x| <= 1 by their Taylor series through x^12 and x^11 (truncation below 2e-10,
// then float32 rounding of the Horner steps).
__device__ inline void cos_sin_small(float x, float& c, float& s) {
  const float z = x * x;
  float ps = -1.0f / 39916800.0f;
  ps = fmaf(ps, z, 1.0f / 362880.0f);
  ps = fmaf(ps, z, -1.0f / 5040.0f);
  ps = fmaf(ps, z, 1.0f / 120.0f);
  ps = fmaf(ps, z, -1.0f / 6.0f);
  s = fmaf(x * z, ps, x);
  float pc = 1.0f / 479001600.0f;
  pc = fmaf(pc, z, -1.0f / 3628800.0f);
  pc = fmaf(pc, z, 1.0f / 40320.0f);
  pc = fmaf(pc, z, -1.0f / 720.0f);
  pc = fmaf(pc, z, 1.0f / 24.0f);
  pc = fmaf(pc, z, -0.5f);
  c = fmaf(z, pc, 1.0f);
}

// Empty register barrier: the compiler must assume `v` changed here, so values it decoded from
// `v` before this point are decoded again afterwards instead of being held in extra VGPRs
// across the row reduction.  Emits no instruction.
__device__ inline void forget(u32x4& v) { asm volatile("" : "+v"(v)); }

// Sum over the 64 lanes of a wave; the result is wave-uniform.  Requires all lanes active.
__device__ inline float wave_sum(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_move<0x124>(v);  // row_ror:4
  v += dpp_move<0x128>(v);  // row_ror:8  -> each lane holds its 16-lane row's sum
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}

// Sum over the `tpr` threads of row group `grp` (threads grp*tpr .. grp*tpr+tpr-1, whole waves).
// `red` holds one float per wave of the block; the caller alternates buffers between calls
// that reuse it so one barrier per call suffices.
__device__ inline float row_sum(float v, int tpr, int grp, float* red) {
  v = wave_sum(v);
  if (tpr > kWave) {
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
    __syncthreads();
    const int wpr = tpr / kWave;
    const float* p = red + grp * wpr;
    float t = p[0];
    for (int i = 1; i < wpr; ++i) t += p[i];
    v = t;
  }
  return v;
}

// ------------------------------------------------------------------------------------------
// Host side: errors, device facts.
// ------------------------------------------------------------------------------------------
inline thread_local char g_last_error[512] = "";

inline int32_t fail(int32_t code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
inline int32_t fail(int32_t code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

inline void clear_error() { g_last_error[0] = '\0'; }

inline int32_t check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail((int32_t)e, "%s: launch failed: %s", what, hipGetErrorString(e));
  clear_error();
  return 0;
}

constexpr int kMaxDevices = 64;
inline std::atomic<int> g_cu_count[kMaxDevices];

inline int cu_count(int device) {
  if (device < 0 || device >= kMaxDevices) return 0;
  int v = g_cu_count[device].load(std::memory_order_relaxed);
  if (v > 0) return v;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      v <= 0)
    return 0;
  g_cu_count[device].store(v, std::memory_order_relaxed);
  return v;
}

inline int env_int(const char* name, int dflt, int lo, int hi) {
  const char* s = getenv(name);
  if (s == nullptr || *s == '\0') return dflt;
  const long v = strtol(s, nullptr, 10);
  if (v < lo || v > hi) return dflt;
  return (int)v;
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

inline int elem_bytes_of(int32_t dt) {
  switch (dt) {
    case VELOGRAD_DTYPE_F32: return 4;
    case VELOGRAD_DTYPE_F16: return 2;
    case VELOGRAD_DTYPE_BF16: return 2;
    default: return 0;
  }
}

}  // namespace vg

#endif  // VELOGRAD_COMMON_H
