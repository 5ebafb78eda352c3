// Fused RMSNorm + residual add, forward and backward, hand-written for gfx950 (CDNA4, wave64).
//
// Math (reference: python/velograd/kernels/fused.py:28-66):
//   forward   h = x + residual;  inv_rms = 1 / sqrt(mean(h^2) + eps);  y = (h * inv_rms) * w
//             (the residual-free module form, python/velograd/nn.py:338-355, first floors
//             mean(h^2) at a minimum: see floor_mean_sq)
//   backward  gw = g * w;  m = mean(gw * xhat);  dx = inv_rms * (gw - xhat * m)
//             dweight = sum over rows of g * xhat,  with xhat = h * inv_rms
// Every operation is fp32 and rounds where the NumPy reference rounds (this file is built with
// -ffp-contract=off so no multiply-add pair is fused behind the code's back); stores round to
// nearest even.  Only the order of the row sums differs from NumPy's pairwise summation.  The
// exceptions are the norm + RoPE kernels, whose walks are bound by their vector instructions:
// they fuse multiply-adds explicitly (one rounding where the reference has two).
//
// Kernels
//   fwd_vec_kernel      one row per `tpr` threads (1..16 wave64), `groups` rows per workgroup;
//                       each thread holds NV 16-byte chunks of the row in registers, so every
//                       element moves through HBM exactly once (read x, residual; write h, y).
//   bwd_vec_kernel      persistent: each row slot walks rows slot, slot + S, ... with the next
//                       row's loads in flight while the current row reduces; the weight chunk and
//                       the fp32 dweight column accumulators stay in registers for the whole walk;
//                       each slot finally writes one fp32 partial row (no atomics).
//   bwd_ring_kernel     the same walk for rows of whole 16-byte chunks (some lanes may idle;
//                       2-byte rows of 8n + 4 elements in 8-byte halves) with a ring of three
//                       row buffers (two rows in flight while one reduces) in a branch-free
//                       steady loop, 512-thread workgroups, one per CU: the backward's default
//                       where the rows suit it.
//   fwd_rope_kernel     the forward with the model's interleaved RoPE on y: strided row walks
//                       with the rotation advanced by a recurrence.
//   bwd_rope_ring_kernel  its backward (grad_y rotated back, then the norm's backward) in
//                       bwd_ring_kernel's walk, one or two chunks per thread (rows of up to
//                       1024 chunks), one workgroup per CU (two of one chunk and under 512
//                       threads);
//                       bwd_vec_kernel with kRopeG where the rows or positions do not suit it.
//   dweight_reduce      stage 2: sums the partial rows in a fixed order -> dweight[dim].
//   *_generic_kernel    any dim and any alignment: the same arithmetic with scalar accesses.
// Row sums: DPP inside each 16-lane row of the wave, readlane across the four rows, LDS only
// across the waves that share a row; every order is fixed, so results are bitwise reproducible.

#include <mutex>
#include <type_traits>

#include "common.h"
#include "fp8_e4m3.h"
#include "mx_formats.h"

#define VG_VERSION_STRING "velograd_amd 0.1.0 fused-rmsnorm-residual gfx950"

namespace {

using namespace vg;
using vg_fp8::inverse_scale;
using vg_fp8::kE4M3Max;
using vg_plan::BwdPlan;
using vg_plan::kGenericBlock;
using vg_plan::kMaxNV;
using vg_plan::kMaxWavesPerRow;
using vg_plan::kWave;
using vg_plan::max_block_for_nv;
using vg_plan::RowPlan;

// The weight values of one activation chunk (kVec(DT) columns), kept packed in registers: one
// 16-byte vector when the weight has the activation dtype, kVec/4 vectors when it is fp32.
// No weight (NULL) reads as 1.0, which leaves (h * r) * w == h * r and g * w == g exactly.
template <int DT, int WDT>
struct WeightChunk {
  static_assert(WDT == DT || WDT == VELOGRAD_DTYPE_F32, "weight is the activation dtype or fp32");
  static constexpr int kParts = (WDT == DT) ? 1 : Codec<DT>::kVec / 4;
  u32x4 q[kParts];

  __device__ inline void load(const void* w, int64_t col0) {
    if (w == nullptr) {
      // fp32 1.0 in every slot, decoded through the fp32 codec below
#pragma unroll
      for (int i = 0; i < kParts; ++i) q[i] = u32x4{0u, 0u, 0u, 0u};
      return;
    }
#pragma unroll
    for (int i = 0; i < kParts; ++i) q[i] = load16<WDT>(w, col0 + i * Codec<WDT>::kVec);
  }
  __device__ inline void unpack(bool has_w, float* f) const {
    if (!has_w) {
#pragma unroll
      for (int i = 0; i < Codec<DT>::kVec; ++i) f[i] = 1.0f;
      return;
    }
#pragma unroll
    for (int i = 0; i < kParts; ++i) Codec<WDT>::unpack(q[i], f + i * Codec<WDT>::kVec);
  }
};

// Where element `elem` of a stream starts inside its 16-byte line (the generic kernels' aligned
// middle of a row, see fwd_generic_kernel).
__device__ inline uintptr_t row_offset16(const void* base, int64_t elem, int elem_bytes) {
  return (reinterpret_cast<uintptr_t>(base) + (uintptr_t)(elem * elem_bytes)) & 15u;
}

// The 16 bytes at p whatever its 2-byte alignment (`align` = p's offset in its 16-byte line, the
// same on every lane), in the widest loads that alignment allows: the generic kernels' weight
// values for a body chunk, which sits elsewhere in its line than the row's chunk.
__device__ inline u32x4 load16_unaligned(const char* p, uintptr_t align) {
  if (align == 0) return *reinterpret_cast<const u32x4*>(p);
  if ((align & 7) == 0) {
    const u32x2 lo = *reinterpret_cast<const u32x2*>(p);
    const u32x2 hi = *reinterpret_cast<const u32x2*>(p + 8);
    return u32x4{lo.x, lo.y, hi.x, hi.y};
  }
  if ((align & 3) == 0) {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
    return u32x4{q[0], q[1], q[2], q[3]};
  }
  const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
  u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = (uint32_t)h[2 * i] | ((uint32_t)h[2 * i + 1] << 16);
  return v;
}

// The weight values of the body chunk at element j (Codec<DT>::kVec of them) into f, for the
// generic kernels: one to four loads of 16 bytes' worth instead of one per element.  `align` is
// the weight's offset inside its 16-byte line at the row's first body element (uniform).
template <int DT, int WDT>
__device__ inline void weight_run(const void* w, int64_t j, uintptr_t align, float* f) {
  constexpr int kParts = (Codec<DT>::kVec * Codec<WDT>::kBytes) / 16;
  const char* p = static_cast<const char*>(w) + j * Codec<WDT>::kBytes;
#pragma unroll
  for (int q = 0; q < kParts; ++q)
    Codec<WDT>::unpack(load16_unaligned(p + 16 * q, align), f + q * Codec<WDT>::kVec);
}

// Largest |value| over the `tpr` threads of row group `grp`, on the bit patterns of |value|
// (sign cleared): for non-negative IEEE floats the unsigned order is the numeric order, and
// every NaN pattern lies above +inf, so a NaN anywhere in the row wins (NaN propagates).
template <int CTRL>
__device__ inline uint32_t dpp_move_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

__device__ inline uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

__device__ inline uint32_t row_max_abs_bits(uint32_t v, int tpr, int grp, uint32_t* red) {
  v = umax(v, dpp_move_u32<0xB1>(v));
  v = umax(v, dpp_move_u32<0x4E>(v));
  v = umax(v, dpp_move_u32<0x124>(v));
  v = umax(v, dpp_move_u32<0x128>(v));
  v = umax(umax((uint32_t)__builtin_amdgcn_readlane((int)v, 0),
                (uint32_t)__builtin_amdgcn_readlane((int)v, 16)),
           umax((uint32_t)__builtin_amdgcn_readlane((int)v, 32),
                (uint32_t)__builtin_amdgcn_readlane((int)v, 48)));
  if (tpr > kWave) {
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
    __syncthreads();
    const int wpr = tpr / kWave;
    const uint32_t* p = red + grp * wpr;
    uint32_t t = p[0];
    for (int i = 1; i < wpr; ++i) t = umax(t, p[i]);
    v = t;
  }
  return v;
}

// ------------------------------------------------------------------------------------------
// fp8 E4M3 codes on the device.  gfx950's v_cvt_pk_fp8_f32 converts two fp32 values to OCP
// e4m3fn with round to nearest even (one instruction per pair instead of the integer steps of
// vg_fp8::e4m3_encode, which the CPU tests pin against the oracle).  It is not saturating, and
// needs not be here: the inputs are y * (1 / scale) with |y| <= amax, so |y * inv| <=
// 448 * (1 + 2^-22), which rounds to 448 (values up to the 464 midpoint do); the exception,
// inv = 1 for a row whose scale is below the smallest normal float, has |y| < 2^-117.  NaN
// converts to a NaN code.  Build with -DVG_FP8_SOFT_ENCODE=1 to use the integer encoder.
// ------------------------------------------------------------------------------------------
#ifndef VG_FP8_SOFT_ENCODE
#define VG_FP8_SOFT_ENCODE 0
#endif

__device__ inline uint32_t e4m3x4(float a, float b, float c, float d) {
#if VG_FP8_SOFT_ENCODE
  return vg_fp8::e4m3_encode(a) | (vg_fp8::e4m3_encode(b) << 8) | (vg_fp8::e4m3_encode(c) << 16) |
         (vg_fp8::e4m3_encode(d) << 24);
#else
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
#endif
}

__device__ inline uint32_t e4m3x1(float a) {
#if VG_FP8_SOFT_ENCODE
  return vg_fp8::e4m3_encode(a);
#else
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, a, 0, false) & 0xffu;
#endif
}

// fp4 E2M1 nibbles on the device: gfx950's v_cvt_scalef32_pk_fp4_f32 converts two fp32 values
// divided by a scale to E2M1, round to nearest even, saturating, the first value in the low
// nibble of the selected byte (checked against the oracle's nearest-value encoder on every
// midpoint and a dense sweep at scales 0.5..4).  The block factor 2^-s is applied by an exact
// multiplication first and the instruction's scale is 1.  Build with -DVG_FP4_SOFT_ENCODE=1 to
// use vg_mx::e2m1_encode (the comparison chain the CPU tests pin) instead.
#ifndef VG_FP4_SOFT_ENCODE
#define VG_FP4_SOFT_ENCODE 0
#endif

template <int SEL>
__device__ inline uint32_t e2m1x2(uint32_t old, float a, float b) {
#if VG_FP4_SOFT_ENCODE
  return old | ((vg_mx::e2m1_encode(a) | (vg_mx::e2m1_encode(b) << 4)) << (8 * SEL));
#else
  return (uint32_t)__builtin_amdgcn_cvt_scalef32_pk_fp4_f32(old, a, b, 1.0f, SEL);
#endif
}

// The reference module's `mean_sq = max(1e-12, sum(x ** 2) / dim)` (python/velograd/nn.py:349),
// for a floor given > 0.  Python's max keeps its first argument unless the second compares
// greater, so a NaN mean square becomes the floor there, and here.  floor == 0 (the fused
// functions, which have no clamp, fused.py:41-42) leaves mean_sq untouched, NaN included.
__device__ __forceinline__ float floor_mean_sq(float mean_sq, float floor) {
  return (floor > 0.0f && !(mean_sq > floor)) ? floor : mean_sq;
}

// ------------------------------------------------------------------------------------------
// Kernel arguments.
// ------------------------------------------------------------------------------------------
struct FwdArgs {
  const void* x;
  const void* res;
  const void* w;
  void* y;          // activation dtype, or fp8 e4m3 codes (one byte each) for the fp8 epilogue
  void* h;
  float* inv_rms;
  float* y_scale;   // fp8 epilogue: per-row dequantisation scale amax(|y|) / 448
  uint8_t* mx_scale;  // MX epilogues: E8M0 scale codes, one per 32 elements of a row
  int64_t ld_mx;      // row stride of mx_scale in bytes
  int64_t rows;
  int64_t ld_x, ld_res, ld_y, ld_h;
  int32_t dim;
  int32_t tpr;
  float eps;
  float ms_floor;   // > 0: floor on mean(h^2) before eps (the reference module's clamp)
  int64_t rope_seq;       // kOutRopeI: positions per outer index (row position = row % rope_seq)
  int32_t rope_half;      // kOutRopeI: dim / 2
  float rope_c_hi, rope_c_lo;  // kOutRopeI: log2(base) / half as an unevaluated float sum
};

struct BwdArgs {
  const void* g;
  const void* saved;
  const void* w;
  const float* inv_rms;
  const void* gh;  // residual-stream gradient added to dx, or null
  void* dx;
  void* dres;
  float* partial;  // [slots, dim] fp32 or null
  int64_t rows;
  int64_t ld_g, ld_s, ld_gh, ld_dx, ld_dres;
  int32_t dim;
  int32_t tpr;
  int32_t iters;  // rows visited per slot = ceil(rows / slots)
  int64_t rope_seq;            // kRopeG: positions per outer index (row position = row % rope_seq)
  float rope_c_hi, rope_c_lo;  // kRopeG: log2(base) / half as an unevaluated float sum
};

// Output modes of the forward kernels.
constexpr int kOutDtype = 0;   // y in the activation dtype
constexpr int kOutFp8Row = 1;  // y as e4m3 codes with one fp32 scale per row
constexpr int kOutMxE4M3 = 2;  // MXFP8: e4m3 codes, one E8M0 scale per 32 elements
constexpr int kOutMxE2M1 = 3;  // MXFP4: e2m1 nibbles (two per byte), one E8M0 scale per 32
constexpr int kOutRopeI = 4;   // y rotated by the reference model's interleaved RoPE
constexpr int kOutDtypeLateH = 5;  // as kOutDtype, with h stored after the row reduction
// y rotated by the interleaved RoPE with each pair's (cos, sin) evaluated directly: rows too wide
// for fwd_rope_kernel's walk (more than one 16-byte chunk per thread)
constexpr int kOutRopeDirect = 6;

// The reference model's RoPE applied to y in registers (python/velograd/functional.py:287-315;
// models/llama.py:48-49 rotates the normalised attention input): the pair (y_2i, y_2i+1) of a
// row at position pos turns by pos * freq_i, freq_i = base^(-2i/dim) = 2^-(i * c) with
// c = log2(base) / half.  c arrives as c_hi + c_lo (from double on the host); freq_i and the
// angle pos * freq_i are formed in double, as the reference's Python floats are, and the angle is
// reduced exactly to [-1/2, 1/2] revolutions before a float32 sincospi, so cos and sin are within
// a few float32 ulps at any position (a float32 angle would carry pos * freq_i * 2^-24 radians of
// error: 0.016 rad at position 2.6e5).
constexpr double kInv2PiD = 0.159154943091895335768883763372514362;
__device__ __forceinline__ double rope_freq(int i, float c_hi, float c_lo) {
  return exp2(-(double)i * ((double)c_hi + (double)c_lo));
}

// cos and sin of pair i's angle at position pos.
__device__ __forceinline__ void rope_cos_sin(int64_t pos, int i, float c_hi, float c_lo, float& c,
                                             float& s) {
  const double rev = (double)pos * rope_freq(i, c_hi, c_lo) * kInv2PiD;
  sincospif(2.0f * (float)(rev - rint(rev)), &s, &c);
}

// The frequencies of a thread's pairs in a strided loop (pairs i0, i0 + stride, ...): the first
// from exp2, each next one the previous times base^(-2 stride / dim), in double (a few double
// ulps over a row, far below the float32 rotation's rounding), so the generic kernels pay one
// double exp2 per row and thread instead of one per pair.
struct RopeFreqWalk {
  double f, ratio;
  __device__ RopeFreqWalk(int i0, int stride, float c_hi, float c_lo) {
    const double c = (double)c_hi + (double)c_lo;
    f = exp2(-(double)i0 * c);
    ratio = exp2(-(double)stride * c);
  }
  __device__ double next() {
    const double v = f;
    f *= ratio;
    return v;
  }
};

// cos and sin at position pos of the pair whose frequency is fr (as rope_cos_sin)
__device__ __forceinline__ void rope_cos_sin_f(int64_t pos, double fr, float& c, float& s) {
  const double rev = (double)pos * fr * kInv2PiD;
  sincospif(2.0f * (float)(rev - rint(rev)), &s, &c);
}

// Largest value over aligned groups of L lanes (L = 4 or 8), on every lane of the group.
template <int L>
__device__ inline uint32_t lane_group_max(uint32_t v) {
  static_assert(L == 4 || L == 8, "MX blocks span 4 or 8 lanes");
  v = umax(v, dpp_move_u32<0xB1>(v));     // quad_perm [1,0,3,2]
  v = umax(v, dpp_move_u32<0x4E>(v));     // quad_perm [2,3,0,1]
  if constexpr (L == 8) v = umax(v, dpp_move_u32<0x141>(v));  // row_half_mirror
  return v;
}

// ------------------------------------------------------------------------------------------
// Forward, register-resident row.
// ------------------------------------------------------------------------------------------
// OUT selects the epilogue.  kOutFp8Row: y is not stored in the activation dtype; a second row
// reduction finds amax = max |y| over the row (fp32 y, before any rounding), the row's scale is
// amax / 448, and y * (1 / scale) is stored as e4m3 codes: 8 bytes per bf16/fp16 chunk, 4 per
// fp32 chunk.  kOutMxE4M3 / kOutMxE2M1: the 32 elements of an MX block are the chunks of 4
// (bf16/fp16) or 8 (fp32) consecutive lanes, whose amax is reduced with DPP inside the group.
// X8: rows of a 2-byte dtype that start on 8-byte boundaries only, dim = n * V + V / 2 (hidden
// sizes such as 4100; plain outputs only): the row plan covers the n whole chunks, each moved as
// two 8-byte halves, and the row's last V / 2 elements form an extra half chunk of lane 0 of the
// row group (every lane of the group loads the same 8 bytes: one request per wave).
template <int DT, int WDT, int NV, int OUT, bool X8 = false>
__global__ __launch_bounds__(max_block_for_nv(NV)) void fwd_vec_kernel(const FwdArgs a) {
  using C = Codec<DT>;
  constexpr int V = C::kVec;
  constexpr int VH = V / 2;
  static_assert(!X8 || ((OUT == kOutDtype || OUT == kOutDtypeLateH) && C::kBytes == 2),
                "rows of 8-byte alignment: plain outputs of a 2-byte dtype");
  __shared__ float red[kMaxWavesPerRow];

  const int tpr = a.tpr;
  const int grp = threadIdx.x / tpr;
  const int lt = threadIdx.x - grp * tpr;
  const int groups = blockDim.x / tpr;
  const int64_t row = (int64_t)blockIdx.x * groups + grp;
  const bool row_ok = row < a.rows;
  const int nchunk = a.dim / V;
  const bool has_res = a.res != nullptr;
  const bool has_w = a.w != nullptr;
  const int64_t xcol = (int64_t)a.dim - VH;  // X8: the extra half chunk's first column
  const bool own_x = X8 && lt == 0;
  // One chunk of a stream: 16 bytes, or two 8-byte halves for X8 rows.
  auto load_chunk = [&](const void* base, int64_t e) -> u32x4 {
    if constexpr (X8) {
      const u32x2 lo = load8_stream<DT>(base, e);
      const u32x2 hi = load8_stream<DT>(base, e + VH);
      return u32x4{lo.x, lo.y, hi.x, hi.y};
    } else {
      return load16_stream<DT>(base, e);
    }
  };
  auto store_chunk = [&](void* base, int64_t e, const u32x4 v) {
    if constexpr (X8) {
      store8_stream<DT>(base, e, u32x2{v.x, v.y});
      store8_stream<DT>(base, e + VH, u32x2{v.z, v.w});
    } else {
      store16_stream<DT>(base, e, v);
    }
  };

  // Only the packed 16-byte chunks stay live across the row reduction; fp32 h is formed again
  // after it (the same single fp32 add, so the same bits), which keeps VGPRs low enough for
  // up to 8 chunks per thread.
  u32x4 xv[NV], rv[NV];
  WeightChunk<DT, WDT> wc[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c = lt + k * tpr;
    xv[k] = u32x4{0u, 0u, 0u, 0u};
    rv[k] = u32x4{0u, 0u, 0u, 0u};
    if (row_ok && c < nchunk) {
      xv[k] = load_chunk(a.x, row * a.ld_x + (int64_t)c * V);
      if (has_res) rv[k] = load_chunk(a.res, row * a.ld_res + (int64_t)c * V);
    }
  }
  u32x2 xx = u32x2{0u, 0u}, rx = u32x2{0u, 0u};
  float wfx[VH];
  if constexpr (X8) {
    if (row_ok) {
      xx = load8_stream<DT>(a.x, row * a.ld_x + xcol);
      if (has_res) rx = load8_stream<DT>(a.res, row * a.ld_res + xcol);
    }
#pragma unroll
    for (int i = 0; i < VH; ++i) wfx[i] = 1.0f;
    if (has_w) {
      if constexpr (WDT == VELOGRAD_DTYPE_F32) {
        Codec<VELOGRAD_DTYPE_F32>::unpack(load16<VELOGRAD_DTYPE_F32>(a.w, xcol), wfx);
      } else {
        const u32x2 q = *reinterpret_cast<const u32x2*>(static_cast<const char*>(a.w) +
                                                        xcol * Codec<WDT>::kBytes);
        float t[V];
        Codec<WDT>::unpack(u32x4{q.x, q.y, 0u, 0u}, t);
#pragma unroll
        for (int i = 0; i < VH; ++i) wfx[i] = t[i];
      }
    }
  }
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c = lt + k * tpr;
    wc[k].load((has_w && c < nchunk) ? a.w : nullptr, (int64_t)c * V);
  }

  // the extra half chunk's h (X8), in the first VH of V slots, the rest 0
  auto make_hx = [&](float* hf) {
    C::unpack(u32x4{xx.x, xx.y, 0u, 0u}, hf);
    if (has_res) {
      float rf[V];
      C::unpack(u32x4{rx.x, rx.y, 0u, 0u}, rf);
#pragma unroll
      for (int i = 0; i < VH; ++i) hf[i] = hf[i] + rf[i];
    }
  };
  auto make_h = [&](int k, float* hf) {
    C::unpack(xv[k], hf);
    if (has_res) {
      float rf[V];
      C::unpack(rv[k], rf);
#pragma unroll
      for (int i = 0; i < V; ++i) hf[i] = hf[i] + rf[i];
    }
  };

  const bool write_h = has_res && a.h != nullptr;
  constexpr bool kLateH = OUT == kOutDtypeLateH;
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float hf[V];
    make_h(k, hf);
#pragma unroll
    for (int i = 0; i < V; ++i) ss += hf[i] * hf[i];
    const int c = lt + k * tpr;
    if (!kLateH && write_h && row_ok && c < nchunk)
      store_chunk(a.h, row * a.ld_h + (int64_t)c * V, C::pack(hf));
  }
  if constexpr (X8) {
    float hf[V];
    make_hx(hf);
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < VH; ++i) p += hf[i] * hf[i];
    ss += own_x ? p : 0.0f;
    if (!kLateH && write_h && row_ok && own_x) {
      const u32x4 pv = C::pack(hf);
      store8_stream<DT>(a.h, row * a.ld_h + xcol, u32x2{pv.x, pv.y});
    }
  }

  ss = row_sum(ss, tpr, grp, red);
  const float mean_sq = floor_mean_sq(ss / (float)a.dim, a.ms_floor);
  const float r = 1.0f / __builtin_sqrtf(mean_sq + a.eps);
  if (row_ok && lt == 0 && a.inv_rms != nullptr) a.inv_rms[row] = r;

#pragma unroll
  for (int k = 0; k < NV; ++k) {
    forget(xv[k]);
    forget(rv[k]);
#pragma unroll
    for (int i = 0; i < WeightChunk<DT, WDT>::kParts; ++i) forget(wc[k].q[i]);
  }
  auto make_y = [&](int k, float* yf) {
    float hf[V], wf[V];
    make_h(k, hf);
    wc[k].unpack(has_w, wf);
#pragma unroll
    for (int i = 0; i < V; ++i) yf[i] = (hf[i] * r) * wf[i];
  };

  static_assert(OUT != kOutRopeI, "the RoPE output runs in fwd_rope_kernel");
  if constexpr (OUT == kOutDtype || OUT == kOutDtypeLateH || OUT == kOutRopeDirect) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = lt + k * tpr;
      if (row_ok && c < nchunk) {
        if (kLateH && write_h) {
          float hf[V];
          make_h(k, hf);
          store_chunk(a.h, row * a.ld_h + (int64_t)c * V, C::pack(hf));
        }
        float yf[V];
        make_y(k, yf);
        if constexpr (OUT == kOutRopeDirect) {
          // pairs c * V/2 + q at position row % rope_seq (functional.py:302-314): double
          // frequency and angle, exact reduction, float sincospi, as rope_cos_sin
          const int64_t pos = row % a.rope_seq;
          RopeFreqWalk fw(c * (V / 2), 1, a.rope_c_hi, a.rope_c_lo);
#pragma unroll
          for (int q = 0; q < V / 2; ++q) {
            float cs, sn;
            rope_cos_sin_f(pos, fw.next(), cs, sn);
            const float y0 = yf[2 * q], y1 = yf[2 * q + 1];
            yf[2 * q] = y0 * cs - y1 * sn;                                 // functional.py:313
            yf[2 * q + 1] = y0 * sn + y1 * cs;                             // functional.py:314
          }
        }
        store_chunk(a.y, row * a.ld_y + (int64_t)c * V, C::pack(yf));
      }
    }
    if constexpr (X8) {
      if (row_ok && own_x) {
        float hf[V];
        make_hx(hf);
        if (kLateH && write_h) {
          const u32x4 pv = C::pack(hf);
          store8_stream<DT>(a.h, row * a.ld_h + xcol, u32x2{pv.x, pv.y});
        }
        float yf[V];
#pragma unroll
        for (int i = 0; i < VH; ++i) yf[i] = (hf[i] * r) * wfx[i];
#pragma unroll
        for (int i = VH; i < V; ++i) yf[i] = 0.0f;
        const u32x4 pv = C::pack(yf);
        store8_stream<DT>(a.y, row * a.ld_y + xcol, u32x2{pv.x, pv.y});
      }
    }
  } else if constexpr (OUT == kOutMxE4M3 || OUT == kOutMxE2M1) {
    constexpr int kEmax = OUT == kOutMxE4M3 ? vg_mx::kEmaxE4M3 : vg_mx::kEmaxE2M1;
    constexpr int kLanes = vg_mx::kBlock / V;  // lanes per MX block
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = lt + k * tpr;
      float yf[V];
      make_y(k, yf);
      uint32_t am = 0;
#pragma unroll
      for (int i = 0; i < V; ++i) am = umax(am, __builtin_bit_cast(uint32_t, yf[i]) & 0x7fffffffu);
      am = lane_group_max<kLanes>(am);  // every lane, before any divergence
      if (row_ok && c < nchunk) {
        const bool finite = am < 0x7f800000u;
        const float f = finite ? vg_mx::inverse_scale(vg_mx::shared_exp(am, kEmax)) : 0.0f;
        uint8_t* dst = static_cast<uint8_t*>(a.y) + row * a.ld_y;
        if constexpr (OUT == kOutMxE4M3) {
          uint32_t words[V / 4];
#pragma unroll
          for (int j = 0; j < V / 4; ++j) {
            float q[4];
#pragma unroll
            for (int t = 0; t < 4; ++t)
              q[t] = __builtin_fminf(__builtin_fmaxf(yf[4 * j + t] * f, -kE4M3Max), kE4M3Max);
            words[j] = finite ? e4m3x4(q[0], q[1], q[2], q[3]) : 0u;
          }
          if constexpr (V == 8) {
            const u32x2 w2 = {words[0], words[1]};
            __builtin_nontemporal_store(w2, reinterpret_cast<u32x2*>(dst + (int64_t)c * V));
          } else {
            __builtin_nontemporal_store(words[0], reinterpret_cast<uint32_t*>(dst + (int64_t)c * V));
          }
        } else {
          uint32_t word = 0;
          word = e2m1x2<0>(word, yf[0] * f, yf[1] * f);
          word = e2m1x2<1>(word, yf[2] * f, yf[3] * f);
          if constexpr (V == 8) {
            word = e2m1x2<2>(word, yf[4] * f, yf[5] * f);
            word = e2m1x2<3>(word, yf[6] * f, yf[7] * f);
          }
          if (!finite) word = 0;
          if constexpr (V == 8) {
            __builtin_nontemporal_store(word, reinterpret_cast<uint32_t*>(dst + (int64_t)c * 4));
          } else {
            __builtin_nontemporal_store((uint16_t)word,
                                        reinterpret_cast<uint16_t*>(dst + (int64_t)c * 2));
          }
        }
        if (lt % kLanes == 0)
          a.mx_scale[row * a.ld_mx + c / kLanes] = (uint8_t)vg_mx::scale_code(am, kEmax);
      }
    }
  } else {
    // y stays in registers from the amax pass to the encoding (NV * V floats).
    __shared__ uint32_t red_max[kMaxWavesPerRow];
    float yf[NV][V];
    uint32_t am = 0;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = lt + k * tpr;
      make_y(k, yf[k]);
      if (row_ok && c < nchunk) {
#pragma unroll
        for (int i = 0; i < V; ++i)
          am = umax(am, __builtin_bit_cast(uint32_t, yf[k][i]) & 0x7fffffffu);
      }
    }
    am = row_max_abs_bits(am, tpr, grp, red_max);
    const float scale = __builtin_bit_cast(float, am) / kE4M3Max;
    const float inv = inverse_scale(scale);
    if (row_ok && lt == 0) a.y_scale[row] = scale;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = lt + k * tpr;
      if (row_ok && c < nchunk) {
        uint32_t words[V / 4];
#pragma unroll
        for (int j = 0; j < V / 4; ++j) {
          words[j] = e4m3x4(yf[k][4 * j] * inv, yf[k][4 * j + 1] * inv, yf[k][4 * j + 2] * inv,
                            yf[k][4 * j + 3] * inv);
        }
        uint8_t* dst = static_cast<uint8_t*>(a.y) + row * a.ld_y + (int64_t)c * V;
        if constexpr (V == 8) {
          const u32x2 w2 = {words[0], words[1]};
          __builtin_nontemporal_store(w2, reinterpret_cast<u32x2*>(dst));
        } else {
          __builtin_nontemporal_store(words[0], reinterpret_cast<uint32_t*>(dst));
        }
      }
    }
  }
}

// ------------------------------------------------------------------------------------------
// Forward with the model's RoPE on y (kOutRopeI), one 16-byte chunk per thread.  Workgroup b of
// G walks up to W rows b, b + G, b + 2G, ... (W = 16, or 32 for long tensors of wide rows:
// launch_plan.h fwd_rope_walk_rows): at each step the resident workgroups
// touch adjacent rows, one compact address front that HBM serves better than runs of
// consecutive rows per workgroup (those spread the front over 16 rows per workgroup).  The next
// rows' chunks are in flight while the current one reduces.  Each thread keeps the rotation
// (cos, sin) of its pairs (in double for fp32 outputs, in float32 for bf16/fp16 ones) and
// advances it by G positions per step (the rotation through G * freq_j, evaluated once per walk),
// so trigonometry runs only before the walk; evaluated per (row, pair) it made the fused pass
// VALU-bound, no faster than two passes.  The walk's first angle is the double pos * freq_j
// reduced exactly before a float sincospi (a few float32 ulps), and so is the step's; the
// recurrence adds ~1e-16 per step in double, about 3 float32 ulps of the pair in float32, over
// at most W - 1 steps from an exact value.  Where a step crosses
// the end of a sequence (row position = row % rope_seq) and G is a multiple or a divisor of
// rope_seq, the position returns to the walk's first one and so does the rotation (kept); any
// other crossing re-evaluates the angle at the new position.
// The pass is bound by its vector instructions as much as by HBM, so each row's arithmetic is
// kept short: the weight is decoded once per walk, h stays in registers across the reduction,
// sums of products and the rotation use fused multiply-adds, and for a power-of-two dim the mean
// is sum * (1 / dim), exact, instead of a division.
// A whole walk whose positions only advance or return to the start (the usual case) runs as
// straight-line code over its rows with a ring of three row buffers, two rows' loads in flight
// while one reduces, and no branch around a global memory operation (the residual and h are
// compile-time flags RF; the walk's inv_rms values wait in LDS and are stored after it), so
// each row waits for its own loads only instead of draining every load and store at each row.
// Shorter walks and walks that re-evaluate angles take the guarded loop.
// ------------------------------------------------------------------------------------------
constexpr int kRopeRes = 1;     // RF: a residual is added
constexpr int kRopeWriteH = 2;  // RF: h is stored
constexpr int kRopeDimPow2 = 4; // RF: dim is a power of two

template <int DT, int WDT, int RF, int W>
__global__ __launch_bounds__(max_block_for_nv(1)) void fwd_rope_kernel(const FwdArgs a) {
  static_assert(W == vg_plan::kNormRopeRows || W == vg_plan::kNormRopeLongRows,
                "walks of 16 or 32 rows");
  using C = Codec<DT>;
  constexpr int V = C::kVec;
  constexpr int PP = V / 2;  // pairs per chunk
  __shared__ float red[2][kMaxWavesPerRow];
  const int tpr = blockDim.x;  // one row group per workgroup, one chunk per thread
  const int lt = threadIdx.x;
  const int nchunk = a.dim / V;
  const bool lane_ok = lt < nchunk;
  constexpr bool has_res = (RF & kRopeRes) != 0;
  constexpr bool write_h = has_res && (RF & kRopeWriteH) != 0;
  const bool has_w = a.w != nullptr;
  const int64_t G = gridDim.x;   // row step of the walk
  const int64_t row0 = blockIdx.x;
  const int64_t left = (a.rows - row0 + G - 1) / G;
  const int nrows = (int)(left < W ? left : W);
  const int64_t col = (int64_t)lt * V;
  const int64_t seq = a.rope_seq;
  const int64_t pos0 = row0 % seq;
  // the positions of the walk only advance by G or return to pos0
  const bool back_to_start = (seq % G == 0) || (G % seq == 0);
  // 1 / dim is exact for a power of two, so sum * (1 / dim) has the bits of sum / dim
  const float inv_dim = (RF & kRopeDimPow2) ? 1.0f / (float)a.dim : 0.0f;

  u32x4 xv = u32x4{0u, 0u, 0u, 0u}, rv = u32x4{0u, 0u, 0u, 0u};
  if (lane_ok) {
    xv = load16_stream<DT>(a.x, row0 * a.ld_x + col);
    if constexpr (has_res) rv = load16_stream<DT>(a.res, row0 * a.ld_res + col);
  }
  float wf[V];
  {
    WeightChunk<DT, WDT> wc;
    wc.load((has_w && lane_ok) ? a.w : nullptr, col);
    wc.unpack(has_w, wf);
  }
  // The rotation state: double for fp32 outputs; float32 for bf16/fp16 ones, within about 3
  // float32 ulps of the pair per step over at most W - 1 = 31 steps (~2^-17.5 of the pair), far
  // below their output's rounding (2^-9 for bf16, 2^-12 for fp16).  Re-evaluating it at the 16th
  // row of a 32-row walk cost 2-5 us at 16384 rows (trigonometry set aside for it before the
  // walk; placed in the unrolled loop it stopped the unrolling).
  using RotT = std::conditional_t<DT == VELOGRAD_DTYPE_F32, double, float>;
  auto rot_fma = [](RotT x, RotT y, RotT z) {
    if constexpr (DT == VELOGRAD_DTYPE_F32) return __builtin_fma(x, y, z);
    else return __builtin_fmaf(x, y, z);
  };
  RotT cr[PP], sr[PP], cst[PP], sst[PP];
  float c0[PP], s0[PP];  // the rotation at pos0
  // the rotation at pos: double angle, reduced exactly, float sincospi
  auto rotation_at = [&](int64_t pos, int q, float& c, float& s) {
    const double rev = (double)pos * rope_freq(lt * PP + q, a.rope_c_hi, a.rope_c_lo) * kInv2PiD;
    sincospif(2.0f * (float)(rev - rint(rev)), &s, &c);
  };
#pragma unroll
  for (int q = 0; q < PP; ++q) {
    // the rotation through G positions: double for fp32 outputs, else as rotation_at
    if constexpr (DT == VELOGRAD_DTYPE_F32) {
      double sv, cv;
      sincos((double)G * rope_freq(lt * PP + q, a.rope_c_hi, a.rope_c_lo), &sv, &cv);
      cst[q] = cv;
      sst[q] = sv;
    } else {
      float sv, cv;
      rotation_at(G, q, cv, sv);
      cst[q] = cv;
      sst[q] = sv;
    }
    rotation_at(pos0, q, c0[q], s0[q]);
    cr[q] = c0[q];
    sr[q] = s0[q];
  }

  auto make_h = [&](const u32x4& xq, const u32x4& rq, float* hf) {
    C::unpack(xq, hf);
    if constexpr (has_res) {
      float rf[V];
      C::unpack(rq, rf);
#pragma unroll
      for (int i = 0; i < V; ++i) hf[i] = hf[i] + rf[i];
    }
  };
  auto sum_sq = [&](const float* hf) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i) ss = __builtin_fmaf(hf[i], hf[i], ss);
    return ss;
  };
  auto inv_rms_of = [&](float ss) {
    const float mean = (RF & kRopeDimPow2) ? ss * inv_dim : ss / (float)a.dim;
    return 1.0f / __builtin_sqrtf(floor_mean_sq(mean, a.ms_floor) + a.eps);
  };
  // y = (h * r) * w turned by the current angles
  auto make_y = [&](const float* hf, float r, float* yf) {
#pragma unroll
    for (int i = 0; i < V; ++i) yf[i] = (hf[i] * r) * wf[i];
#pragma unroll
    for (int q = 0; q < PP; ++q) {
      const float cv = (float)cr[q], sv = (float)sr[q];
      const float y0 = yf[2 * q], y1 = yf[2 * q + 1];
      yf[2 * q] = __builtin_fmaf(y0, cv, -(y1 * sv));                    // functional.py:313
      yf[2 * q + 1] = __builtin_fmaf(y0, sv, y1 * cv);                   // functional.py:314
    }
  };
  // the angles of the next row of the walk: pos advances by G; past the end of the sequence it
  // returns to pos0 (back_to_start) or, with ANCHOR, lands anywhere and is evaluated afresh
  auto advance = [&](int64_t& pos, auto anchor) {
    pos += G;
    if (pos < seq) {
#pragma unroll
      for (int q = 0; q < PP; ++q) {
        const RotT cn = rot_fma(cr[q], cst[q], -(sr[q] * sst[q]));
        sr[q] = rot_fma(sr[q], cst[q], cr[q] * sst[q]);
        cr[q] = cn;
      }
    } else if (!decltype(anchor)::value || back_to_start) {
      pos = pos0;
#pragma unroll
      for (int q = 0; q < PP; ++q) {
        cr[q] = c0[q];
        sr[q] = s0[q];
      }
    } else {
      pos %= seq;
#pragma unroll
      for (int q = 0; q < PP; ++q) {
        float c, s;
        rotation_at(pos, q, c, s);
        cr[q] = c;
        sr[q] = s;
      }
    }
  };

  const bool walk_ok = back_to_start || pos0 + (int64_t)(W - 1) * G < seq;
  if (nrows == W && nchunk == tpr && walk_ok) {
    __shared__ float inv_lds[W];
    constexpr int RB = 3;
    u32x4 xb[RB], rb[RB];
    xb[0] = xv;
    rb[0] = rv;
    xb[1] = load16_stream<DT>(a.x, (row0 + G) * a.ld_x + col);
    if constexpr (has_res) rb[1] = load16_stream<DT>(a.res, (row0 + G) * a.ld_res + col);
    int64_t pos = pos0;
#pragma unroll
    for (int it = 0; it < W; ++it) {
      const int b = it % RB;
      const int64_t row = row0 + it * G;
      if (it + 2 < W) {
        const int nb = (it + 2) % RB;
        xb[nb] = load16_stream<DT>(a.x, (row + 2 * G) * a.ld_x + col);
        if constexpr (has_res) rb[nb] = load16_stream<DT>(a.res, (row + 2 * G) * a.ld_res + col);
      }
      float hf[V];
      make_h(xb[b], rb[b], hf);
      if constexpr (write_h) store16_stream<DT>(a.h, row * a.ld_h + col, C::pack(hf));
      const float r = inv_rms_of(row_sum(sum_sq(hf), tpr, 0, red[it & 1]));
      if (lt == 0) inv_lds[it] = r;
      float yf[V];
      make_y(hf, r, yf);
      store16_stream<DT>(a.y, row * a.ld_y + col, C::pack(yf));
      if (it + 1 < W) advance(pos, std::false_type{});
    }
    // thread 0 wrote inv_lds; threads 1..W-1 of its wave read it in program order
    if (lt < W && a.inv_rms != nullptr) a.inv_rms[row0 + lt * G] = inv_lds[lt];
    return;
  }

  int64_t pos = pos0;
  for (int it = 0; it < nrows; ++it) {
    const int64_t row = row0 + it * G;
    u32x4 xn = u32x4{0u, 0u, 0u, 0u}, rn = u32x4{0u, 0u, 0u, 0u};
    if (it + 1 < nrows && lane_ok) {
      xn = load16_stream<DT>(a.x, (row + G) * a.ld_x + col);
      if constexpr (has_res) rn = load16_stream<DT>(a.res, (row + G) * a.ld_res + col);
    }
    float hf[V];
    make_h(xv, rv, hf);
    if (write_h && lane_ok) store16_stream<DT>(a.h, row * a.ld_h + col, C::pack(hf));
    const float r = inv_rms_of(row_sum(sum_sq(hf), tpr, 0, red[it & 1]));
    if (lt == 0 && a.inv_rms != nullptr) a.inv_rms[row] = r;
    float yf[V];
    make_y(hf, r, yf);
    if (lane_ok) store16_stream<DT>(a.y, row * a.ld_y + col, C::pack(yf));
    if (it + 1 < nrows) advance(pos, std::true_type{});
    xv = xn;
    rv = rn;
  }
}

// ------------------------------------------------------------------------------------------
// Forward, rows of any length and alignment up to 4096 elements that the chunked kernels cannot
// take (odd lengths, streams that start anywhere inside a 16-byte line): one-shot rows as in
// fwd_vec_kernel, several short rows a workgroup, with bwd_ring_elem_kernel's element-strided
// lanes (lane lt of a row group holds columns lt, lt + tpr, ..., M of them), so each of a
// wave's element loads and stores moves one contiguous run of 64 elements.  y in the activation
// dtype (the plain output) only; short rows (kFwdElemMaxDim), where the generic kernel's one row
// per workgroup is bound by each row's latency.
// ------------------------------------------------------------------------------------------
constexpr int64_t kFwdElemMaxDim = 1024;  // the host plans it for rows of at most this length

template <int DT, int WDT, int M>
__global__ __launch_bounds__(vg_plan::kRingBlock) void fwd_elem_kernel(const FwdArgs a) {
  using C = Codec<DT>;
  using Raw = std::conditional_t<C::kBytes == 2, uint16_t, uint32_t>;
  static_assert(M == 4 || M == 8, "four or eight elements a lane");
  __shared__ float red[kMaxWavesPerRow];
  const int tpr = a.tpr;
  const int grp = threadIdx.x / tpr;
  const int lt = threadIdx.x - grp * tpr;
  const int groups = blockDim.x / tpr;
  const int64_t row = (int64_t)blockIdx.x * groups + grp;
  const bool row_ok = row < a.rows;
  const int64_t rw = row_ok ? row : a.rows - 1;  // a row group past the end reads the last row
  const bool has_res = a.res != nullptr;
  const bool write_h = has_res && a.h != nullptr;
  int col[M];
  bool own[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int c = lt + m * tpr;
    own[m] = c < a.dim;
    col[m] = own[m] ? c : a.dim - 1;
  }
  auto decode = [&](uint32_t u) -> float {
    if constexpr (DT == VELOGRAD_DTYPE_BF16) {
      return __builtin_bit_cast(float, u << 16);
    } else if constexpr (DT == VELOGRAD_DTYPE_F16) {
      return (float)__builtin_bit_cast(_Float16, (uint16_t)u);
    } else {
      return __builtin_bit_cast(float, u);
    }
  };
  auto load_raw = [&](const void* base, int64_t i) -> uint32_t {
    return (uint32_t)__builtin_nontemporal_load(static_cast<const Raw*>(base) + i);
  };
  auto store_one = [&](void* base, int64_t i, float f) {
    Raw v;
    if constexpr (DT == VELOGRAD_DTYPE_BF16) v = __builtin_bit_cast(uint16_t, (__bf16)f);
    else if constexpr (DT == VELOGRAD_DTYPE_F16) v = __builtin_bit_cast(uint16_t, (_Float16)f);
    else v = __builtin_bit_cast(uint32_t, f);
    __builtin_nontemporal_store(v, static_cast<Raw*>(base) + i);
  };

  uint32_t xr[M], rr[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    xr[m] = load_raw(a.x, rw * a.ld_x + col[m]);
    rr[m] = has_res ? load_raw(a.res, rw * a.ld_res + col[m]) : 0u;
  }
  float wf[M];
#pragma unroll
  for (int m = 0; m < M; ++m) wf[m] = a.w != nullptr ? Codec<WDT>::load1(a.w, col[m]) : 1.0f;
  float hf[M];
  float ss = 0.0f;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    hf[m] = decode(xr[m]);
    if (has_res) hf[m] = hf[m] + decode(rr[m]);
    const float t = hf[m] * hf[m];
    ss += own[m] ? t : 0.0f;
  }
  ss = row_sum(ss, tpr, grp, red);
  const float mean_sq = floor_mean_sq(ss / (float)a.dim, a.ms_floor);
  const float r = 1.0f / __builtin_sqrtf(mean_sq + a.eps);
  if (row_ok && lt == 0 && a.inv_rms != nullptr) a.inv_rms[row] = r;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    if (row_ok && own[m]) {
      if (write_h) store_one(a.h, row * a.ld_h + col[m], hf[m]);
      store_one(a.y, row * a.ld_y + col[m], (hf[m] * r) * wf[m]);
    }
  }
}

// ------------------------------------------------------------------------------------------
// Forward, any dim / alignment: one row per workgroup, two passes over the row (the second
// re-reads x and residual, normally from L2, and recomputes the identical fp32 h).
// ------------------------------------------------------------------------------------------
template <int DT, int WDT, int OUT>
__global__ __launch_bounds__(kGenericBlock) void fwd_generic_kernel(const FwdArgs a) {
  using C = Codec<DT>;
  using CW = Codec<WDT>;
  __shared__ float red[kGenericBlock / kWave];
  const int64_t row = blockIdx.x;
  const bool has_res = a.res != nullptr;
  const bool has_w = a.w != nullptr;
  const bool write_h = has_res && a.h != nullptr;

  // The plain output moves the row's 16-byte-aligned middle with 16-byte accesses when every
  // stream's row starts at the same offset inside a 16-byte line (contiguous tensors of one dtype
  // whose rows are not 16-byte multiples): `head` elements up to the first boundary and the `tail`
  // past the last whole chunk go element by element.  Other layouts stay element-wise.
  int head = a.dim, nbody = 0;
  if constexpr (OUT == kOutDtype) {
    const uintptr_t mis = row_offset16(a.x, row * a.ld_x, C::kBytes);
    if (mis % C::kBytes == 0 && (!has_res || row_offset16(a.res, row * a.ld_res, C::kBytes) == mis) &&
        row_offset16(a.y, row * a.ld_y, C::kBytes) == mis &&
        (!write_h || row_offset16(a.h, row * a.ld_h, C::kBytes) == mis)) {
      head = (int)(((16 - mis) & 15) / C::kBytes);
      if (head > a.dim) head = a.dim;
      nbody = (a.dim - head) / C::kVec;
    }
  }
  const int tail = head + nbody * C::kVec;  // first element after the body
  auto scalar_j = [&](int t) { return t < head ? t : tail + (t - head); };
  const int nscalar = a.dim - nbody * C::kVec;
  // the weight at the body's chunks: where it sits in its 16-byte lines (2-byte aligned at least)
  const uintptr_t w_align = has_w ? row_offset16(a.w, head, CW::kBytes) : 0;

  // A thread's first KR body chunks stay in registers from the first pass to the second (rows
  // of up to KR * 256 chunks: 8192 bf16/fp16 or 4096 fp32 elements read once); chunks past
  // them are read again in the second pass.  That re-read finds them in L2 when the first pass
  // reads with the normal cache policy and the second non-temporally (its last use): 147.6
  // against 174.9 us the other way round at 16384 x 4100 bf16, before the registers.
  constexpr int KR = OUT == kOutDtype ? 4 : 0;
  u32x4 xk[KR > 0 ? KR : 1], rk[KR > 0 ? KR : 1];
#pragma unroll
  for (int k = 0; k < KR; ++k) {
    const int c = threadIdx.x + k * blockDim.x;
    xk[k] = u32x4{0u, 0u, 0u, 0u};
    rk[k] = u32x4{0u, 0u, 0u, 0u};
    if (c < nbody) {
      const int64_t j = head + (int64_t)c * C::kVec;
      xk[k] = load16_stream<DT>(a.x, row * a.ld_x + j);
      if (has_res) rk[k] = load16_stream<DT>(a.res, row * a.ld_res + j);
    }
  }
  // With a body, the head and tail are fewer than two chunks' worth of elements: one per thread
  // at most, loaded with the body, so a row waits for memory once per pass.
  const bool few_scalar = KR > 0 && nbody > 0;
  int j_s = 0;
  float h_s = 0.0f, w_s = 1.0f;
  if (few_scalar && (int)threadIdx.x < nscalar) {
    j_s = scalar_j(threadIdx.x);
    h_s = C::load1(a.x, row * a.ld_x + j_s);
    if (has_res) h_s = h_s + C::load1(a.res, row * a.ld_res + j_s);
    if (has_w) w_s = CW::load1(a.w, j_s);
  }
  // h of register chunk k (the same single fp32 add as every other path)
  auto h_reg = [&](int k, float* hf) {
    C::unpack(xk[k], hf);
    if (has_res) {
      float rf[C::kVec];
      C::unpack(rk[k], rf);
#pragma unroll
      for (int i = 0; i < C::kVec; ++i) hf[i] = hf[i] + rf[i];
    }
  };
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < KR; ++k) {
    const int c = threadIdx.x + k * blockDim.x;
    if (c < nbody) {
      float hf[C::kVec];
      h_reg(k, hf);
      if (write_h) store16_stream<DT>(a.h, row * a.ld_h + head + (int64_t)c * C::kVec, C::pack(hf));
#pragma unroll
      for (int i = 0; i < C::kVec; ++i) ss += hf[i] * hf[i];
    }
  }
  for (int c = threadIdx.x + KR * blockDim.x; c < nbody; c += blockDim.x) {
    const int64_t j = head + (int64_t)c * C::kVec;
    float hf[C::kVec];
    C::unpack(load16<DT>(a.x, row * a.ld_x + j), hf);
    if (has_res) {
      float rf[C::kVec];
      C::unpack(load16<DT>(a.res, row * a.ld_res + j), rf);
#pragma unroll
      for (int i = 0; i < C::kVec; ++i) hf[i] = hf[i] + rf[i];
    }
    if (write_h) store16_stream<DT>(a.h, row * a.ld_h + j, C::pack(hf));
#pragma unroll
    for (int i = 0; i < C::kVec; ++i) ss += hf[i] * hf[i];
  }
  if (few_scalar) {
    if ((int)threadIdx.x < nscalar) {
      if (write_h) C::store1(a.h, row * a.ld_h + j_s, h_s);
      ss += h_s * h_s;
    }
  } else {
    for (int t = threadIdx.x; t < nscalar; t += blockDim.x) {
      const int j = scalar_j(t);
      float hx = C::load1(a.x, row * a.ld_x + j);
      if (has_res) hx = hx + C::load1(a.res, row * a.ld_res + j);
      if (write_h) C::store1(a.h, row * a.ld_h + j, hx);
      ss += hx * hx;
    }
  }
  ss = row_sum(ss, blockDim.x, 0, red);
  const float mean_sq = floor_mean_sq(ss / (float)a.dim, a.ms_floor);
  const float r = 1.0f / __builtin_sqrtf(mean_sq + a.eps);
  if (threadIdx.x == 0 && a.inv_rms != nullptr) a.inv_rms[row] = r;

  auto y_at = [&](int j) {
    float hx = C::load1(a.x, row * a.ld_x + j);
    if (has_res) hx = hx + C::load1(a.res, row * a.ld_res + j);
    const float n = hx * r;
    return has_w ? n * CW::load1(a.w, j) : n;
  };
  if constexpr (OUT == kOutDtype) {
#pragma unroll
    for (int k = 0; k < KR; ++k) {
      const int c = threadIdx.x + k * blockDim.x;
      if (c < nbody) {
        const int64_t j = head + (int64_t)c * C::kVec;
        float hf[C::kVec], wf[C::kVec];
        h_reg(k, hf);
        if (has_w) weight_run<DT, WDT>(a.w, j, w_align, wf);
#pragma unroll
        for (int i = 0; i < C::kVec; ++i) {
          const float n = hf[i] * r;
          hf[i] = has_w ? n * wf[i] : n;
        }
        store16_stream<DT>(a.y, row * a.ld_y + j, C::pack(hf));
      }
    }
    // the chunks past the registers: x and the residual read again (normally from L2)
    for (int c = threadIdx.x + KR * blockDim.x; c < nbody; c += blockDim.x) {
      const int64_t j = head + (int64_t)c * C::kVec;
      float hf[C::kVec];
      C::unpack(load16_stream<DT>(a.x, row * a.ld_x + j), hf);
      if (has_res) {
        float rf[C::kVec];
        C::unpack(load16_stream<DT>(a.res, row * a.ld_res + j), rf);
#pragma unroll
        for (int i = 0; i < C::kVec; ++i) hf[i] = hf[i] + rf[i];
      }
      float wf[C::kVec];
      if (has_w) weight_run<DT, WDT>(a.w, j, w_align, wf);
#pragma unroll
      for (int i = 0; i < C::kVec; ++i) {
        const float n = hf[i] * r;
        hf[i] = has_w ? n * wf[i] : n;
      }
      store16_stream<DT>(a.y, row * a.ld_y + j, C::pack(hf));
    }
    if (few_scalar) {
      if ((int)threadIdx.x < nscalar) {
        const float n = h_s * r;  // y_at's arithmetic on the register copies
        C::store1(a.y, row * a.ld_y + j_s, has_w ? n * w_s : n);
      }
    } else {
      for (int t = threadIdx.x; t < nscalar; t += blockDim.x) {
        const int j = scalar_j(t);
        C::store1(a.y, row * a.ld_y + j, y_at(j));
      }
    }
  } else if constexpr (OUT == kOutRopeI) {
    const int64_t pos = row % a.rope_seq;
    RopeFreqWalk fw(threadIdx.x, blockDim.x, a.rope_c_hi, a.rope_c_lo);
    for (int i = threadIdx.x; i < a.rope_half; i += blockDim.x) {
      const float x0 = y_at(2 * i), x1 = y_at(2 * i + 1);
      float c, sn;
      rope_cos_sin_f(pos, fw.next(), c, sn);
      C::store1(a.y, row * a.ld_y + 2 * i, x0 * c - x1 * sn);       // functional.py:313
      C::store1(a.y, row * a.ld_y + 2 * i + 1, x0 * sn + x1 * c);   // functional.py:314
    }
  } else if constexpr (OUT == kOutMxE4M3 || OUT == kOutMxE2M1) {
    // MX epilogue (see fwd_vec_kernel): a third pass, one 32-element block per thread.
    constexpr int kEmax = OUT == kOutMxE4M3 ? vg_mx::kEmaxE4M3 : vg_mx::kEmaxE2M1;
    uint8_t* yq = static_cast<uint8_t*>(a.y) + row * a.ld_y;
    for (int b = threadIdx.x; b < a.dim / vg_mx::kBlock; b += blockDim.x) {
      const int j0 = b * vg_mx::kBlock;
      uint32_t am = 0;
      for (int i = 0; i < vg_mx::kBlock; ++i)
        am = umax(am, __builtin_bit_cast(uint32_t, y_at(j0 + i)) & 0x7fffffffu);
      const bool finite = am < 0x7f800000u;
      const float f = finite ? vg_mx::inverse_scale(vg_mx::shared_exp(am, kEmax)) : 0.0f;
      for (int i = 0; i < vg_mx::kBlock; i += 2) {
        const float v0 = y_at(j0 + i) * f, v1 = y_at(j0 + i + 1) * f;
        if constexpr (OUT == kOutMxE4M3) {
          yq[j0 + i] = finite ? (uint8_t)e4m3x1(__builtin_fminf(__builtin_fmaxf(v0, -kE4M3Max), kE4M3Max)) : 0;
          yq[j0 + i + 1] = finite ? (uint8_t)e4m3x1(__builtin_fminf(__builtin_fmaxf(v1, -kE4M3Max), kE4M3Max)) : 0;
        } else {
          yq[(j0 + i) / 2] = finite ? (uint8_t)e2m1x2<0>(0u, v0, v1) : 0;
        }
      }
      a.mx_scale[row * a.ld_mx + b] = (uint8_t)vg_mx::scale_code(am, kEmax);
    }
  } else {
    // fp8 epilogue (see fwd_vec_kernel): a third pass stores the codes.
    __shared__ uint32_t red_max[kGenericBlock / kWave];
    uint32_t am = 0;
    for (int j = threadIdx.x; j < a.dim; j += blockDim.x)
      am = umax(am, __builtin_bit_cast(uint32_t, y_at(j)) & 0x7fffffffu);
    am = row_max_abs_bits(am, blockDim.x, 0, red_max);
    const float scale = __builtin_bit_cast(float, am) / kE4M3Max;
    const float inv = inverse_scale(scale);
    if (threadIdx.x == 0) a.y_scale[row] = scale;
    uint8_t* yq = static_cast<uint8_t*>(a.y) + row * a.ld_y;
    for (int j = threadIdx.x; j < a.dim; j += blockDim.x)
      yq[j] = (uint8_t)e4m3x1(y_at(j) * inv);
  }
}

// ------------------------------------------------------------------------------------------
// Backward, register-resident row, persistent row slots.
// FLAGS: kSavedIsH (the saved tensor is h, xhat = h * inv_rms is formed in registers),
//        kGradH (a residual-stream gradient grad_h is added to dx in the same pass).
// ------------------------------------------------------------------------------------------
constexpr int kSavedIsH = 1;
constexpr int kGradH = 2;
// kRopeG: grad_y is the gradient of the interleaved-RoPE-rotated output (the model's
// F.apply_rotary_emb(attention_norm(x)), models/llama.py:48-49), rotated back in registers
// before use: the backward of the rotation (functional.py:316-345) fused into the norm's.
constexpr int kRopeG = 4;
// kRopeDirect: as kRopeG with each pair's rotation evaluated directly where g is decoded (both
// passes), no walk state and no LDS table: rows too wide for the walk's launch bound.
constexpr int kRopeDirect = 16;
// Rows of the RoPE-gradient walk between direct evaluations of the rotation state.
constexpr int kRopeAnchor = 16;

template <int DT, int WDT, int NV, int FLAGS>
__global__ __launch_bounds__((FLAGS & kRopeG) ? vg_plan::max_block_for_nv_rope(NV)
                                               : max_block_for_nv(NV)) void bwd_vec_kernel(const BwdArgs a) {
  using C = Codec<DT>;
  constexpr int V = C::kVec;
  constexpr bool SAVED_IS_H = (FLAGS & kSavedIsH) != 0;
  constexpr bool HAS_GH = (FLAGS & kGradH) != 0;
  constexpr bool ROPE = (FLAGS & kRopeG) != 0;
  constexpr bool RD = (FLAGS & kRopeDirect) != 0;
  static_assert(!(ROPE && RD), "one RoPE mode");
  constexpr int NH = HAS_GH ? NV : 1;  // grad_h chunks (a dummy slot when absent)
  constexpr int P = V / 2;             // RoPE pairs per chunk
  constexpr int NR = ROPE ? NV : 1;    // rotation state slots (a dummy slot without RoPE)
  __shared__ float red[2][kMaxWavesPerRow];
  // dim floats of dynamic LDS: with kRopeG the walk's step rotations (cos, sin per pair), then
  // (after a barrier) the combine of the row groups' dweight columns.
  extern __shared__ __align__(16) float dyn_lds[];

  const int tpr = a.tpr;
  const int grp = threadIdx.x / tpr;
  const int lt = threadIdx.x - grp * tpr;
  const int groups = blockDim.x / tpr;
  const int64_t slot = (int64_t)blockIdx.x * groups + grp;
  const int64_t nslots = (int64_t)gridDim.x * groups;
  const int nchunk = a.dim / V;
  const bool has_w = a.w != nullptr;
  const bool has_dres = a.dres != nullptr;

  // RoPE: each thread holds (cos, sin) of its pairs at the current row's position and advances
  // them by the rotation through nslots positions (the walk's row step) from the LDS table; they
  // are evaluated directly where the position wraps to a new outer index and on every
  // kRopeAnchor-th row of the walk.  Float32 state: each step adds about an ulp, so re-anchoring
  // keeps the drift under kRopeAnchor ulps however long the walk (the sequence length over the
  // slot count), far below the output rounding of bf16/fp16 and the fp32 dx tolerance.
  float rc[NR][P], rs[NR][P];
  if constexpr (ROPE) {
    for (int q = threadIdx.x; q < a.dim / 2; q += blockDim.x) {
      double sv, cv;
      sincos((double)nslots * rope_freq(q, a.rope_c_hi, a.rope_c_lo), &sv, &cv);
      dyn_lds[2 * q] = (float)cv;
      dyn_lds[2 * q + 1] = (float)sv;
    }
    __syncthreads();
  }
  auto rope_start = [&](int64_t pos) {
    if constexpr (ROPE) {
#pragma unroll
      for (int k = 0; k < NR; ++k) {
#pragma unroll
        for (int p = 0; p < P; ++p)
          rope_cos_sin(pos, (lt + k * tpr) * P + p, a.rope_c_hi, a.rope_c_lo, rc[k][p],
                       rs[k][p]);
      }
    }
  };
  auto rope_step = [&]() {
    if constexpr (ROPE) {
#pragma unroll
      for (int k = 0; k < NR; ++k) {
        const int c = lt + k * tpr;
        if (c < nchunk) {
#pragma unroll
          for (int p = 0; p < P; ++p) {
            const float sc = dyn_lds[2 * (c * P + p)], ss = dyn_lds[2 * (c * P + p) + 1];
            const float cn = rc[k][p] * sc - rs[k][p] * ss;
            rs[k][p] = rs[k][p] * sc + rc[k][p] * ss;
            rc[k][p] = cn;
          }
        }
      }
    }
  };

  // Packed weight chunks and the fp32 dweight column accumulators live for the whole walk; the
  // row's g and saved chunks stay packed and are decoded once per pass.
  WeightChunk<DT, WDT> wc[NV];
  float acc[NV][V];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c = lt + k * tpr;
    wc[k].load((has_w && c < nchunk) ? a.w : nullptr, (int64_t)c * V);
#pragma unroll
    for (int i = 0; i < V; ++i) acc[k][i] = 0.0f;
  }

  // Loads of one row into (gv, sv, hv, rr); zeros outside the tensor.
  auto load_row = [&](int64_t row, u32x4* gv, u32x4* sv, u32x4* hv, float& rr) {
    const bool ok = row < a.rows;
    rr = ok ? a.inv_rms[row] : 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = lt + k * tpr;
      gv[k] = u32x4{0u, 0u, 0u, 0u};
      sv[k] = u32x4{0u, 0u, 0u, 0u};
      if constexpr (HAS_GH) hv[k] = u32x4{0u, 0u, 0u, 0u};
      if (ok && c < nchunk) {
        gv[k] = load16_stream<DT>(a.g, row * a.ld_g + (int64_t)c * V);
        sv[k] = load16_stream<DT>(a.saved, row * a.ld_s + (int64_t)c * V);
        if constexpr (HAS_GH) hv[k] = load16_stream<DT>(a.gh, row * a.ld_gh + (int64_t)c * V);
      }
    }
  };
  // kRopeDirect: the current row's position, each chunk's first pair frequency (double) and
  // the ratio between consecutive pairs' frequencies, base^(-2/dim)
  int64_t rd_pos = 0;
  double rd_f0[RD ? NV : 1], rd_ratio = 0.0;
  if constexpr (RD) {
    const double cc = (double)a.rope_c_hi + (double)a.rope_c_lo;
    rd_ratio = exp2(-cc);
#pragma unroll
    for (int k = 0; k < NV; ++k) rd_f0[k] = exp2(-(double)((lt + k * tpr) * P) * cc);
  }
  // Decoded chunk k of the current row: g, xhat (h * inv_rms when h was saved), weight.
  auto decode = [&](const u32x4* gv, const u32x4* sv, float rr, int k, float* gf, float* xh,
                    float* wf) {
    C::unpack(gv[k], gf);
    if constexpr (RD) {
      // inverse rotation, each pair's (cos, sin) from its double angle (as rope_cos_sin)
      double f = rd_f0[k];
#pragma unroll
      for (int p = 0; p < P; ++p) {
        float cs, sn;
        rope_cos_sin_f(rd_pos, f, cs, sn);
        f *= rd_ratio;
        const float g0 = gf[2 * p], g1 = gf[2 * p + 1];
        gf[2 * p] = g0 * cs + g1 * sn;
        gf[2 * p + 1] = g1 * cs - g0 * sn;
      }
    }
    if constexpr (ROPE) {
      // inverse rotation of each pair (y0, y1) -> (y0 c + y1 s, y1 c - y0 s)
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const float g0 = gf[2 * p], g1 = gf[2 * p + 1];
        gf[2 * p] = g0 * rc[k][p] + g1 * rs[k][p];
        gf[2 * p + 1] = g1 * rc[k][p] - g0 * rs[k][p];
      }
    }
    C::unpack(sv[k], xh);
    if constexpr (SAVED_IS_H) {
#pragma unroll
      for (int i = 0; i < V; ++i) xh[i] = xh[i] * rr;
    }
    wc[k].unpack(has_w, wf);
  };

  int64_t row = slot;
  u32x4 gv[NV], sv[NV], hv[NH];
  float rr;
  load_row(row, gv, sv, hv, rr);
  int64_t pos = ROPE ? row % a.rope_seq : 0;
  rope_start(pos);

  for (int it = 0; it < a.iters; ++it) {
    const bool ok = row < a.rows;
    if constexpr (RD) rd_pos = row % a.rope_seq;
    const int64_t nrow = row + nslots;
    u32x4 gn[NV], sn[NV], hn[NH];
    float rn = 0.0f;
    if (it + 1 < a.iters) {
      load_row(nrow, gn, sn, hn, rn);
    } else {
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        gn[k] = u32x4{0u, 0u, 0u, 0u};
        sn[k] = u32x4{0u, 0u, 0u, 0u};
        if constexpr (HAS_GH) hn[k] = u32x4{0u, 0u, 0u, 0u};
      }
    }

    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      float gf[V], xh[V], wf[V];
      decode(gv, sv, rr, k, gf, xh, wf);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float gw = gf[i] * wf[i];
        s += gw * xh[i];
      }
    }
    s = row_sum(s, tpr, grp, red[it & 1]);
    const float m = s / (float)a.dim;

#pragma unroll
    for (int k = 0; k < NV; ++k) {
      forget(gv[k]);
      forget(sv[k]);
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = lt + k * tpr;
      float gf[V], xh[V], wf[V];
      decode(gv, sv, rr, k, gf, xh, wf);
      if (ok && c < nchunk) {
        float d[V];
#pragma unroll
        for (int i = 0; i < V; ++i) {
          const float gw = gf[i] * wf[i];
          d[i] = rr * (gw - xh[i] * m);
        }
        if constexpr (HAS_GH) {
          float ghf[V];
          C::unpack(hv[k], ghf);
#pragma unroll
          for (int i = 0; i < V; ++i) d[i] = d[i] + ghf[i];
        }
        const u32x4 pv = C::pack(d);
        store16_stream<DT>(a.dx, row * a.ld_dx + (int64_t)c * V, pv);
        if (has_dres) store16_stream<DT>(a.dres, row * a.ld_dres + (int64_t)c * V, pv);
      }
#pragma unroll
      for (int i = 0; i < V; ++i) acc[k][i] += gf[i] * xh[i];
    }

    if constexpr (ROPE) {
      pos += nslots;
      if (pos >= a.rope_seq) {
        pos = nrow % a.rope_seq;
        rope_start(pos);
      } else if ((it + 1) % kRopeAnchor == 0) {
        rope_start(pos);
      } else {
        rope_step();
      }
    }
    row = nrow;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      gv[k] = gn[k];
      sv[k] = sn[k];
      if constexpr (HAS_GH) hv[k] = hn[k];
    }
    rr = rn;
  }

  if (a.partial == nullptr) return;
  // One fp32 partial row per workgroup.  Row groups are added in group order through LDS
  // (dim floats of dynamic LDS), so the partial does not depend on timing.
  float* prow = a.partial + (int64_t)blockIdx.x * a.dim;
  if (groups == 1) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = lt + k * tpr;
      if (c < nchunk) {
#pragma unroll
        for (int q = 0; q < V / 4; ++q)
          store16<VELOGRAD_DTYPE_F32>(prow, (int64_t)c * V + 4 * q,
                                      Codec<VELOGRAD_DTYPE_F32>::pack(&acc[k][4 * q]));
      }
    }
    return;
  }
  float* comb = dyn_lds;
  if constexpr (ROPE) __syncthreads();  // every thread is done with the step table
  for (int gi = 0; gi < groups; ++gi) {
    if (grp == gi) {
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int c = lt + k * tpr;
        if (c < nchunk) {
#pragma unroll
          for (int i = 0; i < V; ++i)
            comb[c * V + i] = (gi == 0) ? acc[k][i] : comb[c * V + i] + acc[k][i];
        }
      }
    }
    __syncthreads();
  }
  for (int q = threadIdx.x; q < a.dim / 4; q += blockDim.x)
    store16<VELOGRAD_DTYPE_F32>(prow, 4 * (int64_t)q, *reinterpret_cast<const u32x4*>(comb + 4 * q));
}

// ------------------------------------------------------------------------------------------
// Backward, ring-pipelined (launch_plan.h: plan_bwd_ring).  Each row slot walks rows slot,
// slot + S, ... as in bwd_vec_kernel, but keeps a ring of PF + 1 = 3 row buffers (2 with
// grad_h): while a row reduces, the next two rows' loads are in flight.  Rows are of whole
// 16-byte chunks, dim <= NV * tpr * V (kRingTail where lanes are left idle; kRing8 for rows of
// 8-byte alignment with a half chunk at their end), and the steady loop
// covers only iterations in which every slot has a row, loading prefetch rows past the end from
// the last row instead (never used), so it is free of branches around memory operations: the
// wait for a row's data then counts exactly the later loads and stores instead of draining them,
// which a guarded loop forces.  The loop is unrolled by the ring length so the buffers are
// indexed at compile time.  kRingDres: dres is written too.
// ------------------------------------------------------------------------------------------
constexpr int kRingDres = 8;
constexpr int kRingTail = 32;
constexpr int kRing8 = 64;

template <int DT, int WDT, int NV, int FLAGS>
__global__ __launch_bounds__(vg_plan::kRingBlock) void bwd_ring_kernel(const BwdArgs a) {
  using C = Codec<DT>;
  constexpr int V = C::kVec;
  constexpr bool SAVED_IS_H = (FLAGS & kSavedIsH) != 0;
  constexpr bool HAS_GH = (FLAGS & kGradH) != 0;
  constexpr bool HAS_DRES = (FLAGS & kRingDres) != 0;
  // kRingTail: rows of fewer chunks than the row group's lanes (launch_plan.h ring_eligible):
  // an idle lane loads the row's last chunk instead (no branch around the load), adds nothing
  // and stores nothing
  constexpr bool TAIL = (FLAGS & kRingTail) != 0;
  // kRing8: rows of a 2-byte dtype that start on 8-byte boundaries only, dim = n * V + V / 2
  // (hidden sizes such as 4100): each of the n whole chunks moves as two 8-byte halves, and the
  // row's last V / 2 elements form an extra half chunk that lane 0 of the row group owns; every
  // lane of the group loads those same 8 bytes (one request per wave), so no branch guards the
  // load.  The row group is laid out over the n whole chunks.
  constexpr bool X8 = (FLAGS & kRing8) != 0;
  static_assert(!X8 || C::kBytes == 2, "rows of 8-byte alignment are of a 2-byte dtype");
  constexpr int VH = V / 2;
  constexpr int NH = HAS_GH ? NV : 1;  // grad_h chunks (a dummy slot when absent)
  // With grad_h a third stream fills the ring: one row ahead keeps it within 256 VGPRs.
  constexpr int PF = HAS_GH ? 1 : vg_plan::kRingPrefetch;
  constexpr int R = PF + 1;
  constexpr int RX = X8 ? R : 1;  // extra half-chunk buffers (a dummy slot without kRing8)
  static_assert((FLAGS & kRopeG) == 0, "the RoPE gradient runs in bwd_vec_kernel");
  __shared__ float red[2][kMaxWavesPerRow];
  extern __shared__ __align__(16) float dyn_lds[];  // dim floats: the row groups' combine

  const int tpr = a.tpr;
  const int grp = threadIdx.x / tpr;
  const int lt = threadIdx.x - grp * tpr;
  const int groups = blockDim.x / tpr;
  const int64_t slot = (int64_t)blockIdx.x * groups + grp;
  const int64_t nslots = (int64_t)gridDim.x * groups;
  const bool has_w = a.w != nullptr;
  const int64_t last = a.rows - 1;
  // chunk k of this lane (the row's last whole one for an idle lane) and whether it is its own
  const int nfull = a.dim / V;
  int chunk[NV];
  bool own[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c = lt + k * tpr;
    own[k] = !TAIL || c < nfull;
    chunk[k] = own[k] ? c : nfull - 1;
  }
  const int64_t xcol = (int64_t)a.dim - VH;  // kRing8: the extra half chunk's first column
  const bool own_x = X8 && lt == 0;

  WeightChunk<DT, WDT> wc[NV];
  float acc[NV][V];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    wc[k].load(has_w ? a.w : nullptr, (int64_t)chunk[k] * V);
#pragma unroll
    for (int i = 0; i < V; ++i) acc[k][i] = 0.0f;
  }
  float wfx[VH], accx[VH];
  if constexpr (X8) {
#pragma unroll
    for (int i = 0; i < VH; ++i) {
      wfx[i] = 1.0f;
      accx[i] = 0.0f;
    }
    if (has_w) {
      if constexpr (WDT == VELOGRAD_DTYPE_F32) {
        Codec<VELOGRAD_DTYPE_F32>::unpack(load16<VELOGRAD_DTYPE_F32>(a.w, xcol), wfx);
      } else {
        const u32x2 q = *reinterpret_cast<const u32x2*>(static_cast<const char*>(a.w) +
                                                        xcol * Codec<WDT>::kBytes);
        float t[V];
        Codec<WDT>::unpack(u32x4{q.x, q.y, 0u, 0u}, t);
#pragma unroll
        for (int i = 0; i < VH; ++i) wfx[i] = t[i];
      }
    }
  }

  u32x4 gr[R][NV], sr[R][NV], hr[R][NH];
  u32x2 gx[RX][HAS_GH ? 3 : 2];  // kRing8: the extra half chunk's g, saved (and grad_h)
  float rr[R];
  // One chunk of a stream: 16 bytes, or two 8-byte halves for kRing8 rows.
  auto load_chunk = [&](const void* base, int64_t e) -> u32x4 {
    if constexpr (X8) {
      const u32x2 lo = load8_stream<DT>(base, e);
      const u32x2 hi = load8_stream<DT>(base, e + VH);
      return u32x4{lo.x, lo.y, hi.x, hi.y};
    } else {
      return load16_stream<DT>(base, e);
    }
  };
  auto store_chunk = [&](void* base, int64_t e, const u32x4 v) {
    if constexpr (X8) {
      store8_stream<DT>(base, e, u32x2{v.x, v.y});
      store8_stream<DT>(base, e + VH, u32x2{v.z, v.w});
    } else {
      store16_stream<DT>(base, e, v);
    }
  };
  // Row `row`'s g, saved, grad_h chunks and inv_rms; rows past the end read the last row.
  auto load_row = [&](int64_t row, u32x4* gv, u32x4* sv, u32x4* hv, float& r, u32x2* xv) {
    const int64_t rw = row < a.rows ? row : last;
    r = a.inv_rms[rw];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int64_t col = (int64_t)chunk[k] * V;
      gv[k] = load_chunk(a.g, rw * a.ld_g + col);
      sv[k] = load_chunk(a.saved, rw * a.ld_s + col);
      if constexpr (HAS_GH) hv[k] = load_chunk(a.gh, rw * a.ld_gh + col);
    }
    if constexpr (X8) {
      xv[0] = load8_stream<DT>(a.g, rw * a.ld_g + xcol);
      xv[1] = load8_stream<DT>(a.saved, rw * a.ld_s + xcol);
      if constexpr (HAS_GH) xv[2] = load8_stream<DT>(a.gh, rw * a.ld_gh + xcol);
    }
  };
  auto decode = [&](const u32x4* gv, const u32x4* sv, float r, int k, float* gf, float* xh,
                    float* wf) {
    C::unpack(gv[k], gf);
    C::unpack(sv[k], xh);
    if constexpr (SAVED_IS_H) {
#pragma unroll
      for (int i = 0; i < V; ++i) xh[i] = xh[i] * r;
    }
    wc[k].unpack(has_w, wf);
  };
  // The backward of one row (as bwd_vec_kernel's loop body); `ok` = the row exists.  The row's
  // decoded g * w and xhat stay in registers across the reduction (one workgroup per CU leaves
  // 256 VGPRs a lane): decoding them again after it, as bwd_vec_kernel does to save registers,
  // ran 16384 x 4096 bf16 in 69.2 us against 68.5 and 16384 x 5120 in 92.7 against 85.1.
  auto process = [&](u32x4* gv, u32x4* sv, const u32x4* hv, float r, const u32x2* xv,
                     int64_t row, bool ok, int it) {
    float s = 0.0f;
    float gfk[NV][V], xhk[NV][V], gwk[NV][V];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      float wf[V];
      decode(gv, sv, r, k, gfk[k], xhk[k], wf);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        gwk[k][i] = gfk[k][i] * wf[i];
        if constexpr (TAIL) {
          const float t = gwk[k][i] * xhk[k][i];
          s += own[k] ? t : 0.0f;
        } else {
          s += gwk[k][i] * xhk[k][i];
        }
      }
    }
    float gfx[VH], xhx[VH], gwx[VH];
    if constexpr (X8) {
      float t[V];
      C::unpack(u32x4{xv[0].x, xv[0].y, 0u, 0u}, t);
#pragma unroll
      for (int i = 0; i < VH; ++i) gfx[i] = t[i];
      C::unpack(u32x4{xv[1].x, xv[1].y, 0u, 0u}, t);
#pragma unroll
      for (int i = 0; i < VH; ++i) {
        xhx[i] = SAVED_IS_H ? t[i] * r : t[i];
        gwx[i] = gfx[i] * wfx[i];
        const float p = gwx[i] * xhx[i];
        s += own_x ? p : 0.0f;
      }
    }
    s = row_sum(s, tpr, grp, red[it & 1]);
    const float m = s / (float)a.dim;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int64_t col = (int64_t)chunk[k] * V;
      const float* gf = gfk[k];
      const float* xh = xhk[k];
      float d[V];
#pragma unroll
      for (int i = 0; i < V; ++i) d[i] = r * (gwk[k][i] - xh[i] * m);
      if constexpr (HAS_GH) {
        float ghf[V];
        C::unpack(hv[k], ghf);
#pragma unroll
        for (int i = 0; i < V; ++i) d[i] = d[i] + ghf[i];
      }
      const u32x4 pv = C::pack(d);
      const bool store = TAIL ? ok && own[k] : ok;
      if (store) {
        store_chunk(a.dx, row * a.ld_dx + col, pv);
        if constexpr (HAS_DRES) store_chunk(a.dres, row * a.ld_dres + col, pv);
      }
#pragma unroll
      for (int i = 0; i < V; ++i) acc[k][i] += store ? gf[i] * xh[i] : 0.0f;
    }
    if constexpr (X8) {
      float d[V];
#pragma unroll
      for (int i = 0; i < VH; ++i) d[i] = r * (gwx[i] - xhx[i] * m);
#pragma unroll
      for (int i = VH; i < V; ++i) d[i] = 0.0f;
      if constexpr (HAS_GH) {
        float t[V];
        C::unpack(u32x4{xv[2].x, xv[2].y, 0u, 0u}, t);
#pragma unroll
        for (int i = 0; i < VH; ++i) d[i] = d[i] + t[i];
      }
      const u32x4 pv = C::pack(d);
      const bool sx = ok && own_x;
      if (sx) {
        store8_stream<DT>(a.dx, row * a.ld_dx + xcol, u32x2{pv.x, pv.y});
        if constexpr (HAS_DRES)
          store8_stream<DT>(a.dres, row * a.ld_dres + xcol, u32x2{pv.x, pv.y});
      }
#pragma unroll
      for (int i = 0; i < VH; ++i) accx[i] += sx ? gfx[i] * xhx[i] : 0.0f;
    }
  };

  // Row j of the walk sits in buffer j % R; processing row j first issues row j + PF's loads
  // into buffer (j + PF) % R, the one row j - 1 has just released.
  const int full = (int)(a.rows / nslots);  // iterations in which every slot has a row
#pragma unroll
  for (int j = 0; j < PF; ++j)
    load_row(slot + (int64_t)j * nslots, gr[j], sr[j], hr[j], rr[j], gx[X8 ? j : 0]);
  int it = 0;
  for (; it + R <= full; it += R) {
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int nb = (u + PF) % R;
      load_row(slot + (int64_t)(it + u + PF) * nslots, gr[nb], sr[nb], hr[nb], rr[nb],
               gx[X8 ? nb : 0]);
      process(gr[u], sr[u], hr[u], rr[u], gx[X8 ? u : 0], slot + (int64_t)(it + u) * nslots, true,
              it + u);
    }
  }
  // The last (up to R) iterations, some of whose slots may have no row.
#pragma unroll
  for (int u = 0; u < R; ++u) {
    if (it + u < a.iters) {
      const int nb = (u + PF) % R;
      if (it + u + PF < a.iters)
        load_row(slot + (int64_t)(it + u + PF) * nslots, gr[nb], sr[nb], hr[nb], rr[nb],
                 gx[X8 ? nb : 0]);
      const int64_t row = slot + (int64_t)(it + u) * nslots;
      process(gr[u], sr[u], hr[u], rr[u], gx[X8 ? u : 0], row, row < a.rows, it + u);
    }
  }

  if (a.partial == nullptr) return;
  // One fp32 partial row per workgroup; row groups added in group order through LDS.
  float* prow = a.partial + (int64_t)blockIdx.x * a.dim;
  if (groups == 1) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      if (!own[k]) continue;
      const int c = chunk[k];
#pragma unroll
      for (int q = 0; q < V / 4; ++q)
        store16<VELOGRAD_DTYPE_F32>(prow, (int64_t)c * V + 4 * q,
                                    Codec<VELOGRAD_DTYPE_F32>::pack(&acc[k][4 * q]));
    }
    if constexpr (X8) {
      if (own_x) store16<VELOGRAD_DTYPE_F32>(prow, xcol, Codec<VELOGRAD_DTYPE_F32>::pack(accx));
    }
    return;
  }
  float* comb = dyn_lds;
  for (int gi = 0; gi < groups; ++gi) {
    if (grp == gi) {
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        if (!own[k]) continue;
        const int c = chunk[k];
#pragma unroll
        for (int i = 0; i < V; ++i)
          comb[c * V + i] = (gi == 0) ? acc[k][i] : comb[c * V + i] + acc[k][i];
      }
      if constexpr (X8) {
        if (own_x) {
#pragma unroll
          for (int i = 0; i < VH; ++i)
            comb[xcol + i] = (gi == 0) ? accx[i] : comb[xcol + i] + accx[i];
        }
      }
    }
    __syncthreads();
  }
  for (int q = threadIdx.x; q < a.dim / 4; q += blockDim.x)
    store16<VELOGRAD_DTYPE_F32>(prow, 4 * (int64_t)q, *reinterpret_cast<const u32x4*>(comb + 4 * q));
}

// ------------------------------------------------------------------------------------------
// Backward, rows of any length and alignment that bwd_ring_kernel cannot take (odd lengths,
// streams that start anywhere in a 16-byte line), in bwd_ring_kernel's walk and ring
// (launch_plan.h: plan_bwd_ring_elem).  Element-strided lanes: lane lt of a row group holds
// columns lt, lt + tpr, ..., lt + (M - 1) tpr, so each element load or store of a wave moves
// one contiguous run of 64 elements; a column past the row's end loads the row's last element
// (no branch around a load) and adds and stores nothing.  Rows of M * tpr elements at most: M 4
// or 8 (106-232 VGPRs; sixteen spilled 21-258 VGPRs a lane even one row ahead), so rows of up
// to 4096 elements.
// ------------------------------------------------------------------------------------------
template <int DT, int WDT, int M, int FLAGS>
__global__ __launch_bounds__(vg_plan::kRingBlock) void bwd_ring_elem_kernel(const BwdArgs a) {
  using C = Codec<DT>;
  using Raw = std::conditional_t<C::kBytes == 2, uint16_t, uint32_t>;
  constexpr bool SAVED_IS_H = (FLAGS & kSavedIsH) != 0;
  constexpr bool HAS_GH = (FLAGS & kGradH) != 0;
  constexpr bool HAS_DRES = (FLAGS & kRingDres) != 0;
  constexpr int MH = HAS_GH ? M : 1;  // grad_h elements (a dummy slot when absent)
  constexpr int PF = HAS_GH ? 1 : vg_plan::kRingPrefetch;
  constexpr int R = PF + 1;
  static_assert((FLAGS & (kRopeG | kRingTail | kRing8)) == 0, "plain rows only");
  static_assert(M == 4 || M == 8, "sixteen elements a lane spill past 256 VGPRs");
  __shared__ float red[2][kMaxWavesPerRow];
  extern __shared__ __align__(16) float dyn_lds[];  // dim floats: the row groups' combine

  const int tpr = a.tpr;
  const int grp = threadIdx.x / tpr;
  const int lt = threadIdx.x - grp * tpr;
  const int groups = blockDim.x / tpr;
  const int64_t slot = (int64_t)blockIdx.x * groups + grp;
  const int64_t nslots = (int64_t)gridDim.x * groups;
  const bool has_w = a.w != nullptr;
  const int64_t last = a.rows - 1;
  // column m of this lane (the row's last one past its end) and whether it is the lane's own
  int col[M];
  bool own[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int c = lt + m * tpr;
    own[m] = c < a.dim;
    col[m] = own[m] ? c : a.dim - 1;
  }
  float wf[M], acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    wf[m] = has_w ? Codec<WDT>::load1(a.w, col[m]) : 1.0f;
    acc[m] = 0.0f;
  }
  auto load_raw = [&](const void* base, int64_t i) -> uint32_t {
    return (uint32_t)__builtin_nontemporal_load(static_cast<const Raw*>(base) + i);
  };
  auto decode = [&](uint32_t u) -> float {
    if constexpr (DT == VELOGRAD_DTYPE_BF16) {
      return __builtin_bit_cast(float, u << 16);
    } else if constexpr (DT == VELOGRAD_DTYPE_F16) {
      return (float)__builtin_bit_cast(_Float16, (uint16_t)u);
    } else {
      return __builtin_bit_cast(float, u);
    }
  };
  auto store_one = [&](void* base, int64_t i, float f) {
    Raw v;
    if constexpr (DT == VELOGRAD_DTYPE_BF16) v = __builtin_bit_cast(uint16_t, (__bf16)f);
    else if constexpr (DT == VELOGRAD_DTYPE_F16) v = __builtin_bit_cast(uint16_t, (_Float16)f);
    else v = __builtin_bit_cast(uint32_t, f);
    __builtin_nontemporal_store(v, static_cast<Raw*>(base) + i);
  };

  uint32_t gr[R][M], sr[R][M], hr[R][MH];
  float rr[R];
  // Row `row`'s g, saved, grad_h elements and inv_rms; rows past the end read the last row.
  auto load_row = [&](int64_t row, uint32_t* gv, uint32_t* sv, uint32_t* hv, float& r) {
    const int64_t rw = row < a.rows ? row : last;
    r = a.inv_rms[rw];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      gv[m] = load_raw(a.g, rw * a.ld_g + col[m]);
      sv[m] = load_raw(a.saved, rw * a.ld_s + col[m]);
      if constexpr (HAS_GH) hv[m] = load_raw(a.gh, rw * a.ld_gh + col[m]);
    }
  };
  // The backward of one row (bwd_ring_kernel's, element by element); `ok` = the row exists.
  auto process = [&](const uint32_t* gv, const uint32_t* sv, const uint32_t* hv, float r,
                     int64_t row, bool ok, int it) {
    float gf[M], xh[M], gw[M];
    float s = 0.0f;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      gf[m] = decode(gv[m]);
      xh[m] = decode(sv[m]);
      if constexpr (SAVED_IS_H) xh[m] = xh[m] * r;
      gw[m] = gf[m] * wf[m];
      const float t = gw[m] * xh[m];
      s += own[m] ? t : 0.0f;
    }
    s = row_sum(s, tpr, grp, red[it & 1]);
    const float mean = s / (float)a.dim;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float d = r * (gw[m] - xh[m] * mean);
      if constexpr (HAS_GH) d = d + decode(hv[m]);
      const bool store = ok && own[m];
      if (store) {
        store_one(a.dx, row * a.ld_dx + col[m], d);
        if constexpr (HAS_DRES) store_one(a.dres, row * a.ld_dres + col[m], d);
      }
      acc[m] += store ? gf[m] * xh[m] : 0.0f;
    }
  };

  // The walk and ring of bwd_ring_kernel.
  const int full = (int)(a.rows / nslots);
#pragma unroll
  for (int j = 0; j < PF; ++j) load_row(slot + (int64_t)j * nslots, gr[j], sr[j], hr[j], rr[j]);
  int it = 0;
  for (; it + R <= full; it += R) {
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int nb = (u + PF) % R;
      load_row(slot + (int64_t)(it + u + PF) * nslots, gr[nb], sr[nb], hr[nb], rr[nb]);
      process(gr[u], sr[u], hr[u], rr[u], slot + (int64_t)(it + u) * nslots, true, it + u);
    }
  }
#pragma unroll
  for (int u = 0; u < R; ++u) {
    if (it + u < a.iters) {
      const int nb = (u + PF) % R;
      if (it + u + PF < a.iters)
        load_row(slot + (int64_t)(it + u + PF) * nslots, gr[nb], sr[nb], hr[nb], rr[nb]);
      const int64_t row = slot + (int64_t)(it + u) * nslots;
      process(gr[u], sr[u], hr[u], rr[u], row, row < a.rows, it + u);
    }
  }

  if (a.partial == nullptr) return;
  // One fp32 partial row per workgroup; row groups added in group order through LDS.
  float* prow = a.partial + (int64_t)blockIdx.x * a.dim;
  if (groups == 1) {
#pragma unroll
    for (int m = 0; m < M; ++m)
      if (own[m]) prow[col[m]] = acc[m];
    return;
  }
  float* comb = dyn_lds;
  for (int gi = 0; gi < groups; ++gi) {
    if (grp == gi) {
#pragma unroll
      for (int m = 0; m < M; ++m)
        if (own[m]) comb[col[m]] = (gi == 0) ? acc[m] : comb[col[m]] + acc[m];
    }
    __syncthreads();
  }
  for (int q = threadIdx.x; q < a.dim; q += blockDim.x) prow[q] = comb[q];
}

// ------------------------------------------------------------------------------------------
// Backward with the fused RoPE gradient, ring-pipelined (launch_plan.h: plan_bwd_rope_ring):
// whole rows of NV (1 or 2) 16-byte chunks per thread, the saved tensor h, no grad_h or dres (the
// module's backward).  The walk, ring and steady loop are bwd_ring_kernel's: slot s walks rows
// s, s + S, ... (S slots), three row buffers, rows past the end read the last row, no branch
// around a memory operation in the steady loop.  Each thread keeps the rotation (cos, sin) of
// its pairs at the current row's position in float32 and advances it by S positions per row with
// the rotation through S * freq_j (formed in double once per walk, rounded to float).  Where a
// walk crosses the end of a sequence, S is a multiple or a divisor of rope_seq (rope_walk_ok: the
// host plans this kernel only then, or when no walk reaches a sequence end), so the position
// returns to the walk's first one and the rotation to its first value (kept in LDS with one
// chunk per thread, evaluated afresh with two); a walk that goes kRopeAnchorRows rows without
// such a return evaluates its angles afresh (double angle, exact reduction, float sincospi), so
// no state is more than kRopeAnchorRows - 1 float steps from an exact value (about 3 * 2^-24 of
// the pair per step).  The row group is a whole number of waves, so slots, rows and positions are
// wave-uniform and the walk's bookkeeping is scalar.  The walk is bound by its vector
// instructions as much as by HBM, so the row's decoded, rotated chunks stay in registers across
// the reduction, the weight is decoded once, sums of products use fused multiply-adds, and for a
// power-of-two dim the mean is s * (1 / dim), exact.  One chunk per thread runs within 128 VGPRs
// (two workgroups of fewer than 512 threads fit a CU); two chunks per thread, one workgroup per
// CU, within 256.
// ------------------------------------------------------------------------------------------
template <int DT, int WDT, int NV>
__global__ __launch_bounds__(vg_plan::kRingBlock, NV == 1 ? 4 : 2) void bwd_rope_ring_kernel(
    const BwdArgs a) {
  using C = Codec<DT>;
  constexpr int V = C::kVec;
  constexpr int P = V / 2;    // RoPE pairs per chunk
  constexpr int NP = NV * P;  // RoPE pairs per thread: pair e = k * P + q of chunk lt + k * tpr
  // One chunk per thread keeps its pair frequencies and first rotations in LDS; with two, they
  // would not fit 64 KiB beside the step rotations, so the frequencies are formed again where
  // the angles are evaluated and the first rotation is evaluated afresh at a return.
  constexpr bool kTablesInLds = NV == 1;
  constexpr int PF = vg_plan::kRingPrefetch;
  constexpr int R = PF + 1;
  constexpr int kRopeAnchorRows = 16;
  static_assert(NV == 1 || NV == 2, "the RoPE ring takes one or two chunks per thread");
  __shared__ float red[2][kMaxWavesPerRow];
  // Dynamic LDS, pair-major so a wave reads consecutive 8-byte entries: with one chunk per thread
  // each thread's pair frequencies (doubles), then step and first rotations (float pairs); with
  // two, the step rotations only; then with several row groups dim floats for their combine
  // (plan_bwd_rope_ring's lds_bytes).
  extern __shared__ __align__(16) float dyn_lds[];

  const int tpr = a.tpr;
  const int grp = __builtin_amdgcn_readfirstlane((int)threadIdx.x / tpr);
  const int lt = threadIdx.x - grp * tpr;
  const int groups = blockDim.x / tpr;
  const int64_t slot = (int64_t)blockIdx.x * groups + grp;
  const int64_t S = (int64_t)gridDim.x * groups;
  const int64_t last = a.rows - 1;
  const int64_t seq = a.rope_seq;
  const int64_t pos0 = slot % seq;
  const int bd = blockDim.x;
  const int tid = threadIdx.x;
  double* freq_lds = reinterpret_cast<double*>(dyn_lds);  // [P][bd], one chunk per thread
  float2* step_lds = kTablesInLds ? reinterpret_cast<float2*>(freq_lds + P * bd)
                                  : reinterpret_cast<float2*>(dyn_lds);  // [NP][bd]
  float2* first_lds = step_lds + NP * bd;  // [P][bd], one chunk per thread
  float* comb = reinterpret_cast<float*>(kTablesInLds ? first_lds + P * bd : first_lds);
  // 1 / dim is exact for a power of two, so s * (1 / dim) has the bits of s / dim
  const bool dim_pow2 = (a.dim & (a.dim - 1)) == 0;
  const float inv_dim = 1.0f / (float)a.dim;
  auto col_of = [&](int k) { return (int64_t)(lt + k * tpr) * V; };
  // pair e's frequency: base^(-2i/dim), i its pair index in the row
  auto freq_of = [&](int e) {
    if constexpr (kTablesInLds) return freq_lds[e * bd + tid];
    else return rope_freq((lt + (e / P) * tpr) * P + e % P, a.rope_c_hi, a.rope_c_lo);
  };

  float wf[NV][V], acc[NV][V];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    WeightChunk<DT, WDT> wc;
    wc.load(a.w, col_of(k));
    wc.unpack(a.w != nullptr, wf[k]);
#pragma unroll
    for (int i = 0; i < V; ++i) acc[k][i] = 0.0f;
  }
  // one pair at a time (a double sincos holds many registers; the walk needs them)
#pragma unroll 1
  for (int e = 0; e < NP; ++e) {
    const double f = rope_freq((lt + (e / P) * tpr) * P + e % P, a.rope_c_hi, a.rope_c_lo);
    double sv, cv;
    sincos((double)S * f, &sv, &cv);
    step_lds[e * bd + tid] = float2{(float)cv, (float)sv};
    if constexpr (kTablesInLds) {
      freq_lds[e * bd + tid] = f;
      // the rotation at the walk's first position: double angle, reduced exactly, float sincospi
      const double rev = (double)pos0 * f * kInv2PiD;
      float s0, c0;
      sincospif(2.0f * (float)(rev - rint(rev)), &s0, &c0);
      first_lds[e * bd + tid] = float2{c0, s0};
    }
  }
  float cr[NP], sr[NP];
  // the rotations at position p evaluated afresh: double angle, exact reduction, float sincospi
  auto evaluate_at = [&](int64_t p) {
#pragma unroll
    for (int e = 0; e < NP; ++e) {
      const double rev = (double)p * freq_of(e) * kInv2PiD;
      sincospif(2.0f * (float)(rev - rint(rev)), &sr[e], &cr[e]);
    }
  };
  auto restore_first = [&]() {
    if constexpr (kTablesInLds) {
#pragma unroll
      for (int e = 0; e < NP; ++e) {
        const float2 f0 = first_lds[e * bd + tid];
        cr[e] = f0.x;
        sr[e] = f0.y;
      }
    } else {
      evaluate_at(pos0);
    }
  };
  restore_first();
  int64_t pos = pos0;
  int since = 0;  // float steps taken since the state was last exact

  u32x4 gr[R][NV], hr[R][NV];
  float rr[R];
  // Row `row`'s grad_y and h chunks and inv_rms; rows past the end read the last row.
  auto load_row = [&](int64_t row, u32x4* gv, u32x4* hv, float& r) {
    const int64_t rw = row < a.rows ? row : last;
    r = a.inv_rms[rw];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      gv[k] = load16_stream<DT>(a.g, rw * a.ld_g + col_of(k));
      hv[k] = load16_stream<DT>(a.saved, rw * a.ld_s + col_of(k));
    }
  };
  // The backward of one row (bwd_vec_kernel's with kSavedIsH | kRopeG); `ok` = the row exists.
  auto process = [&](const u32x4* gv, const u32x4* hv, float r, int64_t row, bool ok, int it) {
    float gf[NV][V], xh[NV][V];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      C::unpack(gv[k], gf[k]);
      // inverse rotation of each pair (y0, y1) -> (y0 c + y1 s, y1 c - y0 s)
#pragma unroll
      for (int q = 0; q < P; ++q) {
        const float c = cr[k * P + q], sn = sr[k * P + q];
        const float g0 = gf[k][2 * q], g1 = gf[k][2 * q + 1];
        gf[k][2 * q] = __builtin_fmaf(g0, c, g1 * sn);
        gf[k][2 * q + 1] = __builtin_fmaf(g1, c, -(g0 * sn));
      }
      C::unpack(hv[k], xh[k]);
#pragma unroll
      for (int i = 0; i < V; ++i) xh[k][i] = xh[k][i] * r;
#pragma unroll
      for (int i = 0; i < V; ++i) s = __builtin_fmaf(gf[k][i] * wf[k][i], xh[k][i], s);
    }
    s = row_sum(s, tpr, grp, red[it & 1]);
    const float m = dim_pow2 ? s * inv_dim : s / (float)a.dim;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      float d[V];
#pragma unroll
      for (int i = 0; i < V; ++i) d[i] = r * __builtin_fmaf(-xh[k][i], m, gf[k][i] * wf[k][i]);
      if (ok) store16_stream<DT>(a.dx, row * a.ld_dx + col_of(k), C::pack(d));
#pragma unroll
      for (int i = 0; i < V; ++i) {
        acc[k][i] = ok ? __builtin_fmaf(gf[k][i], xh[k][i], acc[k][i]) : acc[k][i];
        // the row's sums are done here: its g and xhat are not held into the next row
        asm volatile("" : "+v"(acc[k][i]));
      }
    }
    // the next row's angles: the walk's first position again, evaluated afresh after
    // kRopeAnchorRows - 1 steps, or one float step of S positions on (each thread reads only the
    // LDS entries it wrote, in program order: no barrier)
    pos += S;
    ++since;
    if (pos >= seq) {
      pos = pos0;
      since = 0;
      restore_first();
    } else if (since == kRopeAnchorRows) {
      since = 0;
      evaluate_at(pos);
    } else {
#pragma unroll
      for (int e = 0; e < NP; ++e) {
        const float2 st = step_lds[e * bd + tid];
        const float cn = __builtin_fmaf(cr[e], st.x, -(sr[e] * st.y));
        sr[e] = __builtin_fmaf(sr[e], st.x, cr[e] * st.y);
        cr[e] = cn;
      }
    }
  };

  // Row j of the walk sits in buffer j % R; processing row j first issues row j + PF's loads
  // into buffer (j + PF) % R, the one row j - 1 has just released.
  const int full = (int)(a.rows / S);  // iterations in which every slot has a row
#pragma unroll
  for (int j = 0; j < PF; ++j) load_row(slot + (int64_t)j * S, gr[j], hr[j], rr[j]);
  int it = 0;
  for (; it + R <= full; it += R) {
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int nb = (u + PF) % R;
      load_row(slot + (int64_t)(it + u + PF) * S, gr[nb], hr[nb], rr[nb]);
      process(gr[u], hr[u], rr[u], slot + (int64_t)(it + u) * S, true, it + u);
    }
  }
  // The last (up to R) iterations, some of whose slots may have no row.
#pragma unroll
  for (int u = 0; u < R; ++u) {
    if (it + u < a.iters) {
      const int nb = (u + PF) % R;
      if (it + u + PF < a.iters)
        load_row(slot + (int64_t)(it + u + PF) * S, gr[nb], hr[nb], rr[nb]);
      const int64_t row = slot + (int64_t)(it + u) * S;
      process(gr[u], hr[u], rr[u], row, row < a.rows, it + u);
    }
  }

  if (a.partial == nullptr) return;
  // One fp32 partial row per workgroup; row groups added in group order through LDS.
  float* prow = a.partial + (int64_t)blockIdx.x * a.dim;
  if (groups == 1) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
#pragma unroll
      for (int q = 0; q < V / 4; ++q)
        store16<VELOGRAD_DTYPE_F32>(prow, col_of(k) + 4 * q,
                                    Codec<VELOGRAD_DTYPE_F32>::pack(&acc[k][4 * q]));
    }
    return;
  }
  for (int gi = 0; gi < groups; ++gi) {
    if (grp == gi) {
#pragma unroll
      for (int k = 0; k < NV; ++k) {
#pragma unroll
        for (int i = 0; i < V; ++i)
          comb[col_of(k) + i] = (gi == 0) ? acc[k][i] : comb[col_of(k) + i] + acc[k][i];
      }
    }
    __syncthreads();
  }
  for (int q = threadIdx.x; q < a.dim / 4; q += blockDim.x)
    store16<VELOGRAD_DTYPE_F32>(prow, 4 * (int64_t)q, *reinterpret_cast<const u32x4*>(comb + 4 * q));
}

// ------------------------------------------------------------------------------------------
// Backward, any dim / alignment: one row slot per workgroup, two passes per row; the slot's
// dweight partial row is accumulated in place (each column owned by one thread).
// ------------------------------------------------------------------------------------------
template <int DT, int WDT, int FLAGS>
__global__ __launch_bounds__(kGenericBlock) void bwd_generic_kernel(const BwdArgs a) {
  using C = Codec<DT>;
  using CW = Codec<WDT>;
  constexpr bool SAVED_IS_H = (FLAGS & kSavedIsH) != 0;
  constexpr bool HAS_GH = (FLAGS & kGradH) != 0;
  constexpr bool ROPE = (FLAGS & kRopeG) != 0;
  __shared__ float red[2][kGenericBlock / kWave];
  // The dweight columns of the slot's rows, summed in row order: in dynamic LDS (dim floats)
  // where the launch gave it (vg_plan::generic_bwd_lds_bytes), else in the slot's partial row
  // in global memory, each column then always touched by the same thread.
  extern __shared__ __align__(16) float acc_lds[];
  const int64_t slot = blockIdx.x;
  const int64_t nslots = gridDim.x;
  const bool has_w = a.w != nullptr;
  const bool has_dres = a.dres != nullptr;
  float* prow = a.partial != nullptr ? a.partial + slot * (int64_t)a.dim : nullptr;
  const bool acc_in_lds = vg_plan::generic_bwd_lds_bytes(a.dim, prow != nullptr) != 0;
  auto accumulate = [&](int j, float p, int it) {
    if (acc_in_lds) acc_lds[j] = (it == 0) ? p : acc_lds[j] + p;
    else prow[j] = (it == 0) ? p : prow[j] + p;
  };
  // the 16-byte middle of a row (see fwd_generic_kernel) moves a column between threads from
  // row to row, so it needs the LDS sums when dweight is requested
  const bool body_allowed = !ROPE && (prow == nullptr || acc_in_lds);

  for (int it = 0; it < a.iters; ++it) {
    const int64_t row = slot + (int64_t)it * nslots;
    if (row >= a.rows) break;  // uniform across the workgroup
    const float rr = a.inv_rms[row];
    // element j's contributions given its (rotated-back) gradient gf: to the row sum, then to
    // dx, dres and the partial row
    auto xh_at = [&](int j) {
      float xh = C::load1(a.saved, row * a.ld_s + j);
      if constexpr (SAVED_IS_H) xh = xh * rr;
      return xh;
    };
    auto sum_term = [&](int j, float gf) {
      const float gw = has_w ? gf * CW::load1(a.w, j) : gf;
      return gw * xh_at(j);
    };
    auto finish = [&](int j, float gf, float m) {
      const float xh = xh_at(j);
      const float gw = has_w ? gf * CW::load1(a.w, j) : gf;
      float d = rr * (gw - xh * m);
      if constexpr (HAS_GH) d = d + C::load1(a.gh, row * a.ld_gh + j);
      C::store1(a.dx, row * a.ld_dx + j, d);
      if (has_dres) C::store1(a.dres, row * a.ld_dres + j, d);
      if (prow != nullptr) accumulate(j, gf * xh, it);
    };
    float s = 0.0f;
    if constexpr (ROPE) {
      // one rotation per pair (y0, y1) -> (y0 c + y1 s, y1 c - y0 s) and pass
      const int64_t pos = row % a.rope_seq;
      const int half = a.dim / 2;
      auto grad_pair = [&](int i, double fr, float& g0, float& g1) {
        float c, sn;
        rope_cos_sin_f(pos, fr, c, sn);
        const float y0 = C::load1(a.g, row * a.ld_g + 2 * i);
        const float y1 = C::load1(a.g, row * a.ld_g + 2 * i + 1);
        g0 = y0 * c + y1 * sn;
        g1 = y1 * c - y0 * sn;
      };
      RopeFreqWalk fw(threadIdx.x, blockDim.x, a.rope_c_hi, a.rope_c_lo);
      for (int i = threadIdx.x; i < half; i += blockDim.x) {
        float g0, g1;
        grad_pair(i, fw.next(), g0, g1);
        s += sum_term(2 * i, g0);
        s += sum_term(2 * i + 1, g1);
      }
      s = row_sum(s, blockDim.x, 0, red[it & 1]);
      const float m = s / (float)a.dim;
      RopeFreqWalk fw2(threadIdx.x, blockDim.x, a.rope_c_hi, a.rope_c_lo);
      for (int i = threadIdx.x; i < half; i += blockDim.x) {
        float g0, g1;
        grad_pair(i, fw2.next(), g0, g1);
        finish(2 * i, g0, m);
        finish(2 * i + 1, g1, m);
      }
    } else {
      int head = a.dim, nbody = 0;
      if (body_allowed) {
        const uintptr_t mis = row_offset16(a.g, row * a.ld_g, C::kBytes);
        if (mis % C::kBytes == 0 && row_offset16(a.saved, row * a.ld_s, C::kBytes) == mis &&
            row_offset16(a.dx, row * a.ld_dx, C::kBytes) == mis &&
            (!has_dres || row_offset16(a.dres, row * a.ld_dres, C::kBytes) == mis) &&
            (!HAS_GH || row_offset16(a.gh, row * a.ld_gh, C::kBytes) == mis)) {
          head = (int)(((16 - mis) & 15) / C::kBytes);
          if (head > a.dim) head = a.dim;
          nbody = (a.dim - head) / C::kVec;
        }
      }
      const int tail = head + nbody * C::kVec;
      const int nscalar = a.dim - nbody * C::kVec;
      auto scalar_j = [&](int t) { return t < head ? t : tail + (t - head); };
      const uintptr_t w_align = has_w ? row_offset16(a.w, head, CW::kBytes) : 0;
      // A thread's first KR body chunks of g and the saved tensor stay in registers from the
      // first pass to the second (rows of up to KR * 256 chunks read once); chunks past them
      // are read in the first pass with the normal cache policy and again, non-temporally,
      // in the second (normally from L2).
      constexpr int KR = 4;
      // (grad_h's register chunks too, loaded with them: its loads in the second pass, after
      // the row reduction, cost a memory wait per row)
      u32x4 gk[KR], sk[KR], hk[HAS_GH ? KR : 1];
#pragma unroll
      for (int k = 0; k < KR; ++k) {
        const int c = threadIdx.x + k * blockDim.x;
        gk[k] = u32x4{0u, 0u, 0u, 0u};
        sk[k] = u32x4{0u, 0u, 0u, 0u};
        if constexpr (HAS_GH) hk[k] = u32x4{0u, 0u, 0u, 0u};
        if (c < nbody) {
          const int64_t j = head + (int64_t)c * C::kVec;
          gk[k] = load16_stream<DT>(a.g, row * a.ld_g + j);
          sk[k] = load16_stream<DT>(a.saved, row * a.ld_s + j);
          if constexpr (HAS_GH) hk[k] = load16_stream<DT>(a.gh, row * a.ld_gh + j);
        }
      }
      // With a body, the head and tail are fewer than two chunks' worth of elements (one per
      // thread at most): loaded with the body chunks, so a row waits for memory once per pass
      // instead of three times.
      const bool few_scalar = nbody > 0;
      int j_s = 0;
      float g_s = 0.0f, x_s = 0.0f, w_s = 1.0f;
      float gh_s = 0.0f;
      if (few_scalar && (int)threadIdx.x < nscalar) {
        j_s = scalar_j(threadIdx.x);
        g_s = C::load1(a.g, row * a.ld_g + j_s);
        x_s = C::load1(a.saved, row * a.ld_s + j_s);
        if (has_w) w_s = CW::load1(a.w, j_s);
        if constexpr (HAS_GH) gh_s = C::load1(a.gh, row * a.ld_gh + j_s);
        if constexpr (SAVED_IS_H) x_s = x_s * rr;
      }
      // the body chunk at element j: g and x-hat decoded, g * w formed as sum_term and finish do
      auto body_chunk = [&](const u32x4& gq, const u32x4& sq, int64_t j, float* gf, float* gw,
                            float* xh) {
        C::unpack(gq, gf);
        C::unpack(sq, xh);
        float wf[C::kVec];
        if (has_w) weight_run<DT, WDT>(a.w, j, w_align, wf);
#pragma unroll
        for (int i = 0; i < C::kVec; ++i) {
          if constexpr (SAVED_IS_H) xh[i] = xh[i] * rr;
          gw[i] = has_w ? gf[i] * wf[i] : gf[i];
        }
      };
#pragma unroll
      for (int k = 0; k < KR; ++k) {
        const int c = threadIdx.x + k * blockDim.x;
        if (c < nbody) {
          float gf[C::kVec], gw[C::kVec], xh[C::kVec];
          body_chunk(gk[k], sk[k], head + (int64_t)c * C::kVec, gf, gw, xh);
#pragma unroll
          for (int i = 0; i < C::kVec; ++i) s += gw[i] * xh[i];
        }
      }
      for (int c = threadIdx.x + KR * blockDim.x; c < nbody; c += blockDim.x) {
        const int64_t j = head + (int64_t)c * C::kVec;
        float gf[C::kVec], gw[C::kVec], xh[C::kVec];
        body_chunk(load16<DT>(a.g, row * a.ld_g + j), load16<DT>(a.saved, row * a.ld_s + j), j,
                   gf, gw, xh);
#pragma unroll
        for (int i = 0; i < C::kVec; ++i) s += gw[i] * xh[i];
      }
      if (few_scalar) {
        if ((int)threadIdx.x < nscalar) s += (has_w ? g_s * w_s : g_s) * x_s;
      } else {
        for (int t = threadIdx.x; t < nscalar; t += blockDim.x) {
          const int j = scalar_j(t);
          s += sum_term(j, C::load1(a.g, row * a.ld_g + j));
        }
      }
      s = row_sum(s, blockDim.x, 0, red[it & 1]);
      const float m = s / (float)a.dim;
      // dx of a body chunk, its stores and its dweight terms
      // `ghq`: the chunk's grad_h when it is already in registers, else null (loaded here)
      auto finish_chunk = [&](int64_t j, const float* gf, const float* gw, const float* xh,
                              const u32x4* ghq) {
        float d[C::kVec];
#pragma unroll
        for (int i = 0; i < C::kVec; ++i) d[i] = rr * (gw[i] - xh[i] * m);
        if constexpr (HAS_GH) {
          float ghf[C::kVec];
          C::unpack(ghq != nullptr ? *ghq : load16_stream<DT>(a.gh, row * a.ld_gh + j), ghf);
#pragma unroll
          for (int i = 0; i < C::kVec; ++i) d[i] = d[i] + ghf[i];
        }
        const u32x4 pk = C::pack(d);
        store16_stream<DT>(a.dx, row * a.ld_dx + j, pk);
        if (has_dres) store16_stream<DT>(a.dres, row * a.ld_dres + j, pk);
        if (prow != nullptr) {
          float pv[C::kVec];
#pragma unroll
          for (int i = 0; i < C::kVec; ++i) pv[i] = gf[i] * xh[i];
          // the widest LDS accesses the chunk's first column allows: the dweight reduction costs
          // 11.9 / 13.8 / 27.0 us at 16384 x 4100 / 4102 / 4099 bf16, whose chunks start 16-byte
          // / 8-byte / any aligned in LDS; one word per element in a layout that spreads a
          // chunk's columns across lanes (no bank conflicts, 8 accesses a chunk) cost ~25 us at
          // all three
          if (acc_in_lds && (j & 3) == 0) {
            float4* a4 = reinterpret_cast<float4*>(acc_lds + j);
#pragma unroll
            for (int q = 0; q < C::kVec / 4; ++q) {
              const float4 pq = {pv[4 * q], pv[4 * q + 1], pv[4 * q + 2], pv[4 * q + 3]};
              a4[q] = (it == 0) ? pq : a4[q] + pq;
            }
          } else if (acc_in_lds && (j & 1) == 0) {
            float2* a2 = reinterpret_cast<float2*>(acc_lds + j);
#pragma unroll
            for (int q = 0; q < C::kVec / 2; ++q) {
              const float2 pq = {pv[2 * q], pv[2 * q + 1]};
              a2[q] = (it == 0) ? pq : a2[q] + pq;
            }
          } else {
#pragma unroll
            for (int i = 0; i < C::kVec; ++i) accumulate((int)j + i, pv[i], it);
          }
        }
      };
#pragma unroll
      for (int k = 0; k < KR; ++k) {
        const int c = threadIdx.x + k * blockDim.x;
        if (c < nbody) {
          const int64_t j = head + (int64_t)c * C::kVec;
          float gf[C::kVec], gw[C::kVec], xh[C::kVec];
          body_chunk(gk[k], sk[k], j, gf, gw, xh);
          finish_chunk(j, gf, gw, xh, HAS_GH ? &hk[k] : nullptr);
        }
      }
      for (int c = threadIdx.x + KR * blockDim.x; c < nbody; c += blockDim.x) {
        const int64_t j = head + (int64_t)c * C::kVec;
        float gf[C::kVec], gw[C::kVec], xh[C::kVec];
        body_chunk(load16_stream<DT>(a.g, row * a.ld_g + j),
                   load16_stream<DT>(a.saved, row * a.ld_s + j), j, gf, gw, xh);
        finish_chunk(j, gf, gw, xh, nullptr);
      }
      if (few_scalar) {
        if ((int)threadIdx.x < nscalar) {
          // finish's arithmetic on the register copies
          const float gw = has_w ? g_s * w_s : g_s;
          float d = rr * (gw - x_s * m);
          if constexpr (HAS_GH) d = d + gh_s;
          C::store1(a.dx, row * a.ld_dx + j_s, d);
          if (has_dres) C::store1(a.dres, row * a.ld_dres + j_s, d);
          if (prow != nullptr) accumulate(j_s, g_s * x_s, it);
        }
      } else {
        for (int t = threadIdx.x; t < nscalar; t += blockDim.x) {
          const int j = scalar_j(t);
          finish(j, C::load1(a.g, row * a.ld_g + j), m);
        }
      }
    }
  }
  if (acc_in_lds) {
    __syncthreads();
    for (int j = threadIdx.x; j < a.dim; j += blockDim.x) prow[j] = acc_lds[j];
  }
}

// ------------------------------------------------------------------------------------------
// dweight stage 2: dweight[j] = sum over partial rows p = 0..nparts-1, in a fixed order.
// A workgroup owns 64 columns; wave w sums rows p = w, w + W, ... and the W wave sums are
// added in wave order.
// ------------------------------------------------------------------------------------------
constexpr int kReduceBlock = 1024;
__global__ __launch_bounds__(kReduceBlock) void dweight_reduce_kernel(const float* partial,
                                                                       int32_t nparts,
                                                                       int32_t dim,
                                                                       float* dweight) {
  __shared__ float red[kReduceBlock / kWave][kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  const int col = blockIdx.x * kWave + lane;
  float s = 0.0f;
  if (col < dim) {
    // Batches of 16 loads in flight per lane (one HBM round trip for the usual 256 partial rows
    // over 16 waves); the additions keep ascending p order.
    constexpr int kBatch = 16;
    int p = wave;
    for (; p + (kBatch - 1) * nw < nparts; p += kBatch * nw) {
      float v[kBatch];
#pragma unroll
      for (int b = 0; b < kBatch; ++b) v[b] = partial[(int64_t)(p + b * nw) * dim + col];
#pragma unroll
      for (int b = 0; b < kBatch; ++b) s += v[b];
    }
    for (; p < nparts; p += nw) s += partial[(int64_t)p * dim + col];
  }
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && col < dim) {
    float t = red[0][lane];
    for (int w = 1; w < nw; ++w) t += red[w][lane];
    dweight[col] = t;
  }
}

// Launch-shape knobs, read once per process from the environment (for tuning sweeps; the
// defaults are the measured best on MI355X).  Results do not depend on them except through the
// dweight summation order, which stays fixed for a given setting.
struct Tuning {
  int fwd_nv;             // preferred 16-byte chunks per thread, forward (0 = automatic)
  int bwd_nv;             // same, backward
  int bwd_waves_per_cu;   // resident waves per CU targeted by the persistent backward grid
  int bwd_block;          // upper bound on backward workgroup size (row groups per workgroup)
  int bwd_ring;           // 1: the ring-pipelined backward where the rows suit it
  int ring_block;         // upper bound on the ring backward's workgroup size
  int ring_wgs_per_cu;    // ring backward workgroups per CU (1 or 2)
  int fwd_elem;           // 1: the element-strided forward where the chunked kernels cannot go
};

const Tuning& tuning() {
  static const Tuning t = {
      env_int("VELOGRAD_FWD_NV", 0, 0, kMaxNV),
      env_int("VELOGRAD_BWD_NV", 0, 0, kMaxNV),
      env_int("VELOGRAD_BWD_WAVES_PER_CU", 16, 1, 64),
      env_int("VELOGRAD_BWD_BLOCK", 1024, 64, 1024),
      env_int("VELOGRAD_BWD_RING", 1, 0, 1),
      env_int("VELOGRAD_BWD_RING_BLOCK", vg_plan::kRingBlock, 64, vg_plan::kRingBlock),
      env_int("VELOGRAD_BWD_RING_WGS_PER_CU", 1, 1, 2),
      env_int("VELOGRAD_FWD_ELEM", 1, 0, 1),
  };
  return t;
}

// `one_stream`: no residual, so the row kernel reads x and writes y only.  `epilogue`: a
// quantised output (fp8 per row, MX), whose two row reductions prefer fewer waves per row.
RowPlan plan_fwd(int64_t dim, int elem_bytes, bool aligned, bool one_stream, bool epilogue) {
  return vg_plan::plan_rows(dim, elem_bytes, aligned, tuning().fwd_nv,
                            epilogue     ? vg_plan::kFwdOrderEpilogue
                            : one_stream ? vg_plan::kFwdOrderOneStream
                                         : vg_plan::kFwdOrder);
}

// `aligned8`: every stream starts on an 8-byte boundary (the weight on a 16-byte one), the
// condition of the ring's kRing8 rows.
BwdPlan plan_bwd(int64_t rows, int64_t dim, int elem_bytes, bool aligned, bool aligned8, int cus,
                 bool rope, int64_t rope_seq) {
  const Tuning& t = tuning();
  if (!rope && t.bwd_ring) {
    const BwdPlan r = vg_plan::plan_bwd_ring(rows, dim, elem_bytes, aligned, cus, t.bwd_nv,
                                             t.ring_block, t.ring_wgs_per_cu);
    if (r.ring) return r;
    if (aligned8) {
      const BwdPlan r8 = vg_plan::plan_bwd_ring8(rows, dim, elem_bytes, cus, t.ring_block,
                                                 t.ring_wgs_per_cu);
      if (r8.ring) return r8;
    }
  }
  if (rope && t.bwd_ring) {
    const BwdPlan r = vg_plan::plan_bwd_rope_ring(rows, dim, elem_bytes, aligned, cus);
    if (r.ring && vg_plan::rope_walk_ok(rows, r.wgs * r.rp.groups, rope_seq)) return r;
  }
  if (rope)
    return vg_plan::plan_bwd_rope(rows, dim, elem_bytes, aligned, cus, t.bwd_nv, t.bwd_block,
                                  t.bwd_waves_per_cu);
  const BwdPlan p = vg_plan::plan_bwd(rows, dim, elem_bytes, aligned, cus, t.bwd_nv, t.bwd_block,
                                      t.bwd_waves_per_cu);
  // rows the chunked kernels cannot take: the element-strided ring where it fits
  if (!p.rp.vec && t.bwd_ring) {
    const BwdPlan e = vg_plan::plan_bwd_ring_elem(rows, dim, elem_bytes, cus);
    if (e.elem_m > 0) return e;
  }
  return p;
}

bool ld_ok(int64_t ld, int elem_bytes) { return ((ld * elem_bytes) & 15) == 0; }
bool ld_ok8(int64_t ld, int elem_bytes) { return ((ld * elem_bytes) & 7) == 0; }
bool aligned8p(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7) == 0; }

// ------------------------------------------------------------------------------------------
// Typed launchers.
// ------------------------------------------------------------------------------------------
template <int DT, int WDT, int OUT>
void launch_fwd(const FwdArgs& a, const RowPlan& p, hipStream_t st) {
  if (!p.vec) {
    hipLaunchKernelGGL((fwd_generic_kernel<DT, WDT, OUT>), dim3((uint32_t)a.rows), dim3(p.block),
                       0, st, a);
    return;
  }
  if constexpr (OUT == kOutRopeI) {
    // One chunk per thread (rows up to 1024 chunks: 8192 bf16/fp16, 4096 fp32 elements); more
    // chunks would hold 16 more doubles per chunk and spill, so longer rows take the generic
    // kernel.
    if (p.nv != 1) {
      // wider rows: the register-resident one-shot rows with each pair's rotation evaluated
      // directly (1024-thread row groups, two to four chunks per thread)
      const dim3 grid((uint32_t)((a.rows + p.groups - 1) / p.groups)), block(p.block);
      switch (p.nv) {
        case 2:
          hipLaunchKernelGGL((fwd_vec_kernel<DT, WDT, 2, kOutRopeDirect>), grid, block, 0, st, a);
          break;
        case 3:
          hipLaunchKernelGGL((fwd_vec_kernel<DT, WDT, 3, kOutRopeDirect>), grid, block, 0, st, a);
          break;
        default:
          hipLaunchKernelGGL((fwd_vec_kernel<DT, WDT, 4, kOutRopeDirect>), grid, block, 0, st, a);
          break;
      }
      return;
    }
    const int w = vg_plan::fwd_rope_walk_rows(a.rows, p.tpr);
    const dim3 grid((uint32_t)((a.rows + w - 1) / w)), block(p.tpr);
    const int rf = (a.res == nullptr ? 0 : a.h == nullptr ? kRopeRes : kRopeRes | kRopeWriteH) |
                   ((a.dim & (a.dim - 1)) == 0 ? kRopeDimPow2 : 0);
    switch (rf * 2 + (w == vg_plan::kNormRopeLongRows ? 1 : 0)) {
#define VG_ROPE_FWD(F)                                                                      \
  case 2 * (F):                                                                             \
    hipLaunchKernelGGL((fwd_rope_kernel<DT, WDT, F, vg_plan::kNormRopeRows>), grid, block, 0, \
                       st, a);                                                              \
    break;                                                                                  \
  case 2 * (F) + 1:                                                                         \
    hipLaunchKernelGGL((fwd_rope_kernel<DT, WDT, F, vg_plan::kNormRopeLongRows>), grid,       \
                       block, 0, st, a);                                                    \
    break;
      VG_ROPE_FWD(0)
      VG_ROPE_FWD(kRopeRes)
      VG_ROPE_FWD(kRopeRes | kRopeWriteH)
      VG_ROPE_FWD(kRopeDimPow2)
      VG_ROPE_FWD(kRopeDimPow2 | kRopeRes)
      VG_ROPE_FWD(kRopeDimPow2 | kRopeRes | kRopeWriteH)
#undef VG_ROPE_FWD
      default: break;
    }
  } else {
    const dim3 grid((uint32_t)((a.rows + p.groups - 1) / p.groups));
    const dim3 block(p.block);
    if constexpr (OUT == kOutDtype) {
      if (vg_plan::fwd_late_h(p)) {
        switch (p.nv) {
#define VG_LATE_H(N)                                                                          \
  case N:                                                                                     \
    hipLaunchKernelGGL((fwd_vec_kernel<DT, WDT, N, kOutDtypeLateH>), grid, block, 0, st, a); \
    break;
          VG_LATE_H(1)
          VG_LATE_H(2)
          VG_LATE_H(3)
          default: VG_LATE_H(4)
#undef VG_LATE_H
        }
        return;
      }
    }
    switch (p.nv) {
      case 1: hipLaunchKernelGGL((fwd_vec_kernel<DT, WDT, 1, OUT>), grid, block, 0, st, a); break;
      case 2: hipLaunchKernelGGL((fwd_vec_kernel<DT, WDT, 2, OUT>), grid, block, 0, st, a); break;
      case 3: hipLaunchKernelGGL((fwd_vec_kernel<DT, WDT, 3, OUT>), grid, block, 0, st, a); break;
      default: hipLaunchKernelGGL((fwd_vec_kernel<DT, WDT, 4, OUT>), grid, block, 0, st, a); break;
    }
  }
}

// Rows of 8-byte alignment (fwd_vec_kernel's X8): `p` lays out the dim - V / 2 columns of whole
// chunks.
template <int DT, int WDT>
void launch_fwd_x8(const FwdArgs& a, const RowPlan& p, hipStream_t st) {
  if constexpr (Codec<DT>::kBytes == 2) {
    const dim3 grid((uint32_t)((a.rows + p.groups - 1) / p.groups)), block(p.block);
    const bool late = vg_plan::fwd_late_h(p);
    switch (p.nv * 2 + (late ? 1 : 0)) {
#define VG_FWD_X8(N)                                                                          \
  case 2 * (N):                                                                               \
    hipLaunchKernelGGL((fwd_vec_kernel<DT, WDT, N, kOutDtype, true>), grid, block, 0, st, a); \
    break;                                                                                    \
  case 2 * (N) + 1:                                                                           \
    hipLaunchKernelGGL((fwd_vec_kernel<DT, WDT, N, kOutDtypeLateH, true>), grid, block, 0, st, \
                       a);                                                                    \
    break;
      VG_FWD_X8(1)
      VG_FWD_X8(2)
      VG_FWD_X8(3)
      VG_FWD_X8(4)
#undef VG_FWD_X8
      default: break;
    }
  }
}

// Rows of element-strided lanes (fwd_elem_kernel): `p` from plan_elem_rows, m elements a lane.
template <int DT, int WDT>
void launch_fwd_elem(const FwdArgs& a, const RowPlan& p, int m, hipStream_t st) {
  const dim3 grid((uint32_t)((a.rows + p.groups - 1) / p.groups)), block(p.block);
  if (m == 4)
    hipLaunchKernelGGL((fwd_elem_kernel<DT, WDT, 4>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((fwd_elem_kernel<DT, WDT, 8>), grid, block, 0, st, a);
}

template <int DT, int WDT, int F>
void launch_bwd_ring(const BwdArgs& a, const BwdPlan& b, hipStream_t st) {
  const dim3 grid((uint32_t)b.wgs), block(b.rp.block);
  if constexpr (Codec<DT>::kBytes == 2) {
    // rows of 8-byte alignment with a half chunk at their end: one chunk per thread
    if (b.x8) {
      if ((int64_t)b.rp.tpr * Codec<DT>::kVec != a.dim - Codec<DT>::kVec / 2)
        hipLaunchKernelGGL((bwd_ring_kernel<DT, WDT, 1, F | kRing8 | kRingTail>), grid, block,
                           b.lds_bytes, st, a);
      else
        hipLaunchKernelGGL((bwd_ring_kernel<DT, WDT, 1, F | kRing8>), grid, block, b.lds_bytes,
                           st, a);
      return;
    }
  }
  // rows of fewer chunks than the row group's lanes take the idle-lane variant
  if ((int64_t)b.rp.nv * b.rp.tpr * Codec<DT>::kVec != a.dim) {
    if (b.rp.nv == 1)
      hipLaunchKernelGGL((bwd_ring_kernel<DT, WDT, 1, F | kRingTail>), grid, block, b.lds_bytes,
                         st, a);
    else
      hipLaunchKernelGGL((bwd_ring_kernel<DT, WDT, 2, F | kRingTail>), grid, block, b.lds_bytes,
                         st, a);
    return;
  }
  if (b.rp.nv == 1)
    hipLaunchKernelGGL((bwd_ring_kernel<DT, WDT, 1, F>), grid, block, b.lds_bytes, st, a);
  else
    hipLaunchKernelGGL((bwd_ring_kernel<DT, WDT, 2, F>), grid, block, b.lds_bytes, st, a);
}

template <int DT, int WDT, int F>
void launch_bwd_ring_elem(const BwdArgs& a, const BwdPlan& b, hipStream_t st) {
  const dim3 grid((uint32_t)b.wgs), block(b.rp.block);
  if (b.elem_m == 4)
    hipLaunchKernelGGL((bwd_ring_elem_kernel<DT, WDT, 4, F>), grid, block, b.lds_bytes, st, a);
  else
    hipLaunchKernelGGL((bwd_ring_elem_kernel<DT, WDT, 8, F>), grid, block, b.lds_bytes, st, a);
}

template <int DT, int WDT, int F>
void launch_bwd_flags(const BwdArgs& a, const BwdPlan& b, hipStream_t st) {
  const RowPlan& p = b.rp;
  const dim3 grid((uint32_t)b.wgs);
  const dim3 block(p.block);
  const size_t lds = b.lds_bytes;
  if constexpr ((F & kRopeG) == 0) {
    if (b.elem_m > 0) {
      if (a.dres != nullptr)
        launch_bwd_ring_elem<DT, WDT, F | kRingDres>(a, b, st);
      else
        launch_bwd_ring_elem<DT, WDT, F>(a, b, st);
      return;
    }
  }
  if (!p.vec) {
    hipLaunchKernelGGL((bwd_generic_kernel<DT, WDT, F>), grid, block,
                       vg_plan::generic_bwd_lds_bytes(a.dim, a.partial != nullptr), st, a);
    return;
  }
  if constexpr ((F & kRopeG) == 0) {
    if (b.ring) {
      if (a.dres != nullptr)
        launch_bwd_ring<DT, WDT, F | kRingDres>(a, b, st);
      else
        launch_bwd_ring<DT, WDT, F>(a, b, st);
      return;
    }
  }
  if constexpr ((F & kRopeG) != 0) {
    if (b.ring) {
      if (p.nv == 2)
        hipLaunchKernelGGL((bwd_rope_ring_kernel<DT, WDT, 2>), grid, block, lds, st, a);
      else
        hipLaunchKernelGGL((bwd_rope_ring_kernel<DT, WDT, 1>), grid, block, lds, st, a);
      return;
    }
    if (b.rope_direct) {
      constexpr int FD = (F & ~kRopeG) | kRopeDirect;
      switch (p.nv) {
        case 1: hipLaunchKernelGGL((bwd_vec_kernel<DT, WDT, 1, FD>), grid, block, lds, st, a); break;
        case 2: hipLaunchKernelGGL((bwd_vec_kernel<DT, WDT, 2, FD>), grid, block, lds, st, a); break;
        case 3: hipLaunchKernelGGL((bwd_vec_kernel<DT, WDT, 3, FD>), grid, block, lds, st, a); break;
        default: hipLaunchKernelGGL((bwd_vec_kernel<DT, WDT, 4, FD>), grid, block, lds, st, a); break;
      }
      return;
    }
    // NV 4 is never planned with the RoPE gradient (max_block_for_nv_rope); it is not compiled
    switch (p.nv) {
      case 1: hipLaunchKernelGGL((bwd_vec_kernel<DT, WDT, 1, F>), grid, block, lds, st, a); break;
      case 2: hipLaunchKernelGGL((bwd_vec_kernel<DT, WDT, 2, F>), grid, block, lds, st, a); break;
      default: hipLaunchKernelGGL((bwd_vec_kernel<DT, WDT, 3, F>), grid, block, lds, st, a); break;
    }
  } else {
    switch (p.nv) {
      case 1: hipLaunchKernelGGL((bwd_vec_kernel<DT, WDT, 1, F>), grid, block, lds, st, a); break;
      case 2: hipLaunchKernelGGL((bwd_vec_kernel<DT, WDT, 2, F>), grid, block, lds, st, a); break;
      case 3: hipLaunchKernelGGL((bwd_vec_kernel<DT, WDT, 3, F>), grid, block, lds, st, a); break;
      default: hipLaunchKernelGGL((bwd_vec_kernel<DT, WDT, 4, F>), grid, block, lds, st, a); break;
    }
  }
}

template <int DT, int WDT>
void launch_bwd(const BwdArgs& a, bool saved_is_h, bool rope, const BwdPlan& b, hipStream_t st) {
  if (rope) {  // the module form: the saved tensor is h, no residual-stream gradient
    launch_bwd_flags<DT, WDT, kSavedIsH | kRopeG>(a, b, st);
    return;
  }
  const int flags = (saved_is_h ? kSavedIsH : 0) | (a.gh != nullptr ? kGradH : 0);
  switch (flags) {
    case 0: launch_bwd_flags<DT, WDT, 0>(a, b, st); break;
    case kSavedIsH: launch_bwd_flags<DT, WDT, kSavedIsH>(a, b, st); break;
    case kGradH: launch_bwd_flags<DT, WDT, kGradH>(a, b, st); break;
    default: launch_bwd_flags<DT, WDT, kSavedIsH | kGradH>(a, b, st); break;
  }
}

// Supported (dtype, w_dtype) pairs: weight in the activation dtype, or fp32.
bool types_ok(int32_t dt, int32_t wdt) {
  if (elem_bytes_of(dt) == 0) return false;
  return wdt == dt || wdt == VELOGRAD_DTYPE_F32;
}

#define VG_DISPATCH_TYPES(DT, WDT, CALL)                                       \
  do {                                                                         \
    if ((DT) == VELOGRAD_DTYPE_F32) {                                          \
      constexpr int kD = VELOGRAD_DTYPE_F32, kW = VELOGRAD_DTYPE_F32;          \
      CALL;                                                                    \
    } else if ((DT) == VELOGRAD_DTYPE_BF16 && (WDT) == VELOGRAD_DTYPE_BF16) {  \
      constexpr int kD = VELOGRAD_DTYPE_BF16, kW = VELOGRAD_DTYPE_BF16;        \
      CALL;                                                                    \
    } else if ((DT) == VELOGRAD_DTYPE_BF16) {                                  \
      constexpr int kD = VELOGRAD_DTYPE_BF16, kW = VELOGRAD_DTYPE_F32;         \
      CALL;                                                                    \
    } else if ((WDT) == VELOGRAD_DTYPE_F16) {                                  \
      constexpr int kD = VELOGRAD_DTYPE_F16, kW = VELOGRAD_DTYPE_F16;          \
      CALL;                                                                    \
    } else {                                                                   \
      constexpr int kD = VELOGRAD_DTYPE_F16, kW = VELOGRAD_DTYPE_F32;          \
      CALL;                                                                    \
    }                                                                          \
  } while (0)

size_t workspace_bytes_for(int64_t rows, int64_t dim, int cus) {
  const Tuning& t = tuning();
  return vg_plan::bwd_workspace_bytes(rows, dim, cus, t.bwd_nv, t.bwd_block, t.bwd_waves_per_cu,
                                      t.ring_block, t.ring_wgs_per_cu);
}

// ------------------------------------------------------------------------------------------
// Scratch of the allocation-free backward (velograd_rmsnorm_residual_bwd_noalloc): the dweight
// partial rows live in this file-scope device array instead of a caller workspace.  Each GPU
// the library runs on holds its own copy, at its own address, until the process ends.  In host
// code `scratch` names a host-side stand-in, never the device memory: the device address comes
// from hipGetSymbolAddress, once per device with that device current, and only that address is
// passed to kernels.  Nothing in it needs to start at zero (stage 1 writes every partial row it
// hands to stage 2 before stage 2 reads it), so no call clears it.  Calls that overlap on one
// GPU (two streams, or two host threads) share the array and race.
// ------------------------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

// Device address of `scratch` on `device` (the current device), or null with the HIP error.
void* scratch_on(int device, hipError_t* err) {
  std::call_once(g_scratch_once[device], [device] {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_err[device] = e;
    g_scratch_ptr[device] = (e == hipSuccess) ? p : nullptr;
  });
  *err = g_scratch_err[device];
  return g_scratch_ptr[device];
}

// Shared by the forward entry points.  `out` is the epilogue (kOut*): for kOutFp8Row y holds one
// e4m3 byte per element and y_scale one fp32 per row; for the MX modes y holds e4m3 bytes or
// e2m1 nibbles and mx_scale one E8M0 byte per 32 elements.  ld_y (and ld_mx) count bytes then.
int32_t run_fwd(const char* what, int out, const void* x, const void* residual,
                const void* weight, void* y, float* y_scale, uint8_t* mx_scale, int64_t ld_mx,
                void* h, float* inv_rms, int64_t rows, int64_t dim, int64_t ld_x,
                int64_t ld_res, int64_t ld_y, int64_t ld_h, int32_t dtype, int32_t w_dtype,
                float eps, float ms_floor, void* hip_stream, int64_t rope_seq = 0,
                float rope_theta = 0.0f) {
  const bool mx = out == kOutMxE4M3 || out == kOutMxE2M1;
  if (!types_ok(dtype, w_dtype))
    return fail(VELOGRAD_ERR_UNSUPPORTED_DTYPE,
                "%s: unsupported dtype/w_dtype pair (%d, %d): weight must be the activation "
                "dtype or fp32",
                what, (int)dtype, (int)w_dtype);
  if (rows < 0 || dim <= 0 || dim > INT32_MAX)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "%s: invalid shape rows=%lld dim=%lld", what,
                (long long)rows, (long long)dim);
  if (!(ms_floor >= 0.0f) || !__builtin_isfinite(ms_floor))
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT,
                "%s: min_mean_sq=%g must be finite and >= 0", what, (double)ms_floor);
  if (out == kOutRopeI && (dim % 2 != 0 || rope_seq < 1 || (rows > 0 && rows % rope_seq != 0) ||
                           !(rope_theta > 0.0f) || !__builtin_isfinite(rope_theta)))
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT,
                "%s: RoPE needs an even dim (%lld), seq >= 1 dividing rows (seq=%lld rows=%lld) "
                "and a finite base > 0 (%g)",
                what, (long long)dim, (long long)rope_seq, (long long)rows, (double)rope_theta);
  if (mx && dim % vg_mx::kBlock != 0)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT,
                "%s: dim=%lld must be a multiple of the 32-element MX block", what,
                (long long)dim);
  if (rows == 0) {
    clear_error();
    return 0;
  }
  if (x == nullptr || y == nullptr)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "%s: x and y must not be NULL", what);
  if (out == kOutFp8Row && y_scale == nullptr)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "%s: y_scale must not be NULL", what);
  if (mx && mx_scale == nullptr)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "%s: scales must not be NULL", what);
  if (residual == nullptr) h = nullptr;  // h is x itself
  const int64_t y_row = out == kOutMxE2M1 ? dim / 2 : dim;  // y row length in its own units
  if (ld_x < dim || ld_y < y_row || (residual && ld_res < dim) || (h && ld_h < dim) ||
      (mx && ld_mx < dim / vg_mx::kBlock))
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT,
                "%s: row strides too small (ld_x=%lld ld_res=%lld ld_y=%lld ld_h=%lld "
                "ld_scales=%lld for dim=%lld)",
                what, (long long)ld_x, (long long)ld_res, (long long)ld_y, (long long)ld_h,
                (long long)ld_mx, (long long)dim);
  const void* extra_out = out == kOutFp8Row ? (const void*)y_scale : (const void*)mx_scale;
  if (y == x || y == residual || (h && (h == x || h == residual || h == y)) ||
      (extra_out && (extra_out == x || extra_out == residual || extra_out == y ||
                     (h && extra_out == h))))
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "%s: outputs must not alias inputs", what);
  if (rows > INT32_MAX)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "%s: rows=%lld exceeds the grid limit", what,
                (long long)rows);

  const int eb = elem_bytes_of(dtype);
  // Bytes of y per 16-byte input chunk: 16 (activation dtype), 16 / eb (e4m3), 8 / eb (e2m1).
  bool y_aligned;
  if (out == kOutDtype) {
    y_aligned = aligned16(y) && ld_ok(ld_y, eb);
  } else {
    const int64_t cb = out == kOutMxE2M1 ? 8 / eb : 16 / eb;
    y_aligned = ((uintptr_t)y % (uintptr_t)cb) == 0 && ld_y % cb == 0;
  }
  const bool aligned = aligned16(x) && ld_ok(ld_x, eb) && y_aligned &&
                       (!residual || (aligned16(residual) && ld_ok(ld_res, eb))) &&
                       (!h || (aligned16(h) && ld_ok(ld_h, eb))) && (!weight || aligned16(weight));
  // The fused norm + RoPE kernel holds one chunk per thread, so it keeps the residual order
  // (one chunk first) either way.
  RowPlan p = plan_fwd(dim, eb, aligned, residual == nullptr && out != kOutRopeI,
                       out == kOutFp8Row || mx);
  // Rows of 8n + 4 two-byte elements on 8-byte boundaries (fwd_vec_kernel's X8): the plan of
  // their whole chunks, the last 4 elements an extra half chunk.
  const bool aligned8 = aligned8p(x) && ld_ok8(ld_x, eb) && aligned8p(y) && ld_ok8(ld_y, eb) &&
                        (!residual || (aligned8p(residual) && ld_ok8(ld_res, eb))) &&
                        (!h || (aligned8p(h) && ld_ok8(ld_h, eb))) &&
                        (!weight || aligned16(weight));
  bool x8 = false;
  if (!p.vec && out == kOutDtype && eb == 2 && dim >= 12 && dim % 8 == 4 && aligned8) {
    const RowPlan px = plan_fwd(dim - 4, eb, true, residual == nullptr, false);
    if (px.vec) {
      p = px;
      x8 = true;
    }
  }
  // other short rows the chunked kernels cannot take: element-strided lanes, several rows a
  // workgroup.  Longer rows keep the generic kernel, whose row middles move in 16-byte accesses:
  // bf16 16384 x 99 10.6 us against 38.6 in the generic kernel, 255 13.3 against 40.2, 1001 46.6
  // against 49.2, but 2047 85.9 against 60.2, 3001 154.3 against 81.4, 4095 161.5 against 100.4.
  int elem_m = 0;
  if (!p.vec && !x8 && out == kOutDtype && (eb == 2 || eb == 4) && dim <= kFwdElemMaxDim &&
      tuning().fwd_elem) {
    elem_m = vg_plan::elem_per_lane(dim);
    if (elem_m > 0) p = vg_plan::plan_elem_rows(dim);
  }
  const bool elem_ok = p.tpr % kWave == 0 && p.tpr >= kWave && p.groups >= 1 &&
                       p.block == p.tpr * p.groups && p.block <= vg_plan::kRingBlock &&
                       (int64_t)elem_m * p.tpr >= dim;
  if (elem_m > 0 ? !elem_ok : !vg_plan::row_plan_valid(p, x8 ? dim - 4 : dim, eb))
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "%s: internal launch plan rejected (dim=%lld)",
                what, (long long)dim);

  FwdArgs a;
  a.x = x;
  a.res = residual;
  a.w = weight;
  a.y = y;
  a.h = h;
  a.inv_rms = inv_rms;
  a.y_scale = y_scale;
  a.mx_scale = mx_scale;
  a.ld_mx = ld_mx;
  a.rows = rows;
  a.ld_x = ld_x;
  a.ld_res = ld_res;
  a.ld_y = ld_y;
  a.ld_h = ld_h;
  a.dim = (int32_t)dim;
  a.tpr = p.tpr;
  a.eps = eps;
  a.ms_floor = ms_floor;
  a.rope_seq = rope_seq > 0 ? rope_seq : 1;
  a.rope_half = (int32_t)(dim / 2);
  const double c = (rope_theta > 0.0f && dim >= 2) ? log2((double)rope_theta) / (double)(dim / 2)
                                                   : 0.0;
  a.rope_c_hi = (float)c;
  a.rope_c_lo = (float)(c - (double)a.rope_c_hi);
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  switch (out) {
    case kOutFp8Row: VG_DISPATCH_TYPES(dtype, w_dtype, (launch_fwd<kD, kW, kOutFp8Row>(a, p, st))); break;
    case kOutMxE4M3: VG_DISPATCH_TYPES(dtype, w_dtype, (launch_fwd<kD, kW, kOutMxE4M3>(a, p, st))); break;
    case kOutMxE2M1: VG_DISPATCH_TYPES(dtype, w_dtype, (launch_fwd<kD, kW, kOutMxE2M1>(a, p, st))); break;
    case kOutRopeI: VG_DISPATCH_TYPES(dtype, w_dtype, (launch_fwd<kD, kW, kOutRopeI>(a, p, st))); break;
    default:
      if (x8)
        VG_DISPATCH_TYPES(dtype, w_dtype, (launch_fwd_x8<kD, kW>(a, p, st)));
      else if (elem_m > 0)
        VG_DISPATCH_TYPES(dtype, w_dtype, (launch_fwd_elem<kD, kW>(a, p, elem_m, st)));
      else
        VG_DISPATCH_TYPES(dtype, w_dtype, (launch_fwd<kD, kW, kOutDtype>(a, p, st)));
      break;
  }
  return check_launch(what);
}

// The backward behind both C entry points.  rope_seq > 0: grad_y is the gradient of the
// interleaved-RoPE output (velograd_rmsnorm_rope_bwd); the saved tensor is then h.
int32_t run_bwd(const void* grad_y, const void* saved, int32_t saved_is_h, const void* weight,
                const float* inv_rms, const void* grad_h, void* dx, void* dres, float* dweight,
                void* workspace, size_t ws_bytes, int64_t rows, int64_t dim, int64_t ld_g,
                int64_t ld_saved, int64_t ld_grad_h, int64_t ld_dx, int64_t ld_dres,
                int32_t dtype, int32_t w_dtype, void* hip_stream, int64_t rope_seq = 0,
                float rope_base = 0.0f, bool static_scratch = false) {
  if (!types_ok(dtype, w_dtype))
    return fail(VELOGRAD_ERR_UNSUPPORTED_DTYPE,
                "bwd: unsupported dtype/w_dtype pair (%d, %d): weight must be the activation "
                "dtype or fp32",
                (int)dtype, (int)w_dtype);
  if (rows < 0 || dim <= 0 || dim > INT32_MAX)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "bwd: invalid shape rows=%lld dim=%lld",
                (long long)rows, (long long)dim);
  if (weight == nullptr) dweight = nullptr;  // no weight, no weight gradient (fused.py:62-65)
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  if (rows == 0) {
    // Sum over zero rows: dweight = 0, written by stage 2 with no partial rows.
    if (dweight != nullptr) {
      hipLaunchKernelGGL(dweight_reduce_kernel, dim3((uint32_t)((dim + kWave - 1) / kWave)),
                         dim3(kReduceBlock), 0, st, (const float*)nullptr, 0, (int32_t)dim,
                         dweight);
      return check_launch("velograd_rmsnorm_residual_bwd(dweight)");
    }
    clear_error();
    return 0;
  }
  if (grad_y == nullptr || saved == nullptr || inv_rms == nullptr || dx == nullptr)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT,
                "bwd: grad_y, saved, inv_rms and dx must not be NULL");
  if (ld_g < dim || ld_saved < dim || ld_dx < dim || (dres && ld_dres < dim) ||
      (grad_h && ld_grad_h < dim))
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT,
                "bwd: row strides must be >= dim (ld_g=%lld ld_saved=%lld ld_grad_h=%lld "
                "ld_dx=%lld ld_dres=%lld)",
                (long long)ld_g, (long long)ld_saved, (long long)ld_grad_h, (long long)ld_dx,
                (long long)ld_dres);
  // dx may be grad_h itself (accumulating in place: each element is read before it is written
  // by the same thread); no other output may alias an input.
  if (dx == grad_y || dx == saved || dx == dres ||
      (dres && (dres == grad_y || dres == saved || dres == grad_h)))
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "bwd: outputs must not alias inputs");
  if (grad_h == dx && ld_grad_h != ld_dx)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT,
                "bwd: dx may alias grad_h only with the same row stride");

  int device = 0;
  if (hipGetDevice(&device) != hipSuccess)
    return fail(VELOGRAD_ERR_DEVICE_QUERY, "bwd: hipGetDevice failed");
  const int cus = cu_count(device);
  if (cus <= 0) return fail(VELOGRAD_ERR_DEVICE_QUERY, "bwd: cannot query the CU count");

  const int eb = elem_bytes_of(dtype);
  const bool aligned = aligned16(grad_y) && aligned16(saved) && aligned16(dx) &&
                       ld_ok(ld_g, eb) && ld_ok(ld_saved, eb) && ld_ok(ld_dx, eb) &&
                       (!dres || (aligned16(dres) && ld_ok(ld_dres, eb))) &&
                       (!grad_h || (aligned16(grad_h) && ld_ok(ld_grad_h, eb))) &&
                       (!weight || aligned16(weight));
  const bool aligned8 = aligned8p(grad_y) && aligned8p(saved) && aligned8p(dx) &&
                        ld_ok8(ld_g, eb) && ld_ok8(ld_saved, eb) && ld_ok8(ld_dx, eb) &&
                        (!dres || (aligned8p(dres) && ld_ok8(ld_dres, eb))) &&
                        (!grad_h || (aligned8p(grad_h) && ld_ok8(ld_grad_h, eb))) &&
                        (!weight || aligned16(weight));
  const bool rope = rope_seq > 0;
  BwdPlan plan = plan_bwd(rows, dim, eb, aligned, aligned8, cus, rope, rope_seq);
  const int64_t plan_dim = plan.x8 ? dim - 4 : dim;  // the columns the row plan lays out
  // bwd_vec_kernel's RoPE walk keeps its step rotations (two floats per pair: dim floats) in the
  // same dynamic LDS as the group combine, one after the other.
  if (rope && plan.rp.vec && !plan.ring && !plan.rope_direct)
    plan.lds_bytes = (size_t)dim * sizeof(float);
  const bool elem_ok =
      plan.elem_m > 0 && !rope && plan.rp.tpr % kWave == 0 && plan.rp.tpr >= kWave &&
      plan.rp.groups >= 1 && plan.rp.block == plan.rp.tpr * plan.rp.groups &&
      plan.rp.block <= vg_plan::kRingBlock && (int64_t)plan.elem_m * plan.rp.tpr >= dim;
  if ((plan.elem_m > 0 ? !elem_ok : !vg_plan::row_plan_valid(plan.rp, plan_dim, eb)) ||
      plan.wgs < 1 || plan.wgs > INT32_MAX || plan.lds_bytes > 64 * 1024 ||
      (plan.ring && !rope && (!vg_plan::ring_eligible(plan.rp, plan_dim, eb) ||
                              plan.rp.block > vg_plan::kRingBlock)) ||
      (plan.x8 && (rope || !plan.ring || eb != 2 || dim % 8 != 4 || plan.rp.nv != 1 ||
                   !aligned8)) ||
      (plan.ring && rope && (!vg_plan::rope_ring_eligible(plan.rp, dim, eb) ||
                             !vg_plan::rope_walk_ok(rows, plan.wgs * plan.rp.groups, rope_seq))) ||
      (rope && plan.rp.vec && !plan.ring && !plan.rope_direct &&
       plan.rp.block > vg_plan::max_block_for_nv_rope(plan.rp.nv)) ||
      (plan.rope_direct && (!rope || plan.rp.block > vg_plan::max_block_for_nv(plan.rp.nv))))
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "bwd: internal launch plan rejected (dim=%lld)",
                (long long)dim);
  const int64_t slots = plan.wgs * plan.rp.groups;  // row slots walking the rows

  float* partial = nullptr;
  if (dweight != nullptr) {
    const size_t need = (size_t)plan.wgs * (size_t)dim * sizeof(float);
    if (static_scratch) {
      // velograd_rmsnorm_residual_bwd_noalloc: the partial rows go to the library's own array
      if (need > kNoAllocScratchBytes)
        return fail(VELOGRAD_ERR_WORKSPACE_TOO_SMALL,
                    "bwd_noalloc: dweight needs %zu bytes of scratch for rows=%lld dim=%lld, above "
                    "the fixed maximum of %zu bytes; pass a workspace to "
                    "velograd_rmsnorm_residual_bwd instead",
                    need, (long long)rows, (long long)dim, kNoAllocScratchBytes);
      if (device < 0 || device >= kMaxDevices)
        return fail(VELOGRAD_ERR_DEVICE_QUERY, "bwd_noalloc: device %d out of range", device);
      hipError_t e = hipSuccess;
      workspace = scratch_on(device, &e);
      if (workspace == nullptr)
        return fail((int32_t)e, "bwd_noalloc: hipGetSymbolAddress of the scratch failed: %s",
                    hipGetErrorString(e));
      ws_bytes = kNoAllocScratchBytes;
    }
    if (workspace == nullptr || ws_bytes < need)
      return fail(VELOGRAD_ERR_WORKSPACE_TOO_SMALL,
                  "bwd: workspace of %zu bytes given, %zu needed", ws_bytes, need);
    if (!aligned16(workspace))
      return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "bwd: workspace must be 16-byte aligned");
    partial = static_cast<float*>(workspace);
  }

  BwdArgs a;
  a.g = grad_y;
  a.saved = saved;
  a.w = weight;
  a.inv_rms = inv_rms;
  a.gh = grad_h;
  a.dx = dx;
  a.dres = dres;
  a.partial = partial;
  a.rows = rows;
  a.ld_g = ld_g;
  a.ld_gh = ld_grad_h;
  a.ld_s = ld_saved;
  a.ld_dx = ld_dx;
  a.ld_dres = ld_dres;
  a.dim = (int32_t)dim;
  a.tpr = plan.rp.tpr;
  a.iters = (int32_t)((rows + slots - 1) / slots);
  a.rope_seq = rope ? rope_seq : 1;
  const double c = rope ? log2((double)rope_base) / (double)(dim / 2) : 0.0;
  a.rope_c_hi = (float)c;
  a.rope_c_lo = (float)(c - (double)a.rope_c_hi);
  VG_DISPATCH_TYPES(dtype, w_dtype, (launch_bwd<kD, kW>(a, saved_is_h != 0, rope, plan, st)));
  int32_t rc = check_launch(rope ? "velograd_rmsnorm_rope_bwd" : "velograd_rmsnorm_residual_bwd");
  if (rc != 0 || dweight == nullptr) return rc;
  hipLaunchKernelGGL(dweight_reduce_kernel, dim3((uint32_t)((dim + kWave - 1) / kWave)),
                     dim3(kReduceBlock), 0, st, (const float*)partial, (int32_t)plan.wgs,
                     (int32_t)dim, dweight);
  return check_launch("velograd_rmsnorm_residual_bwd(dweight)");
}

}  // namespace

// ------------------------------------------------------------------------------------------
// C ABI.
// ------------------------------------------------------------------------------------------
extern "C" {

VELOGRAD_API const char* velograd_kernels_version(void) { return VG_VERSION_STRING; }

VELOGRAD_API const char* velograd_kernels_last_error(void) { return g_last_error; }

VELOGRAD_API size_t velograd_rmsnorm_residual_bwd_workspace_bytes(int64_t rows, int64_t dim,
                                                                  int32_t device) {
  return workspace_bytes_for(rows, dim, cu_count(device));
}

VELOGRAD_API int32_t velograd_rmsnorm_residual_fwd(const void* x, const void* residual,
                                                   const void* weight, void* y, void* h,
                                                   float* inv_rms, int64_t rows, int64_t dim,
                                                   int64_t ld_x, int64_t ld_res, int64_t ld_y,
                                                   int64_t ld_h, int32_t dtype, int32_t w_dtype,
                                                   float eps, void* hip_stream) {
  return run_fwd("velograd_rmsnorm_residual_fwd", kOutDtype, x, residual, weight, y, nullptr,
                 nullptr, 0, h, inv_rms, rows, dim, ld_x, ld_res, ld_y, ld_h, dtype, w_dtype,
                 eps, 0.0f, hip_stream);
}

VELOGRAD_API int32_t velograd_rmsnorm_fwd(const void* x, const void* residual,
                                          const void* weight, void* y, void* h, float* inv_rms,
                                          int64_t rows, int64_t dim, int64_t ld_x,
                                          int64_t ld_res, int64_t ld_y, int64_t ld_h,
                                          int32_t dtype, int32_t w_dtype, float eps,
                                          float min_mean_sq, void* hip_stream) {
  return run_fwd("velograd_rmsnorm_fwd", kOutDtype, x, residual, weight, y, nullptr, nullptr, 0,
                 h, inv_rms, rows, dim, ld_x, ld_res, ld_y, ld_h, dtype, w_dtype, eps,
                 min_mean_sq, hip_stream);
}

VELOGRAD_API int32_t velograd_rmsnorm_rope_fwd(
    const void* x, const void* residual, const void* weight, void* y, void* h, float* inv_rms,
    int64_t rows, int64_t dim, int64_t ld_x, int64_t ld_res, int64_t ld_y, int64_t ld_h,
    int64_t seq, int32_t dtype, int32_t w_dtype, float eps, float min_mean_sq, float base,
    void* hip_stream) {
  return run_fwd("velograd_rmsnorm_rope_fwd", kOutRopeI, x, residual, weight, y, nullptr,
                 nullptr, 0, h, inv_rms, rows, dim, ld_x, ld_res, ld_y, ld_h, dtype, w_dtype, eps,
                 min_mean_sq, hip_stream, seq, base);
}

VELOGRAD_API int32_t velograd_rmsnorm_residual_fwd_fp8(
    const void* x, const void* residual, const void* weight, uint8_t* y_fp8, float* y_scale,
    void* h, float* inv_rms, int64_t rows, int64_t dim, int64_t ld_x, int64_t ld_res,
    int64_t ld_y, int64_t ld_h, int32_t dtype, int32_t w_dtype, float eps, void* hip_stream) {
  return run_fwd("velograd_rmsnorm_residual_fwd_fp8", kOutFp8Row, x, residual, weight, y_fp8,
                 y_scale, nullptr, 0, h, inv_rms, rows, dim, ld_x, ld_res, ld_y, ld_h, dtype,
                 w_dtype, eps, 0.0f, hip_stream);
}

VELOGRAD_API int32_t velograd_rmsnorm_residual_fwd_mx(
    const void* x, const void* residual, const void* weight, uint8_t* y_q, uint8_t* y_scales,
    void* h, float* inv_rms, int64_t rows, int64_t dim, int64_t ld_x, int64_t ld_res,
    int64_t ld_yq, int64_t ld_scales, int64_t ld_h, int32_t dtype, int32_t w_dtype,
    int32_t mx_format, float eps, void* hip_stream) {
  if (mx_format != VELOGRAD_MX_E4M3 && mx_format != VELOGRAD_MX_E2M1)
    return fail(VELOGRAD_ERR_UNSUPPORTED_DTYPE,
                "velograd_rmsnorm_residual_fwd_mx: unsupported mx_format %d", (int)mx_format);
  return run_fwd("velograd_rmsnorm_residual_fwd_mx",
                 mx_format == VELOGRAD_MX_E4M3 ? kOutMxE4M3 : kOutMxE2M1, x, residual, weight,
                 y_q, nullptr, y_scales, ld_scales, h, inv_rms, rows, dim, ld_x, ld_res, ld_yq,
                 ld_h, dtype, w_dtype, eps, 0.0f, hip_stream);
}

VELOGRAD_API int32_t velograd_rmsnorm_residual_bwd(
    const void* grad_y, const void* saved, int32_t saved_is_h, const void* weight,
    const float* inv_rms, const void* grad_h, void* dx, void* dres, float* dweight,
    void* workspace, size_t ws_bytes, int64_t rows, int64_t dim, int64_t ld_g, int64_t ld_saved,
    int64_t ld_grad_h, int64_t ld_dx, int64_t ld_dres, int32_t dtype, int32_t w_dtype,
    void* hip_stream) {
  return run_bwd(grad_y, saved, saved_is_h, weight, inv_rms, grad_h, dx, dres, dweight, workspace,
                 ws_bytes, rows, dim, ld_g, ld_saved, ld_grad_h, ld_dx, ld_dres, dtype, w_dtype,
                 hip_stream);
}

VELOGRAD_API int32_t velograd_rmsnorm_residual_bwd_noalloc(
    const void* grad_y, const void* saved, int32_t saved_is_h, const void* weight,
    const float* inv_rms, const void* grad_h, void* dx, void* dres, float* dweight, int64_t rows,
    int64_t dim, int64_t ld_g, int64_t ld_saved, int64_t ld_grad_h, int64_t ld_dx,
    int64_t ld_dres, int32_t dtype, int32_t w_dtype, void* hip_stream) {
  return run_bwd(grad_y, saved, saved_is_h, weight, inv_rms, grad_h, dx, dres, dweight, nullptr,
                 0, rows, dim, ld_g, ld_saved, ld_grad_h, ld_dx, ld_dres, dtype, w_dtype,
                 hip_stream, 0, 0.0f, /*static_scratch=*/true);
}

VELOGRAD_API int32_t velograd_rmsnorm_rope_bwd(
    const void* grad_y, const void* h, const void* weight, const float* inv_rms, void* dx,
    float* dweight, void* workspace, size_t ws_bytes, int64_t rows, int64_t dim, int64_t ld_g,
    int64_t ld_h, int64_t ld_dx, int64_t seq, int32_t dtype, int32_t w_dtype, float base,
    void* hip_stream) {
  if (dim % 2 != 0 || seq < 1 || (rows > 0 && rows % seq != 0) || !(base > 0.0f) ||
      !__builtin_isfinite(base))
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT,
                "velograd_rmsnorm_rope_bwd: RoPE needs an even dim (%lld), seq >= 1 dividing rows "
                "(seq=%lld rows=%lld) and a finite base > 0 (%g)",
                (long long)dim, (long long)seq, (long long)rows, (double)base);
  return run_bwd(grad_y, h, 1, weight, inv_rms, nullptr, dx, nullptr, dweight, workspace,
                 ws_bytes, rows, dim, ld_g, ld_h, dim, ld_dx, dim, dtype, w_dtype, hip_stream,
                 seq, base);
}

}  // extern "C"
