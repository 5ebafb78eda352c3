// Fused rotary position embedding (RoPE), "rotate half" pairing, hand-written for gfx950.
//
// Math (reference: python/velograd/kernels/fused.py:72-130, fused_rope_forward):
//   for every head vector x[o, s, h, :] at position s, pair j < half = rot_dim / 2:
//     freq_j = 1 / theta^(2j / rot_dim),  angle = s * freq_j          (fp32, fused.py:98-103)
//     (x_j, x_{j+half}) -> (x_j cos - x_{j+half} sin,  x_j sin + x_{j+half} cos)
//   elements at rot_dim and beyond are copied (fused.py:119-120).
// The inverse rotation (sin -> -sin) is the backward: the adjoint of a rotation is its inverse
// (the reference's rotary backward, src/ops.rs:501-530, for its own pairing).
//
// Layout: [outer, seq, heads, dim] contiguous; a "token" is the heads * dim elements of one
// (o, s).  A workgroup takes `tpb` consecutive tokens: it first writes freq_j and then cos/sin of
// every (token, pair) it needs into LDS (each computed once per workgroup instead of once per
// head), then streams the tokens' elements with 16-byte loads and stores, every element moving
// through HBM once.  The kernel is HBM-bound: ~6 flops per element pair.
//
// Numerics: freq_j = 1 / powf(theta, e) in float32, as the reference forms it with NumPy's
// float32 power (faithful, within 1 ulp; so is ocml's powf: the two may differ by an ulp or
// two, which moves the angle by that many ulps of |angle|); the angle is the float32 product
// s * freq_j as np.outer forms it; sincosf is ocml's (a few ulps); products and sums round as
// NumPy's float32 ufuncs do (-ffp-contract=off).  A double-precision pow was measured to cost
// 89 VGPRs (5 waves per SIMD) against 50 (8 waves) for powf.

#include "common.h"

namespace {

using namespace vg;

constexpr int kRopeBlock = 256;
constexpr int kRopeMaxHalf = 2048;       // rot_dim <= 4096
constexpr int kRopeLdsFloats = 8192;     // bound on freq[half] + cos/sin[tpb][half]: 32 KiB
static_assert(3 * kRopeMaxHalf <= kRopeLdsFloats, "one token's tables must fit the LDS array");
constexpr int kRopeTargetElems = 4096;   // elements per workgroup the token grouping aims at

struct RopeArgs {
  const void* x;
  void* out;
  int64_t tokens;   // outer * seq
  int32_t seq;
  int32_t heads;
  int32_t dim;
  int32_t half;
  int32_t tpb;      // tokens per workgroup
  int32_t copy_tail;
  float theta;
  float sin_sign;   // +1 forward, -1 inverse
};

// Fills freq[half], then cos/sin[t * half + j] for the workgroup's tokens.
__device__ inline void rope_tables(const RopeArgs& a, int64_t tok0, int ntok, float* freq,
                                   float* cs, float* sn) {
  for (int j = threadIdx.x; j < a.half; j += blockDim.x) {
    const float e = (2.0f * (float)j) / (float)(2 * a.half);          // fused.py:100
    const float p = powf(a.theta, e);
    freq[j] = 1.0f / p;
  }
  __syncthreads();
  const int n = ntok * a.half;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int t = i / a.half;
    const int j = i - t * a.half;
    const float pos = (float)((tok0 + t) % a.seq);                       // fused.py:98
    float s, c;
    sincosf(pos * freq[j], &s, &c);                                      // fused.py:101-103
    cs[i] = c;
    sn[i] = a.sin_sign * s;
  }
  __syncthreads();
}

// Item `it` of a workgroup: token t, head h, chunk c of that head (chunks < rot_items are pairs
// of rotated chunks, the rest pass-through chunks).
struct RopeItem {
  int t, c;
  int64_t head0;  // element offset of the head vector
};

__device__ inline RopeItem rope_item(const RopeArgs& a, int64_t tok0, int it, int per_tok,
                                     int per_head) {
  RopeItem r;
  r.t = it / per_tok;
  const int rest = it - r.t * per_tok;
  const int h = rest / per_head;
  r.c = rest - h * per_head;
  r.head0 = ((tok0 + r.t) * a.heads + h) * (int64_t)a.dim;
  return r;
}

// VEC: 16-byte chunks (needs half and dim multiples of the chunk, 16-byte aligned tensors);
// otherwise one element (pair) per item.  The first kPrefetch items of every thread are loaded
// before the tables are built, so the table work overlaps their HBM latency.
constexpr int kPrefetch = 2;

template <int DT, bool VEC>
__global__ __launch_bounds__(kRopeBlock) void rope_kernel(const RopeArgs a) {
  using C = Codec<DT>;
  constexpr int V = VEC ? C::kVec : 1;
  extern __shared__ float lds[];  // freq[half], cos[tpb][half], sin[tpb][half]
  const int64_t tok0 = (int64_t)blockIdx.x * a.tpb;
  const int ntok = (int)((a.tokens - tok0) < a.tpb ? (a.tokens - tok0) : a.tpb);
  float* freq = lds;
  float* cs = lds + a.half;
  float* sn = cs + a.tpb * a.half;

  const int rot_items = a.half / V;                                     // per head
  const int tail_items = a.copy_tail ? (a.dim - 2 * a.half) / V : 0;   // per head
  const int per_head = rot_items + tail_items;
  const int per_tok = a.heads * per_head;
  const int n = ntok * per_tok;

  auto rotate_store = [&](const RopeItem& r, const u32x4 va, const u32x4 vb) {
    const int j0 = r.c * V;
    const float* cp = cs + r.t * a.half + j0;
    const float* sp = sn + r.t * a.half + j0;
    float x1[C::kVec], x2[C::kVec], r1[C::kVec], r2[C::kVec];
    C::unpack(va, x1);
    C::unpack(vb, x2);
#pragma unroll
    for (int i = 0; i < C::kVec; ++i) {
      const float cv = cp[i], sv = sp[i];
      r1[i] = x1[i] * cv - x2[i] * sv;                                   // fused.py:116
      r2[i] = x1[i] * sv + x2[i] * cv;                                   // fused.py:117
    }
    store16_stream<DT>(a.out, r.head0 + j0, C::pack(r1));
    store16_stream<DT>(a.out, r.head0 + a.half + j0, C::pack(r2));
  };

  if constexpr (VEC) {
    u32x4 pa[kPrefetch], pb[kPrefetch];
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p) {
      const int it = threadIdx.x + p * blockDim.x;
      pa[p] = u32x4{0u, 0u, 0u, 0u};
      pb[p] = u32x4{0u, 0u, 0u, 0u};
      if (it < n) {
        const RopeItem r = rope_item(a, tok0, it, per_tok, per_head);
        if (r.c < rot_items) {
          pa[p] = load16_stream<DT>(a.x, r.head0 + r.c * V);
          pb[p] = load16_stream<DT>(a.x, r.head0 + a.half + r.c * V);
        } else {
          pa[p] = load16_stream<DT>(a.x, r.head0 + 2 * a.half + (int64_t)(r.c - rot_items) * V);
        }
      }
    }
    rope_tables(a, tok0, ntok, freq, cs, sn);
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p) {
      const int it = threadIdx.x + p * blockDim.x;
      if (it < n) {
        const RopeItem r = rope_item(a, tok0, it, per_tok, per_head);
        if (r.c < rot_items)
          rotate_store(r, pa[p], pb[p]);
        else
          store16_stream<DT>(a.out, r.head0 + 2 * a.half + (int64_t)(r.c - rot_items) * V, pa[p]);
      }
    }
    for (int it = threadIdx.x + kPrefetch * blockDim.x; it < n; it += blockDim.x) {
      const RopeItem r = rope_item(a, tok0, it, per_tok, per_head);
      if (r.c < rot_items) {
        rotate_store(r, load16_stream<DT>(a.x, r.head0 + r.c * V),
                     load16_stream<DT>(a.x, r.head0 + a.half + r.c * V));
      } else {
        const int64_t e0 = r.head0 + 2 * a.half + (int64_t)(r.c - rot_items) * V;
        store16_stream<DT>(a.out, e0, load16_stream<DT>(a.x, e0));
      }
    }
  } else {
    rope_tables(a, tok0, ntok, freq, cs, sn);
    for (int it = threadIdx.x; it < n; it += blockDim.x) {
      const RopeItem r = rope_item(a, tok0, it, per_tok, per_head);
      if (r.c < rot_items) {
        const float* cp = cs + r.t * a.half + r.c;
        const float* sp = sn + r.t * a.half + r.c;
        const float x1 = C::load1(a.x, r.head0 + r.c);
        const float x2 = C::load1(a.x, r.head0 + a.half + r.c);
        C::store1(a.out, r.head0 + r.c, x1 * cp[0] - x2 * sp[0]);
        C::store1(a.out, r.head0 + a.half + r.c, x1 * sp[0] + x2 * cp[0]);
      } else {
        const int64_t e0 = r.head0 + 2 * a.half + (r.c - rot_items);
        C::store1(a.out, e0, C::load1(a.x, e0));
      }
    }
  }
}

template <int DT>
void launch_rope(const RopeArgs& a, bool vec, hipStream_t st) {
  const dim3 grid((uint32_t)((a.tokens + a.tpb - 1) / a.tpb));
  const size_t lds = (size_t)(a.half + 2 * a.tpb * a.half) * sizeof(float);
  if (vec)
    hipLaunchKernelGGL((rope_kernel<DT, true>), grid, dim3(kRopeBlock), lds, st, a);
  else
    hipLaunchKernelGGL((rope_kernel<DT, false>), grid, dim3(kRopeBlock), lds, st, a);
}

}  // namespace

extern "C" {

VELOGRAD_API int32_t velograd_rope(const void* x, void* out, int64_t outer, int64_t seq,
                                   int64_t heads, int64_t dim, int64_t rot_dim, float theta,
                                   int32_t inverse, int32_t dtype, void* hip_stream) {
  const int eb = elem_bytes_of(dtype);
  if (eb == 0)
    return fail(VELOGRAD_ERR_UNSUPPORTED_DTYPE, "rope: unsupported dtype %d", (int)dtype);
  if (outer < 0 || seq < 0 || heads < 0 || dim < 0)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT,
                "rope: invalid shape outer=%lld seq=%lld heads=%lld dim=%lld", (long long)outer,
                (long long)seq, (long long)heads, (long long)dim);
  if (outer == 0 || seq == 0 || heads == 0 || dim == 0) {
    clear_error();
    return 0;
  }
  if (rot_dim < 2 || rot_dim % 2 != 0 || rot_dim > dim || rot_dim / 2 > kRopeMaxHalf)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT,
                "rope: rot_dim=%lld must be even, >= 2, <= dim=%lld and <= %d",
                (long long)rot_dim, (long long)dim, 2 * kRopeMaxHalf);
  if (x == nullptr || out == nullptr)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "rope: x and out must not be NULL");
  if (!(theta > 0.0f))
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "rope: theta must be positive");
  if (seq > INT32_MAX || heads > INT32_MAX || dim > INT32_MAX)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "rope: seq, heads and dim must fit in int32");
  const int64_t tok_elems = heads * dim;
  if (tok_elems > INT32_MAX / 2 || outer > INT64_MAX / seq)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "rope: tensor too large");

  RopeArgs a;
  a.x = x;
  a.out = out;
  a.tokens = outer * seq;
  a.seq = (int32_t)seq;
  a.heads = (int32_t)heads;
  a.dim = (int32_t)dim;
  a.half = (int32_t)(rot_dim / 2);
  a.copy_tail = (out != x && rot_dim < dim) ? 1 : 0;
  a.theta = theta;
  a.sin_sign = inverse ? -1.0f : 1.0f;
  // Tokens per workgroup: about kRopeTargetElems elements, bounded by the LDS tables
  // (freq[half] + cos/sin[tpb][half]) and by the items a workgroup indexes in int32.
  int64_t tpb = (kRopeTargetElems + tok_elems - 1) / tok_elems;
  const int64_t lds_cap = (kRopeLdsFloats - a.half) / (2 * a.half);
  if (tpb > lds_cap) tpb = lds_cap;
  if (tpb > 64) tpb = 64;
  if (tpb < 1) tpb = 1;
  a.tpb = (int32_t)tpb;
  const int64_t grid = (a.tokens + tpb - 1) / tpb;
  if (grid > INT32_MAX)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "rope: %lld tokens exceed the grid limit",
                (long long)a.tokens);

  const int vec_elems = 16 / eb;
  const bool vec = aligned16(x) && aligned16(out) && a.half % vec_elems == 0 &&
                   a.dim % vec_elems == 0;
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  switch (dtype) {
    case VELOGRAD_DTYPE_F32: launch_rope<VELOGRAD_DTYPE_F32>(a, vec, st); break;
    case VELOGRAD_DTYPE_F16: launch_rope<VELOGRAD_DTYPE_F16>(a, vec, st); break;
    default: launch_rope<VELOGRAD_DTYPE_BF16>(a, vec, st); break;
  }
  return check_launch("velograd_rope");
}

}  // extern "C"
