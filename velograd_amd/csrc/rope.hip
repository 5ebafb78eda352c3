// Fused rotary position embedding (RoPE), hand-written for gfx950, in the reference's two
// pairings of a head vector's elements.
//
// Math, for every head vector x[o, s, h, :] at position s and pair j < half = rot_dim / 2:
//     freq_j = 1 / theta^(2j / rot_dim),  angle = s * freq_j
//     (fp32 for rotate half, fused.py:98-103; double for interleaved, functional.py:302-305)
//     (a, b) -> (a cos - b sin,  a sin + b cos)
//   "rotate half" (python/velograd/kernels/fused.py:72-130, src/cuda/fused_kernels.cu:145-181):
//     (a, b) = (x_j, x_{j+half}); elements at rot_dim and beyond are copied (fused.py:119-120).
//   interleaved (python/velograd/functional.py:287-315, the LLaMA model's RoPE, and
//     src/ops.rs:465-499): (a, b) = (x_{2j}, x_{2j+1}), both in the same 16-byte chunk.
// The inverse rotation (sin -> -sin) is the backward: the adjoint of a rotation is its inverse
// (the reference's rotary backward, src/ops.rs:501-530, for its own pairing).
//
// Layout: [outer, seq, heads, dim] contiguous; a "token" is the heads * dim elements of one
// (o, s).  A workgroup takes `tpb` consecutive tokens: it first writes freq_j and then cos/sin of
// every (token, pair) it needs into LDS (each computed once per workgroup instead of once per
// head), then streams the tokens' elements with 16-byte loads and stores, every element moving
// through HBM once.  The kernel is HBM-bound: ~6 flops per element pair.
//
// Numerics of rotate half: freq_j = 1 / powf(theta, e) in float32, as the reference forms it with NumPy's
// float32 power (faithful, within 1 ulp; so is ocml's powf: the two may differ by an ulp or
// two, which moves the angle by that many ulps of |angle|); the angle is the float32 product
// s * freq_j as np.outer forms it; sincosf is ocml's (a few ulps); products and sums round as
// NumPy's float32 ufuncs do (-ffp-contract=off).  A double-precision pow was measured to cost
// 89 VGPRs (5 waves per SIMD) against 50 (8 waves) for powf.

#include "common.h"

namespace {

using namespace vg;

constexpr int kRopeBlock = 256;
constexpr int kRopeMaxHalf = 4096;       // rot_dim <= 8192 (a whole hidden vector, interleaved)
constexpr int kRopeLdsFloats = 12288;    // bound on freq[half] + cos/sin[tpb][half]: 48 KiB
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
  int32_t interleaved;  // pairs (2j, 2j+1) instead of (j, j + half)
};

constexpr double kInv2Pi = 0.159154943091895335768883763372514362;  // 1 / (2 pi)

// Fills freq[half], then cos/sin[t * half + j] for the workgroup's tokens.  Rotate-half forms
// them in float32 as its reference does (fused.py:98-103); the interleaved pairing forms freq_j
// and the angle in double, as its reference's Python floats do (functional.py:302-305), and
// reduces the angle exactly to [-1/2, 1/2] revolutions before a float32 sincospi, so cos and
// sin are within a few float32 ulps at any position (the 16-byte path, rope_run_kernel, walks
// the same double-precision angles).
__device__ inline void rope_tables(const RopeArgs& a, int64_t tok0, int ntok, float* freq,
                                   float* cs, float* sn) {
  if (a.interleaved) {
    const double log2_theta = log2((double)a.theta);
    const int n = ntok * a.half;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      const int t = i / a.half;
      const int j = i - t * a.half;
      const double fr = exp2(-(double)j / (double)a.half * log2_theta);  // 1/theta^(2j/rot_dim)
      const double rev = (double)((tok0 + t) % a.seq) * fr * kInv2Pi;
      float s, c;
      sincospif(2.0f * (float)(rev - rint(rev)), &s, &c);
      cs[i] = c;
      sn[i] = a.sin_sign * s;
    }
    __syncthreads();
    return;
  }
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

template <int DT, bool VEC, bool INTERLEAVED>
__global__ __launch_bounds__(kRopeBlock) void rope_kernel(const RopeArgs a) {
  using C = Codec<DT>;
  constexpr int V = VEC ? C::kVec : 1;
  extern __shared__ float lds[];  // freq[half], cos[tpb][half], sin[tpb][half]
  const int64_t tok0 = (int64_t)blockIdx.x * a.tpb;
  const int ntok = (int)((a.tokens - tok0) < a.tpb ? (a.tokens - tok0) : a.tpb);
  float* freq = lds;
  float* cs = lds + a.half;
  float* sn = cs + a.tpb * a.half;

  if constexpr (INTERLEAVED) {
    // Scalar interleaved path (rows that do not split into whole 16-byte pairs of chunks): one
    // item = one pair of the rotated region [0, 2 * half), then the pass-through elements.  The
    // 16-byte path is rope_run_kernel.
    static_assert(!VEC, "interleaved 16-byte chunks go through rope_run_kernel");
    const int rot_items = a.half;
    const int tail_items = a.copy_tail ? a.dim - 2 * a.half : 0;
    const int per_head = rot_items + tail_items;
    const int per_tok = a.heads * per_head;
    const int n = ntok * per_tok;
    rope_tables(a, tok0, ntok, freq, cs, sn);
    for (int it = threadIdx.x; it < n; it += blockDim.x) {
      const RopeItem r = rope_item(a, tok0, it, per_tok, per_head);
      if (r.c < rot_items) {
        const float cv = cs[r.t * a.half + r.c], sv = sn[r.t * a.half + r.c];
        const float x1 = C::load1(a.x, r.head0 + 2 * r.c);
        const float x2 = C::load1(a.x, r.head0 + 2 * r.c + 1);
        C::store1(a.out, r.head0 + 2 * r.c, x1 * cv - x2 * sv);           // functional.py:313
        C::store1(a.out, r.head0 + 2 * r.c + 1, x1 * sv + x2 * cv);       // functional.py:314
      } else {
        const int64_t e0 = r.head0 + 2 * a.half + (r.c - rot_items);
        C::store1(a.out, e0, C::load1(a.x, e0));
      }
    }
    return;
  }

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

// Interleaved pairs, 16-byte path: a thread owns one chunk column (V / 2 pairs) of the token
// vector (heads * dim elements) of one outer index and walks the positions w, w + G, w + 2G, ...
// (G = ceil(seq / kRopeRun) position groups, about kRopeRun positions per thread), so that at any
// moment the whole grid works on a compact band of rows.  Its rotation (cos, sin) starts from a
// double-precision sincos of angle w * freq_j and advances by the rotation through G * freq_j,
// also in double (about 1e-16 drift per step): no per-(position, pair) sincos is evaluated.
// With the whole hidden vector rotated (the reference model's RoPE) there is no sharing across
// heads to amortise rope_kernel's tables, whose sincosf per (position, pair) bound that kernel
// by VALU at a quarter of the copy speed.  The angles come out closer to the reference's
// double-precision ones (functional.py:302-305) than a float32 angle does.  kRopeDepth loads
// stay in flight per thread; they are issued before the double-precision set-up.  The kernel is
// latency-bound on its loads, so the launch bounds ask for 4 waves per SIMD (128 VGPRs, no
// spills; 138 VGPRs and 3 waves ran 10% slower).
constexpr int kRopeRun = 32;
constexpr int kRopeDepth = 4;

template <int DT>
__global__ __launch_bounds__(kRopeBlock, 4) void rope_run_kernel(const RopeArgs a,
                                                                 int64_t col_blocks,
                                                                 int64_t groups) {
  using C = Codec<DT>;
  constexpr int V = C::kVec;
  constexpr int P = V / 2;
  const int64_t tok_elems = (int64_t)a.heads * a.dim;
  const int64_t tok_chunks = tok_elems / V;
  const int64_t blk = blockIdx.x;
  const int64_t run = blk / col_blocks;
  const int64_t col = (blk - run * col_blocks) * blockDim.x + threadIdx.x;
  if (col >= tok_chunks) return;
  const int64_t o = run / groups;
  const int64_t w = run - o * groups;                // first position; the walk strides by groups
  const int ns = (int)((a.seq - w + groups - 1) / groups);
  const int chunks_per_head = a.dim / V;
  const int h = (int)(col / chunks_per_head);
  const int c = (int)(col - (int64_t)h * chunks_per_head);
  const int64_t base0 = ((o * a.seq + w) * a.heads + h) * (int64_t)a.dim + (int64_t)c * V;
  const int64_t stride = groups * tok_elems;

  if (c * V >= 2 * a.half) {  // pass-through chunk past rot_dim
    if (!a.copy_tail) return;
    for (int t = 0; t < ns; ++t) {
      const int64_t e = base0 + (int64_t)t * stride;
      store16_stream<DT>(a.out, e, load16_stream<DT>(a.x, e));
    }
    return;
  }
  u32x4 buf[kRopeDepth];
#pragma unroll
  for (int u = 0; u < kRopeDepth; ++u)
    buf[u] = u < ns ? load16_stream<DT>(a.x, base0 + (int64_t)u * stride) : u32x4{0u, 0u, 0u, 0u};
  double cr[P], sr[P], cstep[P], sstep[P];
  const double log2_theta = log2((double)a.theta);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int j = c * P + p;
    const double fr = exp2(-(double)j / (double)a.half * log2_theta);  // 1/theta^(2j/rot_dim)
    double sv, cv;
    sincos((double)w * fr, &sv, &cv);
    cr[p] = cv;
    sr[p] = (double)a.sin_sign * sv;
    sincos((double)groups * fr, &sv, &cv);
    cstep[p] = cv;
    sstep[p] = (double)a.sin_sign * sv;
  }
  for (int t = 0; t < ns; t += kRopeDepth) {
#pragma unroll
    for (int u = 0; u < kRopeDepth; ++u) {
      const int tt = t + u;
      if (tt < ns) {
        float f[V];
        C::unpack(buf[u], f);
        if (tt + kRopeDepth < ns)
          buf[u] = load16_stream<DT>(a.x, base0 + (int64_t)(tt + kRopeDepth) * stride);
#pragma unroll
        for (int p = 0; p < P; ++p) {
          const float cv = (float)cr[p], sv = (float)sr[p];
          const float x1 = f[2 * p], x2 = f[2 * p + 1];
          f[2 * p] = x1 * cv - x2 * sv;                                  // functional.py:313
          f[2 * p + 1] = x1 * sv + x2 * cv;                              // functional.py:314
          const double cn = cr[p] * cstep[p] - sr[p] * sstep[p];
          sr[p] = sr[p] * cstep[p] + cr[p] * sstep[p];
          cr[p] = cn;
        }
        store16_stream<DT>(a.out, base0 + (int64_t)tt * stride, C::pack(f));
      }
    }
  }
}

template <int DT>
void launch_rope(const RopeArgs& a, bool vec, hipStream_t st) {
  const dim3 grid((uint32_t)((a.tokens + a.tpb - 1) / a.tpb));
  const size_t lds = (size_t)(a.half + 2 * a.tpb * a.half) * sizeof(float);
  if (a.interleaved) {
    if (vec) {
      const int64_t col_blocks =
          ((int64_t)a.heads * a.dim / Codec<DT>::kVec + kRopeBlock - 1) / kRopeBlock;
      const int64_t groups = (a.seq + kRopeRun - 1) / kRopeRun;
      const int64_t outer = a.tokens / a.seq;
      hipLaunchKernelGGL((rope_run_kernel<DT>), dim3((uint32_t)(col_blocks * groups * outer)),
                         dim3(kRopeBlock), 0, st, a, col_blocks, groups);
    } else {
      hipLaunchKernelGGL((rope_kernel<DT, false, true>), grid, dim3(kRopeBlock), lds, st, a);
    }
  } else {
    if (vec)
      hipLaunchKernelGGL((rope_kernel<DT, true, false>), grid, dim3(kRopeBlock), lds, st, a);
    else
      hipLaunchKernelGGL((rope_kernel<DT, false, false>), grid, dim3(kRopeBlock), lds, st, a);
  }
}

}  // namespace

extern "C" {

VELOGRAD_API int32_t velograd_rope(const void* x, void* out, int64_t outer, int64_t seq,
                                   int64_t heads, int64_t dim, int64_t rot_dim, float theta,
                                   int32_t inverse, int32_t pairing, int32_t dtype,
                                   void* hip_stream) {
  const int eb = elem_bytes_of(dtype);
  if (eb == 0)
    return fail(VELOGRAD_ERR_UNSUPPORTED_DTYPE, "rope: unsupported dtype %d", (int)dtype);
  if (pairing != VELOGRAD_ROPE_HALF && pairing != VELOGRAD_ROPE_INTERLEAVED)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "rope: unknown pairing %d", (int)pairing);
  if (outer < 0 || seq < 0 || heads < 0 || dim < 0)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT,
                "rope: invalid shape outer=%lld seq=%lld heads=%lld dim=%lld", (long long)outer,
                (long long)seq, (long long)heads, (long long)dim);
  if (outer == 0 || seq == 0 || heads == 0 || dim == 0) {
    clear_error();
    return 0;
  }
  if (rot_dim < 2 || rot_dim % 2 != 0 || rot_dim > dim)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT,
                "rope: rot_dim=%lld must be even, >= 2 and <= dim=%lld", (long long)rot_dim,
                (long long)dim);
  // The table kernels hold one token's frequencies and (cos, sin) in LDS: rot_dim <= 8192.  The
  // interleaved pairing on 16-byte chunks walks positions without tables (rope_run_kernel), so it
  // takes any rot_dim (a whole hidden vector of 16384, say).
  const int vec_chunk = 16 / eb;
  const bool run_path = pairing == VELOGRAD_ROPE_INTERLEAVED && aligned16(x) && aligned16(out) &&
                        dim % vec_chunk == 0 && rot_dim % vec_chunk == 0;
  if (rot_dim / 2 > kRopeMaxHalf && !run_path)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT,
                "rope: rot_dim=%lld above %d needs the interleaved pairing on 16-byte aligned, "
                "16-byte multiple rows",
                (long long)rot_dim, 2 * kRopeMaxHalf);
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
  a.interleaved = pairing == VELOGRAD_ROPE_INTERLEAVED ? 1 : 0;
  // Tokens per workgroup: about kRopeTargetElems elements, bounded by the LDS tables
  // (freq[half] + cos/sin[tpb][half]) and by the items a workgroup indexes in int32.
  int64_t tpb = (kRopeTargetElems + tok_elems - 1) / tok_elems;
  const int64_t lds_cap = a.half <= kRopeMaxHalf ? (kRopeLdsFloats - a.half) / (2 * a.half) : 1;
  if (tpb > lds_cap) tpb = lds_cap;
  if (tpb > 64) tpb = 64;
  if (tpb < 1) tpb = 1;
  a.tpb = (int32_t)tpb;
  const int64_t grid = (a.tokens + tpb - 1) / tpb;
  if (grid > INT32_MAX)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "rope: %lld tokens exceed the grid limit",
                (long long)a.tokens);

  const int vec_elems = 16 / eb;
  if (pairing == VELOGRAD_ROPE_INTERLEAVED) {
    const int64_t run_blocks = ((tok_elems / vec_elems + kRopeBlock - 1) / kRopeBlock) *
                               ((seq + kRopeRun - 1) / kRopeRun) * outer;
    if (run_blocks > INT32_MAX)
      return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "rope: tensor too large for the grid");
  }
  // 16-byte chunks must not straddle the rotated region's boundaries: rotate-half needs each
  // half chunk-aligned, interleaved the whole region (a chunk then holds whole pairs).
  const bool vec = aligned16(x) && aligned16(out) && a.dim % vec_elems == 0 &&
                   (a.interleaved ? (2 * a.half) % vec_elems == 0 : a.half % vec_elems == 0);
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  switch (dtype) {
    case VELOGRAD_DTYPE_F32: launch_rope<VELOGRAD_DTYPE_F32>(a, vec, st); break;
    case VELOGRAD_DTYPE_F16: launch_rope<VELOGRAD_DTYPE_F16>(a, vec, st); break;
    default: launch_rope<VELOGRAD_DTYPE_BF16>(a, vec, st); break;
  }
  return check_launch("velograd_rope");
}

}  // extern "C"
