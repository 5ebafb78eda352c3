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
// sin are within a few float32 ulps at any position (the 16-byte path, rope_tile_kernel, forms
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
    // 16-byte path is rope_tile_kernel.
    static_assert(!VEC, "interleaved 16-byte chunks go through rope_tile_kernel");
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

// Interleaved pairs, 16-byte path: a one-pass grid of short tiles.  A thread owns one chunk
// column (P = V / 2 pairs) of kRopeTileRows consecutive positions of one sequence: it issues the
// tile's loads back to back (a position past the sequence's end re-reads the last one and stores
// nothing), forms its pairs' frequencies and rotations while they are in flight, then rotates
// and stores each position.  A 256-thread workgroup takes 256 chunk columns of one tile (or, for
// token vectors of fewer than 256 chunks, whole token vectors of several tiles), so consecutive
// workgroups sweep the tensor front to back as the copy kernels do.  Short-lived threads whose
// loads are all in flight at once keep HBM busier than long walks down the positions (each thread
// walking ~32 positions with 4 loads in flight ran 49.5-49.8 us at [16384, 4096] bf16 against
// 44.2-44.4 us here; the 1R1W copy takes 43.4-44.0).
//
// Angles, as the reference's Python floats form them (functional.py:302-305): the pair frequency
// in revolutions per position, g_j = theta^(-j / half) / (2 pi), in double (one exp2 per chunk,
// then the chunk's next pairs by the double ratio theta^(-1 / half)); the angle of position s is
// s * g_j in double, reduced exactly to [-1/2, 1/2] revolutions (rev - rint(rev) is exact) before
// a float32 sincospi, so cos and sin are within a few float32 ulps at any position.
//   fp32 outputs: every position evaluates its own angle that way.
//   bf16/fp16 outputs: the tile's first position does; the next ones advance the float32
//   rotation by the step rotation (cos g_j 2pi, sin g_j 2pi), at most kRopeTileRows - 1 steps of
//   a few float32 ulps each, far below those formats' rounding.  The step's angle g_j 2pi is at
//   most 1 radian when theta >= 1 and takes the Taylor series of cos and sin (below); a base under
//   1 reduces it as the anchors are reduced.
constexpr int kRopeTileRows = 3;
constexpr double kTwoPi = 6.283185307179586476925286766559005768;

// cos and sin of 2 pi rev for any double rev: exact reduction to [-1/2, 1/2], then sincospi.
__device__ inline void cos_sin_rev(double rev, float& c, float& s) {
  sincospif(2.0f * (float)(rev - rint(rev)), &s, &c);
}

struct RopeTileGrid {
  int32_t tok_chunks;   // 16-byte chunks per token vector (heads * dim / V)
  int32_t col_blocks;   // workgroups per tile when tok_chunks >= kRopeBlock, else 0
  int32_t tiles_per_block;  // tiles per workgroup when tok_chunks < kRopeBlock, else 1
  int64_t row_tiles;    // tiles per sequence: ceil(seq / kRopeTileRows)
  int64_t tiles;        // outer * row_tiles
  double g_log2_step;   // -log2(theta) / half: g_j = 2^(j * g_log2_step) / (2 pi)
  double g_ratio;       // theta^(-1 / half): g_{j+1} = g_j * g_ratio
};

template <int DT>
__global__ __launch_bounds__(kRopeBlock) void rope_tile_kernel(const RopeArgs a,
                                                               const RopeTileGrid gd) {
  using C = Codec<DT>;
  constexpr int V = C::kVec;
  constexpr int P = V / 2;
  constexpr int R = kRopeTileRows;
  int64_t tile;
  int32_t col;
  if (gd.col_blocks > 0) {
    const int64_t blk = blockIdx.x;
    tile = blk / gd.col_blocks;
    col = (int32_t)(blk - tile * gd.col_blocks) * kRopeBlock + (int32_t)threadIdx.x;
    if (col >= gd.tok_chunks) return;
  } else {
    const int32_t t = (int32_t)threadIdx.x / gd.tok_chunks;
    if (t >= gd.tiles_per_block) return;
    col = (int32_t)threadIdx.x - t * gd.tok_chunks;
    tile = (int64_t)blockIdx.x * gd.tiles_per_block + t;
    if (tile >= gd.tiles) return;
  }
  const int64_t o = tile / gd.row_tiles;
  const int64_t s0 = (tile - o * gd.row_tiles) * R;
  const int ns = (int)((a.seq - s0) < R ? (a.seq - s0) : R);   // >= 1
  const int64_t tok_elems = (int64_t)gd.tok_chunks * V;
  const int64_t base = (o * a.seq + s0) * tok_elems + (int64_t)col * V;
  const int32_t c = col % (a.dim / V);
  if (c * V >= 2 * a.half) {  // pass-through chunk past rot_dim
    if (!a.copy_tail) return;
    u32x4 buf[R];
#pragma unroll
    for (int u = 0; u < R; ++u)
      buf[u] = load16_stream<DT>(a.x, base + (int64_t)(u < ns ? u : ns - 1) * tok_elems);
#pragma unroll
    for (int u = 0; u < R; ++u)
      if (u < ns) store16_stream<DT>(a.out, base + (int64_t)u * tok_elems, buf[u]);
    return;
  }
  // Every load is issued before any arithmetic (no branch between them, so no wait either).
  u32x4 buf[R];
#pragma unroll
  for (int u = 0; u < R; ++u)
    buf[u] = load16_stream<DT>(a.x, base + (int64_t)(u < ns ? u : ns - 1) * tok_elems);
  double g = exp2((double)(c * P) * gd.g_log2_step) * kInv2Pi;
  if constexpr (DT == VELOGRAD_DTYPE_F32) {
    double gp[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      gp[p] = g;
      g *= gd.g_ratio;
    }
#pragma unroll
    for (int u = 0; u < R; ++u) {
      if (u < ns) {
        float f[V];
        C::unpack(buf[u], f);
#pragma unroll
        for (int p = 0; p < P; ++p) {
          float cv, sv;
          cos_sin_rev((double)(s0 + u) * gp[p], cv, sv);
          sv *= a.sin_sign;
          const float x1 = f[2 * p], x2 = f[2 * p + 1];
          f[2 * p] = x1 * cv - x2 * sv;                                  // functional.py:313
          f[2 * p + 1] = x1 * sv + x2 * cv;                              // functional.py:314
        }
        store16_stream<DT>(a.out, base + (int64_t)u * tok_elems, C::pack(f));
      }
    }
  } else {
    float cr[P], sr[P], cs[P], ss[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      float cv, sv;
      cos_sin_rev((double)s0 * g, cv, sv);
      cr[p] = cv;
      sr[p] = a.sin_sign * sv;
      if (a.theta >= 1.0f)
        cos_sin_small((float)(g * kTwoPi), cv, sv);
      else
        cos_sin_rev(g, cv, sv);
      cs[p] = cv;
      ss[p] = a.sin_sign * sv;
      g *= gd.g_ratio;
    }
#pragma unroll
    for (int u = 0; u < R; ++u) {
      if (u < ns) {
        float f[V];
        C::unpack(buf[u], f);
#pragma unroll
        for (int p = 0; p < P; ++p) {
          const float x1 = f[2 * p], x2 = f[2 * p + 1];
          f[2 * p] = x1 * cr[p] - x2 * sr[p];                            // functional.py:313
          f[2 * p + 1] = x1 * sr[p] + x2 * cr[p];                        // functional.py:314
          if (u + 1 < R) {
            const float cn = fmaf(cr[p], cs[p], -(sr[p] * ss[p]));
            sr[p] = fmaf(sr[p], cs[p], cr[p] * ss[p]);
            cr[p] = cn;
          }
        }
        store16_stream<DT>(a.out, base + (int64_t)u * tok_elems, C::pack(f));
      }
    }
  }
}

RopeTileGrid rope_tile_grid(const RopeArgs& a, int vec) {
  RopeTileGrid g;
  g.tok_chunks = (int32_t)((int64_t)a.heads * a.dim / vec);
  g.col_blocks = g.tok_chunks >= kRopeBlock ? (g.tok_chunks + kRopeBlock - 1) / kRopeBlock : 0;
  g.tiles_per_block = g.tok_chunks >= kRopeBlock ? 1 : kRopeBlock / g.tok_chunks;
  g.row_tiles = (a.seq + kRopeTileRows - 1) / kRopeTileRows;
  g.tiles = (a.tokens / a.seq) * g.row_tiles;
  g.g_log2_step = -log2((double)a.theta) / (double)a.half;
  g.g_ratio = exp2(g.g_log2_step);
  return g;
}

int64_t rope_tile_blocks(const RopeTileGrid& g) {
  return g.col_blocks > 0 ? g.tiles * g.col_blocks
                          : (g.tiles + g.tiles_per_block - 1) / g.tiles_per_block;
}

template <int DT>
void launch_rope(const RopeArgs& a, bool vec, hipStream_t st) {
  const dim3 grid((uint32_t)((a.tokens + a.tpb - 1) / a.tpb));
  const size_t lds = (size_t)(a.half + 2 * a.tpb * a.half) * sizeof(float);
  if (a.interleaved) {
    if (vec) {
      const RopeTileGrid gd = rope_tile_grid(a, Codec<DT>::kVec);
      hipLaunchKernelGGL((rope_tile_kernel<DT>), dim3((uint32_t)rope_tile_blocks(gd)),
                         dim3(kRopeBlock), 0, st, a, gd);
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
  // interleaved pairing on 16-byte chunks forms its angles without tables (rope_tile_kernel), so
  // it takes any rot_dim (a whole hidden vector of 16384, say).
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
  const int vec_elems = 16 / eb;
  const int64_t grid = run_path ? rope_tile_blocks(rope_tile_grid(a, vec_elems))
                                : (a.tokens + tpb - 1) / tpb;
  if (grid > INT32_MAX)
    return fail(VELOGRAD_ERR_INVALID_ARGUMENT, "rope: %lld tokens exceed the grid limit",
                (long long)a.tokens);

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
