// Launch plans of the fused RMSNorm + residual kernels (host-only C++, no HIP dependency), so
// the planner can be compiled and checked on a CPU (tests/plan_check.cpp, under ASan/UBSan).
//
// A row of `dim` elements is cut into 16-byte chunks (8 bf16/fp16 or 4 fp32 elements).  The
// register-resident kernels give each row `tpr` threads (whole wave64s) and each thread NV
// chunks, c = lane + k * tpr for k < NV, so that consecutive lanes touch consecutive 16-byte
// chunks (coalesced 1 KiB per wave instruction).  Rows whose length is not a multiple of the
// chunk, misaligned rows, and rows too long for registers use the generic looping kernels.
#ifndef VELOGRAD_LAUNCH_PLAN_H
#define VELOGRAD_LAUNCH_PLAN_H

#include <stddef.h>
#include <stdint.h>

#ifndef VG_HOST_DEVICE
#define VG_HOST_DEVICE
#endif

namespace vg_plan {

constexpr int kWave = 64;
constexpr int kMaxWavesPerRow = 16;  // 1024 threads per row at most
// 16-byte chunks per thread in the register-resident path.  Capped at 4: the one-wave-per-row
// forward with 8 chunks per thread (191 VGPRs) made an illegal memory access on MI355X although
// its launch plan was correct (checked on the CPU by intercepting the launch); until that is
// understood, NV 5..8 are neither planned nor compiled.
constexpr int kMaxNV = 4;
constexpr int kGenericBlock = 256;
// The generic backward sums a slot's dweight columns in dynamic LDS (dim floats) for rows of up
// to kGenericLdsCols elements (64 KiB of LDS a workgroup, less its static row-sum buffers), else
// in its partial row in global memory.  Returns the launch's dynamic LDS bytes.
constexpr int kGenericLdsCols = 16000;
VG_HOST_DEVICE constexpr size_t generic_bwd_lds_bytes(int64_t dim, bool dweight) {
  return dweight && dim > 0 && dim <= kGenericLdsCols ? (size_t)dim * sizeof(float) : 0;
}

// Workgroup size bound of the register-resident kernels, so that a thread's packed chunks fit
// its VGPR budget (512 VGPRs per SIMD lane shared by the block's waves on that SIMD):
// NV <= 2 -> 1024 threads (128 VGPRs), NV 3..4 -> 512 (256).
VG_HOST_DEVICE constexpr int max_block_for_nv(int nv) { return nv <= 2 ? 1024 : 512; }

// The same bound for the backward with the fused inverse RoPE of grad_y: its rotation state
// (cos and sin per pair) takes more VGPRs, so NV 1 -> 1024 threads (95 VGPRs used),
// NV 2 and 3 -> 512 (256); with NV 4 the kernel would spill, so those rows take the generic
// kernel.
VG_HOST_DEVICE constexpr int max_block_for_nv_rope(int nv) {
  return nv <= 1 ? 1024 : (nv <= 3 ? 512 : 0);
}

struct RowPlan {
  bool vec;    // register-resident path
  int nv;      // 16-byte chunks per thread
  int tpr;     // threads per row
  int groups;  // rows per workgroup
  int block;   // threads per workgroup = tpr * groups
};

// Automatic orders in which chunks-per-thread values are tried (measured on MI355X, bf16 rows of
// 4096 and 8192): the forward with a residual (two streams read, two written) is fastest with
// one chunk per thread (more waves per row, all of a row's loads in one instruction per lane);
// without one (x read, y written) with two, since one 16-byte load per lane leaves too few
// bytes in flight (16384 x 4096: 44.5 us against 51.0 us, the plain copy's speed); the
// persistent backward with two (it keeps the next row's chunks in flight too, so it trades
// waves for bytes per lane).
constexpr int kFwdOrder[kMaxNV] = {1, 2, 3, 4};
constexpr int kFwdOrderOneStream[kMaxNV] = {2, 4, 3, 1};
// The quantised epilogues (fp8 per row, MXFP8, MXFP4) reduce each row twice (sum of squares,
// then amax), so fewer waves per row pay off there: two chunks per thread against one ran
// 76.9 / 301.5 / 39.9 us against 79.6 / 335.0 / 42.5 us for the per-row fp8 forward at configs
// C / D / B (and MXFP4 at D 280 against 314); four chunks were within 1% at C and D and 2-3%
// slower at B.
constexpr int kFwdOrderEpilogue[kMaxNV] = {2, 4, 3, 1};
constexpr int kBwdOrder[kMaxNV] = {2, 3, 4, 1};
// The backward with the fused RoPE gradient prefers one chunk per thread: its rotation state
// then fits 1024-thread workgroups (16384 x 4096 bf16: 84.0 us against 89.7 us at two chunks
// in 768-thread workgroups).
constexpr int kBwdOrderRope[kMaxNV] = {1, 2, 3, 4};

// Register-resident layout for rows of `dim` elements of `elem_bytes` bytes, or the generic
// plan when the row does not split into 16-byte chunks or does not fit in registers.
// `prefer_nv` (1..kMaxNV, 0 = automatic) is tried first, then `auto_order`; the first choice
// whose idle lanes stay under 1/8 wins, else the least idle one.
inline RowPlan plan_rows(int64_t dim, int elem_bytes, bool aligned, int prefer_nv,
                         const int (&auto_order)[kMaxNV]) {
  RowPlan p{false, 0, kGenericBlock, 1, kGenericBlock};
  if (elem_bytes != 2 && elem_bytes != 4) return p;
  const int V = 16 / elem_bytes;
  if (!aligned || dim <= 0 || dim % V != 0) return p;
  const int64_t chunks = dim / V;
  int order[1 + kMaxNV];
  int n = 0;
  if (prefer_nv >= 1 && prefer_nv <= kMaxNV) order[n++] = prefer_nv;
  for (int i = 0; i < kMaxNV; ++i)
    if (auto_order[i] != prefer_nv) order[n++] = auto_order[i];
  int best_nv = 0, best_wpr = 0;
  int64_t best_waste = -1;
  for (int i = 0; i < n; ++i) {
    const int nv = order[i];
    const int64_t wpr = (chunks + (int64_t)kWave * nv - 1) / ((int64_t)kWave * nv);
    if (wpr * kWave > max_block_for_nv(nv)) continue;
    const int64_t slots = wpr * kWave * nv;
    const int64_t waste = slots - chunks;
    if (waste * 8 <= slots) {
      best_nv = nv;
      best_wpr = (int)wpr;
      break;
    }
    if (best_waste < 0 || waste < best_waste) {
      best_waste = waste;
      best_nv = nv;
      best_wpr = (int)wpr;
    }
  }
  if (best_nv == 0) return p;
  p.vec = true;
  p.nv = best_nv;
  p.tpr = best_wpr * kWave;
  p.groups = p.tpr >= 256 ? 1 : 256 / p.tpr;
  p.block = p.tpr * p.groups;
  return p;
}

// Where the register-resident forward stores h: after the row reduction, beside y, when a row
// takes at most kLateHMaxTpr threads; before it otherwise.  Measured on MI355X (bf16, A/B in
// one process, batched launches over rotating buffer sets, 6 rounds): after is faster at dim
// 2048 (86.6 against 87.5 us for 32768 rows) and 4096 (86.0 against 86.8 us at 16384 rows;
// 44.9 against 45.2 at 8192), equal at 3072 (65.2 / 65.1 us), slower at 5120 (110.7 against
// 109.5) and 8192 (179.1 against 172.7).
constexpr int kLateHMaxTpr = 512;

inline bool fwd_late_h(const RowPlan& p) { return p.vec && p.tpr <= kLateHMaxTpr; }

// The facts the kernels' indexing relies on; the C entry points refuse to launch a plan that
// breaks one of them.
inline bool row_plan_valid(const RowPlan& p, int64_t dim, int elem_bytes) {
  if (!p.vec)
    return p.tpr == kGenericBlock && p.groups == 1 && p.block == kGenericBlock;
  if (elem_bytes != 2 && elem_bytes != 4) return false;
  const int V = 16 / elem_bytes;
  return dim > 0 && dim % V == 0 && p.nv >= 1 && p.nv <= kMaxNV && p.tpr >= kWave &&
         p.tpr % kWave == 0 && p.groups >= 1 && p.block == p.tpr * p.groups &&
         p.block <= max_block_for_nv(p.nv) && (int64_t)p.nv * p.tpr * V >= dim;
}

// Backward launch: row layout, row groups per workgroup, persistent grid size and dynamic LDS.
// The register-resident kernel packs as many row groups into a workgroup as its size bound
// allows (capped by `max_block`), because the groups' dweight columns are combined in LDS and
// each workgroup writes one partial row: fewer, larger workgroups mean fewer partial rows for
// stage 2.  The grid targets `waves_per_cu` resident waves on each of `cus` compute units.
struct BwdPlan {
  RowPlan rp;
  int64_t wgs;       // workgroups = dweight partial rows
  size_t lds_bytes;  // dynamic LDS of the group combine
  bool ring = false; // the ring-pipelined kernel (plan_bwd_ring) instead of bwd_vec_kernel
  // the ring over rows of 8-byte alignment with a half chunk at their end (plan_bwd_ring8): rp
  // lays out the row's whole chunks (dim - 4 elements)
  bool x8 = false;
  // the element-strided ring (plan_bwd_ring_elem): elements per lane, 0 when not planned
  int elem_m = 0;
  // with the RoPE gradient: bwd_vec_kernel's plain plan, each pair's rotation evaluated directly
  // where g is decoded (rows too wide for the RoPE walk's bound)
  bool rope_direct = false;
};

// The ring-pipelined backward (bwd_ring_kernel): a ring of kRingPrefetch + 1 row buffers per
// thread, so two rows are in flight while one reduces, in a branch-free steady loop.  It takes
// rows of whole 16-byte chunks over whole waves (dim <= nv * tpr * V, at most 1/8 of the chunk
// slots idle, or for 2-byte rows of one chunk per thread a partly idle last wave; idle lanes
// reload the row's last chunk, so no branch guards a load), at most two
// chunks per thread, and workgroups of at most kRingBlock threads (its launch bound: 256 VGPRs a lane for
// the three row buffers), one per CU, so each row slot walks twice as many rows as in the
// 1024-thread persistent kernel.  Measured on MI355X at 16384 x 4096 bf16: 69.2 us against 72.4.
constexpr int kRingBlock = 512;
constexpr int kRingMaxNV = 2;
constexpr int kRingPrefetch = 2;

inline BwdPlan plan_bwd(int64_t rows, int64_t dim, int elem_bytes, bool aligned, int cus,
                        int prefer_nv, int max_block, int waves_per_cu,
                        const int (&order)[kMaxNV] = kBwdOrder) {
  BwdPlan b;
  b.rp = plan_rows(dim, elem_bytes, aligned, prefer_nv, order);
  RowPlan& p = b.rp;
  if (p.vec) {
    int mb = max_block_for_nv(p.nv);
    if (max_block < mb) mb = max_block;
    p.groups = mb / p.tpr;
    if (p.groups < 1) p.groups = 1;
    p.block = p.tpr * p.groups;
  }
  const int64_t wgs_needed = rows > 0 ? (rows + p.groups - 1) / p.groups : 1;
  int64_t wg_per_cu = waves_per_cu / (p.block / kWave);
  if (wg_per_cu < 1) wg_per_cu = 1;
  int64_t wgs = (int64_t)(cus > 0 ? cus : 1) * wg_per_cu;
  if (wgs > wgs_needed) wgs = wgs_needed;
  if (wgs < 1) wgs = 1;
  b.wgs = wgs;
  b.lds_bytes = (p.vec && p.groups > 1) ? (size_t)dim * sizeof(float) : 0;
  return b;
}

// Whether a row plan suits the ring-pipelined backward (see kRingBlock).
// Rows may leave lanes idle (whole waves over fewer chunks), at most 1/8 of the row group's
// chunk slots, or for 2-byte rows of one chunk per thread any part of the last wave: the
// kernel's idle-lane variant (kRingTail) reloads the row's last chunk there.  Measured on
// MI355X (bf16, 16384 rows, alternating processes, two runs each), one-chunk row groups with a
// partly idle last wave against the plans before them (two or three chunks per thread in
// bwd_vec_kernel): 640 19.1 against 20.6 us, 768 19.5 against 21.9, 1152 29.6 against 32.4, 1280
// 30.2 against 34.0.
inline bool ring_eligible(const RowPlan& p, int64_t dim, int elem_bytes) {
  if (!p.vec || (elem_bytes != 2 && elem_bytes != 4)) return false;
  const int V = 16 / elem_bytes;
  const int64_t slots = (int64_t)p.nv * p.tpr;
  if (dim % V != 0) return false;
  const int64_t chunks = dim / V;
  return p.nv >= 1 && p.nv <= kRingMaxNV && p.tpr <= kRingBlock && chunks >= 1 &&
         slots >= chunks && slots - chunks < p.tpr &&
         ((p.nv == 1 && elem_bytes == 2) ? slots - chunks < kWave : (slots - chunks) * 8 <= slots);
}

// Whether the ring's idle-lane variant is planned for rows that leave lanes idle (whole rows
// always take the ring).  Measured on MI355X against bwd_vec_kernel (16384 rows, backward only,
// two alternating processes each, best of 3 batched rounds): faster everywhere except (a) rows
// of one chunk per thread in 320-thread row groups, whose workgroup alone on its CU holds five
// waves (2240 bf16: 56.1 us against 51.4; 1120 fp32 56.6 against 50.7), and (b) rows of two
// chunks per thread in row groups of 448 or 512 threads that are not whole 128-byte lines (bf16
// 7160: 131.0 against 125.4, 7176: 132.2 against 127.7, 8184: 150.2 against 148.3), where the
// workgroup's seven or eight waves hold the ring while bwd_vec_kernel keeps twice the waves;
// whole lines there still pay (6272 bf16: 105.8 against 112.9).  Elsewhere, e.g. bf16 4000:
// 71.3 against 73.4, 5000 87.0 against 91.9, 3576 63.2 against 75.8, fp32 2240 74.4 against
// 84.9.
inline bool ring_tail_pays(const RowPlan& p, int64_t dim, int elem_bytes) {
  const int64_t chunks = dim / (16 / elem_bytes);
  if ((int64_t)p.nv * p.tpr == chunks) return true;
  if (p.nv == 1) return (kRingBlock / p.tpr) * p.tpr >= 6 * kWave;
  return p.tpr < 448 || (dim * elem_bytes) % 128 == 0;
}

// Plan of the ring-pipelined backward: row groups packed into workgroups of up to kRingBlock
// threads, one workgroup per CU.  `ring` is false (and the plan unusable) when the row layout
// does not suit it; the caller then plans bwd_vec_kernel.
// `max_block` (at most kRingBlock) bounds the workgroup and `wgs_per_cu` (1 or 2) sets the
// resident workgroups per CU: two 256-thread workgroups per CU hold the same waves as one of 512
// (the ring's registers allow eight waves per CU) without sharing a barrier.
// Without a preference (`prefer_nv` 0), for 2-byte dtypes a ring row group of one chunk per
// thread comes first where it is planned (rows of up to kRingBlock chunks), else the backward's
// order: one chunk per thread in row groups of up to 512 threads beat two in half as many (no
// LDS combine of the row groups' dweight columns when one row group fills the workgroup).
// Measured on MI355X (16384 rows, alternating processes): the bench's config C backward
// 67.3-67.5 us against 68.6-68.7 in three runs each (the step 6094-6098 GB/s against
// 6062-6070), and with batched launches (best of 3 rounds, two runs each) bf16 1024 22.0 against
// 23.5, 1536 30.2 against 36.7, 2048 37.5 against 38.6, 3584 60.1 against 62.7, 4000 68.0
// against 71.5, 4096 68.2 against 69.4, 512, 768, 2560 and 3072 equal.  fp32 rows keep two
// chunks per thread first: one ran 1024 in 39.7 against 37.5 us, 1536 62.2 against 53.4, 2048
// 74.1 against 68.2.  Nor do one-chunk row groups of 320 or 384 threads come first (one
// workgroup of five or six waves a CU): bf16 3000 ran 59.4-59.6 us against 55.8-56.0 with two
// chunks per thread in two 192-thread row groups, 3072 55.6-56.0 against 54.7, and 2560
// 52.6-53.0 against 52.0-52.3 in bwd_vec_kernel; 448-thread ones stay first (3500 70.9-71.6
// against 72.2-72.6, 3584 60.9-62.1 against 62.5-62.7; 3200 within 1%).
// Walks of more than kRingOneChunkMaxIters rows per slot keep the backward's order: one chunk per
// thread halves the row slots, and its walks of 256 rows ran slower than two chunks' walks of 128
// (bf16 65536 x 4096: 265.9-268.3 us against 259.7-260.0; 131072 x 2048: 267.2-269.0 against
// 260.9), while walks of up to 192 rows kept its lead (49152 x 4096: 193.4 against 194.3; 32768
// x 4096: 128.5-128.7 against 130.7-131.2).
constexpr int64_t kRingOneChunkMaxIters = 192;

inline BwdPlan plan_bwd_ring(int64_t rows, int64_t dim, int elem_bytes, bool aligned, int cus,
                             int prefer_nv, int max_block = kRingBlock, int wgs_per_cu = 1) {
  if (max_block > kRingBlock) max_block = kRingBlock;
  if (wgs_per_cu < 1) wgs_per_cu = 1;
  if (wgs_per_cu > 2) wgs_per_cu = 2;
  // The ring's launch over row layout `rp`: `ring` false when the layout does not suit it.
  auto complete = [&](const RowPlan& rp) {
    BwdPlan b;
    b.rp = rp;
    b.wgs = 0;
    b.lds_bytes = 0;
    b.ring = ring_eligible(rp, dim, elem_bytes) && rp.tpr <= max_block &&
             ring_tail_pays(rp, dim, elem_bytes);
    if (!b.ring) return b;
    int wpc = wgs_per_cu;
    if (rp.tpr * wpc > kRingBlock) wpc = 1;  // a row group fills the CU's waves
    RowPlan& p = b.rp;
    p.groups = max_block / p.tpr;
    if (p.groups * wpc * p.tpr > kRingBlock) p.groups = kRingBlock / (wpc * p.tpr);
    p.block = p.tpr * p.groups;
    const int64_t wgs_needed = rows > 0 ? (rows + p.groups - 1) / p.groups : 1;
    int64_t wgs = cus > 0 ? (int64_t)cus * wpc : 1;
    if (wgs > wgs_needed) wgs = wgs_needed;
    b.wgs = wgs;
    b.lds_bytes = p.groups > 1 ? (size_t)dim * sizeof(float) : 0;
    return b;
  };
  if (prefer_nv == 0 && elem_bytes == 2) {
    // one chunk per thread in whole waves, the last one partly idle where the chunks end there
    RowPlan one = plan_rows(dim, elem_bytes, aligned, 1, kBwdOrder);
    if (aligned && dim % 8 == 0 && dim / 8 <= kRingBlock) {
      const int t = (int)((dim / 8 + kWave - 1) / kWave) * kWave;
      one = RowPlan{true, 1, t, 1, t};
    }
    if (one.vec && one.nv == 1 && one.tpr != 320 && one.tpr != 384) {
      const BwdPlan b = complete(one);
      const int64_t slots = b.wgs * b.rp.groups;
      if (b.ring && (rows + slots - 1) / slots <= kRingOneChunkMaxIters) return b;
    }
  }
  return complete(plan_rows(dim, elem_bytes, aligned, prefer_nv, kBwdOrder));
}

// The ring over rows of a 2-byte dtype whose streams start on 8-byte boundaries only and hold
// dim = 8 * n + 4 elements (hidden sizes such as 4100, whose rows alternate between the two
// halves of a 16-byte line): the ring's plan for the n whole chunks (dim - 4 elements, each
// moved as two 8-byte halves), the row's last 4 elements an extra half chunk of the row group's
// lane 0, the group combine over all dim columns.  One chunk per thread: the extra chunk's ring
// buffers and sums fit beside one chunk's, not beside two (the planner asks plan_bwd_ring for
// one, so rows of up to kRingBlock whole chunks, dim <= 4100 bf16, take it).
inline BwdPlan plan_bwd_ring8(int64_t rows, int64_t dim, int elem_bytes, int cus,
                              int max_block = kRingBlock, int wgs_per_cu = 1) {
  BwdPlan b;
  b.rp = RowPlan{false, 0, kGenericBlock, 1, kGenericBlock};
  b.wgs = 0;
  b.lds_bytes = 0;
  if (elem_bytes != 2 || dim < 12 || dim % 8 != 4) return b;
  b = plan_bwd_ring(rows, dim - 4, elem_bytes, true, cus, 1, max_block, wgs_per_cu);
  if (!b.ring || b.rp.nv != 1) {
    b.ring = false;
    return b;
  }
  b.x8 = true;
  b.lds_bytes = b.rp.groups > 1 ? (size_t)dim * sizeof(float) : 0;
  return b;
}

// Element-strided rows (fwd_elem_kernel, bwd_ring_elem_kernel) for rows the chunked kernels
// cannot take (odd lengths, streams that start anywhere in a 16-byte line): M elements a lane,
// 4 for rows of up to 512 elements, else 8 (0: a row longer than kRingElemMaxM * kRingBlock
// elements), row groups of whole waves packed into workgroups of up to kRingBlock threads.
// Eight elements a lane in half the lanes (more row groups a workgroup) ran the backward at bf16
// 16384 x 1535 in 42.3 us against 55.5 with four, 2047 49.4 against 60.5, 1001 30.0 against
// 31.8, and 3001 and 4095 alike.
constexpr int kRingElemMaxM = 8;

inline int elem_per_lane(int64_t dim) {
  if (dim <= 0 || dim > (int64_t)kRingElemMaxM * kRingBlock) return 0;
  return dim > 512 ? 8 : 4;
}

inline RowPlan plan_elem_rows(int64_t dim) {
  RowPlan p{false, 0, kGenericBlock, 1, kGenericBlock};
  const int m = elem_per_lane(dim);
  if (m == 0) return p;
  const int64_t lanes = (dim + m - 1) / m;
  p.tpr = (int)((lanes + kWave - 1) / kWave) * kWave;
  p.groups = kRingBlock / p.tpr;
  p.block = p.tpr * p.groups;
  return p;
}

// The element-strided ring backward: plan_elem_rows' row groups, one workgroup per CU.
inline BwdPlan plan_bwd_ring_elem(int64_t rows, int64_t dim, int elem_bytes, int cus) {
  BwdPlan b;
  b.rp = RowPlan{false, 0, kGenericBlock, 1, kGenericBlock};
  b.wgs = 0;
  b.lds_bytes = 0;
  const int m = elem_per_lane(dim);
  if ((elem_bytes != 2 && elem_bytes != 4) || m == 0) return b;
  b.rp = plan_elem_rows(dim);
  const RowPlan& p = b.rp;
  const int64_t wgs_needed = rows > 0 ? (rows + p.groups - 1) / p.groups : 1;
  int64_t wgs = cus > 0 ? (int64_t)cus : 1;
  if (wgs > wgs_needed) wgs = wgs_needed;
  b.wgs = wgs;
  b.lds_bytes = p.groups > 1 ? (size_t)dim * sizeof(float) : 0;
  b.elem_m = m;
  return b;
}

// The ring-pipelined backward with the fused RoPE gradient (bwd_rope_ring_kernel): whole rows
// of one 16-byte chunk per thread where a row has at most kRingBlock chunks (its rotation state
// and tables keep it at 128 VGPRs), else of two (rows of up to 2 * kRingBlock chunks; 256
// VGPRs), row groups packed into workgroups of up to kRingBlock threads, rope_ring_wgs_per_cu of
// them per CU.  `ring` is false when the row layout does not suit it.  The kernel also needs every
// slot's walk to advance by the slot count or return to its first position (rope_walk_ok).
constexpr int kRopeRingMaxWgsPerCu = 2;

// One chunk per thread: one workgroup per CU when it fills kRingBlock threads (eight waves),
// else two (a 320- to 448-thread workgroup alone would leave the CU five to seven waves).
// Measured on MI355X (bf16, A/B in one process, 4 rounds): one 512-thread workgroup per CU
// against two runs 16384 x 4096 in 71.8 us against 79.0 (and 72.0 against 79.2 as 8 sequences of
// 2048), 8192 x 4096 in 41.7 against 45.1 and 32768 x 2048 in 71.8 against 77.6 (half the partial
// rows, and twice as many rows per walk over the same resident waves); 384-thread workgroups
// (16384 x 3072) run 61.5 us two per CU against 63.4 alone.  Two chunks per thread hold up to
// 256 VGPRs, so one workgroup per CU.
inline int rope_ring_wgs_per_cu(int nv, int block) {
  return nv == 1 && block < kRingBlock ? kRopeRingMaxWgsPerCu : 1;
}

inline BwdPlan plan_bwd_rope_ring(int64_t rows, int64_t dim, int elem_bytes, bool aligned,
                                  int cus) {
  BwdPlan b;
  b.rp = RowPlan{false, 0, kGenericBlock, 1, kGenericBlock};
  b.wgs = 0;
  b.lds_bytes = 0;
  if ((elem_bytes != 2 && elem_bytes != 4) || !aligned || dim <= 0) return b;
  const int V = 16 / elem_bytes;
  if (dim % V != 0) return b;
  const int64_t chunks = dim / V;
  const int nv = chunks <= kRingBlock ? 1 : 2;
  if (chunks % ((int64_t)nv * kWave) != 0 || chunks > (int64_t)nv * kRingBlock) return b;
  RowPlan& p = b.rp;
  p.vec = true;
  p.nv = nv;
  p.tpr = (int)(chunks / nv);
  p.groups = kRingBlock / p.tpr;
  p.block = p.tpr * p.groups;
  const int64_t wgs_needed = rows > 0 ? (rows + p.groups - 1) / p.groups : 1;
  int64_t wgs = (int64_t)(cus > 0 ? cus : 1) * rope_ring_wgs_per_cu(nv, p.block);
  if (wgs > wgs_needed) wgs = wgs_needed;
  b.wgs = wgs;
  // per thread and pair (V / 2 pairs a chunk): with one chunk the double frequency and the float
  // step and first rotations, 24 bytes; with two the float step rotation, 8 bytes; then, with
  // several row groups, their dweight combine
  const int pairs = nv * (V / 2);
  const size_t per_pair = nv == 1 ? sizeof(double) + 4 * sizeof(float) : 2 * sizeof(float);
  b.lds_bytes = (size_t)p.block * pairs * per_pair +
                (p.groups > 1 ? (size_t)dim * sizeof(float) : 0);
  b.ring = true;
  return b;
}

// Whether `slots` row slots walking `rows` rows (slot s: rows s, s + slots, ...) see positions
// (row % seq) that only advance by `slots` or return to the walk's first one: slots is a
// multiple or a divisor of seq, or no walk reaches the end of a sequence.
inline bool rope_walk_ok(int64_t rows, int64_t slots, int64_t seq) {
  if (rows <= 0 || slots <= 0 || seq <= 0) return false;
  if (seq % slots == 0 || slots % seq == 0) return true;
  const int64_t iters = (rows + slots - 1) / slots;
  return iters <= seq / slots;  // iters * slots <= seq
}

// Whether a plan suits bwd_rope_ring_kernel (the facts its indexing relies on).
inline bool rope_ring_eligible(const RowPlan& p, int64_t dim, int elem_bytes) {
  if (!p.vec || (elem_bytes != 2 && elem_bytes != 4)) return false;
  return (p.nv == 1 || p.nv == 2) && p.tpr % kWave == 0 &&
         (int64_t)p.nv * p.tpr * (16 / elem_bytes) == dim && p.block == p.tpr * p.groups &&
         p.block <= kRingBlock;
}

// Backward plan with the fused inverse RoPE: the same layout under max_block_for_nv_rope, or the
// generic plan where a row group does not fit that bound.
inline BwdPlan plan_bwd_rope(int64_t rows, int64_t dim, int elem_bytes, bool aligned, int cus,
                             int prefer_nv, int max_block, int waves_per_cu) {
  RowPlan rp = plan_rows(dim, elem_bytes, aligned, prefer_nv, kBwdOrderRope);
  if (rp.vec && max_block_for_nv_rope(rp.nv) < rp.tpr) {
    // the first chunk count whose row group fits the RoPE walk's bound (rows of 1536 chunks:
    // three chunks per thread in 512 threads, not two in 768)
    rp.vec = false;
    for (int nv = 1; nv <= kMaxNV && !rp.vec; ++nv) {
      const RowPlan q = plan_rows(dim, elem_bytes, aligned, nv, kBwdOrderRope);
      if (q.vec && q.nv == nv && q.tpr <= max_block_for_nv_rope(nv)) rp = q;
    }
    if (!rp.vec) {
      // no chunk count fits the walk (rows of more than 1536 chunks): the plain plan with each
      // pair's rotation evaluated where g is decoded, preferring four chunks per thread (248
      // VGPRs in 512-thread rows; two chunks in 1024-thread rows spill), else the generic kernel
      BwdPlan d = plan_bwd(rows, dim, elem_bytes, aligned, cus, 4, max_block, waves_per_cu);
      if (d.rp.vec) {
        d.rope_direct = true;
        return d;
      }
      return plan_bwd(rows, dim, elem_bytes, false, cus, prefer_nv, max_block,
                      waves_per_cu);  // generic
    }
    prefer_nv = rp.nv;
  }
  int mb = max_block;
  if (rp.vec) {
    const int bound = max_block_for_nv_rope(rp.nv);
    if (bound < mb) mb = bound;
  }
  return plan_bwd(rows, dim, elem_bytes, aligned, cus, prefer_nv, mb, waves_per_cu,
                  kBwdOrderRope);
}

// Rows per walk of the norm + RoPE forward (fwd_rope_kernel: workgroup b walks rows b, b + G, ...
// with G = ceil(rows / W)).  32-row walks halve the workgroups and the per-walk set-up (the
// step and first rotations, a few hundred vector instructions a thread); they pay where a row
// group fills a CU's waves with fewer workgroups (more than 256 threads) and the tensor keeps
// at least two 32-row walks per CU on 256 CUs.  Measured on MI355X (bf16, module form, A/B in one
// process, 3 rounds; 16-row against 32-row walks): 16384 x 4096 51.2 / 50.0 us (one sequence
// 50.3 / 49.8), 16384 x 5120 73.4 / 61.4, 16384 x 7168 98.2 / 89.5, 16384 x 8192 103.8 / 94.1,
// 16384 x 3072 42.1 / 40.3; against: 32768 x 2048 51.6 / 52.2 (256-thread rows), 8192 x 4096
// 27.2 / 31.2 (256 workgroups); 64-row walks lost everywhere (99.6 us at 16384 x 4096).
constexpr int kNormRopeRows = 16;
constexpr int kNormRopeLongRows = 32;
constexpr int64_t kNormRopeLongMinRows = 16384;
inline int fwd_rope_walk_rows(int64_t rows, int tpr) {
  return tpr > 256 && rows >= kNormRopeLongMinRows ? kNormRopeLongRows : kNormRopeRows;
}

// Workspace of the backward's dweight partial rows.  The plan depends on the element size, on
// pointer alignment and on whether the RoPE gradient is fused, which a size query does not know,
// so this is the largest need over every plan the backward can pick for (rows, dim).
inline size_t bwd_workspace_bytes(int64_t rows, int64_t dim, int cus, int prefer_nv,
                                  int max_block, int waves_per_cu, int ring_block = kRingBlock,
                                  int ring_wgs_per_cu = 1) {
  if (rows <= 0 || dim <= 0 || cus <= 0) return 0;
  int64_t most = 0;
  const int sizes[2] = {2, 4};
  for (int si = 0; si < 2; ++si) {
    for (int al = 0; al < 2; ++al) {
      const int64_t n =
          plan_bwd(rows, dim, sizes[si], al != 0, cus, prefer_nv, max_block, waves_per_cu).wgs;
      if (n > most) most = n;
      const int64_t nr = plan_bwd_rope(rows, dim, sizes[si], al != 0, cus, prefer_nv, max_block,
                                       waves_per_cu).wgs;
      if (nr > most) most = nr;
      const BwdPlan rg = plan_bwd_ring(rows, dim, sizes[si], al != 0, cus, prefer_nv,
                                       ring_block, ring_wgs_per_cu);
      if (rg.ring && rg.wgs > most) most = rg.wgs;
      const BwdPlan rr = plan_bwd_rope_ring(rows, dim, sizes[si], al != 0, cus);
      if (rr.ring && rr.wgs > most) most = rr.wgs;
      const BwdPlan r8 = plan_bwd_ring8(rows, dim, sizes[si], cus, ring_block, ring_wgs_per_cu);
      if (r8.ring && r8.wgs > most) most = r8.wgs;
      const BwdPlan re = plan_bwd_ring_elem(rows, dim, sizes[si], cus);
      if (re.elem_m > 0 && re.wgs > most) most = re.wgs;
    }
  }
  return (size_t)most * (size_t)dim * sizeof(float);
}

}  // namespace vg_plan

#endif  // VELOGRAD_LAUNCH_PLAN_H
