// HBM ceilings for bench.py: plain streaming kernels with the byte patterns of the fused
// RMSNorm kernels but no arithmetic dependency between elements.  Not part of the kernels' C ABI.
//
// velograd_stream_probe (the bench's same-run ceilings) runs one fixed shape per pattern:
//   pattern 0  copy     1 read  + 1 write
//   pattern 1  fwd-like 2 reads + 2 writes   (x, residual -> h, y)
//   pattern 2  bwd-like 2 reads + 1 write    (grad_y, h -> dx)
//   pattern 3  read-only  2 reads            (stores only on a 128-bit value random data never
//                                             holds, so the loads cannot be removed)
//   pattern 4  write-only 2 writes
//   pattern 5  grad_h-bwd-like 3 reads + 1 write (grad_y, h, grad_h -> dx)
// Patterns 3 and 4 bound what mixing reads and writes costs: the same streams, one direction.
// That shape is 256-thread workgroups, two 16-byte vectors per thread and stream, non-temporal
// loads and stores, one pass over the buffers (no grid-stride loop), and with two write streams
// the second one's stores rotated by half a workgroup's 8 KiB block, so that the two stores a
// thread issues together fall 4 KiB apart: over buffers whose addresses agree in their low bits
// (large torch allocations are 2 MiB aligned) stores that agree in address bit 12 collide, and
// the rotation speeds the 2-read/2-write pattern up by 4.5% (89.6 -> 85.5 us for 4 x 128 MiB)
// and the write-only one by 2.7%; rotating a read stream changes nothing.
//
// velograd_stream_probe_shape runs any of the shapes a sweep compares (bench.py --probe-sweep):
// 0-3 read streams, 0-2 write streams, workgroups of 256/512/1024 threads, 1/2/4 vectors per
// thread and stream, 16 or 32 contiguous bytes per lane and vector, a one-pass grid or a
// persistent grid of `wgs_per_cu` workgroups per CU walking the tiles, non-temporal or plain
// loads and stores, the second write stream rotated or not, and guarded or flat code.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "velograd_kernels.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kFlagNtLoad = 1;   // non-temporal loads
constexpr int kFlagNtStore = 2;  // non-temporal stores
constexpr int kFlagRotate = 4;   // second write stream rotated by half a tile
constexpr int kFlagFlat = 8;     // whole tiles without per-access guards (no branches)

template <bool NT>
__device__ __forceinline__ u32x4 ld(const u32x4* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <bool NT>
__device__ __forceinline__ void st(u32x4* p, u32x4 v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// One tile = VPT vectors of L 16-byte units per thread of a BLOCK-thread workgroup: tile t covers
// units [t * VPT * BLOCK * L, (t + 1) * VPT * BLOCK * L) of every stream; vector k of thread i is
// units (t * VPT + k) * BLOCK * L + i * L .. + L - 1, so each wave instruction moves 64 * 16 * L
// contiguous bytes.  Units at or past n16 are skipped: in the guarded style every access tests
// its own index (a branch around each vector, after which the compiler waits for all earlier
// memory operations); in the flat style (FLAT) whole tiles take a path with no test and only the
// last tile is guarded.  Which style is faster depends on the shape: for 2-read/2-write over
// 16384 x 4096 bf16, at two vectors per thread guarded 86.6 us and flat 90.6, at four vectors
// flat 85.9 and guarded 94.8.
template <int NR, int NW, int VPT, int L, int BLOCK, bool NTL, bool NTS, bool GUARD = true>
__device__ __forceinline__ void probe_tile(const u32x4* a, const u32x4* b, const u32x4* c,
                                           u32x4* w0, u32x4* w1, int64_t n16, int64_t t,
                                           bool rotate) {
  constexpr int64_t kTile = (int64_t)VPT * BLOCK * L;
  const int64_t base = t * kTile + (int64_t)threadIdx.x * L;
  // every load is issued before any value is combined, so all of a thread's loads are in flight
  // together (adding as they arrive made each vector wait for the previous one's loads)
  u32x4 va[VPT][L], vb[VPT][L], vc[VPT][L];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
#pragma unroll
    for (int l = 0; l < L; ++l) {
      const int64_t i = base + (int64_t)k * BLOCK * L + l;
      va[k][l] = u32x4{(uint32_t)i, 1u, 2u, 3u};
      vb[k][l] = vc[k][l] = u32x4{0u, 0u, 0u, 0u};
      if (!GUARD || i < n16) {
        if (NR >= 1) va[k][l] = ld<NTL>(a + i);
        if (NR >= 2) vb[k][l] = ld<NTL>(b + i);
        if (NR >= 3) vc[k][l] = ld<NTL>(c + i);
      }
    }
  }
  // the second write stream's vector for slot k: slot (k + VPT / 2) % VPT of the same tile
  // (whole tiles only, so it stays in bounds)
  const bool whole = (t + 1) * kTile <= n16;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
#pragma unroll
    for (int l = 0; l < L; ++l) {
      const int64_t i = base + (int64_t)k * BLOCK * L + l;
      if (!GUARD || i < n16) {
        const u32x4 x = va[k][l] + vb[k][l] + vc[k][l];
        if (NW == 0) {
          if (x.x == 0x9E3779B9u && x.y == 0x7F4A7C15u && x.z == 0xF39CC060u &&
              x.w == 0x5CEDC834u)
            w0[i] = x;
        } else {
          st<NTS>(w0 + i, x);
          if (NW == 2) {
            const int64_t j = (whole && rotate && VPT >= 2)
                                  ? base + (int64_t)((k + VPT / 2) % VPT) * BLOCK * L + l
                                  : i;
            st<NTS>(w1 + j, x ^ u32x4{1u, 1u, 1u, 1u});
          }
        }
      }
    }
  }
}

template <int NR, int NW, int VPT, int L, int BLOCK, bool NTL, bool NTS, bool FLAT>
__device__ __forceinline__ void probe_tile_style(const u32x4* a, const u32x4* b,
                                                 const u32x4* c, u32x4* w0, u32x4* w1,
                                                 int64_t n16, int64_t t, bool rotate) {
  if (FLAT && (t + 1) * ((int64_t)VPT * BLOCK * L) <= n16)
    probe_tile<NR, NW, VPT, L, BLOCK, NTL, NTS, false>(a, b, c, w0, w1, n16, t, rotate);
  else
    probe_tile<NR, NW, VPT, L, BLOCK, NTL, NTS, true>(a, b, c, w0, w1, n16, t, rotate);
}

// One workgroup per tile (a one-pass grid).
template <int NR, int NW, int VPT, int L, int BLOCK, bool NTL, bool NTS, bool ROT, bool FLAT>
__global__ __launch_bounds__(BLOCK) void probe_kernel(const u32x4* a, const u32x4* b,
                                                      const u32x4* c, u32x4* w0, u32x4* w1,
                                                      int64_t n16) {
  probe_tile_style<NR, NW, VPT, L, BLOCK, NTL, NTS, FLAT>(a, b, c, w0, w1, n16, blockIdx.x, ROT);
}

// A persistent grid: workgroup g walks tiles g, g + gridDim.x, ...
template <int NR, int NW, int VPT, int L, int BLOCK, bool NTL, bool NTS, bool ROT, bool FLAT>
__global__ __launch_bounds__(BLOCK) void probe_walk_kernel(const u32x4* a, const u32x4* b,
                                                           const u32x4* c, u32x4* w0,
                                                           u32x4* w1, int64_t n16,
                                                           int64_t tiles) {
  for (int64_t t = blockIdx.x; t < tiles; t += gridDim.x)
    probe_tile_style<NR, NW, VPT, L, BLOCK, NTL, NTS, FLAT>(a, b, c, w0, w1, n16, t, ROT);
}

struct ProbeLaunch {
  dim3 grid;
  bool persistent;
  bool flat;
  int64_t tiles;
  hipStream_t st;
  const u32x4 *a, *b, *c;
  u32x4 *w0, *w1;
  int64_t n16;
};

template <int NR, int NW, int VPT, int L, int BLOCK, bool NTL, bool NTS, bool ROT, bool FLAT>
hipError_t launch_style(const ProbeLaunch& p) {
  if (p.persistent)
    hipLaunchKernelGGL((probe_walk_kernel<NR, NW, VPT, L, BLOCK, NTL, NTS, ROT, FLAT>), p.grid,
                       dim3(BLOCK), 0, p.st, p.a, p.b, p.c, p.w0, p.w1, p.n16, p.tiles);
  else
    hipLaunchKernelGGL((probe_kernel<NR, NW, VPT, L, BLOCK, NTL, NTS, ROT, FLAT>), p.grid,
                       dim3(BLOCK), 0, p.st, p.a, p.b, p.c, p.w0, p.w1, p.n16);
  return hipGetLastError();
}

template <int NR, int NW, int VPT, int L, int BLOCK, bool NTL, bool NTS, bool ROT>
hipError_t launch_one(const ProbeLaunch& p) {
  if (p.flat) return launch_style<NR, NW, VPT, L, BLOCK, NTL, NTS, ROT, true>(p);
  return launch_style<NR, NW, VPT, L, BLOCK, NTL, NTS, ROT, false>(p);
}

// Cache policies and the rotation: all combinations for the bench's shape (256 threads, two
// vectors of 16 bytes), non-temporal and rotated for the others.
template <int NR, int NW, int VPT, int L, int BLOCK>
hipError_t launch_policy(int flags, const ProbeLaunch& p) {
  const bool ntl = (flags & kFlagNtLoad) != 0, nts = (flags & kFlagNtStore) != 0;
  const bool rot = (flags & kFlagRotate) != 0;
  if (ntl && nts && rot) return launch_one<NR, NW, VPT, L, BLOCK, true, true, true>(p);
  if constexpr (VPT == 2 && L == 1 && BLOCK == 256) {
    if (ntl && nts) return launch_one<NR, NW, 2, 1, 256, true, true, false>(p);
    if (ntl && rot) return launch_one<NR, NW, 2, 1, 256, true, false, true>(p);
    if (ntl) return launch_one<NR, NW, 2, 1, 256, true, false, false>(p);
    if (nts && rot) return launch_one<NR, NW, 2, 1, 256, false, true, true>(p);
    if (nts) return launch_one<NR, NW, 2, 1, 256, false, true, false>(p);
    if (rot) return launch_one<NR, NW, 2, 1, 256, false, false, true>(p);
    return launch_one<NR, NW, 2, 1, 256, false, false, false>(p);
  }
  return hipErrorInvalidValue;
}

template <int NR, int NW, int VPT, int L>
hipError_t launch_block(int block, int flags, const ProbeLaunch& p) {
  switch (block) {
    case 256: return launch_policy<NR, NW, VPT, L, 256>(flags, p);
    case 512: return launch_policy<NR, NW, VPT, L, 512>(flags, p);
    default: return launch_policy<NR, NW, VPT, L, 1024>(flags, p);
  }
}

template <int NR, int NW, int VPT>
hipError_t launch_l(int lane_bytes, int block, int flags, const ProbeLaunch& p) {
  if (lane_bytes == 32) return launch_block<NR, NW, VPT, 2>(block, flags, p);
  return launch_block<NR, NW, VPT, 1>(block, flags, p);
}

template <int NR, int NW>
hipError_t launch_v(int vpt, int lane_bytes, int block, int flags, const ProbeLaunch& p) {
  switch (vpt) {
    case 1: return launch_l<NR, NW, 1>(lane_bytes, block, flags, p);
    case 2: return launch_l<NR, NW, 2>(lane_bytes, block, flags, p);
    default: return launch_l<NR, NW, 4>(lane_bytes, block, flags, p);
  }
}

// The bench's fixed shapes (velograd_stream_probe): 256-thread workgroups, two 16-byte vectors
// per thread and stream, non-temporal, one pass, the second write stream rotated, every access
// guarded by its index, all of a thread's loads issued before its stores.  Kept as its own
// kernel so the bench's ceilings stay comparable across builds: the sweep kernel above, at the
// same shape, runs the 2-read/2-write pattern in 88 us against 85.7 us for this one (one
// process, one box).
constexpr int kPerThread = 2;
constexpr int kBlock = 256;

template <int NR, int NW>
__global__ __launch_bounds__(kBlock) void stream_kernel(const u32x4* a, const u32x4* b,
                                                        const u32x4* e, u32x4* c, u32x4* d,
                                                        int64_t n16) {
  const int64_t base = (int64_t)blockIdx.x * kBlock * kPerThread + threadIdx.x;
  u32x4 va[kPerThread], vb[kPerThread], ve[kPerThread];
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int64_t i = base + (int64_t)k * kBlock;
    va[k] = u32x4{(uint32_t)i, 1u, 2u, 3u};
    if (i < n16) {
      if (NR >= 1) va[k] = __builtin_nontemporal_load(a + i);
      if (NR >= 2) vb[k] = __builtin_nontemporal_load(b + i);
      if (NR == 3) ve[k] = __builtin_nontemporal_load(e + i);
    }
  }
  // d's vector for slot k: the block's other half (whole blocks only, so it stays in bounds)
  const bool whole = (int64_t)(blockIdx.x + 1) * kBlock * kPerThread <= n16;
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int64_t i = base + (int64_t)k * kBlock;
    if (i < n16) {
      u32x4 v = va[k];
      if (NR >= 2) v += vb[k];
      if (NR == 3) v += ve[k];
      if (NW == 0) {
        if (v.x == 0x9E3779B9u && v.y == 0x7F4A7C15u && v.z == 0xF39CC060u && v.w == 0x5CEDC834u)
          c[i] = v;
      } else {
        __builtin_nontemporal_store(v, c + i);
        if (NW == 2) {
          const int64_t j = whole ? base + (int64_t)((k + 1) % kPerThread) * kBlock : i;
          __builtin_nontemporal_store(v ^ u32x4{1u, 1u, 1u, 1u}, d + j);
        }
      }
    }
  }
}


int cu_count() {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return v;
}

}  // namespace

// Any probe shape: `nread` streams read from rd[0..nread-1], `nwrite` streams written to
// wr[0..nwrite-1], n16 16-byte units each.  block in {256, 512, 1024}, vpt in {1, 2, 4},
// lane_bytes in {16, 32}; wgs_per_cu 0 launches one workgroup per tile, else that many
// workgroups per CU walk the tiles.  flags: 1 non-temporal loads, 2 non-temporal stores,
// 4 rotate the second write stream, 8 the flat style (whole tiles without per-access guards);
// the policies other than 1 | 2 | 4 are built for the bench's shape (256 threads, 2 vectors of
// 16 bytes per thread) only.  Returns 0, -1 for a bad
// argument, or the hipError_t of the launch.
extern "C" VELOGRAD_API int32_t velograd_stream_probe_shape(
    int32_t nread, int32_t nwrite, const void* const* rd, void* const* wr, int64_t n16,
    int32_t block, int32_t vpt, int32_t lane_bytes, int32_t wgs_per_cu, int32_t flags,
    void* hip_stream) {
  if (n16 <= 0 || nread < 0 || nread > 3 || nwrite < 0 || nwrite > 2 || nread + nwrite == 0 ||
      (nread == 0 && nwrite != 2) || (nwrite == 0 && nread != 2) ||
      (block != 256 && block != 512 && block != 1024) || (vpt != 1 && vpt != 2 && vpt != 4) ||
      (lane_bytes != 16 && lane_bytes != 32) || wgs_per_cu < 0 || wgs_per_cu > 64)
    return -1;
  if (nread > 0 && rd == nullptr) return -1;
  if (wr == nullptr) return -1;
  for (int i = 0; i < nread; ++i)
    if (rd[i] == nullptr) return -1;
  // a read-only shape still names one buffer to write to (its stores never happen)
  for (int i = 0; i < (nwrite > 0 ? nwrite : 1); ++i)
    if (wr[i] == nullptr) return -1;
  const int64_t tile_units = (int64_t)vpt * block * (lane_bytes / 16);
  const int64_t tiles = (n16 + tile_units - 1) / tile_units;
  int64_t grid = tiles;
  if (wgs_per_cu > 0) {
    const int cus = cu_count();
    if (cus <= 0) return -1;
    grid = (int64_t)cus * wgs_per_cu;
    if (grid > tiles) grid = tiles;
  }
  if (grid > INT32_MAX) return -1;
  ProbeLaunch p;
  p.grid = dim3((uint32_t)grid);
  p.persistent = wgs_per_cu > 0;
  p.flat = (flags & kFlagFlat) != 0;
  p.tiles = tiles;
  p.st = static_cast<hipStream_t>(hip_stream);
  p.a = nread > 0 ? static_cast<const u32x4*>(rd[0]) : nullptr;
  p.b = nread > 1 ? static_cast<const u32x4*>(rd[1]) : nullptr;
  p.c = nread > 2 ? static_cast<const u32x4*>(rd[2]) : nullptr;
  p.w0 = static_cast<u32x4*>(wr[0]);
  p.w1 = nwrite > 1 ? static_cast<u32x4*>(wr[1]) : nullptr;
  p.n16 = n16;
  hipError_t e;
  if (nread == 1 && nwrite == 1) e = launch_v<1, 1>(vpt, lane_bytes, block, flags, p);
  else if (nread == 2 && nwrite == 2) e = launch_v<2, 2>(vpt, lane_bytes, block, flags, p);
  else if (nread == 2 && nwrite == 1) e = launch_v<2, 1>(vpt, lane_bytes, block, flags, p);
  else if (nread == 3 && nwrite == 1) e = launch_v<3, 1>(vpt, lane_bytes, block, flags, p);
  else if (nread == 2 && nwrite == 0) e = launch_v<2, 0>(vpt, lane_bytes, block, flags, p);
  else if (nread == 0 && nwrite == 2) e = launch_v<0, 2>(vpt, lane_bytes, block, flags, p);
  else return -1;
  return (int32_t)e;
}

// The bench's fixed shapes (pattern numbers above) over streams a, b (read), c, d (written);
// pattern 5 reads a, b and d and writes c.
extern "C" VELOGRAD_API int32_t velograd_stream_probe(int32_t pattern, const void* a,
                                                      const void* b, void* c, void* d,
                                                      int64_t n16, void* hip_stream) {
  if (n16 <= 0 || a == nullptr || c == nullptr) return -1;
  if ((pattern == 1 || pattern == 2 || pattern == 3 || pattern == 5) && b == nullptr) return -1;
  if ((pattern == 1 || pattern == 4 || pattern == 5) && d == nullptr) return -1;
  const int64_t grid = (n16 + (int64_t)kBlock * kPerThread - 1) / ((int64_t)kBlock * kPerThread);
  if (grid > INT32_MAX) return -1;
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  const u32x4* A = static_cast<const u32x4*>(a);
  const u32x4* B = static_cast<const u32x4*>(b);
  u32x4* C = static_cast<u32x4*>(c);
  u32x4* D = static_cast<u32x4*>(d);
  const dim3 g((uint32_t)grid), blk(kBlock);
  switch (pattern) {
    case 0: hipLaunchKernelGGL((stream_kernel<1, 1>), g, blk, 0, st, A, B, nullptr, C, D, n16); break;
    case 1: hipLaunchKernelGGL((stream_kernel<2, 2>), g, blk, 0, st, A, B, nullptr, C, D, n16); break;
    case 2: hipLaunchKernelGGL((stream_kernel<2, 1>), g, blk, 0, st, A, B, nullptr, C, D, n16); break;
    case 3: hipLaunchKernelGGL((stream_kernel<2, 0>), g, blk, 0, st, A, B, nullptr, C, D, n16); break;
    case 4: hipLaunchKernelGGL((stream_kernel<0, 2>), g, blk, 0, st, A, B, nullptr, C, D, n16); break;
    case 5: hipLaunchKernelGGL((stream_kernel<3, 1>), g, blk, 0, st, A, B, D, C, nullptr, n16); break;
    default: return -1;
  }
  return (int32_t)hipGetLastError();
}
