// Same-run HBM ceiling for bench.py: plain streaming kernels with the byte pattern of the fused
// RMSNorm kernels but no arithmetic dependency between elements:
//   pattern 0  copy     1 read  + 1 write
//   pattern 1  fwd-like 2 reads + 2 writes   (x, residual -> h, y)
//   pattern 2  bwd-like 2 reads + 1 write    (grad_y, h -> dx)
//   pattern 3  read-only  2 reads            (stores only on a 128-bit value random data never
//                                             holds, so the loads cannot be removed)
//   pattern 4  write-only 2 writes
// Patterns 3 and 4 bound what mixing reads and writes costs: the same streams, one direction.
// Each thread moves two 16-byte vectors per stream with non-temporal accesses, one pass over
// the buffers (no grid-stride loop): the fastest shape found by a sweep over vectors per
// thread, workgroup size, grid size and cache policy on MI355X.  With two write streams the
// second one's stores are rotated by half a workgroup's 8 KiB block, so that the two stores a
// thread issues together fall 4 KiB apart: over buffers whose addresses agree in their low bits
// (large torch allocations are 2 MiB aligned) stores that agree in address bit 12 collide,
// and the rotation speeds the 2-read/2-write pattern up by 4.5% (89.6 -> 85.5 us for
// 4 x 128 MiB) and the write-only one by 2.7%; rotating a read stream changes nothing.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "velograd_kernels.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kPerThread = 2;
constexpr int kBlock = 256;

template <int NR, int NW>
__global__ __launch_bounds__(kBlock) void stream_kernel(const u32x4* a, const u32x4* b,
                                                        u32x4* c, u32x4* d, int64_t n16) {
  const int64_t base = (int64_t)blockIdx.x * kBlock * kPerThread + threadIdx.x;
  u32x4 va[kPerThread], vb[kPerThread];
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int64_t i = base + (int64_t)k * kBlock;
    va[k] = u32x4{(uint32_t)i, 1u, 2u, 3u};
    if (i < n16) {
      if (NR >= 1) va[k] = __builtin_nontemporal_load(a + i);
      if (NR == 2) vb[k] = __builtin_nontemporal_load(b + i);
    }
  }
  // d's vector for slot k: the block's other half (whole blocks only, so it stays in bounds)
  const bool whole = (int64_t)(blockIdx.x + 1) * kBlock * kPerThread <= n16;
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int64_t i = base + (int64_t)k * kBlock;
    if (i < n16) {
      u32x4 v = va[k];
      if (NR == 2) v += vb[k];
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

}  // namespace

// Bench helper, not part of the kernels' ABI: launches one pass of `pattern` over n16 16-byte
// vectors per stream (a, b read; c, d written) on `hip_stream`.  Returns 0, -1 for a bad
// argument, or the hipError_t of the launch.
extern "C" VELOGRAD_API int32_t velograd_stream_probe(int32_t pattern, const void* a,
                                                      const void* b, void* c, void* d,
                                                      int64_t n16, void* hip_stream) {
  if (n16 <= 0 || a == nullptr || c == nullptr) return -1;
  if ((pattern == 1 || pattern == 2 || pattern == 3) && b == nullptr) return -1;
  if ((pattern == 1 || pattern == 4) && d == nullptr) return -1;
  const int64_t grid = (n16 + (int64_t)kBlock * kPerThread - 1) / ((int64_t)kBlock * kPerThread);
  if (grid > INT32_MAX) return -1;
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  const u32x4* A = static_cast<const u32x4*>(a);
  const u32x4* B = static_cast<const u32x4*>(b);
  u32x4* C = static_cast<u32x4*>(c);
  u32x4* D = static_cast<u32x4*>(d);
  switch (pattern) {
    case 0: hipLaunchKernelGGL((stream_kernel<1, 1>), dim3(grid), dim3(kBlock), 0, st, A, B, C, D, n16); break;
    case 1: hipLaunchKernelGGL((stream_kernel<2, 2>), dim3(grid), dim3(kBlock), 0, st, A, B, C, D, n16); break;
    case 2: hipLaunchKernelGGL((stream_kernel<2, 1>), dim3(grid), dim3(kBlock), 0, st, A, B, C, D, n16); break;
    case 3: hipLaunchKernelGGL((stream_kernel<2, 0>), dim3(grid), dim3(kBlock), 0, st, A, B, C, D, n16); break;
    case 4: hipLaunchKernelGGL((stream_kernel<0, 2>), dim3(grid), dim3(kBlock), 0, st, A, B, C, D, n16); break;
    default: return -1;
  }
  return (int32_t)hipGetLastError();
}
