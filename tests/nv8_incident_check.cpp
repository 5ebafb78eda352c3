// CPU check of the forward fault recorded for 8 chunks per thread (one wave per row): what the
// host side of that tuning build handed to the GPU, rebuilt from the source of that build.
//
// That build planned rows with a preference order written into `int order[4]`; a preference of
// 5..8 wrote a fifth entry past the array's end (undefined behaviour, since fixed: the planner now
// lives in velograd_amd/csrc/launch_plan.h with room for every entry).  This program
//   1. runs that planner (kMaxNV raised to 8, as the tuning build had it) for the faulting
//      workload, bf16 16384 x 4096 with VELOGRAD_FWD_NV=8, and prints the plan it returns;
//   2. replays the forward kernel's index arithmetic of that build (fwd_vec_kernel<bf16,bf16,8>:
//      row = blockIdx * (blockDim / tpr) + threadIdx / tpr, chunk c = lane + k * tpr, k < 8,
//      guarded by row < rows and c < dim / 8) for every thread of the launch the plan gives, and
//      checks every element it would load or store against the tensors' extents.
// Built and run by tests/test_launch_plan.py at -O0 and -O3 and under ASan/UBSan; the sanitized
// run is expected to report the overflow (it is the bug), the others print the plan and "in
// bounds".  Exit status: 0 = plan as expected and every access in bounds, 1 = not.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

namespace sweep_build {

constexpr int kWave = 64;
constexpr int kMaxWavesPerRow = 16;
constexpr int kMaxNV = 8;  // the tuning build; the library caps it at 4
constexpr int kGenericBlock = 256;

constexpr int max_block_for_nv(int nv) { return nv <= 2 ? 1024 : 512; }

struct RowPlan {
  bool vec;
  int nv;
  int tpr;
  int groups;
  int block;
};

// The planner of that build, unchanged apart from kMaxNV above.
__attribute__((noinline)) RowPlan plan_rows(int64_t dim, int elem_bytes, bool aligned,
                                            int prefer_nv) {
  const int V = 16 / elem_bytes;
  RowPlan p{false, 0, kGenericBlock, 1, kGenericBlock};
  if (!aligned || dim <= 0 || dim % V != 0) return p;
  const int64_t chunks = dim / V;
  if (chunks > (int64_t)kMaxWavesPerRow * kWave * kMaxNV) return p;
  const int order_auto[4] = {2, 3, 4, 1};
  int order[4];
  int n = 0;
  if (prefer_nv > 0) order[n++] = prefer_nv;
  for (int i = 0; i < 4; ++i)
    if (order_auto[i] != prefer_nv) order[n++] = order_auto[i];  // n reaches 5: overflow
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

}  // namespace sweep_build

int main() {
  using namespace sweep_build;
  const int64_t rows = 16384, dim = 4096, ld = 4096;
  const int eb = 2, V = 8, NV = 8;
  volatile int prefer = 8;  // VELOGRAD_FWD_NV=8, read at run time as the library read it
  const RowPlan p = plan_rows(dim, eb, true, prefer);
  const int64_t grid = p.groups > 0 ? (rows + p.groups - 1) / p.groups : 0;
  printf("plan: vec=%d nv=%d tpr=%d groups=%d block=%d grid=%lld\n", (int)p.vec, p.nv, p.tpr,
         p.groups, p.block, (long long)grid);
  const bool expected = p.vec && p.nv == 8 && p.tpr == 64 && p.groups == 4 && p.block == 256 &&
                        grid == 4096;
  if (!expected) {
    printf("plan differs from the launch intercepted in that build\n");
    return 1;
  }
  // Replay the kernel's accesses.  Extents in elements: x, residual, h, y are rows * ld;
  // weight is dim; inv_rms is rows.
  const int64_t act_extent = rows * ld;
  const int nchunk = (int)(dim / V);
  int64_t checked = 0, bad = 0;
  int64_t rows_seen = 0;
  for (int64_t bid = 0; bid < grid; ++bid) {
    for (int tid = 0; tid < p.block; ++tid) {
      const int tpr = p.tpr;
      const int grp = tid / tpr;
      const int lt = tid - grp * tpr;
      const int groups = p.block / tpr;
      const int64_t row = bid * groups + grp;
      const bool row_ok = row < rows;
      if (row_ok && lt == 0) {
        ++rows_seen;
        if (row < 0 || row >= rows) ++bad;  // inv_rms[row]
      }
      for (int k = 0; k < NV; ++k) {
        const int c = lt + k * tpr;
        if (c < nchunk) {  // weight chunk, loaded for every row slot
          const int64_t w0 = (int64_t)c * V;
          ++checked;
          if (w0 < 0 || w0 + V > dim) ++bad;
        }
        if (!(row_ok && c < nchunk)) continue;
        const int64_t e0 = row * ld + (int64_t)c * V;  // x, residual, h, y alike
        ++checked;
        if (e0 < 0 || e0 + V > act_extent) ++bad;
      }
    }
  }
  printf("accesses checked: %lld, out of bounds: %lld, rows covered: %lld of %lld\n",
         (long long)checked, (long long)bad, (long long)rows_seen, (long long)rows);
  if (bad != 0 || rows_seen != rows) return 1;
  printf("in bounds\n");
  return 0;
}
