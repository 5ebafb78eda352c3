// CPU check of the kernels' launch planner (velograd_amd/csrc/launch_plan.h), built by
// tests/test_launch_plan.py with AddressSanitizer and UBSan.  For every row length, element
// size, alignment, tuning preference and row count it checks the facts the kernels rely on:
//   * the register-resident plan covers every 16-byte chunk of a row exactly once, with whole
//     wave64s per row, and its workgroup fits the kernel's launch bound for that NV;
//   * the backward's workgroups, LDS and partial rows fit the workspace the size query reports.
#include <algorithm>
#include <stdio.h>
#include <stdlib.h>

#include <vector>

#include "launch_plan.h"

using namespace vg_plan;

static int failures = 0;

#define CHECK(cond, ...)                                   \
  do {                                                     \
    if (!(cond)) {                                         \
      if (failures < 20) {                                 \
        fprintf(stderr, "FAIL %s:%d: %s: ", __FILE__, __LINE__, #cond); \
        fprintf(stderr, __VA_ARGS__);                      \
        fputc('\n', stderr);                               \
      }                                                    \
      ++failures;                                          \
    }                                                      \
  } while (0)

static void check_row_plan(const RowPlan& p, int64_t dim, int eb, bool aligned) {
  const int V = 16 / eb;
  CHECK(row_plan_valid(p, dim, eb), "row_plan_valid rejects a plan the planner made (dim=%lld)",
        (long long)dim);
  if (!p.vec) {
    CHECK(p.block == kGenericBlock && p.groups == 1 && p.tpr == kGenericBlock,
          "generic plan shape dim=%lld", (long long)dim);
    return;
  }
  CHECK(aligned && dim % V == 0, "vector plan for unaligned/ragged dim=%lld", (long long)dim);
  CHECK(p.nv >= 1 && p.nv <= kMaxNV, "nv=%d", p.nv);
  CHECK(p.tpr >= kWave && p.tpr % kWave == 0, "tpr=%d", p.tpr);
  CHECK(p.groups >= 1 && p.block == p.tpr * p.groups, "groups=%d block=%d", p.groups, p.block);
  CHECK(p.block <= max_block_for_nv(p.nv), "block %d over bound for nv %d", p.block, p.nv);
  const int64_t nchunk = dim / V;
  CHECK((int64_t)p.nv * p.tpr >= nchunk, "plan covers %lld of %lld chunks",
        (long long)p.nv * p.tpr, (long long)nchunk);
  // Exactly-once coverage of the chunks by (lane, k) as the kernels index them.
  if (nchunk <= 4096) {
    std::vector<int> seen((size_t)nchunk, 0);
    for (int lt = 0; lt < p.tpr; ++lt)
      for (int k = 0; k < p.nv; ++k) {
        const int64_t c = lt + (int64_t)k * p.tpr;
        if (c < nchunk) seen[(size_t)c]++;
      }
    for (int64_t c = 0; c < nchunk; ++c)
      CHECK(seen[(size_t)c] == 1, "chunk %lld seen %d times (dim=%lld)", (long long)c,
            seen[(size_t)c], (long long)dim);
  }
}

int main() {
  const int cus_list[3] = {1, 80, 256};
  const int64_t rows_list[6] = {1, 7, 64, 257, 16384, 32768};
  long plans = 0;
  for (int eb = 2; eb <= 4; eb += 2) {
    for (int aligned = 0; aligned < 2; ++aligned) {
      for (int64_t dim = 1; dim <= 70000; dim += (dim < 2048 ? 1 : 61)) {
        for (int prefer = -1; prefer <= kMaxNV + 1; ++prefer) {
          check_row_plan(plan_rows(dim, eb, aligned != 0, prefer, kFwdOrder), dim, eb,
                         aligned != 0);
          check_row_plan(plan_rows(dim, eb, aligned != 0, prefer, kFwdOrderOneStream), dim, eb,
                         aligned != 0);
          check_row_plan(plan_rows(dim, eb, aligned != 0, prefer, kBwdOrder), dim, eb,
                         aligned != 0);
          check_row_plan(plan_rows(dim, eb, aligned != 0, prefer, kFwdOrderEpilogue), dim, eb,
                         aligned != 0);
          plans += 4;
        }
      }
    }
  }
  // Backward plans and the workspace query, on the dims the benchmarks and tests use plus a
  // spread of others, for every tuning knob value range.
  const int64_t dims[] = {1,    4,    13,   16,   64,    100,   512,   768,  1024, 2048,
                          2560, 3072, 4096, 4104, 5120,  6144,  7168,  8192, 9216, 16384,
                          20000, 40000};
  for (int64_t dim : dims) {
    for (int64_t rows : rows_list) {
      for (int cus : cus_list) {
        for (int prefer = 0; prefer <= kMaxNV; ++prefer) {
          for (int max_block = 64; max_block <= 1024; max_block *= 2) {
            for (int waves = 1; waves <= 64; waves *= 2) {
              const size_t ws = bwd_workspace_bytes(rows, dim, cus, prefer, max_block, waves);
              for (int eb = 2; eb <= 4; eb += 2) {
                for (int aligned = 0; aligned < 2; ++aligned) {
                  const BwdPlan b =
                      plan_bwd(rows, dim, eb, aligned != 0, cus, prefer, max_block, waves);
                  check_row_plan(b.rp, dim, eb, aligned != 0);
                  CHECK(b.wgs >= 1 && b.wgs <= (rows + b.rp.groups - 1) / b.rp.groups,
                        "wgs=%lld rows=%lld groups=%d", (long long)b.wgs, (long long)rows,
                        b.rp.groups);
                  CHECK((size_t)b.wgs * (size_t)dim * sizeof(float) <= ws,
                        "partials %lld x %lld exceed workspace %zu", (long long)b.wgs,
                        (long long)dim, ws);
                  CHECK(b.lds_bytes <= 64 * 1024, "lds %zu", b.lds_bytes);
                  CHECK(b.lds_bytes == 0 || (b.rp.vec && b.rp.groups > 1),
                        "lds without a group combine");
                  // the fused-RoPE plan: same facts, its own block bound, and its step table
                  // (dim floats of LDS) within 64 KiB; or, for rows no walk plan fits, the plain
                  // plan with the rotation evaluated directly (no step table)
                  const BwdPlan br =
                      plan_bwd_rope(rows, dim, eb, aligned != 0, cus, prefer, max_block, waves);
                  check_row_plan(br.rp, dim, eb, aligned != 0);
                  if (br.rope_direct) {
                    CHECK(br.rp.vec && br.rp.block <= max_block_for_nv(br.rp.nv) &&
                              br.lds_bytes <= 64 * 1024,
                          "rope direct block %d nv %d lds %zu", br.rp.block, br.rp.nv,
                          br.lds_bytes);
                  } else {
                    CHECK(!br.rp.vec || br.rp.block <= max_block_for_nv_rope(br.rp.nv),
                          "rope block %d over its bound for nv %d", br.rp.block, br.rp.nv);
                    CHECK(!br.rp.vec || dim * 4 <= 64 * 1024, "rope step table %lld floats",
                          (long long)dim);
                  }
                  CHECK((size_t)br.wgs * (size_t)dim * sizeof(float) <= ws,
                        "rope partials %lld x %lld exceed workspace %zu", (long long)br.wgs,
                        (long long)dim, ws);
                  // the ring-pipelined plan: whole rows, its own block bound, one workgroup per
                  // CU at most, its partials within the workspace
                  const BwdPlan rg = plan_bwd_ring(rows, dim, eb, aligned != 0, cus, prefer);
                  if (rg.ring) {
                    check_row_plan(rg.rp, dim, eb, aligned != 0);
                    CHECK(ring_eligible(rg.rp, dim, eb), "ring plan not eligible dim=%lld",
                          (long long)dim);
                    {
                      // whole waves over the row's chunks, at most 1/8 of the slots idle (for
                      // 2-byte rows of one chunk per thread, less than the last wave), and fewer
                      // idle slots than one chunk per lane
                      const int64_t slots = (int64_t)rg.rp.nv * rg.rp.tpr;
                      const int64_t chunks = dim / (16 / eb);
                      const bool part_wave = rg.rp.nv == 1 && eb == 2 && slots - chunks < kWave;
                      CHECK(dim % (16 / eb) == 0 && slots >= chunks &&
                                ((slots - chunks) * 8 <= slots || part_wave) &&
                                slots - chunks < rg.rp.tpr,
                            "ring plan idle lanes dim=%lld slots=%lld", (long long)dim,
                            (long long)slots);
                    }
                    CHECK(rg.rp.block <= kRingBlock && rg.rp.nv <= kRingMaxNV,
                          "ring block %d nv %d", rg.rp.block, rg.rp.nv);
                    CHECK(rg.wgs >= 1 && rg.wgs <= cus &&
                              rg.wgs <= (rows + rg.rp.groups - 1) / rg.rp.groups,
                          "ring wgs=%lld", (long long)rg.wgs);
                    CHECK((size_t)rg.wgs * (size_t)dim * sizeof(float) <= ws,
                          "ring partials %lld x %lld exceed workspace %zu", (long long)rg.wgs,
                          (long long)dim, ws);
                    CHECK(rg.lds_bytes <= 64 * 1024 &&
                              (rg.lds_bytes == 0) == (rg.rp.groups == 1),
                          "ring lds %zu", rg.lds_bytes);
                  } else {
                    CHECK(!ring_eligible(rg.rp, dim, eb) || !ring_tail_pays(rg.rp, dim, eb),
                          "eligible ring plan refused");
                  }
                  // the ring plan under its tuning knobs (workgroup bound, workgroups per CU):
                  // the same facts, at most two workgroups of at most kRingBlock / 2 threads per
                  // CU (so a CU's resident waves stay eight), and a workspace query made with
                  // the same knobs covering its partial rows
                  for (int rb = 64; rb <= kRingBlock; rb *= 2) {
                    for (int wpc = 1; wpc <= 2; ++wpc) {
                      const BwdPlan rk = plan_bwd_ring(rows, dim, eb, aligned != 0, cus, prefer,
                                                       rb, wpc);
                      if (!rk.ring) {
                        CHECK(!ring_eligible(rk.rp, dim, eb) || rk.rp.tpr > rb ||
                                  !ring_tail_pays(rk.rp, dim, eb),
                              "ring refused under knobs rb=%d wpc=%d dim=%lld", rb, wpc,
                              (long long)dim);
                        continue;
                      }
                      check_row_plan(rk.rp, dim, eb, aligned != 0);
                      const int64_t per_cu = rk.wgs > cus ? 2 : 1;
                      CHECK(rk.rp.block <= rb && rk.rp.block <= kRingBlock &&
                                rk.rp.block * per_cu <= kRingBlock &&
                                rk.wgs >= 1 && rk.wgs <= (int64_t)cus * wpc &&
                                rk.wgs <= (rows + rk.rp.groups - 1) / rk.rp.groups,
                            "ring under knobs rb=%d wpc=%d: block %d wgs %lld", rb, wpc,
                            rk.rp.block, (long long)rk.wgs);
                      CHECK(rk.lds_bytes <= 64 * 1024 &&
                                (rk.lds_bytes == 0) == (rk.rp.groups == 1),
                            "ring lds under knobs %zu", rk.lds_bytes);
                      const size_t wsk = bwd_workspace_bytes(rows, dim, cus, prefer, max_block,
                                                             waves, rb, wpc);
                      CHECK((size_t)rk.wgs * (size_t)dim * sizeof(float) <= wsk,
                            "ring partials under knobs exceed workspace %zu", wsk);
                    }
                  }
                  // the ring-pipelined plan with the fused RoPE gradient: whole rows of one
                  // chunk per thread (two for rows of 513 to 1024 chunks), one workgroup per
                  // CU, two for one chunk per thread in workgroups under 512 threads (or as
                  // many as there are row groups' rows), its tables and combine within 64 KiB
                  // of LDS, its partials within the workspace
                  const BwdPlan rr = plan_bwd_rope_ring(rows, dim, eb, aligned != 0, cus);
                  if (rr.ring) {
                    check_row_plan(rr.rp, dim, eb, aligned != 0);
                    CHECK(rope_ring_eligible(rr.rp, dim, eb), "rope ring plan not eligible");
                    const int64_t chunks = dim / (16 / eb);
                    CHECK(rr.rp.nv == (chunks <= kRingBlock ? 1 : 2) &&
                              (int64_t)rr.rp.nv * rr.rp.tpr * (16 / eb) == dim &&
                              rr.rp.block <= kRingBlock,
                          "rope ring nv %d tpr %d block %d dim=%lld", rr.rp.nv, rr.rp.tpr,
                          rr.rp.block, (long long)dim);
                    const int64_t per_cu = rr.rp.nv == 1 && rr.rp.block < kRingBlock ? 2 : 1;
                    const int64_t need = (rows + rr.rp.groups - 1) / rr.rp.groups;
                    CHECK(rr.wgs == std::min<int64_t>((int64_t)(cus > 0 ? cus : 1) * per_cu, need) &&
                              rr.wgs <= (int64_t)cus * kRopeRingMaxWgsPerCu,
                          "rope ring wgs=%lld block %d", (long long)rr.wgs, rr.rp.block);
                    CHECK((size_t)rr.wgs * (size_t)dim * sizeof(float) <= ws,
                          "rope ring partials %lld x %lld exceed workspace %zu",
                          (long long)rr.wgs, (long long)dim, ws);
                    const size_t tables = rr.rp.nv == 1
                                              ? (size_t)rr.rp.block * (16 / eb / 2) * 24
                                              : (size_t)rr.rp.block * (16 / eb) * 8;
                    CHECK(rr.lds_bytes <= 64 * 1024 &&
                              rr.lds_bytes == tables + (rr.rp.groups > 1 ? dim * 4 : 0),
                          "rope ring lds %zu", rr.lds_bytes);
                  } else {
                    CHECK(!(aligned && eb == 2 && dim % 512 == 0 && dim <= 4096) &&
                              !(aligned && eb == 4 && dim % 256 == 0 && dim <= 2048) &&
                              !(aligned && eb == 2 && dim % 1024 == 0 && dim <= 8192) &&
                              !(aligned && eb == 4 && dim % 512 == 0 && dim <= 4096),
                          "rope ring plan refused dim=%lld eb=%d", (long long)dim, eb);
                  }
                  ++plans;
                }
              }
            }
          }
        }
      }
    }
  }
  // rope_walk_ok: where it holds, the RoPE ring kernel's position rule (start at slot % seq,
  // add S per row, back to the start where that reaches seq) gives row % seq for every row of
  // every slot's walk.
  const int64_t slot_counts[] = {1, 2, 3, 5, 64, 100, 128, 512, 600, 1024, 4096};
  const int64_t seqs[] = {1, 2, 3, 7, 64, 100, 300, 1000, 1024, 2048, 3000, 16384};
  const int64_t walk_rows[] = {1, 5, 64, 1000, 5000, 16384};
  long walks = 0;
  for (int64_t S : slot_counts) {
    for (int64_t seq : seqs) {
      for (int64_t rows : walk_rows) {
        if (!rope_walk_ok(rows, S, seq)) continue;
        const int64_t iters = (rows + S - 1) / S;
        for (int64_t slot = 0; slot < S && slot < rows; ++slot) {
          const int64_t pos0 = slot % seq;
          int64_t pos = pos0;
          for (int64_t j = 0; j < iters; ++j) {
            const int64_t row = slot + j * S;
            if (row < rows)
              CHECK(pos == row % seq, "walk S=%lld seq=%lld rows=%lld slot %lld row %lld: "
                    "pos %lld", (long long)S, (long long)seq, (long long)rows, (long long)slot,
                    (long long)row, (long long)pos);
            pos += S;
            if (pos >= seq) pos = pos0;
          }
          ++walks;
        }
      }
    }
  }
  CHECK(rope_walk_ok(16384, 512, 16384) && rope_walk_ok(16384, 512, 2048) &&
            rope_walk_ok(16448, 2048, 64) && !rope_walk_ok(6000, 512, 1000),
        "rope_walk_ok on the test shapes");
  printf("rope walks checked: %ld\n", walks);
  // The ring over rows of 8-byte alignment (kRing8): 2-byte dims of 8n + 4 only, one chunk per
  // thread over the n whole chunks (a ring plan of dim - 4 columns), LDS for all dim columns when
  // row groups combine, partial rows within the workspace query; 4100, 2052 and 100 take it with
  // 512-, 256- and 64-thread row groups (at 100, 12 of 64 lanes busy), 4108 (513 whole chunks)
  // does not.
  long ring8 = 0;
  for (int64_t dim = 4; dim <= 8200; dim += 4) {
    for (int64_t rows : {1, 300, 16384}) {
      for (int eb = 2; eb <= 4; eb += 2) {
        const BwdPlan r8 = plan_bwd_ring8(rows, dim, eb, 256);
        if (!r8.ring) {
          CHECK(!r8.x8, "refused ring8 plan marked x8 (dim=%lld)", (long long)dim);
          continue;
        }
        ++ring8;
        CHECK(eb == 2 && dim % 8 == 4 && r8.x8 && r8.rp.nv == 1, "ring8 plan dim=%lld eb=%d",
              (long long)dim, eb);
        check_row_plan(r8.rp, dim - 4, eb, true);
        CHECK(ring_eligible(r8.rp, dim - 4, eb) && r8.rp.block <= kRingBlock,
              "ring8 layout dim=%lld", (long long)dim);
        CHECK(r8.lds_bytes == (r8.rp.groups > 1 ? (size_t)dim * sizeof(float) : 0),
              "ring8 lds %zu dim=%lld", r8.lds_bytes, (long long)dim);
        const size_t ws = bwd_workspace_bytes(rows, dim, 256, 0, 1024, 16);
        CHECK((size_t)r8.wgs * (size_t)dim * sizeof(float) <= ws && r8.wgs <= 256,
              "ring8 partials %lld x %lld exceed workspace %zu", (long long)r8.wgs,
              (long long)dim, ws);
      }
    }
  }
  CHECK(plan_bwd_ring8(16384, 4100, 2, 256).ring && plan_bwd_ring8(16384, 4100, 2, 256).rp.tpr == 512,
        "ring8 at 4100");
  CHECK(plan_bwd_ring8(16384, 2052, 2, 256).ring && plan_bwd_ring8(16384, 2052, 2, 256).rp.tpr == 256,
        "ring8 at 2052");
  CHECK(!plan_bwd_ring8(16384, 4108, 2, 256).ring && !plan_bwd_ring8(16384, 4100, 4, 256).ring &&
            !plan_bwd_ring8(16384, 4104, 2, 256).ring,
        "ring8 refusals");
  CHECK(plan_bwd_ring8(16384, 100, 2, 256).ring && plan_bwd_ring8(16384, 100, 2, 256).rp.tpr == 64,
        "ring8 at 100 (12 whole chunks in one partly idle wave)");
  printf("ring8 plans checked: %ld\n", ring8);
  // The element-strided ring: 4 elements a lane for rows of up to 512, else 8, whole waves
  // with less than one idle, every column covered, workgroups
  // within kRingBlock threads and one per CU, LDS for the combine of several row groups, the
  // partial rows within the workspace query; none past 4096 elements.
  long relem = 0;
  for (int64_t dim = 1; dim <= 4200; dim += (dim < 600 ? 1 : 7)) {
    for (int eb = 2; eb <= 4; eb += 2) {
      for (int64_t rows : {1, 300, 16384}) {
        const BwdPlan e = plan_bwd_ring_elem(rows, dim, eb, 256);
        if (dim > 4096) {
          CHECK(e.elem_m == 0, "element ring past 4096 (dim=%lld)", (long long)dim);
          continue;
        }
        ++relem;
        const int m = e.elem_m;
        const int64_t lanes = (dim + m - 1) / m;
        CHECK(m == (dim <= 512 ? 4 : 8) && e.rp.tpr % kWave == 0 &&
                  e.rp.tpr <= kRingBlock && e.rp.tpr - lanes < kWave && lanes <= e.rp.tpr &&
                  (int64_t)m * e.rp.tpr >= dim,
              "element ring layout dim=%lld m=%d tpr=%d", (long long)dim, m, e.rp.tpr);
        CHECK(e.rp.groups >= 1 && e.rp.block == e.rp.groups * e.rp.tpr &&
                  e.rp.block <= kRingBlock && e.wgs >= 1 && e.wgs <= 256 &&
                  e.wgs <= (rows + e.rp.groups - 1) / e.rp.groups &&
                  e.lds_bytes == (e.rp.groups > 1 ? (size_t)dim * sizeof(float) : 0),
              "element ring launch dim=%lld", (long long)dim);
        CHECK((size_t)e.wgs * (size_t)dim * sizeof(float) <=
                  bwd_workspace_bytes(rows, dim, 256, 0, 1024, 16),
              "element ring partials exceed the workspace (dim=%lld)", (long long)dim);
      }
    }
  }
  printf("element ring plans checked: %ld\n", relem);
  // One chunk per thread first in the ring for 2-byte rows, for walks of up to
  // kRingOneChunkMaxIters rows per slot; longer walks, fp32 rows and an explicit preference
  // keep the backward's order (two chunks per thread first).
  {
    const BwdPlan c = plan_bwd_ring(16384, 4096, 2, true, 256, 0);
    const BwdPlan edge = plan_bwd_ring(49152, 4096, 2, true, 256, 0);
    const BwdPlan longer = plan_bwd_ring(49153, 4096, 2, true, 256, 0);
    const BwdPlan f32 = plan_bwd_ring(16384, 2048, 4, true, 256, 0);
    const BwdPlan asked = plan_bwd_ring(16384, 4096, 2, true, 256, 2);
    CHECK(c.ring && c.rp.nv == 1 && c.rp.tpr == 512 && c.wgs == 256, "config C ring plan");
    CHECK(edge.ring && edge.rp.nv == 1, "one chunk per thread at 192 rows per slot");
    CHECK(longer.ring && longer.rp.nv == 2 && longer.rp.tpr == 256,
          "two chunks per thread past 192 rows per slot");
    CHECK(f32.ring && f32.rp.nv == 2 && asked.ring && asked.rp.nv == 2,
          "fp32 rows and an explicit preference keep two chunks per thread");
  }
  // The ring backward over rows with idle lanes: bf16 rows of 1000, 3000, 4000 and 5000 leave
  // 3, 9, 12 and 15 of their chunk slots idle and take it, and 768 and 1280 32 of one chunk per
  // thread's 128 and 192 (a partly idle last wave); 2056 and 4104 would leave more than 1/8
  // idle, 2240 has one chunk per thread in 320-thread rows and 7160 and 8184 two in 448- and
  // 512-thread rows that are not whole 128-byte lines: those stay on bwd_vec_kernel, as do none
  // of the whole rows (2560 in 320-thread rows, 8192).
  for (int64_t dim : {1000, 3000, 4000, 5000, 768, 1280, 2056, 4104, 2240, 7160, 8184, 2560,
                      8192, 6272, 3576}) {
    const BwdPlan rg = plan_bwd_ring(16384, dim, 2, true, 256, 0);
    const int64_t idle = (int64_t)rg.rp.nv * rg.rp.tpr - dim / 8;
    const bool want = dim == 1000 || dim == 3000 || dim == 4000 || dim == 5000 || dim == 2560 ||
                      dim == 8192 || dim == 6272 || dim == 3576 || dim == 768 || dim == 1280;
    CHECK(rg.ring == want, "ring plan over %lld bf16 columns: %d", (long long)dim, (int)rg.ring);
    CHECK(!want || idle == (dim == 1000 ? 3 : dim == 3000 ? 9 : dim == 4000 ? 12 :
                            dim == 5000 ? 15 : dim == 6272 ? 112 : dim == 3576 ? 1 :
                            dim == 768 || dim == 1280 ? 32 : 0),
          "idle chunk slots at %lld: %lld", (long long)dim, (long long)idle);
  }
  // Where the forward stores h: after the reduction for the measured bf16 rows of 2048, 3072
  // and 4096 (whole rows of at most 512 threads), before it for 5120, 7168 and 8192, and never
  // on the generic path.
  for (int64_t dim : {2048, 3072, 4096, 5120, 7168, 8192}) {
    const RowPlan p = plan_rows(dim, 2, true, 0, kFwdOrder);
    CHECK(fwd_late_h(p) == (dim <= 4096), "fwd_late_h dim=%lld tpr=%d", (long long)dim, p.tpr);
  }
  CHECK(!fwd_late_h(plan_rows(4096, 2, false, 0, kFwdOrder)), "fwd_late_h on the generic plan");
  // the norm + RoPE forward's walk length: 32 rows for row groups of more than 256 threads over
  // at least 16384 rows, else 16; the walk's inv_rms stores need a thread per row of the walk
  for (int tpr = 64; tpr <= 1024; tpr += 64) {
    for (int64_t rows : {1, 15, 16, 4096, 16383, 16384, 16385, 262147}) {
      const int w = fwd_rope_walk_rows(rows, tpr);
      CHECK(w == ((tpr > 256 && rows >= 16384) ? 32 : 16) && w <= tpr,
            "fwd_rope_walk_rows rows=%lld tpr=%d -> %d", (long long)rows, tpr, w);
    }
  }
  // Wide norm + RoPE rows (tests/test_gpu_rmsnorm_rope.py): the backward's walk takes three
  // chunks per thread up to 1536 chunks; past that the plain plan with each pair's rotation
  // evaluated directly, two chunks per thread in 832-thread rows at 1540 chunks and four in
  // 512-thread rows at 2048; the forward's direct rows take three or four chunks per thread in
  // 512-thread rows when VELOGRAD_FWD_NV asks for them.
  {
    const BwdPlan a = plan_bwd_rope(64, 12288, 2, true, 256, 0, 1024, 16);
    CHECK(a.rp.vec && !a.rope_direct && a.rp.nv == 3 && a.rp.tpr == 512, "rope bwd 12288");
    const BwdPlan b = plan_bwd_rope(64, 12320, 2, true, 256, 0, 1024, 16);
    CHECK(b.rp.vec && b.rope_direct && b.rp.nv == 2 && b.rp.tpr == 832 &&
              b.rp.block <= max_block_for_nv(2),
          "rope bwd 12320: direct %d nv %d tpr %d", (int)b.rope_direct, b.rp.nv, b.rp.tpr);
    const BwdPlan c = plan_bwd_rope(64, 16384, 2, true, 256, 0, 1024, 16);
    CHECK(c.rp.vec && c.rope_direct && c.rp.nv == 4 && c.rp.tpr == 512, "rope bwd 16384");
    const RowPlan f3 = plan_rows(12288, 2, true, 3, kFwdOrder);
    CHECK(f3.vec && f3.nv == 3 && f3.tpr == 512 && f3.block <= max_block_for_nv(3),
          "fwd nv 3 at 12288: nv %d tpr %d", f3.nv, f3.tpr);
    const RowPlan f4 = plan_rows(16384, 2, true, 4, kFwdOrder);
    CHECK(f4.vec && f4.nv == 4 && f4.tpr == 512 && f4.block <= max_block_for_nv(4),
          "fwd nv 4 at 16384: nv %d tpr %d", f4.nv, f4.tpr);
    const RowPlan f4s = plan_rows(8192, 4, true, 4, kFwdOrder);
    CHECK(f4s.vec && f4s.nv == 4 && f4s.tpr == 512, "fwd nv 4 at fp32 8192");
  }
  // The allocation-free backward refuses fp32 2048 x 16384 (tests/test_zz_no_alloc.py): on 256
  // CUs with the default tuning, every plan the backward can pick for that shape (aligned or
  // not, with or without the ring) needs more partial rows than its 16 MiB scratch holds, while
  // fp32 8192 (its documented bound) fits.
  {
    const int64_t rows = 2048, dim = 16384;
    const size_t scratch = (size_t)16 << 20;
    for (int aligned = 0; aligned < 2; ++aligned) {
      const BwdPlan b = plan_bwd(rows, dim, 4, aligned != 0, 256, 0, 1024, 16);
      CHECK((size_t)b.wgs * dim * sizeof(float) > scratch,
            "no-alloc refusal shape plans %lld partial rows, within the scratch",
            (long long)b.wgs);
      const BwdPlan rg = plan_bwd_ring(rows, dim, 4, aligned != 0, 256, 0);
      CHECK(!rg.ring, "no-alloc refusal shape got a ring plan");
    }
    // the bounds the header states, on the plans the backward picks (no RoPE): 16-byte aligned
    // rows up to 8192 fp32 or 16384 bf16/fp16 elements, other rows up to 4096
    for (int64_t r : {1, 64, 2048, 16384, 262144}) {
      for (int eb = 2; eb <= 4; eb += 2) {
        for (int aligned = 0; aligned < 2; ++aligned) {
          const int64_t dim = aligned ? (eb == 4 ? 8192 : 16384) : 4096;
          const BwdPlan rg = plan_bwd_ring(r, dim, eb, aligned != 0, 256, 0);
          const BwdPlan b = rg.ring ? rg : plan_bwd(r, dim, eb, aligned != 0, 256, 0, 1024, 16);
          CHECK((size_t)b.wgs * dim * sizeof(float) <= scratch,
                "no-alloc bound: eb %d aligned %d dim %lld rows %lld plans %lld partial rows",
                eb, aligned, (long long)dim, (long long)r, (long long)b.wgs);
        }
      }
    }
  }
  if (failures) {
    fprintf(stderr, "%d failures over %ld plans\n", failures, plans);
    return 1;
  }
  printf("plan_check ok: %ld plans\n", plans);
  return 0;
}
