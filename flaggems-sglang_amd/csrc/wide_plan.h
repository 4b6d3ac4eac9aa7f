// Tile plan of the 4-wave GEMMs (gemm_wide.hip): its layout, and the one-wave
// routine that writes it from per-row-block costs. Two producers use it:
// wide_plan_kernel (from the padded order, ahead of a GEMM) and the
// alignment kernels (align.hip: from the per-expert counts, for both GEMMs of
// a call at once, which saves the two plan launches).
#pragma once

#include "fgs_common.h"

namespace fgs {

constexpr int kPlanMaxRows = 64;  // row blocks a launch may have for a plan
constexpr int kPlanWords = 9;
constexpr int kPlanClaimStride = 64;  // ints: one 256-byte slot per XCD counter
constexpr int kPlanClaimTail = 64;    // positions at the end of a range that are claimed
// row-block cost = base + ceil(live 32-row blocks / 2): a block of a few
// rows costs 6/9 of a full one in GEMM1 (measured 0.65-0.72) and 16/19 in
// GEMM2 (measured 0.80-0.85: its k rows are longer)
constexpr int kPlanBaseGemm1 = 5;
constexpr int kPlanBaseGemm2 = 15;

// One GEMM's plan as the alignment writes it: the plan words (null: no
// plan), the launch's column tiles, the most positions an XCD's range may
// hold, and the row-block base cost.
struct WidePlanReq {
  int32_t* plan;
  int32_t n_ct;
  int32_t cap;
  int32_t base;
};

// Row-block cost from its live rows (bm = 256: 32-row groups whose first
// row is live, 1..8, two per 32-row block of a wave row).
__device__ __forceinline__ int wide_plan_cost(int live_rows, int base) {
  const int lb = (live_rows + 31) / 32;
  return base + (lb + 1) / 2;
}

// Run by all 64 lanes of one wave: lane r < rows holds row block r's cost c
// (lanes beyond rows hold 0). Writes plan[0..8], the bounds of the eight
// XCD ranges in row-block-major tile index: equal cost, or equal count when
// an equal-cost range would exceed cap positions; rows outside 1..
// kPlanMaxRows give plan[0] = -1 (no plan: the kernel splits by count).
// Zeroes the claim counters.
__device__ __forceinline__ void wide_plan_write(int lane, int rows, int c, int n_ct, int cap,
                                                int32_t* plan) {
  if (lane < 8) plan[kPlanWords + lane * kPlanClaimStride] = 0;  // nothing claimed yet
  if (rows <= 0 || rows > kPlanMaxRows) {
    if (lane == 0) plan[0] = -1;
    return;
  }
  int incl = c;  // inclusive sums of the row costs
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int o = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += o;
  }
  const int64_t total_cost = static_cast<int64_t>(__shfl(incl, kWave - 1, kWave)) * n_ct;
  const int64_t lo_cost = static_cast<int64_t>(incl - c) * n_ct;
  const int64_t hi_cost = static_cast<int64_t>(incl) * n_ct;
  const int total_tiles = rows * n_ct;
  // bound x: the first tile whose start cost reaches total_cost * x / 8,
  // found in the row whose cost range holds that target (none: target 0)
  int bound[9];
  bound[0] = 0;
  bound[8] = total_tiles;
#pragma unroll
  for (int x = 1; x < 8; ++x) {
    const int64_t target = total_cost * x / 8;
    const bool own = lane < rows && target > lo_cost && target <= hi_cost;
    const int into = own ? static_cast<int>(target - lo_cost) : 0;  // < n_ct * c
    const int cand = own ? lane * n_ct + (into + c - 1) / c : 0;
    const uint64_t m = __ballot(own);
    bound[x] = m ? __shfl(cand, __ffsll(static_cast<long long>(m)) - 1, kWave) : 0;
  }
  if (lane == 0) {
    bool even = false;
#pragma unroll
    for (int x = 0; x < 8; ++x) even |= bound[x + 1] - bound[x] > cap;
#pragma unroll
    for (int x = 0; x <= 8; ++x)
      plan[x] = even ? static_cast<int>(static_cast<int64_t>(total_tiles) * x / 8) : bound[x];
  }
}

}  // namespace fgs
