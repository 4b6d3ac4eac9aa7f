// moe_align_block_size for gfx950.
//
// Replaces the routing conversion of the reference
// (src/flaggems_sglang/ops/fused_moe.py:130-139): a stable argsort of the
// flattened expert ids (:134) and a per-expert histogram (:137-139). The
// output is the block-padded, expert-grouped order the grouped GEMMs consume.
//
// One workgroup of 16 wave64s (and, asked for tile plans, a second that
// writes them). Wave w owns the contiguous slot segment
// [w*seg, (w+1)*seg). Pass 1 counts ids per (wave, expert) in LDS; pass 2
// turns the counts into per-expert padded offsets plus per-wave offsets
// inside each expert (exclusive over waves, so lower slots come first);
// pass 3 walks each segment in slot order, 64 slots at a time, ranking each
// slot among equal ids of the chunk with ballots over the id bits. Nothing
// order-deciding uses atomics, so the result is bit-exact and stable.
#include <mutex>
#include <string>

#include "fgs_common.h"
#include "fgs_moe_kernels.h"

namespace fgs {

// The 4-wave GEMMs' tile plans from the per-expert counts (one wave, once
// the padded offsets are final): lane r costs row block r from the live rows
// the expert holding it has there -- what wide_plan_kernel reads back from
// the padded order -- so the GEMM launches need no plan kernel. The plans
// need block_size 256 (the 4-wave kernel's row block). An extra workgroup of
// the alignment launch writes them: it redoes the counts and the padded
// scan beside the others and stops there, so the plans stay off the
// critical path of the scatter.
__device__ __forceinline__ void align_write_plans(int lane, const int32_t* off,
                                                  const int32_t* tot, int E, int block_size,
                                                  const WidePlanReq& r0, const WidePlanReq& r1) {
  const int rows = off[E] / block_size;
  int live = 0;
  if (rows <= kPlanMaxRows && lane < rows) {
    const int pos = lane * block_size;
    // the expert holding padded position pos: the last e with off[e] <= pos
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (off[mid] <= pos) lo = mid;
      else hi = mid - 1;
    }
    live = min(block_size, tot[lo] - (pos - off[lo]));
  }
  if (r0.plan)
    wide_plan_write(lane, rows, live > 0 ? wide_plan_cost(live, r0.base) : 0, r0.n_ct, r0.cap,
                    r0.plan);
  if (r1.plan)
    wide_plan_write(lane, rows, live > 0 ? wide_plan_cost(live, r1.base) : 0, r1.n_ct, r1.cap,
                    r1.plan);
}

constexpr int kAlignWaves = 16;
constexpr int64_t kAlignMultiMin = 4096;  // slots from which the multi-WG path runs
constexpr int kAlignThreads = kAlignWaves * kWave;

__global__ __launch_bounds__(kAlignThreads) void moe_align_kernel(
    const int32_t* __restrict__ ids, int64_t numel, int num_experts,
    int block_size, int id_bits, int32_t* __restrict__ sorted_ids,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ num_post_pad,
    int64_t max_padded, WidePlanReq plan0, WidePlanReq plan1) {
  // cnt[w * E + e]: pass 1 count, then (after pass 2) the slot cursor.
  extern __shared__ int32_t smem[];
  int32_t* cnt = smem;                                  // [16][E]
  int32_t* off = smem + kAlignWaves * num_experts;      // [E + 1]
  int32_t* tot = off + num_experts + 1;                 // [E]
  __shared__ int32_t scan_tmp[kAlignThreads / kWave];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int E = num_experts;

  for (int i = tid; i < kAlignWaves * E; i += kAlignThreads) cnt[i] = 0;
  __syncthreads();

  // Segment per wave, a multiple of 64 slots.
  const int64_t seg =
      ((numel + kAlignWaves - 1) / kAlignWaves + kWave - 1) / kWave * kWave;
  const int64_t beg = static_cast<int64_t>(wave) * seg;
  const int64_t end = beg + seg < numel ? beg + seg : numel;

  // Pass 1: per-(wave, expert) histogram.
  for (int64_t i = beg + lane; i < end; i += kWave) {
    const int e = ids[i];
    if (e >= 0 && e < E) atomicAdd(&cnt[wave * E + e], 1);
  }
  __syncthreads();

  // Pass 2a: per expert, total and exclusive offsets over waves.
  for (int e = tid; e < E; e += kAlignThreads) {
    int run = 0;
    for (int w = 0; w < kAlignWaves; ++w) {
      const int c = cnt[w * E + e];
      cnt[w * E + e] = run;
      run += c;
    }
    tot[e] = run;
  }
  __syncthreads();

  // Pass 2b: exclusive scan of padded sizes over experts (block scan over
  // chunks of kAlignThreads experts).
  int carry = 0;
  for (int base = 0; base < E; base += kAlignThreads) {
    const int e = base + tid;
    const int padded =
        e < E ? (tot[e] + block_size - 1) / block_size * block_size : 0;
    // inclusive scan within the wave
    int v = padded;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int t = __shfl_up(v, d, kWave);
      if (lane >= d) v += t;
    }
    if (lane == kWave - 1) scan_tmp[wave] = v;
    __syncthreads();
    int wave_base = 0;
    int all = 0;
    for (int w = 0; w < kAlignThreads / kWave; ++w) {
      const int s = scan_tmp[w];
      if (w < wave) wave_base += s;
      all += s;
    }
    if (e < E) off[e] = carry + wave_base + v - padded;
    carry += all;
    __syncthreads();
  }
  if (tid == 0) {
    off[E] = carry;
    if (blockIdx.x == 0) num_post_pad[0] = carry;
  }
  __syncthreads();
  if (blockIdx.x == 1) {  // the plan workgroup
    if (wave == 0) align_write_plans(lane, off, tot, E, block_size, plan0, plan1);
    return;
  }

  const int total_padded = off[E];

  // Pass 2c: sentinel fill of pads and of the tail, and block -> expert map.
  for (int e = wave; e < E; e += kAlignWaves) {
    const int64_t p0 = static_cast<int64_t>(off[e]) + tot[e];
    const int64_t p1 = off[e + 1];
    for (int64_t p = p0 + lane; p < p1; p += kWave)
      sorted_ids[p] = static_cast<int32_t>(numel);
    for (int b = off[e] / block_size + lane; b < off[e + 1] / block_size;
         b += kWave)
      expert_ids[b] = e;
  }
  for (int64_t p = total_padded + tid; p < max_padded; p += kAlignThreads)
    sorted_ids[p] = static_cast<int32_t>(numel);
  for (int64_t b = total_padded / block_size + tid; b < max_padded / block_size;
       b += kAlignThreads)
    expert_ids[b] = -1;

  // Pass 3: stable scatter. Chunks of 64 consecutive slots; rank among equal
  // ids of the chunk from ballots over the id bits.
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
  for (int64_t c0 = beg; c0 < end; c0 += kWave) {
    const int64_t i = c0 + lane;
    int e = -1;
    if (i < end) {
      e = ids[i];
      if (e < 0 || e >= E) e = -1;
    }
    const bool valid = e >= 0;
    uint64_t match = __ballot(valid);
    for (int b = 0; b < id_bits; ++b) {
      const bool bit = valid && ((e >> b) & 1);
      const uint64_t on = __ballot(bit);
      match &= bit ? on : ~on;
    }
    int base = 0;
    if (valid) base = cnt[wave * E + e];
    const int rank = __popcll(match & lt_mask);
    // Highest matching lane advances the cursor after every lane has read it.
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      sorted_ids[off[e] + base + rank] = static_cast<int32_t>(i);
      const bool leader = (match >> lane) == 1ull;
      if (leader) cnt[wave * E + e] = base + __popcll(match);
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// ------------------------------------------------ multi-workgroup variant ---
// For many slots: the ids are cut into chunks of kChunk consecutive slots.
// Kernel 1 counts each chunk's ids per expert (counts[c][e]). Kernel 2 runs
// one workgroup per chunk: it sums the counts of every chunk (totals) and of
// the chunks before its own (its per-expert base, so lower slots come
// first), redoes the padded scan over experts, then ranks its own chunk like
// pass 3 above (per-wave LDS counts, ballots over the id bits) and scatters.
// Pads, the tail and the block -> expert map are split over the
// workgroups. Same output, bit for bit, as moe_align_kernel.
constexpr int kChunkWaves = 4;
constexpr int kChunkThreads = kChunkWaves * kWave;
constexpr int kChunk = 1024;  // slots per chunk (256 per wave)

__global__ __launch_bounds__(kChunkThreads) void moe_align_count_kernel(
    const int32_t* __restrict__ ids, int64_t numel, int num_experts,
    int32_t* __restrict__ counts) {
  extern __shared__ int32_t hist[];  // [E]
  const int E = num_experts;
  for (int e = threadIdx.x; e < E; e += kChunkThreads) hist[e] = 0;
  __syncthreads();
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kChunk;
  for (int64_t i = c0 + threadIdx.x; i < c0 + kChunk && i < numel; i += kChunkThreads) {
    const int e = ids[i];
    if (e >= 0 && e < E) atomicAdd(&hist[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kChunkThreads)
    counts[static_cast<int64_t>(blockIdx.x) * E + e] = hist[e];
}

__global__ __launch_bounds__(kChunkThreads) void moe_align_scatter_kernel(
    const int32_t* __restrict__ ids, int64_t numel, int num_experts,
    int block_size, int id_bits, const int32_t* __restrict__ counts,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ num_post_pad, int64_t max_padded, WidePlanReq plan0,
    WidePlanReq plan1) {
  extern __shared__ int32_t smem[];
  const int E = num_experts;
  int32_t* cnt = smem;                         // [4][E]: wave counts, then cursors
  int32_t* off = cnt + kChunkWaves * E;        // [E + 1] padded expert offsets
  int32_t* tot = off + E + 1;                  // [E]
  int32_t* pre = tot + E;                      // [E] slots of earlier chunks
  __shared__ int32_t scan_tmp[kChunkWaves];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int c = blockIdx.x;
  // with plans, the last workgroup writes them and scatters nothing
  const int nchunks = gridDim.x - (plan0.plan || plan1.plan ? 1 : 0);

  for (int e = tid; e < E; e += kChunkThreads) {
    // 16 chunks' counts in flight at a time (integer sums: any order)
    int before = 0, all = 0;
    int cc = 0;
    for (; cc + 16 <= nchunks; cc += 16) {
      int v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = counts[static_cast<int64_t>(cc + u) * E + e];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        if (cc + u < c) before += v[u];
        all += v[u];
      }
    }
    for (; cc < nchunks; ++cc) {
      const int v = counts[static_cast<int64_t>(cc) * E + e];
      if (cc < c) before += v;
      all += v;
    }
    pre[e] = before;
    tot[e] = all;
  }
  for (int i = tid; i < kChunkWaves * E; i += kChunkThreads) cnt[i] = 0;
  __syncthreads();

  // exclusive scan of padded sizes over experts
  int carry = 0;
  for (int base = 0; base < E; base += kChunkThreads) {
    const int e = base + tid;
    const int padded = e < E ? (tot[e] + block_size - 1) / block_size * block_size : 0;
    int v = padded;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int t = __shfl_up(v, d, kWave);
      if (lane >= d) v += t;
    }
    if (lane == kWave - 1) scan_tmp[wave] = v;
    __syncthreads();
    int wave_base = 0, all = 0;
    for (int w = 0; w < kChunkWaves; ++w) {
      const int sw = scan_tmp[w];
      if (w < wave) wave_base += sw;
      all += sw;
    }
    if (e < E) off[e] = carry + wave_base + v - padded;
    carry += all;
    __syncthreads();
  }
  if (tid == 0) off[E] = carry;
  if (c == 0 && tid == 0) num_post_pad[0] = carry;
  if (c == nchunks) {  // the plan workgroup
    __syncthreads();
    if (wave == 0) align_write_plans(lane, off, tot, E, block_size, plan0, plan1);
    return;
  }

  // this chunk's per-(wave, expert) counts; each wave owns 256 slots
  const int64_t wbeg = static_cast<int64_t>(c) * kChunk + wave * (kChunk / kChunkWaves);
  const int64_t wend = wbeg + kChunk / kChunkWaves < numel ? wbeg + kChunk / kChunkWaves : numel;
  for (int64_t i = wbeg + lane; i < wend; i += kWave) {
    const int e = ids[i];
    if (e >= 0 && e < E) atomicAdd(&cnt[wave * E + e], 1);
  }
  __syncthreads();
  // cursors: expert offset + earlier chunks + earlier waves of this chunk
  for (int e = tid; e < E; e += kChunkThreads) {
    int run = off[e] + pre[e];
    for (int w = 0; w < kChunkWaves; ++w) {
      const int v = cnt[w * E + e];
      cnt[w * E + e] = run;
      run += v;
    }
  }
  __syncthreads();

  // pads and block -> expert map of experts c, c + nchunks, ...; the tail
  const int total_padded = off[E];
  for (int e = c * kChunkWaves + wave; e < E; e += nchunks * kChunkWaves) {
    const int64_t p0 = static_cast<int64_t>(off[e]) + tot[e];
    for (int64_t p = p0 + lane; p < off[e + 1]; p += kWave)
      sorted_ids[p] = static_cast<int32_t>(numel);
    for (int b = off[e] / block_size + lane; b < off[e + 1] / block_size; b += kWave)
      expert_ids[b] = e;
  }
  for (int64_t p = total_padded + static_cast<int64_t>(c) * kChunkThreads + tid;
       p < max_padded; p += static_cast<int64_t>(nchunks) * kChunkThreads)
    sorted_ids[p] = static_cast<int32_t>(numel);
  for (int64_t b = total_padded / block_size + static_cast<int64_t>(c) * kChunkThreads + tid;
       b < max_padded / block_size; b += static_cast<int64_t>(nchunks) * kChunkThreads)
    expert_ids[b] = -1;

  // stable scatter, 64 slots at a time
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
  for (int64_t c0 = wbeg; c0 < wend; c0 += kWave) {
    const int64_t i = c0 + lane;
    int e = -1;
    if (i < wend) {
      e = ids[i];
      if (e < 0 || e >= E) e = -1;
    }
    const bool valid = e >= 0;
    uint64_t match = __ballot(valid);
    for (int b = 0; b < id_bits; ++b) {
      const bool bit = valid && ((e >> b) & 1);
      const uint64_t on = __ballot(bit);
      match &= bit ? on : ~on;
    }
    int base = 0;
    if (valid) base = cnt[wave * E + e];
    const int rank = __popcll(match & lt_mask);
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      sorted_ids[base + rank] = static_cast<int32_t>(i);
      const bool leader = (match >> lane) == 1ull;
      if (leader) cnt[wave * E + e] = base + __popcll(match);
    }
    __builtin_amdgcn_wave_barrier();
  }
}

int64_t align_scratch_bytes(int64_t numel, int num_experts) {
  if (numel < kAlignMultiMin) return 0;
  return (numel + kChunk - 1) / kChunk * num_experts * static_cast<int64_t>(sizeof(int32_t));
}

// Decode-sized inputs (numel <= 64): one wave, no barriers, no loop over
// the slots. Lane i holds slot i's id. Ballots over the id bits, most
// significant first, give each lane the masks of lanes with an equal and
// with a smaller id, hence its expert's count, its stable rank and the
// number of slots before its expert; bit-sliced ballots of the experts' pad
// sizes (< block_size, held by each expert's first slot) add the padding
// before it. The buffers are then written as moe_align_kernel writes them:
// sentinel everywhere (made visible before the slots land on it), slots,
// the block -> expert map and its -1 tail.
__global__ __launch_bounds__(kWave) void moe_align_wave_kernel(
    const int32_t* __restrict__ ids, int numel, int num_experts, int block_size,
    int id_bits, int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ num_post_pad, int64_t max_padded) {
  const int lane = threadIdx.x;
  int e = -1;
  if (lane < numel) {
    e = ids[lane];
    if (e < 0 || e >= num_experts) e = -1;  // dropped slot
  }
  const bool valid = e >= 0;
  uint64_t eq = __ballot(valid);
  uint64_t lt = 0;
  for (int b = id_bits - 1; b >= 0; --b) {
    const bool bit = valid && ((e >> b) & 1);
    const uint64_t on = __ballot(bit);
    if (bit) lt |= eq & ~on;  // same higher bits, this bit clear: smaller id
    eq &= bit ? on : ~on;
  }
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
  const int cnt = valid ? __popcll(eq) : 0;
  const int rank = valid ? __popcll(eq & below) : 0;
  const bool first = valid && rank == 0;
  const int pad = first ? (cnt + block_size - 1) / block_size * block_size - cnt : 0;
  int off = __popcll(lt);  // slots of smaller experts
  int total = __popcll(__ballot(valid));
  for (int k = 0; (1 << k) < block_size; ++k) {
    const uint64_t pk = __ballot(first && ((pad >> k) & 1));
    off += __popcll(lt & pk) << k;
    total += __popcll(pk) << k;
  }
  for (int64_t q = lane; q < max_padded; q += kWave) sorted_ids[q] = numel;
  __builtin_amdgcn_s_waitcnt(0);  // the sentinel fill completes before the slots
  if (valid) sorted_ids[off + rank] = lane;
  if (first)
    for (int blk = off / block_size; blk < (off + cnt + pad) / block_size; ++blk)
      expert_ids[blk] = e;
  for (int64_t blk = total / block_size + lane; blk < max_padded / block_size; blk += kWave)
    expert_ids[blk] = -1;
  if (lane == 0) num_post_pad[0] = total;
}

size_t align_smem_bytes(int num_experts) {
  return sizeof(int32_t) *
         (static_cast<size_t>(kAlignWaves) * num_experts + 2 * num_experts + 1);
}

int launch_align(const int32_t* ids, int64_t numel, int num_experts,
                 int block_size, int32_t* sorted_ids, int32_t* expert_ids,
                 int32_t* num_post_pad, int64_t max_padded,
                 hipStream_t stream, int32_t* scratch, const WidePlanReq* plans,
                 bool* planned) {
  int id_bits = 0;
  while ((1 << id_bits) < num_experts) ++id_bits;
  WidePlanReq plan0{}, plan1{};
  if (plans && block_size == 256) {
    plan0 = plans[0];
    plan1 = plans[1];
  }
  if (planned) *planned = false;
  if (numel <= kWave) {
    hipLaunchKernelGGL(moe_align_wave_kernel, dim3(1), dim3(kWave), 0, stream, ids,
                       static_cast<int>(numel), num_experts, block_size, id_bits,
                       sorted_ids, expert_ids, num_post_pad, max_padded);
    return check_launch("moe_align_wave_kernel");
  }
  if (scratch && numel >= kAlignMultiMin) {
    const int nchunks = static_cast<int>((numel + kChunk - 1) / kChunk);
    const size_t smem1 = sizeof(int32_t) * num_experts;
    const size_t smem2 = sizeof(int32_t) * ((kChunkWaves + 3) * num_experts + 1);
    hipLaunchKernelGGL(moe_align_count_kernel, dim3(nchunks), dim3(kChunkThreads),
                       smem1, stream, ids, numel, num_experts, scratch);
    int rc = check_launch("moe_align_count_kernel");
    if (rc) return rc;
    const bool with_plans = plan0.plan || plan1.plan;
    hipLaunchKernelGGL(moe_align_scatter_kernel, dim3(nchunks + (with_plans ? 1 : 0)),
                       dim3(kChunkThreads),
                       smem2, stream, ids, numel, num_experts, block_size, id_bits,
                       scratch, sorted_ids, expert_ids, num_post_pad, max_padded, plan0, plan1);
    rc = check_launch("moe_align_scatter_kernel");
    if (!rc && planned) *planned = plan0.plan || plan1.plan;
    return rc;
  }
  const size_t smem = align_smem_bytes(num_experts);
  if (smem > 64 * 1024) {
    // gfx950 has 160 KiB of LDS per CU; opt in beyond the 64 KiB default.
    static std::once_flag once;
    static hipError_t attr_err = hipSuccess;
    std::call_once(once, [] {
      attr_err = hipFuncSetAttribute(
          reinterpret_cast<const void*>(&moe_align_kernel),
          hipFuncAttributeMaxDynamicSharedMemorySize,
          static_cast<int>(align_smem_bytes(1024)));
    });
    if (attr_err != hipSuccess)
      return fail(FGS_ELAUNCH, std::string("moe_align_kernel LDS opt-in: ") +
                                   hipGetErrorString(attr_err));
  }
  const bool with_plans = plan0.plan || plan1.plan;
  hipLaunchKernelGGL(moe_align_kernel, dim3(with_plans ? 2 : 1), dim3(kAlignThreads), smem,
                     stream, ids, numel, num_experts, block_size, id_bits,
                     sorted_ids, expert_ids, num_post_pad, max_padded, plan0, plan1);
  const int rc = check_launch("moe_align_kernel");
  if (!rc && planned) *planned = plan0.plan || plan1.plan;
  return rc;
}

}  // namespace fgs
