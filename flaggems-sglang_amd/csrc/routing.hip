// Routing-format conversion for gfx950, both directions.
//
// (topk_weights, topk_ids) -> the triton_kernels routing tuple of the
// reference's _standard_topk_to_triton_kernels (src/flaggems_sglang/ops/
// fused_moe.py:119-146), block metadata included. The reference sorts each
// token's ids (:130-131), takes a stable argsort of the flattened ids (:134),
// its inverse (:135), the gathered weights (:136), a histogram (:137-139) and
// compute_expt_data_torch's tile tables (:140). Here the stable argsort is
// moe_align_block_size itself (align.hip: a bit-exact stable counting sort),
// run with block size 1 over E + 1 id classes:
//   classes 0..E-1: experts 0..E-1, class E: ids outside [0, E).
// Inside a class, slots stay in flat (token-major) order. Slots with ids
// outside [0, E) (not routed here) go behind expert E-1: matmul_ogs reads
// expert e's rows at gathered positions [token_offs_raw[e],
// token_offs_raw[e+1]) with token_offs_raw starting at 0, so they must not
// sit ahead of expert 0 (where the reference's argsort would put negative
// ids; its own callers never produce them).
//
// Then, per sorted position q (slot s = sorted[q] of token t):
//   topk_indx[q] = t*k + rank of s's id among token t's ids (the index the
//                  reference's per-token sort gives the slot),
//   gate_indx[topk_indx[q]] = q, gate_scal[q] = topk_weights[s],
// and one workgroup derives the histogram from the sorted class array
// (binary search) and the tile tables for block_m in {16, 32, 64, 128}:
//   token_offs_raw[e]      = sum of hist below e (E + 1 entries),
//   token_offs_pad[B][e]   = sum of ceil(hist/B) below e (in tiles),
//   block_pid_map[B][tile] = (b << 16) | e for expert e's b-th tile, -1 past
//                            the last tile (max_tiles entries).
//
// The routing tuple -> what the grouped GEMMs consume (routing_order_kernel,
// the direction the reference's matmul_ogs calls take, :205-231): expert e's
// gathered positions [raw[e], raw[e] + hist[e]) of gather_indx.src_indx become
// its segment of the block-padded order, and each flat slot gets back its
// expert id and gate scale.
#include <algorithm>
#include <string>

#include "fgs_moe_kernels.h"

namespace fgs {

constexpr int kRoutingBlockMs[4] = {16, 32, 64, 128};
constexpr int kRoutingMetaThreads = 1024;

__global__ void routing_class_kernel(const int32_t* __restrict__ ids, int64_t numel,
                                     int num_experts, int32_t* __restrict__ cls) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= numel) return;
  const int e = ids[i];
  cls[i] = (e >= 0 && e < num_experts) ? e : num_experts;
}

__global__ void routing_finish_kernel(const int32_t* __restrict__ ids,
                                      const float* __restrict__ weights, int64_t numel,
                                      int topk, const int32_t* __restrict__ sorted,
                                      float* __restrict__ gate_scal,
                                      int32_t* __restrict__ topk_indx,
                                      int32_t* __restrict__ gate_indx) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= numel) return;
  const int64_t s = sorted[q];
  const int64_t t = s / topk;
  const int j = static_cast<int>(s - t * topk);
  const int e = ids[s];
  int rank = 0;
  for (int jj = 0; jj < topk; ++jj) {
    const int o = ids[t * topk + jj];
    rank += (o < e || (o == e && jj < j)) ? 1 : 0;
  }
  const int32_t r = static_cast<int32_t>(t * topk + rank);
  topk_indx[q] = r;
  gate_indx[r] = static_cast<int32_t>(q);
  gate_scal[q] = weights[s];
}

// First position of `cls_sorted` (non-decreasing, n entries) holding a
// class >= c.
__device__ __forceinline__ int64_t lower_bound_class(const int32_t* cls_sorted, int64_t n,
                                                     int c) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (cls_sorted[mid] < c) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// Inclusive prefix sum of v over the workgroup's threads (one value each).
__device__ int block_inclusive_scan(int v, int* tmp) {
  const int tid = threadIdx.x;
  tmp[tid] = v;
  __syncthreads();
  for (int d = 1; d < kRoutingMetaThreads; d <<= 1) {
    const int add = tid >= d ? tmp[tid - d] : 0;
    __syncthreads();
    tmp[tid] += add;
    __syncthreads();
  }
  const int r = tmp[tid];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kRoutingMetaThreads) void routing_meta_kernel(
    const int32_t* __restrict__ cls_sorted, int64_t numel, int num_experts,
    int32_t* __restrict__ hist, int32_t* __restrict__ token_offs_raw,
    int32_t* __restrict__ token_offs_pad, int32_t* __restrict__ block_pid_map,
    int64_t max_tiles) {
  __shared__ int tmp[kRoutingMetaThreads];
  __shared__ int incl[kRoutingMetaThreads];
  const int e = threadIdx.x;  // one expert per thread (num_experts < 1024)
  int h = 0;
  if (e < num_experts)
    h = static_cast<int>(lower_bound_class(cls_sorted, numel, e + 1) -
                         lower_bound_class(cls_sorted, numel, e));
  if (e < num_experts) hist[e] = h;
  const int raw = block_inclusive_scan(h, tmp);
  if (e == 0) token_offs_raw[0] = 0;
  if (e < num_experts) token_offs_raw[e + 1] = raw;
  for (int bi = 0; bi < 4; ++bi) {
    const int bm = kRoutingBlockMs[bi];
    const int tiles = (h + bm - 1) / bm;
    const int inc = block_inclusive_scan(e < num_experts ? tiles : 0, tmp);
    int32_t* pad = token_offs_pad + static_cast<int64_t>(bi) * (num_experts + 1);
    if (e == 0) pad[0] = 0;
    if (e < num_experts) pad[e + 1] = inc;
    incl[e] = inc;
    __syncthreads();
    const int total = incl[num_experts - 1];
    int32_t* map = block_pid_map + static_cast<int64_t>(bi) * max_tiles;
    for (int64_t t = e; t < max_tiles; t += kRoutingMetaThreads) {
      int32_t v = -1;
      if (t < total) {
        // expert of tile t: the first e with incl[e] > t
        int lo = 0, hi = num_experts - 1;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (incl[mid] > t) hi = mid;
          else lo = mid + 1;
        }
        const int first = lo == 0 ? 0 : incl[lo - 1];
        v = (static_cast<int32_t>(t - first) << 16) | lo;
      }
      map[t] = v;
    }
    __syncthreads();
  }
}

int64_t routing_max_tiles(int64_t numel, int num_experts) {
  // compute_expt_data_torch's bound for the smallest block (16): at most
  // ceil((numel - E + 1) / 16) + E - 1 tiles, or numel when numel <= E
  if (numel <= num_experts) return numel;
  return (numel - num_experts + 1 + 15) / 16 + num_experts - 1;
}

int64_t routing_workspace_bytes(int64_t numel, int num_experts) {
  auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
  // classes, sorted positions, class per position, padded total, align scratch
  return 3 * up(numel * 4) + 256 + up(align_scratch_bytes(numel, num_experts + 1));
}

int launch_topk_to_routing(const float* weights, const int32_t* ids, int64_t m, int topk,
                           int num_experts, float* gate_scal, int32_t* topk_indx,
                           int32_t* gate_indx, int32_t* hist, int32_t* token_offs_raw,
                           int32_t* token_offs_pad, int32_t* block_pid_map,
                           int64_t max_tiles, void* workspace, hipStream_t stream) {
  const int64_t numel = m * topk;
  auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  int32_t* cls = reinterpret_cast<int32_t*>(ws);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + up(numel * 4));
  int32_t* cls_sorted = reinterpret_cast<int32_t*>(ws + 2 * up(numel * 4));
  int32_t* npp = reinterpret_cast<int32_t*>(ws + 3 * up(numel * 4));
  int32_t* scratch = align_scratch_bytes(numel, num_experts + 1) > 0
                         ? reinterpret_cast<int32_t*>(ws + 3 * up(numel * 4) + 256)
                         : nullptr;
  constexpr int kThreads = 256;
  const int blocks = static_cast<int>((numel + kThreads - 1) / kThreads);
  if (numel > 0) {
    hipLaunchKernelGGL(routing_class_kernel, dim3(blocks), dim3(kThreads), 0, stream, ids,
                       numel, num_experts, cls);
    int rc = check_launch("routing_class_kernel");
    if (rc) return rc;
    // block size 1: sorted holds every slot, cls_sorted its class
    rc = launch_align(cls, numel, num_experts + 1, 1, sorted, cls_sorted, npp, numel, stream,
                      scratch);
    if (rc) return rc;
    hipLaunchKernelGGL(routing_finish_kernel, dim3(blocks), dim3(kThreads), 0, stream, ids,
                       weights, numel, topk, sorted, gate_scal, topk_indx, gate_indx);
    rc = check_launch("routing_finish_kernel");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(routing_meta_kernel, dim3(1), dim3(kRoutingMetaThreads), 0, stream,
                     cls_sorted, numel, num_experts, hist, token_offs_raw, token_offs_pad,
                     block_pid_map, max_tiles);
  return check_launch("routing_meta_kernel");
}


// ------------------------------------------------ routing tuple -> order ---
constexpr int kOrderThreads = 1024;  // one expert per thread (E <= 1024)

// Inclusive prefix sum over the workgroup (64-bit: a caller's histogram
// may hold anything).
__device__ int64_t block_inclusive_scan64(int64_t v, int64_t* tmp) {
  const int tid = threadIdx.x;
  tmp[tid] = v;
  __syncthreads();
  for (int d = 1; d < static_cast<int>(blockDim.x); d <<= 1) {
    const int64_t add = tid >= d ? tmp[tid - d] : 0;
    __syncthreads();
    tmp[tid] += add;
    __syncthreads();
  }
  const int64_t r = tmp[tid];
  __syncthreads();
  return r;
}

// First index i in [0, n) with incl[i] > x (incl non-decreasing; n when none).
__device__ __forceinline__ int first_above(const int32_t* incl, int n, int64_t x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (incl[mid] > x) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

// Expert e reads gathered positions [raw[e], raw[e] + h[e]) with raw the
// exclusive sums of the histogram (token_offs_raw, as matmul_ogs reads
// them); h is the histogram clamped so every range stays inside [0, numel)
// (negative counts read as 0, sums past numel are cut at numel).
//   order (sorted_ids != null): sorted_ids[pad[e] + i] = src[raw[e] + i] for
//     i < h[e], numel elsewhere (pads, and src entries outside [0, numel));
//     pad[e] = exclusive sums of ceil(h / block) * block; expert_ids[b] = the
//     expert of padded row b * block, -1 past the padded total;
//     *num_post_pad = the padded total;
//   inverse (ids_out != null): for every gathered position p with
//     v = src[p] in [0, numel): ids_out[v] = the expert whose range holds p
//     (-1 past the histogram's total: a slot no expert reads),
//     w_out[v] = gate_scal[p].
// Every workgroup (one thread per expert: blockDim >= E, a power of two up
// to 1024) derives the offsets itself and then walks its share of the
// positions; no atomics, so the result is deterministic.
__global__ __launch_bounds__(kOrderThreads) void routing_order_kernel(
    const float* __restrict__ gate_scal, const int32_t* __restrict__ src,
    const int32_t* __restrict__ hist, int64_t numel, int num_experts, int block,
    int64_t max_padded, int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ num_post_pad, int32_t* __restrict__ ids_out,
    float* __restrict__ w_out) {
  __shared__ int64_t tmp[kOrderThreads];
  __shared__ int32_t raw_incl[kOrderThreads];
  __shared__ int32_t pad_incl[kOrderThreads];
  const int e = threadIdx.x;
  const int E = num_experts;
  int64_t h = e < E ? static_cast<int64_t>(hist[e]) : 0;
  h = h < 0 ? 0 : (h > numel ? numel : h);
  const int64_t r = min(block_inclusive_scan64(h, tmp), numel);
  raw_incl[e] = static_cast<int32_t>(r);
  __syncthreads();
  const int64_t hc = e < E ? r - (e > 0 ? raw_incl[e - 1] : 0) : 0;
  const int64_t pc = (hc + block - 1) / block * block;
  pad_incl[e] = static_cast<int32_t>(block_inclusive_scan64(pc, tmp));
  __syncthreads();
  const int64_t total_raw = raw_incl[E - 1];
  const int64_t total_pad = pad_incl[E - 1];

  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  if (sorted_ids) {
    for (int64_t q = tid; q < max_padded; q += stride) {
      int32_t v = static_cast<int32_t>(numel);
      if (q < total_pad) {
        const int x = first_above(pad_incl, E, q);
        const int64_t i = q - (x > 0 ? pad_incl[x - 1] : 0);
        const int64_t r0 = x > 0 ? raw_incl[x - 1] : 0;
        if (i < raw_incl[x] - r0) {
          const int32_t s = src[r0 + i];
          if (s >= 0 && s < numel) v = s;
        }
      }
      sorted_ids[q] = v;
    }
    for (int64_t b = tid; b < max_padded / block; b += stride)
      expert_ids[b] = b * block < total_pad ? first_above(pad_incl, E, b * block) : -1;
    if (tid == 0) *num_post_pad = static_cast<int32_t>(total_pad);
  }
  if (ids_out) {
    for (int64_t p = tid; p < numel; p += stride) {
      const int32_t s = src[p];
      if (s < 0 || s >= numel) continue;
      ids_out[s] = p < total_raw ? first_above(raw_incl, E, p) : -1;
      w_out[s] = gate_scal[p];
    }
  }
}

int launch_routing_order(const float* gate_scal, const int32_t* src, const int32_t* hist,
                         int64_t numel, int num_experts, int block, int64_t max_padded,
                         int32_t* sorted_ids, int32_t* expert_ids, int32_t* num_post_pad,
                         int32_t* ids_out, float* w_out, hipStream_t stream) {
  if (num_experts < 1 || num_experts > kOrderThreads)
    return fail(FGS_EINVAL, "routing order: num_experts must be in [1, 1024]");
  // one wave for up to 64 experts (its barriers cost next to nothing)
  int threads = 64;
  while (threads < num_experts) threads *= 2;
  const int64_t work = std::max<int64_t>(sorted_ids ? max_padded : 0, numel);
  const int blocks =
      static_cast<int>(std::min<int64_t>(std::max<int64_t>((work + threads - 1) / threads, 1), 1024));
  hipLaunchKernelGGL(routing_order_kernel, dim3(blocks), dim3(threads), 0, stream,
                     gate_scal, src, hist, numel, num_experts, block, max_padded, sorted_ids,
                     expert_ids, num_post_pad, ids_out, w_out);
  return check_launch("routing_order_kernel");
}

}  // namespace fgs
