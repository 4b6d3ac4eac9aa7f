// Router gating: scores -> top-k -> optional renormalisation, one wave per
// token. Produces the (topk_weights, topk_ids) pair the fused MoE consumes
// (the routing the reference's tests build with torch ops,
// tests/test_fused_moe.py:37-41, and that _standard_topk_to_triton_kernels
// converts, src/flaggems_sglang/ops/fused_moe.py:119-146).
//
// Each lane holds experts lane, lane+64, ... (VPL per lane). Selection ranks
// the logits themselves (softmax and sigmoid are monotonic, so this is the
// same set as ranking the scores, and it is exact: no rounding can reorder
// two experts); equal logits go to the lower expert id. Selected experts come
// out in rank order, like torch.topk(sorted=True).
#include <math.h>

#include "fgs_common.h"
#include "fgs_moe_kernels.h"

namespace fgs {

template <int VPL>
__global__ __launch_bounds__(256) void topk_gating_kernel(
    const void* __restrict__ logits, int bf16_in, int64_t m, int num_experts,
    int topk, int sigmoid, int renormalize, float* __restrict__ w_out,
    int32_t* __restrict__ id_out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = blockIdx.x * 4LL + (threadIdx.x >> 6);
  if (row >= m) return;  // whole wave

  float v[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = i * 64 + lane;
    if (e < num_experts) {
      const int64_t at = row * num_experts + e;
      v[i] = bf16_in ? bf16_bits_to_f32(static_cast<const uint16_t*>(logits)[at])
                     : static_cast<const float*>(logits)[at];
    } else {
      v[i] = -INFINITY;
    }
  }

  // scores
  float p[VPL];
  if (sigmoid) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) p[i] = 1.0f / (1.0f + __expf(-v[i]));
  } else {
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPL; ++i) mx = fmaxf(mx, v[i]);
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) mx = fmaxf(mx, __shfl_xor(mx, d, 64));
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      p[i] = i * 64 + lane < num_experts ? __expf(v[i] - mx) : 0.f;
      sum += p[i];
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) sum += __shfl_xor(sum, d, 64);
    const float inv = 1.0f / sum;
#pragma unroll
    for (int i = 0; i < VPL; ++i) p[i] *= inv;
  }

  // top-k by (logit desc, expert id asc); lane r keeps the r-th pick
  uint32_t taken = 0;
  float my_w = 0.f, wsum = 0.f;
  int my_id = 0;
  for (int r = 0; r < topk; ++r) {
    float key = -INFINITY;
    int idx = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int e = i * 64 + lane;
      if (e < num_experts && !(taken & (1u << i)) && (v[i] > key || idx == 0x7fffffff)) {
        key = v[i];
        idx = e;
      }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
      const float ok = __shfl_xor(key, d, 64);
      const int oi = __shfl_xor(idx, d, 64);
      if (ok > key || (ok == key && oi < idx)) {
        key = ok;
        idx = oi;
      }
    }
    // idx is now uniform; its owner lane supplies the score
    float pw = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      if (i == idx / 64) pw = p[i];
    pw = __shfl(pw, idx & 63, 64);
    if (lane == (idx & 63)) taken |= 1u << (idx / 64);
    if (lane == r) {
      my_w = pw;
      my_id = idx;
    }
    wsum += pw;
  }
  if (lane < topk) {
    w_out[row * topk + lane] = renormalize ? my_w / wsum : my_w;
    id_out[row * topk + lane] = my_id;
  }
}

int launch_topk_gating(const void* logits, bool bf16_in, int64_t m,
                       int num_experts, int topk, bool sigmoid,
                       bool renormalize, float* w_out, int32_t* id_out,
                       hipStream_t stream) {
  if (m == 0) return FGS_OK;
  const dim3 grid(static_cast<unsigned>((m + 3) / 4));
  const int vpl = (num_experts + 63) / 64;
#define FGS_GATING_CASE(V)                                                      \
  hipLaunchKernelGGL(topk_gating_kernel<V>, grid, dim3(256), 0, stream, logits, \
                     bf16_in ? 1 : 0, m, num_experts, topk, sigmoid ? 1 : 0,     \
                     renormalize ? 1 : 0, w_out, id_out)
  if (vpl <= 1) FGS_GATING_CASE(1);
  else if (vpl <= 2) FGS_GATING_CASE(2);
  else if (vpl <= 4) FGS_GATING_CASE(4);
  else if (vpl <= 8) FGS_GATING_CASE(8);
  else FGS_GATING_CASE(16);
#undef FGS_GATING_CASE
  return check_launch("topk_gating_kernel");
}

}  // namespace fgs
