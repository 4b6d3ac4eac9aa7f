// Bandwidth-bound kernels of the fused-MoE path: silu_and_mul, moe_sum and
// the dynamic activation quantisers. Every thread moves 16-byte vectors;
// a row is processed by consecutive threads so each wave touches one or two
// contiguous 1 KiB spans per instruction.
#include <string>
#include <type_traits>

#include "fgs_moe_kernels.h"

namespace fgs {

// ----------------------------------------------------------- silu_and_mul ---
// out[r, c] = bf16(silu(f32(in[r, c])) * f32(in[r, n + c]))
// (ops/fused_moe.py:44-63). Requires n % 8 == 0; 8 columns per thread.
__global__ __launch_bounds__(256) void silu_and_mul_kernel(
    const uint16_t* __restrict__ in, uint16_t* __restrict__ out, int64_t rows,
    int64_t n) {
  const int64_t vec_per_row = n / 8;
  const int64_t total = rows * vec_per_row;
  for (int64_t v = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
       v < total; v += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = v / vec_per_row;
    const int64_t c = (v - r * vec_per_row) * 8;
    const u32x4 g = *reinterpret_cast<const u32x4*>(in + r * 2 * n + c);
    const u32x4 u = *reinterpret_cast<const u32x4*>(in + r * 2 * n + n + c);
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float g0 = __uint_as_float(g[j] << 16);
      const float g1 = __uint_as_float(g[j] & 0xffff0000u);
      const float u0 = __uint_as_float(u[j] << 16);
      const float u1 = __uint_as_float(u[j] & 0xffff0000u);
      o[j] = pack_bf16x2(silu_mul(g0, u0), silu_mul(g1, u1));
    }
    *reinterpret_cast<u32x4*>(out + r * n + c) = o;
  }
}

// ---------------------------------------------------------------- moe_sum ---
// out[t, c] = bf16(sum_j f32(in[t, j, c])): the top-k reduction that
// matmul_ogs performs when given scatter_indx (ops/fused_moe.py:224-231).
// Requires k % 8 == 0. With `ids` given, slots whose expert id lies outside
// [0, num_experts) were never computed and contribute nothing. With
// `weights` given each slot is scaled first: out = bf16(sum_j w_j * y_j),
// product and sum each rounded in fp32 in slot order (no fused multiply-add),
// which is the gammas-on-GEMM2 reduction of ops/fused_moe.py:203,224-231.
__global__ __launch_bounds__(256) void moe_sum_kernel(
    const uint16_t* __restrict__ in, uint16_t* __restrict__ out, int64_t m,
    int topk, int64_t k, const int32_t* __restrict__ ids, int num_experts,
    const float* __restrict__ weights) {
  const int64_t vec_per_row = k / 8;
  const int64_t total = m * vec_per_row;
  for (int64_t v = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
       v < total; v += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = v / vec_per_row;
    const int64_t c = (v - t * vec_per_row) * 8;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const uint16_t* src = in + t * topk * k + c;
    for (int j = 0; j < topk; ++j) {
      if (ids) {
        const int e = ids[t * topk + j];
        if (e < 0 || e >= num_experts) continue;
      }
      const u32x4 x = *reinterpret_cast<const u32x4*>(src + j * k);
      if (weights) {
        const float w = weights[t * topk + j];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] = __fadd_rn(acc[2 * q], __fmul_rn(w, __uint_as_float(x[q] << 16)));
          acc[2 * q + 1] =
              __fadd_rn(acc[2 * q + 1], __fmul_rn(w, __uint_as_float(x[q] & 0xffff0000u)));
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] += __uint_as_float(x[q] << 16);
          acc[2 * q + 1] += __uint_as_float(x[q] & 0xffff0000u);
        }
      }
    }
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
    *reinterpret_cast<u32x4*>(out + t * k + c) = o;
  }
}

// moe_sum_kernel for a compile-time top-k: a thread issues its TK row loads
// before any of the dropped-slot checks (a runtime loop with a `continue`
// keeps each load behind the previous slot's check: TK round trips in
// series), then sums in slot order with the same roundings. Every slot has a
// row in `in`, so the loads stay in bounds whatever the ids say.
template <int TK>
__global__ __launch_bounds__(256) void moe_sum_tk_kernel(
    const uint16_t* __restrict__ in, uint16_t* __restrict__ out, int64_t m,
    int64_t k, const int32_t* __restrict__ ids, int num_experts,
    const float* __restrict__ weights) {
  const int64_t vec_per_row = k / 8;
  const int64_t total = m * vec_per_row;
  for (int64_t v = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
       v < total; v += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = v / vec_per_row;
    const int64_t c = (v - t * vec_per_row) * 8;
    const uint16_t* src = in + t * TK * k + c;
    u32x4 x[TK];
#pragma unroll
    for (int j = 0; j < TK; ++j) x[j] = *reinterpret_cast<const u32x4*>(src + j * k);
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < TK; ++j) {
      if (ids) {
        const int e = ids[t * TK + j];
        if (e < 0 || e >= num_experts) continue;
      }
      if (weights) {
        const float w = weights[t * TK + j];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] = __fadd_rn(acc[2 * q], __fmul_rn(w, __uint_as_float(x[j][q] << 16)));
          acc[2 * q + 1] =
              __fadd_rn(acc[2 * q + 1], __fmul_rn(w, __uint_as_float(x[j][q] & 0xffff0000u)));
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] += __uint_as_float(x[j][q] << 16);
          acc[2 * q + 1] += __uint_as_float(x[j][q] & 0xffff0000u);
        }
      }
    }
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
    *reinterpret_cast<u32x4*>(out + t * k + c) = o;
  }
}

// moe_sum over fp32 split-K partials: 4 columns per thread.
__global__ __launch_bounds__(256) void moe_sum_partials_kernel(
    const float* __restrict__ part, int nsplit, uint16_t* __restrict__ out,
    int64_t m, int topk, int64_t k, const int32_t* __restrict__ ids,
    int num_experts, const float* __restrict__ weights) {
  const int64_t vec_per_row = k / 4;
  const int64_t total = m * vec_per_row;
  const int64_t split_stride = m * topk * k;
  for (int64_t v = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
       v < total; v += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = v / vec_per_row;
    const int64_t c = (v - t * vec_per_row) * 4;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < topk; ++j) {
      const int64_t slot = t * topk + j;
      const int e = ids[slot];
      if (e < 0 || e >= num_experts) continue;
      f32x4 y = *reinterpret_cast<const f32x4*>(part + slot * k + c);
      for (int s = 1; s < nsplit; ++s)
        y += *reinterpret_cast<const f32x4*>(part + s * split_stride + slot * k + c);
      const float w = weights ? weights[slot] : 1.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float yb = bf16_bits_to_f32(f32_to_bf16_bits(y[q]));
        acc[q] = weights ? __fadd_rn(acc[q], __fmul_rn(w, yb)) : acc[q] + yb;
      }
    }
    uint2 o;
    o.x = pack_bf16x2(acc[0], acc[1]);
    o.y = pack_bf16x2(acc[2], acc[3]);
    *reinterpret_cast<uint2*>(out + t * k + c) = o;
  }
}

// ------------------------------------------------------ fp8 group quant ---
// Each lane quantises 8 consecutive columns; the group/8 lanes of a group
// (a power of two <= 64, aligned within the wave) reduce its amax with
// butterfly shuffles, so a wave covers 512 columns. A workgroup takes
// 2048 columns of one row (grid: rows x column chunks), so the row and its
// skip test are uniform and no index is divided.
// scale = max(amax, 1e-10) / 448; q = e4m3fn(clamp(x / scale, +-448)).
// With `rows_dev` given, rows >= *rows_dev are skipped (padded-row buffers
// whose live prefix is only known on the device); with `sorted_ids` given,
// so are the pad rows (sorted_ids[r] >= numel), which no GEMM reads.
constexpr int kQuantChunkCols = 256 * 8;  // columns per workgroup
__global__ __launch_bounds__(256) void quant_fp8_group_kernel(
    const uint16_t* __restrict__ x, uint8_t* __restrict__ q,
    float* __restrict__ scales, int64_t rows, int64_t cols, int group,
    const int32_t* __restrict__ rows_dev, const int32_t* __restrict__ sorted_ids,
    int64_t numel, int64_t scale_kstride) {
  const int lane = threadIdx.x & 63;
  const int lanes_per_group = group / 8;
  const int64_t r = blockIdx.x;
  const int64_t live_rows = rows_dev ? min(rows, static_cast<int64_t>(*rows_dev)) : rows;
  if (r >= live_rows) return;
  if (sorted_ids && sorted_ids[r] >= numel) return;
  const int64_t c = (static_cast<int64_t>(blockIdx.y) * kQuantChunkCols) + threadIdx.x * 8;
  // a group lies wholly inside or outside the row (cols % group == 0)
  const bool active = c < cols;
  float f[8];
  float amax = 0.f;
  if (active) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(x + r * cols + c);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[2 * j] = __uint_as_float(w[j] << 16);
      f[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(f[j]));
  }
  for (int d = lanes_per_group / 2; d >= 1; d >>= 1)
    amax = fmaxf(amax, __shfl_xor(amax, d, 64));
  if (!active) return;
  const float scale = fmaxf(amax, 1e-10f) / 448.0f;
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float a = fminf(fmaxf(f[2 * j] / scale, -448.f), 448.f);
    const float b = fminf(fmaxf(f[2 * j + 1] / scale, -448.f), 448.f);
    const uint32_t pk = cvt_pk_fp8(a, b);
    if (j < 2)
      lo |= pk << (16 * j);
    else
      hi |= pk << (16 * (j - 2));
  }
  uint2 o;
  o.x = lo;
  o.y = hi;
  *reinterpret_cast<uint2*>(q + r * cols + c) = o;
  if ((lane & (lanes_per_group - 1)) == 0) {
    const int gshift = __builtin_ctz(group);  // group is a power of two
    const int64_t g = c >> gshift;
    if (scale_kstride > 0) scales[g * scale_kstride + r] = scale;
    else scales[r * (cols >> gshift) + g] = scale;
  }
}

// Activation scales of the padded row order, k-block-major:
// out[kb * stride + r] = xs[sorted_ids[r] / topk][kb] for the rows below
// num_tokens_post_padded; a pad row takes the block's first row's scales
// (any finite value does: pad rows' outputs are never stored). One thread
// per (padded row, k block): blockIdx.y is the k block, so each k block's
// writes are contiguous.
__global__ __launch_bounds__(256) void moe_scale_gather_kernel(
    const float* __restrict__ xs, int kblocks, const int32_t* __restrict__ sorted_ids,
    const int32_t* __restrict__ num_post_pad, int64_t numel, int topk, int block,
    float* __restrict__ out, int64_t stride) {
  const int64_t r = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (r >= num_post_pad[0]) return;
  const int kb = blockIdx.y;
  int sid = sorted_ids[r];
  if (sid >= numel) sid = sorted_ids[r - r % block];
  out[kb * stride + r] = xs[static_cast<int64_t>(sid / topk) * kblocks + kb];
}

// ----------------------------------------------------- int8 token quant ---
constexpr int64_t kInt8WaveRows = 1024;  // rows from which a wave takes a row
// One wave per row (4 rows per workgroup), the row held in registers: NV
// vectors of 8 columns per lane (cols <= 512 * NV, cols % 8 == 0), one read
// of x. With `rows_dev` given, rows >= *rows_dev are skipped; with
// `sorted_ids` given, so are the pad rows (sorted_ids[r] >= numel).
// scale = max(amax, 1e-10) / 127; q = clamp(rne(x / scale), -127, 127).
template <int NV>
__global__ __launch_bounds__(256) void quant_int8_token_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q,
    float* __restrict__ scales, int64_t rows, int64_t cols,
    const int32_t* __restrict__ rows_dev, const int32_t* __restrict__ sorted_ids,
    int64_t numel) {
  const int lane = threadIdx.x & 63;
  const int64_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows || (rows_dev && r >= *rows_dev)) return;
  if (sorted_ids && sorted_ids[r] >= numel) return;
  const uint16_t* src = x + r * cols;
  int8_t* dst = q + r * cols;
  u32x4 w[NV];
  float amax = 0.f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int64_t c = (static_cast<int64_t>(v) * 64 + lane) * 8;
    if (c < cols) {
      w[v] = *reinterpret_cast<const u32x4*>(src + c);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        amax = fmaxf(amax, fabsf(__uint_as_float(w[v][j] << 16)));
        amax = fmaxf(amax, fabsf(__uint_as_float(w[v][j] & 0xffff0000u)));
      }
    }
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) amax = fmaxf(amax, __shfl_xor(amax, d, 64));
  const float scale = fmaxf(amax, 1e-10f) / 127.0f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int64_t c = (static_cast<int64_t>(v) * 64 + lane) * 8;
    if (c >= cols) continue;
    uint32_t packed[2] = {0, 0};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float f = (j & 1) ? __uint_as_float(w[v][j / 2] & 0xffff0000u)
                              : __uint_as_float(w[v][j / 2] << 16);
      float rq = __builtin_rintf(f / scale);
      rq = fminf(fmaxf(rq, -127.f), 127.f);
      const uint32_t b = static_cast<uint32_t>(static_cast<int32_t>(rq)) & 0xffu;
      packed[j / 4] |= b << (8 * (j & 3));
    }
    uint2 o;
    o.x = packed[0];
    o.y = packed[1];
    *reinterpret_cast<uint2*>(dst + c) = o;
  }
  if (lane == 0) scales[r] = scale;
}

// ------------------------------------------------------------- launchers ---
static unsigned grid_for(int64_t work_items, int threads) {
  int64_t g = (work_items + threads - 1) / threads;
  const int64_t cap = 256 * 64;  // enough waves to fill 256 CUs many times
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return static_cast<unsigned>(g);
}

int launch_silu_and_mul(const void* in, void* out, int64_t rows, int64_t n,
                        hipStream_t stream) {
  if (rows == 0) return FGS_OK;
  hipLaunchKernelGGL(silu_and_mul_kernel, dim3(grid_for(rows * (n / 8), 256)),
                     dim3(256), 0, stream, static_cast<const uint16_t*>(in),
                     static_cast<uint16_t*>(out), rows, n);
  return check_launch("silu_and_mul_kernel");
}

int launch_moe_sum_routed(const void* in, void* out, int64_t m, int topk,
                          int64_t k, const int32_t* ids, int num_experts,
                          const float* weights, hipStream_t stream);

int launch_moe_sum(const void* in, void* out, int64_t m, int topk, int64_t k,
                   hipStream_t stream) {
  return launch_moe_sum_routed(in, out, m, topk, k, nullptr, 0, nullptr, stream);
}

int launch_moe_sum_routed(const void* in, void* out, int64_t m, int topk,
                          int64_t k, const int32_t* ids, int num_experts,
                          const float* weights, hipStream_t stream) {
  if (m == 0) return FGS_OK;
  const dim3 grid(grid_for(m * (k / 8), 256));
  const uint16_t* src = static_cast<const uint16_t*>(in);
  uint16_t* dst = static_cast<uint16_t*>(out);
  if (topk == 8) {
    hipLaunchKernelGGL(moe_sum_tk_kernel<8>, grid, dim3(256), 0, stream, src, dst, m, k, ids,
                       num_experts, weights);
    return check_launch("moe_sum_tk_kernel");
  }
  if (topk == 2) {
    hipLaunchKernelGGL(moe_sum_tk_kernel<2>, grid, dim3(256), 0, stream, src, dst, m, k, ids,
                       num_experts, weights);
    return check_launch("moe_sum_tk_kernel");
  }
  hipLaunchKernelGGL(moe_sum_kernel, dim3(grid_for(m * (k / 8), 256)),
                     dim3(256), 0, stream, static_cast<const uint16_t*>(in),
                     static_cast<uint16_t*>(out), m, topk, k, ids, num_experts,
                     weights);
  return check_launch("moe_sum_kernel");
}

int launch_moe_sum_partials(const float* part, int nsplit, void* out, int64_t m,
                            int topk, int64_t k, const int32_t* ids,
                            int num_experts, const float* weights,
                            hipStream_t stream) {
  if (m == 0) return FGS_OK;
  hipLaunchKernelGGL(moe_sum_partials_kernel, dim3(grid_for(m * (k / 4), 256)),
                     dim3(256), 0, stream, part, nsplit,
                     static_cast<uint16_t*>(out), m, topk, k, ids, num_experts,
                     weights);
  return check_launch("moe_sum_partials_kernel");
}

// Few rows (under kInt8WaveRows): a workgroup of 256 threads per row, two
// passes over the row (amax, then quantise), for parallelism at small M.
__global__ __launch_bounds__(256) void quant_int8_token_wg_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q,
    float* __restrict__ scales, int64_t cols, const int32_t* __restrict__ rows_dev,
    const int32_t* __restrict__ sorted_ids, int64_t numel) {
  const int64_t r = blockIdx.x;
  if (rows_dev && r >= *rows_dev) return;
  if (sorted_ids && sorted_ids[r] >= numel) return;
  const uint16_t* src = x + r * cols;
  int8_t* dst = q + r * cols;
  float amax = 0.f;
  for (int64_t c = threadIdx.x * 8; c < cols; c += 256 * 8) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(src + c);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      amax = fmaxf(amax, fabsf(__uint_as_float(w[j] << 16)));
      amax = fmaxf(amax, fabsf(__uint_as_float(w[j] & 0xffff0000u)));
    }
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) amax = fmaxf(amax, __shfl_xor(amax, d, 64));
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float scale = fmaxf(amax, 1e-10f) / 127.0f;
  for (int64_t c = threadIdx.x * 8; c < cols; c += 256 * 8) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(src + c);
    uint32_t packed[2] = {0, 0};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float f = (j & 1) ? __uint_as_float(w[j / 2] & 0xffff0000u)
                              : __uint_as_float(w[j / 2] << 16);
      float rq = __builtin_rintf(f / scale);
      rq = fminf(fmaxf(rq, -127.f), 127.f);
      const uint32_t b = static_cast<uint32_t>(static_cast<int32_t>(rq)) & 0xffu;
      packed[j / 4] |= b << (8 * (j & 3));
    }
    uint2 o;
    o.x = packed[0];
    o.y = packed[1];
    *reinterpret_cast<uint2*>(dst + c) = o;
  }
  if (threadIdx.x == 0) scales[r] = scale;
}

// Calls f(std::integral_constant<int, n>) for a runtime n in [0, N].
template <int N, class F>
static void dispatch_nv(int n, F&& f) {
  if constexpr (N >= 0) {
    if (n == N) {
      f(std::integral_constant<int, N>{});
      return;
    }
    dispatch_nv<N - 1>(n, f);
  }
}

int launch_quant_fp8_group(const void* x, void* q, float* scales,
                           int64_t rows, int64_t cols, int group,
                           hipStream_t stream, const int32_t* rows_dev,
                           const int32_t* sorted_ids, int64_t numel,
                           int64_t scale_kstride) {
  if (rows == 0 || cols == 0) return FGS_OK;
  const int64_t chunks = (cols + kQuantChunkCols - 1) / kQuantChunkCols;
  if (rows > 0x7fffffff || chunks > 0xffff)
    return fail(FGS_EUNSUPPORTED, "fp8 group quantiser: too many rows or columns for its grid");
  hipLaunchKernelGGL(quant_fp8_group_kernel,
                     dim3(static_cast<unsigned>(rows), static_cast<unsigned>(chunks)),
                     dim3(256), 0, stream, static_cast<const uint16_t*>(x),
                     static_cast<uint8_t*>(q), scales, rows, cols, group, rows_dev,
                     sorted_ids, numel, scale_kstride);
  return check_launch("quant_fp8_group_kernel");
}

int launch_scale_gather(const float* xs, int kblocks, const int32_t* sorted_ids,
                        const int32_t* num_post_pad, int64_t numel, int topk, int block,
                        int64_t max_padded, float* out, hipStream_t stream) {
  if (max_padded <= 0 || kblocks <= 0) return FGS_OK;
  hipLaunchKernelGGL(moe_scale_gather_kernel,
                     dim3(static_cast<unsigned>((max_padded + 255) / 256),
                          static_cast<unsigned>(kblocks)),
                     dim3(256), 0, stream,
                     xs, kblocks, sorted_ids, num_post_pad, numel, topk, block, out, max_padded);
  return check_launch("moe_scale_gather_kernel");
}

int launch_quant_int8_token(const void* x, int8_t* q, float* scales,
                            int64_t rows, int64_t cols, hipStream_t stream,
                            const int32_t* rows_dev, const int32_t* sorted_ids,
                            int64_t numel) {
  if (rows == 0) return FGS_OK;
  const uint16_t* xs = static_cast<const uint16_t*>(x);
  // rows too wide for a wave's registers take the workgroup-per-row kernel
  if (rows < kInt8WaveRows || cols > 512 * kInt8QuantMaxVec) {
    hipLaunchKernelGGL(quant_int8_token_wg_kernel, dim3(static_cast<unsigned>(rows)),
                       dim3(256), 0, stream, xs, q, scales, cols, rows_dev, sorted_ids,
                       numel);
    return check_launch("quant_int8_token_wg_kernel");
  }
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  const int nv = static_cast<int>((cols + 511) / 512);
  bool launched = false;
  dispatch_nv<kInt8QuantMaxVec>(nv, [&](auto nv_c) {
    constexpr int NV = decltype(nv_c)::value;
    if constexpr (NV >= 1) {
      hipLaunchKernelGGL(quant_int8_token_kernel<NV>, grid, dim3(256), 0, stream, xs, q,
                         scales, rows, cols, rows_dev, sorted_ids, numel);
      launched = true;
    }
  });
  if (!launched) return fail(FGS_EINVAL, "int8 token quantiser: bad column count");
  return check_launch("quant_int8_token_kernel");
}

}  // namespace fgs
