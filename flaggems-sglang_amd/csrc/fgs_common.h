// Shared definitions of the gfx950 fused-MoE kernels: vector types, MFMA
// wrappers, bf16 / fp8 conversions and the host-side error plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "fgs_moe.h"

namespace fgs {

// ---------------------------------------------------------------- types ----
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) int i32x4;
typedef __attribute__((ext_vector_type(8))) int i32x8;
typedef __attribute__((ext_vector_type(16))) int i32x16;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;

constexpr int kWave = 64;

// bf16 is carried as its 16-bit pattern in memory; conversions are explicit.
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even f32 -> bf16 bit pattern (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two f32 -> one word of two bf16 (round to nearest even, lo in the low
// half): one v_cvt_pk_bf16_f32 (converting the halves separately costs a
// conversion each plus a shift and an or).
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) { return cvt_pk_bf16(lo, hi); }

// The expert whose range of a routing tuple's gathered order holds position
// j: expert e owns [raw[e], raw[e] + h[e]) with raw the running sums of the
// histogram (token_offs_raw, the ranges matmul_ogs reads; counts clamped as
// the routing-order kernel clamps them: negative -> 0, sums capped at
// numel); -1 past the total. A wave-wide computation (64 experts per step,
// DPP-free shuffles); every lane of the wave returns the same value.
__device__ __forceinline__ int routed_expert_of(const int32_t* __restrict__ hist,
                                                int num_experts, int64_t numel, int64_t j) {
  const int lane = threadIdx.x & 63;
  int64_t base = 0;
  for (int e0 = 0; e0 < num_experts; e0 += 64) {
    const int e = e0 + lane;
    const int64_t h = e < num_experts ? static_cast<int64_t>(max(hist[e], 0)) : 0;
    int64_t s = h < numel ? h : numel;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int64_t o = __shfl_up(s, d, 64);
      if (lane >= d) s += o;
    }
    const int64_t incl = base + s < numel ? base + s : numel;
    const uint64_t hit = __ballot(incl > j);
    if (hit) return e0 + __ffsll(static_cast<long long>(hit)) - 1;
    const int64_t tot = __shfl(s, 63, 64);
    base = base + tot < numel ? base + tot : numel;
  }
  return -1;
}

// silu(g) * u in fp32, the activation of the reference's
// _silu_and_mul_kernel (ops/fused_moe.py:58-62): g / (1 + exp(-g)) * u,
// with the division done as a hardware reciprocal (1 ulp).
__device__ __forceinline__ float silu_mul(float g, float u) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

// GEMM1 activations.
enum { kActSilu = 0, kActGelu = 1, kActSwiglu = 2 };

// gelu(g) * u with the exact (erf) gelu: the activation sgl_kernel's
// gelu_and_mul applies (ops/fused_moe.py:219-220).
__device__ __forceinline__ float gelu_mul(float g, float u) {
  return 0.5f * g * (1.0f + erff(g * 0.70710678118654752f)) * u;
}

// GEMM1 epilogue.
// silu / gelu keep the rounding points of the reference's unfused path:
// matmul_ogs writes its output (gate and up halves, gammas applied when the
// router weight goes on the input, ops/fused_moe.py:202-212) in bf16, then
// the activation kernel computes in fp32 from those bf16 values and stores
// bf16 (:58-63, :219-220).
// swiglu is the activation fused into matmul_ogs by the bias variant
// (:274-314): gate g and linear u stay fp32 (biases already added);
// with limit > 0, g = min(g, limit) and u = clamp(u, -limit, limit); out =
// bf16(g * sigmoid(alpha * g) * (u + 1)), times the router weight when it
// goes on the input (matmul_ogs scales its epilogue's output -- the fused
// activation's result -- by the gammas).
__device__ __forceinline__ uint16_t gemm1_epilogue(float g, float u, bool scale,
                                                   float gamma, int act = kActSilu,
                                                   float alpha = 1.f, float limit = 0.f) {
  if (act == kActSwiglu) {
    if (limit > 0.f) {
      g = fminf(g, limit);
      u = fminf(fmaxf(u, -limit), limit);
    }
    const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-alpha * g));
    const float o = g * sg * (u + 1.0f);
    return f32_to_bf16_bits(scale ? o * gamma : o);
  }
  if (scale) {
    g *= gamma;
    u *= gamma;
  }
  g = bf16_bits_to_f32(f32_to_bf16_bits(g));
  u = bf16_bits_to_f32(f32_to_bf16_bits(u));
  return f32_to_bf16_bits(act == kActGelu ? gelu_mul(g, u) : silu_mul(g, u));
}


// gemm1_epilogue's silu path for two adjacent outputs, word-packed: the same
// roundings (g and u to bf16, silu(g) * u in fp32, bf16 out) with the
// conversions done pairwise.
template <bool SCALE>
__device__ __forceinline__ uint32_t silu_mul_bf16x2(float g0, float g1, float u0, float u1,
                                                    float gamma) {
  if (SCALE) {
    g0 *= gamma;
    g1 *= gamma;
    u0 *= gamma;
    u1 *= gamma;
  }
  const uint32_t gp = cvt_pk_bf16(g0, g1);
  const uint32_t up = cvt_pk_bf16(u0, u1);
  const float o0 = silu_mul(__builtin_bit_cast(float, gp << 16),
                            __builtin_bit_cast(float, up << 16));
  const float o1 = silu_mul(__builtin_bit_cast(float, gp & 0xffff0000u),
                            __builtin_bit_cast(float, up & 0xffff0000u));
  return cvt_pk_bf16(o0, o1);
}

// ------------------------------------------------------------------ MFMA ---
// v_mfma_f32_16x16x32_bf16: A 16x32, B 32x16, C 16x16 fp32.
// Lane l holds A row (l & 15) / B column (l & 15), eight consecutive
// k values of lane group (l >> 4); C: column (l & 15), rows 4*(l>>4)+i.
__device__ __forceinline__ f32x4 mfma16_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_32x32x16_bf16: A 32x16, B 16x32, C 32x32 fp32 in 16 regs.
// Lane l holds A row (l & 31), k values 8*(l>>5)..+7; C column (l & 31),
// rows 8*(i>>2) + 4*(l>>5) + (i&3) for register i.
__device__ __forceinline__ f32x16 mfma32_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_16x16x128_f8f6f4 with both operands OCP e4m3 (format 0) and
// unit (e8m0 = 127) block scales: A 16x128, B 128x16, 32 bytes per lane.
__device__ __forceinline__ f32x4 mfma16_fp8(i32x8 a, i32x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0,
                                                          127, 0, 127);
}

// v_mfma_i32_16x16x64_i8: A 16x64, B 64x16 int8, 16 bytes per lane.
__device__ __forceinline__ i32x4 mfma16_i8(i32x4 a, i32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------ fp8 e4m3fn ---
// Two floats -> two OCP e4m3fn bytes (hardware RNE conversion on gfx950),
// placed in the low 16 bits of the result.
__device__ __forceinline__ uint32_t cvt_pk_fp8(float a, float b) {
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false)) &
         0xffffu;
}

// --------------------------------------------------------- host helpers ---
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);
// A schedule tuning aid from the environment: getenv(name) when the
// process runs with FGS_MOE_TUNING=1 (read once), else null -- the
// schedule's compiled-in choices are what every other process runs,
// whatever else its environment holds.
const char* tuning_env(const char* name);

}  // namespace fgs
