// Device helpers shared by the LDS-tiled grouped GEMM kernels
// (gemm_tiled.hip, gemm_wide.hip): wait counters, LDS-DMA, the
// compile-time dispatch of a runtime count and the per-element-type MFMA.
#pragma once

#include <type_traits>

#include "fgs_moe_kernels.h"

namespace fgs {

// Division by topk as a multiply and two shifts (Granlund and Montgomery,
// "Division by Invariant Integers using Multiplication", PLDI 1994, unsigned
// case, exact for every 32-bit numerator): l = ceil(log2 d), magic =
// floor(2^32 (2^l - d) / d) + 1, q = (t + ((n - t) >> min(l, 1))) >>
// max(l - 1, 0) with t = the high word of magic * n. The launch sets the
// magic; the kernels divide token slots by topk with it.
inline void set_topk_magic(GemmParams* q) {
  const uint32_t d = static_cast<uint32_t>(q->topk > 1 ? q->topk : 1);
  int l = 0;
  while ((uint64_t{1} << l) < d) ++l;
  q->topk_magic = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << l) - d)) / d + 1);
  q->topk_sh1 = l < 1 ? l : 1;
  q->topk_sh2 = l > 1 ? l - 1 : 0;
}
__device__ __forceinline__ int div_topk(const GemmParams& p, int n) {
  const uint32_t t = __umulhi(p.topk_magic, static_cast<uint32_t>(n));
  return static_cast<int>((t + ((static_cast<uint32_t>(n) - t) >> p.topk_sh1)) >> p.topk_sh2);
}

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// One wave-wide LDS-DMA load: lane l copies 16 bytes from `src` (its own
// global address) to byte 16*l of the 1 KiB block at `lds_dst` (uniform).
__device__ __forceinline__ void lds_dma16(const void* src, void* lds_dst) {
  __builtin_amdgcn_global_load_lds(
      src, (__attribute__((address_space(3))) void*)(lds_dst), 16, 0, 0);
}

__device__ __forceinline__ void wave_barrier_all() { __builtin_amdgcn_s_barrier(); }

// s_waitcnt lgkmcnt(0): this wave's LDS reads have completed.
__device__ __forceinline__ void wait_lgkm0() {
  __builtin_amdgcn_s_waitcnt((63 & 15) | (7 << 4) | (0 << 8) | ((63 >> 4) << 14));
}

// Calls f(std::integral_constant<int, n>) for a runtime n in [0, N].
template <int N, class F>
__device__ __forceinline__ void dispatch_count(int n, F&& f) {
  if constexpr (N >= 0) {
    if (n == N) {
      f(std::integral_constant<int, N>{});
      return;
    }
    dispatch_count<N - 1>(n, f);
  }
}

// Element types of the tiled kernels. A 32x32 MFMA k step reads 16 bytes
// per lane of each operand (bf16: 8 elements, int8: 16) -- one LDS chunk --
// except fp8, whose 32x32x64 MFMA reads 32 bytes per lane (two chunks).
template <int DT>
struct TiledType;
template <>
struct TiledType<kDtBf16> {
  static constexpr int ESZ = 2, FC = 1;
  using Frag = bf16x8;
  using Acc = f32x16;
  static __device__ __forceinline__ Acc mma(Frag w, Frag x, Acc c) {
    return mfma32_bf16(w, x, c);
  }
};
template <>
struct TiledType<kDtInt8> {
  static constexpr int ESZ = 1, FC = 1;
  using Frag = i32x4;
  using Acc = i32x16;
  // v_mfma_i32_32x32x32_i8: same lane layout as the bf16 32x32x16 form
  // with 16 int8 of k per lane.
  static __device__ __forceinline__ Acc mma(Frag w, Frag x, Acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(w, x, c, 0, 0, 0);
  }
};
template <>
struct TiledType<kDtFp8> {
  static constexpr int ESZ = 1, FC = 2;
  using Frag = i32x8;
  using Acc = f32x16;
  // v_mfma_scale_f32_32x32x64_f8f6f4, both operands OCP e4m3 (format 0),
  // unit e8m0 block scales (127): 32 fp8 of k per lane.
  static __device__ __forceinline__ Acc mma(Frag w, Frag x, Acc c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, x, c, 0, 0, 0, 127,
                                                           0, 127);
  }
};

}  // namespace fgs
