// Streaming grouped GEMMs of the fused-MoE path (decode regime: few rows per
// expert, the layer is bound by reading every touched expert's weights once).
//
// A workgroup owns one row block (16*MT rows of the expert-sorted, padded
// order from moe_align_block_size) and one 16-column output tile (grid x:
// the column tiles, y: the row blocks). Its KW
// waves split the contraction; each wave streams its share of the 16 (or,
// for GEMM1, 16 gate + 16 up) weight rows straight from HBM into MFMA
// operand registers, with no LDS staging. Every weight load instruction
// reads 8 rows x 128 contiguous bytes (whole lines; a 16-rows x 64-byte
// pattern streams ~20 % slower), and two DPP moves per dword between the
// halves of each 16-lane row put row n's bytes into the lanes of MFMA row
// n (lines_to_frag). Partial sums meet in LDS; wave 0 runs the epilogue:
//   GEMM1 (replaces matmul_ogs with gather + _silu_and_mul_triton,
//          ops/fused_moe.py:205-218): a2[row, c] = bf16(silu(g) * u)
//   GEMM2 (replaces matmul_ogs with scatter + gammas, :224-231):
//          y[slot, c] = bf16(acc); the gamma-weighted top-k sum is moe_sum's
//
// Direct rows (one token, DIRECT): the token's top-k slots go to distinct
// experts, so no alignment is needed -- row tile j is slot j alone, its
// expert topk_ids[j], and the activations are compact [slots, k] rows.
// moe_gemm2_direct_kernel also folds the gamma-weighted top-k sum into
// GEMM2: a workgroup owns 16 output columns for every slot.
#include "fgs_moe_kernels.h"

namespace fgs {

template <int DT>
struct StreamTraits;

// bf16: 16x16x32 MFMA, 16 B per lane per MFMA, 4 MFMAs per 128-k step.
template <>
struct StreamTraits<kDtBf16> {
  static constexpr int kLaneBytes = 64;           // bytes per lane per step
  static constexpr int kStepK = 128;              // k elements per step
  static constexpr int kVecs = kLaneBytes / 16;   // u32x4 per lane per step
  typedef f32x4 Acc;
};
// fp8 e4m3: 16x16x128 MFMA, 32 B per lane, one MFMA per 128-k scale group.
template <>
struct StreamTraits<kDtFp8> {
  static constexpr int kLaneBytes = 32;
  static constexpr int kStepK = 128;
  static constexpr int kVecs = 2;
  typedef f32x4 Acc;
};
// int8: 16x16x64 MFMA, 16 B per lane per MFMA, 4 MFMAs per 256-k step.
template <>
struct StreamTraits<kDtInt8> {
  static constexpr int kLaneBytes = 64;
  static constexpr int kStepK = 256;
  static constexpr int kVecs = 4;
  typedef i32x4 Acc;
};

// Weight rows arrive as whole 128-byte lines. For each 128-byte group q of
// a step, f[2q] is loaded from row (lane & 7) of the 16-row tile and
// f[2q + 1] from row 8 + (lane & 7), both at byte (lane >> 3) * 16 of the
// group: one load instruction covers 8 rows x 128 contiguous bytes. `p` is
// this lane's row (lane & 7) at its byte of the step, `row8` the byte
// distance of 8 rows.
template <int DT, int NV>
__device__ __forceinline__ void load_lines(u32x4 (&f)[NV], const uint8_t* p, int64_t row8) {
#pragma unroll
  for (int q = 0; q < NV / 2; ++q) {
    f[2 * q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + q * 128));
    f[2 * q + 1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + row8 + q * 128));
  }
}

// Lines -> MFMA fragments. In each 16-lane row, lane n < 8 holds row n's
// 16-byte chunk 2g of the group (g = lane >> 4) in f[2q] and row n + 8's
// chunk 2g in f[2q + 1]; lane n >= 8 holds row n - 8's chunk 2g + 1 and
// row n's chunk 2g + 1. row_ror:8 pairs lane n with n +- 8, and the bank
// masks write only the half that receives: lanes 8-15 take f[2q + 1] of
// lane n - 8 into f[2q], lanes 0-7 take f[2q] of lane n + 8 into f[2q + 1].
// Then lane (n, g) holds row n's bytes 32g .. 32g + 31 of the group in
// f[2q], f[2q + 1]: the MFMA k index of a lane is the same in every row, so
// activations read with that mapping (read_act_vec) make the contraction
// exact.
template <int NV>
__device__ __forceinline__ void lines_to_frag(u32x4 (&f)[NV]) {
#pragma unroll
  for (int q = 0; q < NV / 2; ++q)
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int a = static_cast<int>(f[2 * q][d]), b = static_cast<int>(f[2 * q + 1][d]);
      f[2 * q][d] = static_cast<unsigned>(__builtin_amdgcn_update_dpp(a, b, 0x128, 0xF, 0xC, false));
      f[2 * q + 1][d] = static_cast<unsigned>(__builtin_amdgcn_update_dpp(b, a, 0x128, 0xF, 0x3, false));
    }
}

// Byte of an operand vector v within a step for lane group g: group v / 2,
// chunk 2g + v % 2 (the weight fragments' k mapping).
__device__ __forceinline__ int frag_byte(int v, int g) { return (v >> 1) * 128 + g * 32 + (v & 1) * 16; }

// Activation fragments (p: the row at this lane's step; lane group g).
template <int NV>
__device__ __forceinline__ void load_act(u32x4 (&f)[NV], const uint8_t* p, int g,
                                         bool valid) {
  if (valid) {
#pragma unroll
    for (int v = 0; v < NV; ++v) f[v] = *reinterpret_cast<const u32x4*>(p + frag_byte(v, g));
  } else {
#pragma unroll
    for (int v = 0; v < NV; ++v) f[v] = u32x4{0, 0, 0, 0};
  }
}

template <int DT, int NV>
__device__ __forceinline__ void mma_step(f32x4& acc, const u32x4 (&a)[NV],
                                         const u32x4 (&b)[NV]) {
  if constexpr (DT == kDtBf16) {
#pragma unroll
    for (int v = 0; v < NV; ++v)
      acc = mfma16_bf16(__builtin_bit_cast(bf16x8, a[v]),
                        __builtin_bit_cast(bf16x8, b[v]), acc);
  }
}

template <int DT, int NV>
__device__ __forceinline__ void mma_step_i8(i32x4& acc, const u32x4 (&a)[NV],
                                            const u32x4 (&b)[NV]) {
#pragma unroll
  for (int v = 0; v < NV; ++v)
    acc = mfma16_i8(__builtin_bit_cast(i32x4, a[v]),
                    __builtin_bit_cast(i32x4, b[v]), acc);
}

__device__ __forceinline__ f32x4 mma_fp8(const u32x4 (&a)[2],
                                         const u32x4 (&b)[2]) {
  i32x8 av, bv;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    av[j] = static_cast<int>(a[0][j]);
    av[4 + j] = static_cast<int>(a[1][j]);
    bv[j] = static_cast<int>(b[0][j]);
    bv[4 + j] = static_cast<int>(b[1][j]);
  }
  return mfma16_fp8(av, bv, f32x4{0.f, 0.f, 0.f, 0.f});
}

// ---- on-the-fly activation quantisation (direct rows, fp8 / int8) ----
// With p.a_src set, a direct-row fp8 kernel reads its activation row in bf16
// and quantises it itself, with the arithmetic of quant_fp8_group_kernel
// (per 128-column group, scale = max(amax, 1e-10) / 448, q =
// e4m3fn(clamp(x / scale, +-448))), so the bytes and scales match that
// kernel's output exactly and the quantiser launches drop out of the
// single-token path; int8 likewise with quant_int8_token_kernel's
// per-token arithmetic (below).
//
// Every lane quantises 2 consecutive values of the step (one 128-column
// group) and the bytes go through the wave's LDS slot to lanes (0, lg),
// whose MFMA row 0 fragments hold the step's bytes 32*lg .. 32*lg + 31.
__device__ __forceinline__ uint32_t load_raw(const uint16_t* row, int64_t k0, int lane) {
  return *reinterpret_cast<const uint32_t*>(row + k0 + lane * 2);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ float quant1_fp8(float f, float scale) {
  return fminf(fmaxf(f / scale, -448.f), 448.f);
}
// One DPP lane move within each row of 16 lanes (CTRL: a quad permutation
// or a row mirror; every source lane exists, so no lane keeps `old`).
template <int CTRL>
__device__ __forceinline__ float dpp_move(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
// Max over the wave, in every lane: quad xor 1 and xor 2, then the row's
// half mirror (max over 8 lanes) and mirror (over 16), then the four rows'
// lanes 0, 16, 32, 48 -- VALU lane moves and readlanes instead of six LDS
// permute round trips. max is exact in any order, so the result is the
// butterfly's bit for bit.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = fmaxf(v, dpp_move<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = fmaxf(v, dpp_move<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_move<0x140>(v));  // row_mirror
  const int b = __float_as_int(v);
  return fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(b, 0)),
                     __int_as_float(__builtin_amdgcn_readlane(b, 16))),
               fmaxf(__int_as_float(__builtin_amdgcn_readlane(b, 32)),
                     __int_as_float(__builtin_amdgcn_readlane(b, 48))));
}

// fp8 step: the group amax over the wave, scale = max(amax, 1e-10) / 448
// (returned, the same in every lane); qb is the wave's 128-byte LDS slot.
__device__ __forceinline__ float quant_step_fp8(uint32_t raw, uint8_t* qb, int lane,
                                               u32x4 (&f)[2]) {
  const float a = bf16_lo(raw), b = bf16_hi(raw);
  const float amax = wave_max(fmaxf(fabsf(a), fabsf(b)));
  const float scale = fmaxf(amax, 1e-10f) / 448.0f;
  reinterpret_cast<uint16_t*>(qb)[lane] =
      static_cast<uint16_t>(cvt_pk_fp8(quant1_fp8(a, scale), quant1_fp8(b, scale)));
  const int lg = lane >> 4;
  const bool row0 = (lane & 15) == 0;
#pragma unroll
  for (int v = 0; v < 2; ++v)
    f[v] = row0 ? *reinterpret_cast<const u32x4*>(qb + frag_byte(v, lg)) : u32x4{0, 0, 0, 0};
  return scale;
}

// int8 (one token, per-token scale like quant_int8_token_kernel): every
// wave reduces the whole bf16 row's amax itself (16 bytes per lane per
// 1 KiB of row), scale = max(amax, 1e-10) / 127, then per 256-column step
// each lane quantises 4 consecutive values, rint(x / scale) clamped to
// +-127, and the bytes reach the row-0 lanes through the wave's 256-byte
// LDS slot.
__device__ __forceinline__ float row_scale_int8(const uint16_t* row, int64_t cols, int lane) {
  float m = 0.f;
  for (int64_t c = lane * 8; c < cols; c += 512) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(row + c);
#pragma unroll
    for (int j = 0; j < 4; ++j) m = fmaxf(m, fmaxf(fabsf(bf16_lo(w[j])), fabsf(bf16_hi(w[j]))));
  }
  return fmaxf(wave_max(m), 1e-10f) / 127.0f;
}

__device__ __forceinline__ uint32_t quant1_int8(float f, float scale) {
  const float r = fminf(fmaxf(__builtin_rintf(f / scale), -127.f), 127.f);
  return static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xffu;
}

__device__ __forceinline__ void quant_step_int8(uint2 raw, float scale, uint8_t* qb, int lane,
                                                u32x4 (&f)[4]) {
  reinterpret_cast<uint32_t*>(qb)[lane] =
      quant1_int8(bf16_lo(raw.x), scale) | quant1_int8(bf16_hi(raw.x), scale) << 8 |
      quant1_int8(bf16_lo(raw.y), scale) << 16 | quant1_int8(bf16_hi(raw.y), scale) << 24;
  const int lg = lane >> 4;
  const bool row0 = (lane & 15) == 0;
#pragma unroll
  for (int v = 0; v < 4; ++v)
    f[v] = row0 ? *reinterpret_cast<const u32x4*>(qb + frag_byte(v, lg)) : u32x4{0, 0, 0, 0};
}

// This lane's raw bf16 values of a step: 2 (fp8, 128 columns) or 4 (int8,
// 256 columns) consecutive ones.
template <int DT>
struct QaRaw {
  typedef uint32_t type;
  static __device__ __forceinline__ uint32_t load(const uint16_t* row, int64_t k0, int lane) {
    return load_raw(row, k0, lane);
  }
};
template <>
struct QaRaw<kDtInt8> {
  typedef uint2 type;
  static __device__ __forceinline__ uint2 load(const uint16_t* row, int64_t k0, int lane) {
    return *reinterpret_cast<const uint2*>(row + k0 + lane * 4);
  }
};

template <int DT, int MT, int KW, bool GEMM1, bool DIRECT, bool QA>
__global__ __launch_bounds__(KW * 64) void moe_gemm_stream_kernel(
    const GemmParams p) {
  typedef StreamTraits<DT> T;
  typedef typename T::Acc Acc;
  constexpr int NB = GEMM1 ? 2 : 1;  // weight row groups: gate/up or one
  constexpr int NV = T::kVecs;
  constexpr int ESZ = (DT == kDtBf16) ? 2 : 1;
  constexpr int BM = 16 * MT;
  static_assert(!DIRECT || MT == 1, "direct rows: one slot per row tile");

  // column tile fastest: the resident workgroups stream neighbouring tiles
  // of a few experts (measured: Qwen2 int8 M=8 356 -> 216 us, Mixtral M=8
  // -15 %, where row-block-fastest had dozens of experts read at one offset)
  const int rb = blockIdx.y;
  const int n0 = blockIdx.x * 16;
  int e;
  if constexpr (DIRECT) {
    if (rb >= p.numel) return;
    if (GEMM1 && p.route_hist) {
      // routing tuple: row rb is gathered position rb; the first column
      // tile records its expert for GEMM2 and the top-k sum
      e = routed_expert_of(p.route_hist, p.num_experts, p.numel, rb);
      if (blockIdx.x == 0 && threadIdx.x == 0) p.route_ids[rb] = e;
    } else {
      e = p.direct_ids[rb];
    }
    if (e < 0 || e >= p.num_experts) return;  // dropped slot: never read
  } else {
    if (rb * BM >= p.num_post_pad[0]) return;
    e = p.expert_ids[rb];
    if (e < 0) return;
  }
  // slot of row r of the tile (p.numel: a pad row)
  auto row_sid = [&](int r) -> int {
    if constexpr (DIRECT) return r == rb * BM ? rb : static_cast<int>(p.numel);
    else return p.sorted_ids[r];
  };
  // activation / scale row of a valid slot: GEMM1 the token, GEMM2 the
  // padded row (direct: the compact slot row)
  auto src_row = [&](int r, int sid) -> int64_t {
    if constexpr (GEMM1) return sid / p.topk;
    else return DIRECT ? sid : r;
  };

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int ln = lane & 15;
  const int lg = lane >> 4;

  // Activation row of lane ln in each row tile.
  const uint8_t* arow[MT];
  bool avalid[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = rb * BM + mt * 16 + ln;
    const int sid = row_sid(r);
    avalid[mt] = sid < p.numel;
    const int64_t src = avalid[mt] ? src_row(r, sid) : 0;
    arow[mt] = p.a + (src * p.kdim) * ESZ;
  }
  // Weight row (lane & 7) of each row group at this lane's line byte.
  const uint8_t* brow[NB];
  const int64_t wbase = static_cast<int64_t>(e) * p.nrows_w;
  const int64_t row8 = 8 * p.kdim * ESZ;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int64_t n = wbase + (nb ? p.n_out : 0) + n0 + (lane & 7);
    brow[nb] = p.w + (n * p.kdim) * ESZ + (lane >> 3) * 16;
  }

  // QA: the direct row's bf16 source (the token for GEMM1, slot rb's a2 row
  // for GEMM2), quantised step by step below
  static_assert(!QA || (DIRECT && MT == 1 && DT != kDtBf16), "on-the-fly quantisation");
  const uint16_t* qrow = nullptr;
  if constexpr (QA) qrow = p.a_src + src_row(rb * BM, rb) * p.kdim;
  __shared__ __attribute__((aligned(16))) uint8_t qlds[QA ? KW : 1][T::kStepK];

  // fp8 / int8 activation scales of this lane's accumulator rows.
  int64_t crow[MT][4];
  bool cvalid[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rb * BM + mt * 16 + lg * 4 + i;
      const int sid = row_sid(r);
      cvalid[mt][i] = sid < p.numel;
      crow[mt][i] = cvalid[mt][i] ? src_row(r, sid) : 0;
    }

  Acc acc[NB][MT];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[nb][mt] = Acc{0, 0, 0, 0};

  const int steps = static_cast<int>(p.kdim / T::kStepK);
  const int s0 = wave * steps / KW;
  const int s1 = (wave + 1) * steps / KW;
  const int64_t step_bytes = static_cast<int64_t>(T::kStepK) * ESZ;
  const int kblocks = static_cast<int>(p.kdim / 128);

  u32x4 bf[2][NB][NV];
  u32x4 af[2][MT][NV];
  typename QaRaw<DT>::type ar[2];  // QA: this lane's raw bf16 values of the step
  // fp8 block scales of a step (one 128-k group), fetched with its operands
  float sw[2][NB], sa[2][MT][4];
  auto load_scales = [&](int buf, int kb) {
    if constexpr (DT == kDtFp8) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int64_t wrow = (nb ? p.n_out : 0) + n0;
        sw[buf][nb] = p.w_scale[(static_cast<int64_t>(e) * (p.nrows_w / 128) +
                                 wrow / 128) * kblocks + kb];
      }
      if constexpr (!QA) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            sa[buf][mt][i] = cvalid[mt][i] ? p.a_scale[crow[mt][i] * kblocks + kb] : 0.f;
      }
    }
  };
  auto load_a = [&](int buf, int st) {
    if constexpr (QA) {
      ar[buf] = QaRaw<DT>::load(qrow, static_cast<int64_t>(st) * T::kStepK, lane);
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        load_act(af[buf][mt], arow[mt] + st * step_bytes, lg, avalid[mt]);
    }
  };
  if (s0 < s1) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      load_lines<DT>(bf[0][nb], brow[nb] + s0 * step_bytes, row8);
    load_a(0, s0);
    load_scales(0, s0);
  }
  // int8 QA: the token's scale (its row loads issued after the first step's)
  float qscale = 0.f;
  if constexpr (QA && DT == kDtInt8) qscale = row_scale_int8(qrow, p.kdim, lane);
  for (int s = s0; s < s1; s += 2) {
    // Two-deep register pipeline: fetch s+1 while s is multiplied.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int cur = s + h;
      if (cur >= s1) break;
      const int nxt = cur + 1;
      if (nxt < s1) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          load_lines<DT>(bf[h ^ 1][nb], brow[nb] + nxt * step_bytes, row8);
        load_a(h ^ 1, nxt);
        load_scales(h ^ 1, nxt);
      }
      if constexpr (QA && DT == kDtFp8) {
        const float sc = quant_step_fp8(ar[h], qlds[wave], lane, af[h][0]);
#pragma unroll
        for (int i = 0; i < 4; ++i) sa[h][0][i] = cvalid[0][i] ? sc : 0.f;
      } else if constexpr (QA) {
        quant_step_int8(ar[h], qscale, qlds[wave], lane, af[h][0]);
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) lines_to_frag(bf[h][nb]);
      if constexpr (DT == kDtBf16) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            mma_step<DT>(acc[nb][mt], af[h][mt], bf[h][nb]);
      } else if constexpr (DT == kDtInt8) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            mma_step_i8<DT>(acc[nb][mt], af[h][mt], bf[h][nb]);
      } else {
        // fp8 block scales: one 128-k group per step (fetched a step ahead).
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            const f32x4 t = mma_fp8(af[h][mt], bf[h][nb]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
              acc[nb][mt][i] += t[i] * (sa[h][mt][i] * sw[h][nb]);
          }
        }
      }
    }
  }

  // Cross-wave reduction of the split contraction.
  __shared__ Acc red[KW > 1 ? KW - 1 : 1][NB][MT][64];
  if (KW > 1) {
    if (wave > 0) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) red[wave - 1][nb][mt][lane] = acc[nb][mt];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < KW - 1; ++w)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[nb][mt] += red[w][nb][mt][lane];
  }

  // Epilogue (wave 0): lane owns column n0+ln, rows lg*4+i of each tile.
  const int col = n0 + ln;
  uint16_t* out = static_cast<uint16_t*>(p.out);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rb * BM + mt * 16 + lg * 4 + i;
      const bool valid = cvalid[mt][i];
      const int sid = row_sid(r);
      float v[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        float x;
        if constexpr (DT == kDtInt8) {
          float sa = 0.f;
          if (valid) sa = QA ? qscale : p.a_scale[crow[mt][i]];
          const float sw = p.w_scale[static_cast<int64_t>(e) * p.nrows_w +
                                     (nb ? p.n_out : 0) + col];
          x = static_cast<float>(acc[nb][mt][i]) * sa * sw;
        } else {
          x = acc[nb][mt][i];
        }
        if (p.bias)  // per-expert fp32 bias (the bias variant)
          x += p.bias[static_cast<int64_t>(e) * p.nrows_w + (nb ? p.n_out : 0) + col];
        v[nb] = x;
      }
      if constexpr (GEMM1) {
        // padded row order; direct rows write the compact slot rows only
        if (!DIRECT || valid)
          out[static_cast<int64_t>(DIRECT ? sid : r) * p.n_out + col] =
              gemm1_epilogue(v[0], v[NB - 1], p.weight_on_input && valid,
                             valid ? p.topk_w[sid] : 0.f, p.act, p.alpha, p.limit);
      } else {
        if (valid)
          out[static_cast<int64_t>(sid) * p.n_out + col] = f32_to_bf16_bits(v[0]);
      }
    }
  }
}

template <int DT, int MT, int KW, bool GEMM1, bool DIRECT, bool QA = false>
static int launch_one(const GemmParams& p, int row_blocks, hipStream_t stream) {
  dim3 grid(static_cast<unsigned>(p.n_out / 16), row_blocks);
  hipLaunchKernelGGL((moe_gemm_stream_kernel<DT, MT, KW, GEMM1, DIRECT, QA>), grid,
                     dim3(KW * 64), 0, stream, p);
  return check_launch("moe_gemm_stream_kernel");
}

template <int DT, bool GEMM1>
static int dispatch_kw(const GemmParams& p, int mt, int kw, int row_blocks,
                       hipStream_t stream) {
  if (p.direct_ids) {
    // direct rows: one slot per 16-row tile; a_src: quantised on the fly
    if constexpr (DT != kDtBf16) {
      if (p.a_src) {
#define FGS_CASE(KW_)             \
  if (mt == 1 && kw == KW_)       \
    return launch_one<DT, 1, KW_, GEMM1, true, true>(p, row_blocks, stream);
        FGS_CASE(1) FGS_CASE(2) FGS_CASE(4) FGS_CASE(8)
#undef FGS_CASE
        return fail(FGS_EUNSUPPORTED, "stream GEMM: no direct-row kernel for this tile");
      }
    }
#define FGS_CASE(KW_) \
  if (mt == 1 && kw == KW_) return launch_one<DT, 1, KW_, GEMM1, true>(p, row_blocks, stream);
    FGS_CASE(1) FGS_CASE(2) FGS_CASE(4) FGS_CASE(8)
#undef FGS_CASE
    return fail(FGS_EUNSUPPORTED, "stream GEMM: no direct-row kernel for this tile");
  }
#define FGS_CASE(MT_, KW_)                                           \
  if (mt == MT_ && kw == KW_)                                        \
    return launch_one<DT, MT_, KW_, GEMM1, false>(p, row_blocks, stream);
  FGS_CASE(1, 1) FGS_CASE(1, 2) FGS_CASE(1, 4) FGS_CASE(1, 8)
  FGS_CASE(2, 1) FGS_CASE(2, 2) FGS_CASE(2, 4) FGS_CASE(2, 8)
  FGS_CASE(4, 1) FGS_CASE(4, 2) FGS_CASE(4, 4) FGS_CASE(4, 8)
#undef FGS_CASE
  return fail(FGS_EUNSUPPORTED, "stream GEMM: no kernel for this tile");
}

// GEMM2 of one token with the top-k sum folded in (direct rows):
//   out[c] = bf16( sum_j gamma_j * (a2[j] . W2[e_j][c]) (+ gamma_j * b2[e_j][c]) )
// gamma_j = topk_w[j] (1 with the router weight on the input), dropped slots
// (ids outside [0, E)) skipped. The sum over slots runs in fp32 in a fixed
// order (slots in a wave, then waves), so it replaces GEMM2's bf16 y rows and
// moe_sum with one pass and no intermediate rounding. A workgroup owns 16
// output columns; with S slots, S <= KW gives each slot KW / S waves that
// split its contraction, S > KW deals whole slots to the waves in turn. Only
// row 0 of the MFMA tile is live (the token; the other activation rows are
// zero).
template <int DT, int KW, bool QA>
__global__ __launch_bounds__(KW * 64) void moe_gemm2_direct_kernel(const GemmParams p) {
  typedef StreamTraits<DT> T;
  typedef typename T::Acc Acc;
  constexpr int NV = T::kVecs;
  constexpr int ESZ = (DT == kDtBf16) ? 2 : 1;
  const int n0 = blockIdx.x * 16;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int ln = lane & 15;
  const int lg = lane >> 4;
  const int col = n0 + ln;
  const int slots = static_cast<int>(p.numel);
  const int steps = static_cast<int>(p.kdim / T::kStepK);
  const int64_t step_bytes = static_cast<int64_t>(T::kStepK) * ESZ;
  const int kblocks = static_cast<int>(p.kdim / 128);

  int j0, jstride, s0, s1;
  if (slots <= KW) {
    const int wps = KW / slots;  // waves per slot
    j0 = wave / wps;             // >= slots: an idle wave (KW % slots != 0)
    jstride = slots;
    const int sub = wave % wps;
    s0 = sub * steps / wps;      // empty for some waves when steps < wps
    s1 = (sub + 1) * steps / wps;
  } else {
    j0 = wave;
    jstride = KW;
    s0 = 0;
    s1 = steps;
  }

  static_assert(!QA || DT != kDtBf16, "on-the-fly quantisation");
  __shared__ __attribute__((aligned(16))) uint8_t qlds[QA ? KW : 1][T::kStepK];

  // slots <= KW: this wave's partial of slot j0's y (un-weighted);
  // slots > KW: the weighted sum of this wave's complete slots
  f32x4 tot = {0.f, 0.f, 0.f, 0.f};
  for (int j = j0; j < slots; j += jstride) {
    const int e = p.direct_ids[j];
    if (e < 0 || e >= p.num_experts) continue;
    const float gamma = p.weight_on_input ? 1.f : p.topk_w[j];
    const uint8_t* brow = p.w + ((static_cast<int64_t>(e) * p.nrows_w + n0 + (lane & 7)) *
                                 p.kdim) * ESZ + (lane >> 3) * 16;
    const int64_t row8 = 8 * p.kdim * ESZ;
    const uint8_t* arow = p.a + (static_cast<int64_t>(j) * p.kdim) * ESZ;
    const bool avalid = ln == 0;  // activation row 0 is the slot's row
    const float* wsc = DT == kDtFp8
                           ? p.w_scale + (static_cast<int64_t>(e) * (p.nrows_w / 128) +
                                          n0 / 128) * kblocks
                           : nullptr;
    Acc acc = {0, 0, 0, 0};
    u32x4 bf[2][NV], af[2][NV];
    typename QaRaw<DT>::type ar[2];  // QA: this lane's raw bf16 values of the step
    const uint16_t* qrow = QA ? p.a_src + static_cast<int64_t>(j) * p.kdim : nullptr;
    float sc[2];  // fp8: activation x weight block scale of the step (QA: weight)
    auto load = [&](int buf, int st) {
      load_lines<DT>(bf[buf], brow + st * step_bytes, row8);
      if constexpr (QA) {
        ar[buf] = QaRaw<DT>::load(qrow, static_cast<int64_t>(st) * T::kStepK, lane);
        if constexpr (DT == kDtFp8) sc[buf] = wsc[st];
      } else {
        load_act(af[buf], arow + st * step_bytes, lg, avalid);
        if constexpr (DT == kDtFp8) sc[buf] = p.a_scale[j * kblocks + st] * wsc[st];
      }
    };
    if (s0 < s1) load(0, s0);
    // int8 QA: the slot row's per-token scale
    float qscale = 0.f;
    if constexpr (QA && DT == kDtInt8) qscale = row_scale_int8(qrow, p.kdim, lane);
    for (int s = s0; s < s1; s += 2) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int cur = s + h;
        if (cur >= s1) break;
        if (cur + 1 < s1) load(h ^ 1, cur + 1);
        lines_to_frag(bf[h]);
        if constexpr (DT == kDtBf16) {
          mma_step<DT>(acc, af[h], bf[h]);
        } else if constexpr (DT == kDtInt8) {
          if constexpr (QA) quant_step_int8(ar[h], qscale, qlds[wave], lane, af[h]);
          mma_step_i8<DT>(acc, af[h], bf[h]);
        } else {
          float scl = sc[h];
          if constexpr (QA) scl = quant_step_fp8(ar[h], qlds[wave], lane, af[h]) * sc[h];
          const f32x4 t = mma_fp8(af[h], bf[h]);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i] += t[i] * scl;
        }
      }
    }
    float f = 1.f;
    if constexpr (DT == kDtInt8)
      f = (QA ? qscale : p.a_scale[j]) * p.w_scale[static_cast<int64_t>(e) * p.nrows_w + col];
    const float b = p.bias ? p.bias[static_cast<int64_t>(e) * p.nrows_w + col] : 0.f;
    if (slots <= KW) {
#pragma unroll
      for (int i = 0; i < 4; ++i) tot[i] = static_cast<float>(acc[i]) * f;
    } else {
      // the slot's whole y in this wave: round it to bf16 (the slot row the
      // unfused GEMM2 writes), then weight it as moe_sum does (product and
      // sum rounded separately)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        tot[i] = __fadd_rn(tot[i], __fmul_rn(gamma, bf16_bits_to_f32(f32_to_bf16_bits(
                                                        static_cast<float>(acc[i]) * f + b))));
    }
  }

  __shared__ f32x4 red[KW][64];
  red[wave][lane] = tot;
  __syncthreads();
  if (wave != 0) return;
  if (slots <= KW) {
    // per slot: its waves' partials in order, the bias, one bf16 rounding,
    // then the weighted sum over the slots in slot order
    const int wps = KW / slots;
    tot = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < slots; ++j) {
      const int e = p.direct_ids[j];
      if (e < 0 || e >= p.num_experts) continue;
      const float gamma = p.weight_on_input ? 1.f : p.topk_w[j];
      const float b = p.bias ? p.bias[static_cast<int64_t>(e) * p.nrows_w + col] : 0.f;
      f32x4 y = red[j * wps][lane];
      for (int w = 1; w < wps; ++w) y += red[j * wps + w][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        tot[i] = __fadd_rn(tot[i], __fmul_rn(gamma, bf16_bits_to_f32(f32_to_bf16_bits(y[i] + b))));
    }
  } else {
#pragma unroll
    for (int w = 1; w < KW; ++w) tot += red[w][lane];
  }
  // row 0 of the tile: lane group 0, register 0
  if (lg == 0) static_cast<uint16_t*>(p.out)[col] = f32_to_bf16_bits(tot[0]);
}

template <int DT, bool QA>
static int launch_gemm2_direct_t(const GemmParams& p, int kw, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.n_out / 16));
#define FGS_CASE(KW_)                                                                   \
  if (kw == KW_) {                                                                      \
    hipLaunchKernelGGL((moe_gemm2_direct_kernel<DT, KW_, QA>), grid, dim3(KW_ * 64), 0, \
                       stream, p);                                                      \
    return check_launch("moe_gemm2_direct_kernel");                                     \
  }
  FGS_CASE(4) FGS_CASE(8) FGS_CASE(16)
#undef FGS_CASE
  return fail(FGS_EUNSUPPORTED, "direct GEMM2: no kernel for this wave count");
}

// GEMM2 of one token with the top-k sum folded in, two slots per MFMA: a
// workgroup owns 8 output columns; slot pair q (slots 2q, 2q+1) puts those
// columns' weight rows of expert topk_ids[2q] in MFMA rows 0-7 and of
// topk_ids[2q+1] in rows 8-15 (one whole-line load instruction each) and the
// two slots' activation rows in A rows 0 and 1, so C[0][c] is slot 2q's
// column c and C[1][8 + c] slot 2q+1's. The same bytes as
// moe_gemm2_direct_kernel on twice the workgroups. pairs <= KW: each pair's
// KW / pairs waves split its contraction; the sum over slots is the same as
// moe_gemm2_direct_kernel's (per slot its waves' partials in order, the
// bias, one bf16 rounding, then gamma-weighted in slot order).
template <int DT>
__device__ __forceinline__ float quant_pair_fp8(uint32_t ra, uint32_t rb, uint8_t* qb, int lane,
                                                u32x4 (&f)[2], float& sb) {
  const float a0 = bf16_lo(ra), a1 = bf16_hi(ra), b0 = bf16_lo(rb), b1 = bf16_hi(rb);
  const float sa = fmaxf(wave_max(fmaxf(fabsf(a0), fabsf(a1))), 1e-10f) / 448.0f;
  sb = fmaxf(wave_max(fmaxf(fabsf(b0), fabsf(b1))), 1e-10f) / 448.0f;
  reinterpret_cast<uint16_t*>(qb)[lane] =
      static_cast<uint16_t>(cvt_pk_fp8(quant1_fp8(a0, sa), quant1_fp8(a1, sa)));
  reinterpret_cast<uint16_t*>(qb + 128)[lane] =
      static_cast<uint16_t>(cvt_pk_fp8(quant1_fp8(b0, sb), quant1_fp8(b1, sb)));
  const int lg = lane >> 4, ln = lane & 15;
#pragma unroll
  for (int v = 0; v < 2; ++v) {
    const u32x4 x = *reinterpret_cast<const u32x4*>(qb + (ln == 1 ? 128 : 0) + frag_byte(v, lg));
    f[v] = ln < 2 ? x : u32x4{0, 0, 0, 0};
  }
  return sa;
}

__device__ __forceinline__ void quant_pair_int8(uint2 ra, uint2 rb, float sa, float sb, uint8_t* qb,
                                                int lane, u32x4 (&f)[4]) {
  reinterpret_cast<uint32_t*>(qb)[lane] =
      quant1_int8(bf16_lo(ra.x), sa) | quant1_int8(bf16_hi(ra.x), sa) << 8 |
      quant1_int8(bf16_lo(ra.y), sa) << 16 | quant1_int8(bf16_hi(ra.y), sa) << 24;
  reinterpret_cast<uint32_t*>(qb + 256)[lane] =
      quant1_int8(bf16_lo(rb.x), sb) | quant1_int8(bf16_hi(rb.x), sb) << 8 |
      quant1_int8(bf16_lo(rb.y), sb) << 16 | quant1_int8(bf16_hi(rb.y), sb) << 24;
  const int lg = lane >> 4, ln = lane & 15;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const u32x4 x = *reinterpret_cast<const u32x4*>(qb + (ln == 1 ? 256 : 0) + frag_byte(v, lg));
    f[v] = ln < 2 ? x : u32x4{0, 0, 0, 0};
  }
}

template <int DT, int KW, bool QA>
__global__ __launch_bounds__(KW * 64) void moe_gemm2_pair_kernel(const GemmParams p) {
  typedef StreamTraits<DT> T;
  typedef typename T::Acc Acc;
  constexpr int NV = T::kVecs;
  constexpr int ESZ = (DT == kDtBf16) ? 2 : 1;
  static_assert(!QA || DT != kDtBf16, "on-the-fly quantisation");
  const int n0 = blockIdx.x * 8;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15;
  const int lg = lane >> 4;
  const int c8 = ln & 7;   // this lane's output column n0 + c8 (rows c8 and 8 + c8)
  const int slots = static_cast<int>(p.numel);
  const int pairs = (slots + 1) / 2;  // <= KW (the launcher checks)
  const int wps = KW / pairs;         // waves per pair
  const int q = wave / wps;           // >= pairs: an idle wave
  const int sub = wave % wps;
  const int steps = static_cast<int>(p.kdim / T::kStepK);
  const int s0 = sub * steps / wps, s1 = (sub + 1) * steps / wps;
  const int64_t step_bytes = static_cast<int64_t>(T::kStepK) * ESZ;
  const int kblocks = static_cast<int>(p.kdim / 128);
  __shared__ __attribute__((aligned(16))) uint8_t qlds[QA ? KW : 1][2 * T::kStepK];
  __shared__ float2 red[KW][64];

  float2 part = {0.f, 0.f};  // (slot 2q, column c8) and (slot 2q + 1, column c8)
  if (q < pairs) {
    const int ja = 2 * q, jb = 2 * q + 1;
    const int ea = p.direct_ids[ja];
    const int eb = jb < slots ? p.direct_ids[jb] : -1;
    const bool va = ea >= 0 && ea < p.num_experts;
    const bool vb = eb >= 0 && eb < p.num_experts;
    if (va || vb) {
      // a dropped (or absent) slot reads the other slot's rows with a zero
      // activation row and is skipped in the sum
      const int xa = va ? ea : eb, xb = vb ? eb : ea;
      const int ra = va ? ja : jb, rb = vb ? jb : ja;
      const uint8_t* brow = p.w + ((static_cast<int64_t>(xa) * p.nrows_w + n0 + (lane & 7)) *
                                   p.kdim) * ESZ + (lane >> 3) * 16;
      const int64_t row8 = (static_cast<int64_t>(xb) - xa) * p.nrows_w * p.kdim * ESZ;
      const bool avalid = (ln == 0 && va) || (ln == 1 && vb);
      const uint8_t* arow = p.a + (static_cast<int64_t>(ln == 1 ? rb : ra) * p.kdim) * ESZ;
      const float* wsa = DT == kDtFp8 ? p.w_scale + (static_cast<int64_t>(xa) * (p.nrows_w / 128) +
                                                      n0 / 128) * kblocks : nullptr;
      const float* wsb = DT == kDtFp8 ? p.w_scale + (static_cast<int64_t>(xb) * (p.nrows_w / 128) +
                                                      n0 / 128) * kblocks : nullptr;
      const uint16_t* qa = QA ? p.a_src + static_cast<int64_t>(ra) * p.kdim : nullptr;
      const uint16_t* qbr = QA ? p.a_src + static_cast<int64_t>(rb) * p.kdim : nullptr;
      Acc acc = {0, 0, 0, 0};
      u32x4 bf[2][NV], af[2][NV];
      typename QaRaw<DT>::type ar[2][2];
      float sc[2][2];  // fp8: the two slots' activation x weight scales of a step (QA: weight)
      auto load = [&](int buf, int st) {
        load_lines<DT>(bf[buf], brow + st * step_bytes, row8);
        if constexpr (QA) {
          ar[buf][0] = QaRaw<DT>::load(qa, static_cast<int64_t>(st) * T::kStepK, lane);
          ar[buf][1] = QaRaw<DT>::load(qbr, static_cast<int64_t>(st) * T::kStepK, lane);
          if constexpr (DT == kDtFp8) {
            sc[buf][0] = wsa[st];
            sc[buf][1] = wsb[st];
          }
        } else {
          load_act(af[buf], arow + st * step_bytes, lg, avalid);
          if constexpr (DT == kDtFp8) {
            sc[buf][0] = p.a_scale[ra * kblocks + st] * wsa[st];
            sc[buf][1] = p.a_scale[rb * kblocks + st] * wsb[st];
          }
        }
      };
      float qsa = 0.f, qsb = 0.f;  // int8 QA: the two slot rows' per-token scales
      if (s0 < s1) load(0, s0);
      if constexpr (QA && DT == kDtInt8) {
        qsa = row_scale_int8(qa, p.kdim, lane);
        qsb = row_scale_int8(qbr, p.kdim, lane);
      }
      for (int s = s0; s < s1; s += 2) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int cur = s + h;
          if (cur >= s1) break;
          if (cur + 1 < s1) load(h ^ 1, cur + 1);
          lines_to_frag(bf[h]);
          if constexpr (DT == kDtBf16) {
            mma_step<DT>(acc, af[h], bf[h]);
          } else if constexpr (DT == kDtInt8) {
            if constexpr (QA) quant_pair_int8(ar[h][0], ar[h][1], qsa, qsb, qlds[wave], lane, af[h]);
            mma_step_i8<DT>(acc, af[h], bf[h]);
          } else {
            float s_a = sc[h][0], s_b = sc[h][1];
            if constexpr (QA) {
              float xb;
              s_a *= quant_pair_fp8<DT>(ar[h][0], ar[h][1], qlds[wave], lane, af[h], xb);
              s_b *= xb;
            }
            const f32x4 t = mma_fp8(af[h], bf[h]);
            acc[0] += t[0] * s_a;
            acc[1] += t[1] * s_b;
          }
        }
      }
      float fa = 1.f, fb = 1.f;
      if constexpr (DT == kDtInt8) {
        fa = (QA ? qsa : p.a_scale[ra]) * p.w_scale[static_cast<int64_t>(xa) * p.nrows_w + n0 + c8];
        fb = (QA ? qsb : p.a_scale[rb]) * p.w_scale[static_cast<int64_t>(xb) * p.nrows_w + n0 + c8];
      }
      part.x = static_cast<float>(acc[0]) * fa;  // C[0][c8] in lane (c8, 0)
      part.y = static_cast<float>(acc[1]) * fb;  // C[1][8 + c8] in lane (8 + c8, 0)
    }
  }
  red[wave][lane] = part;
  __syncthreads();
  if (wave != 0 || lane >= 8) return;
  // lane c: output column n0 + c; slots in order, each its waves' partials
  // in order, the bias, one bf16 rounding, then the weighted sum
  const int col = n0 + lane;
  float tot = 0.f;
  for (int j = 0; j < slots; ++j) {
    const int e = p.direct_ids[j];
    if (e < 0 || e >= p.num_experts) continue;
    const float gamma = p.weight_on_input ? 1.f : p.topk_w[j];
    const float b = p.bias ? p.bias[static_cast<int64_t>(e) * p.nrows_w + col] : 0.f;
    const int qj = j >> 1;
    float y = 0.f;
    for (int w = 0; w < wps; ++w) {
      const float2 v = red[qj * wps + w][(j & 1) ? 8 + lane : lane];
      y += (j & 1) ? v.y : v.x;
    }
    tot = __fadd_rn(tot, __fmul_rn(gamma, bf16_bits_to_f32(f32_to_bf16_bits(y + b))));
  }
  static_cast<uint16_t*>(p.out)[col] = f32_to_bf16_bits(tot);
}

template <int DT, bool QA>
static int launch_gemm2_pair_t(const GemmParams& p, int kw, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.n_out / 8));
#define FGS_CASE(KW_)                                                                 \
  if (kw == KW_) {                                                                    \
    hipLaunchKernelGGL((moe_gemm2_pair_kernel<DT, KW_, QA>), grid, dim3(KW_ * 64), 0, \
                       stream, p);                                                    \
    return check_launch("moe_gemm2_pair_kernel");                                     \
  }
  FGS_CASE(4) FGS_CASE(8) FGS_CASE(16)
#undef FGS_CASE
  return fail(FGS_EUNSUPPORTED, "paired GEMM2: no kernel for this wave count");
}

int launch_gemm2_pair(int dt, const GemmParams& p, int kw, hipStream_t stream) {
  if (!p.direct_ids || p.numel < 1)
    return fail(FGS_EINVAL, "paired GEMM2: needs the slot ids");
  if ((p.numel + 1) / 2 > kw || p.n_out % 8 != 0)
    return fail(FGS_EINVAL, "paired GEMM2: more slot pairs than waves, or n_out % 8 != 0");
  if (p.a_src && (dt == kDtBf16 || p.numel > kQaMaxSlots))
    return fail(FGS_EINVAL, "paired GEMM2: on-the-fly quantisation needs fp8 / int8");
  switch (dt) {
    case kDtBf16: return launch_gemm2_pair_t<kDtBf16, false>(p, kw, stream);
    case kDtFp8:
      return p.a_src ? launch_gemm2_pair_t<kDtFp8, true>(p, kw, stream)
                     : launch_gemm2_pair_t<kDtFp8, false>(p, kw, stream);
    case kDtInt8:
      return p.a_src ? launch_gemm2_pair_t<kDtInt8, true>(p, kw, stream)
                     : launch_gemm2_pair_t<kDtInt8, false>(p, kw, stream);
  }
  return fail(FGS_EUNSUPPORTED, "paired GEMM2: unknown dtype");
}

int launch_gemm2_direct(int dt, const GemmParams& p, int kw, hipStream_t stream) {
  if (!p.direct_ids || p.numel < 1)
    return fail(FGS_EINVAL, "direct GEMM2: needs the slot ids");
  if (p.a_src && (dt == kDtBf16 || p.numel > kQaMaxSlots))
    return fail(FGS_EINVAL, "direct GEMM2: on-the-fly quantisation needs fp8 / int8 and at "
                            "most 64 slots");
  switch (dt) {
    case kDtBf16: return launch_gemm2_direct_t<kDtBf16, false>(p, kw, stream);
    case kDtFp8:
      return p.a_src ? launch_gemm2_direct_t<kDtFp8, true>(p, kw, stream)
                     : launch_gemm2_direct_t<kDtFp8, false>(p, kw, stream);
    case kDtInt8:
      return p.a_src ? launch_gemm2_direct_t<kDtInt8, true>(p, kw, stream)
                     : launch_gemm2_direct_t<kDtInt8, false>(p, kw, stream);
  }
  return fail(FGS_EUNSUPPORTED, "direct GEMM2: unknown dtype");
}

int stream_step_k(int dt) {
  return dt == kDtInt8 ? StreamTraits<kDtInt8>::kStepK : 128;
}

int launch_gemm_stream(int dt, bool gemm1, const GemmParams& p, int mt, int kw,
                       int row_blocks, hipStream_t stream) {
  if (row_blocks <= 0) return FGS_OK;
  if (row_blocks > 65535)
    return fail(FGS_EUNSUPPORTED, "stream GEMM: more than 65535 row blocks (grid y)");
  switch (dt) {
    case kDtBf16:
      return gemm1 ? dispatch_kw<kDtBf16, true>(p, mt, kw, row_blocks, stream)
                   : dispatch_kw<kDtBf16, false>(p, mt, kw, row_blocks, stream);
    case kDtFp8:
      return gemm1 ? dispatch_kw<kDtFp8, true>(p, mt, kw, row_blocks, stream)
                   : dispatch_kw<kDtFp8, false>(p, mt, kw, row_blocks, stream);
    case kDtInt8:
      return gemm1 ? dispatch_kw<kDtInt8, true>(p, mt, kw, row_blocks, stream)
                   : dispatch_kw<kDtInt8, false>(p, mt, kw, row_blocks, stream);
  }
  return fail(FGS_EUNSUPPORTED, "stream GEMM: unknown dtype");
}

}  // namespace fgs
