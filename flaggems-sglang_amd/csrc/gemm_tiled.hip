// LDS-tiled grouped GEMMs of the fused-MoE path (prefill regime: many rows
// per expert, the layer is bound by MFMA throughput).
//
// A workgroup of WM x WN waves owns a BM-row block of the expert-sorted,
// padded row order (one expert per block, from moe_align_block_size) and
// BNR weight rows. Activation and weight tiles stream into a STAGES-deep LDS
// ring with LDS-DMA loads (global_load_lds_dwordx4: no staging registers),
// SK bytes of k per stage (a configuration may add a compact ring with
// fewer activation rows and more slots for blocks that are mostly padding). Each wave multiplies its (BM/WM) x (BNR/WN)
// sub-tile with v_mfma_f32_32x32x16_bf16; the fragments of the next half
// stage are read while the current MFMAs run.
//
// GEMM1 (fused activation): each wave's weight rows are its gate rows
// followed by the matching up rows, so every lane holds the gate and up
// accumulators of the same output element; the epilogue applies the
// reference's rounding points and silu (ops/fused_moe.py:205-218).
// GEMM2: y = a2 W2^T per padded row, stored (bf16) at its top-k slot, or,
// split over k (ksplit > 1, to fill the chip when there are few tiles), as
// fp32 partial sums per split that moe_sum adds in a fixed order.
#include <stdlib.h>

#include <mutex>
#include <string>
#include <type_traits>

#include "gemm_tiled_common.h"

namespace fgs {

// Tile order. The grid is 1-D and padded to a multiple of the 8 XCDs.
// Workgroup `pid` runs on XCD pid % 8, so logical tile
// (pid % 8) * (grid / 8) + pid / 8 gives every XCD a contiguous range of
// tiles. group_m > 0: bands of group_m row blocks, walked column by column
// (row block fastest), so the row blocks of one expert -- adjacent in the
// sorted order -- read each weight tile back to back, and a band's
// activation tiles are reused across its columns. group_m == 0: all row
// blocks walked per group of group_n column tiles (column fastest).
__device__ __forceinline__ bool tile_of(int pid, int grid, int n_rb, int n_ct,
                                        int group_m, int group_n, int* rb, int* ct) {
  const int logical = (pid % 8) * (grid / 8) + pid / 8;
  if (logical >= n_rb * n_ct) return false;
  // both orders computed as values and stored once at the end (stores in
  // each branch were merged into a store through a selected address, which
  // kept rb / ct in scratch memory: a store and reload before every tile's
  // first load)
  int r, c;
  if (group_m > 0) {
    const int band_tiles = group_m * n_ct;
    const int band = logical / band_tiles;
    const int rem = logical - band * band_tiles;
    const int rows = min(group_m, n_rb - band * group_m);
    c = rem / rows;
    r = band * group_m + rem % rows;
  } else {
    const int span = n_rb * group_n;
    const int group = logical / span;
    const int idx = logical - group * span;
    const int gsize = min(group_n, n_ct - group * group_n);
    r = idx / gsize;
    c = group * group_n + idx % gsize;
  }
  *rb = r;
  *ct = c;
  return true;
}

// BMA < BM: a second, compact LDS ring for row blocks whose rows from BMA on
// are all padding -- BMA activation rows per stage in STAGES_C slots (more
// stages in flight than the full ring fits); fuller blocks use the full one.
template <int BM_, int BNR_, int WM_, int WN_, int SK_, int STAGES_, int BMA_ = BM_,
          int STAGES_C_ = STAGES_>
struct TileCfg {
  static constexpr int BM = BM_;        // rows (alignment block size)
  static constexpr int BNR = BNR_;      // weight rows per tile
  static constexpr int WM = WM_, WN = WN_;
  static constexpr int SK = SK_;        // k bytes per LDS stage row
  static constexpr int STAGES = STAGES_;
  static constexpr int BMA = BMA_;      // activation rows of the compact ring
  static constexpr int STAGES_C = STAGES_C_;
  static constexpr int NW = WM * WN;
  static constexpr int CPR = SK / 16;   // 16-byte chunks per stage row
  static constexpr int LR = 64 / CPR;   // rows one LDS-DMA wave load covers
  static constexpr int RPL = 256 / SK;  // stage rows per 256-byte bank line
  static_assert(BMA <= BM && STAGES_C >= 2, "compact ring");
};

// Swizzled position of logical 16-byte chunk c of stage row r. The DMA
// writes rows densely (lane l -> byte 16*l of a 1 KiB block), so rows are
// not padded; gfx950's LDS serves a 16-byte-per-lane read 16 lanes (256
// bytes, all 64 banks) at a time, and the XOR with (r / RPL) % CPR gives
// the 16 consecutive rows such a group reads 16 distinct bank positions.
template <class C>
__device__ __forceinline__ int chunk_pos(int r, int c) {
  return c ^ ((r / C::RPL) % C::CPR);
}

// Bytes of the per-stage scale area (fp8 only): one float slot per lane of
// the workgroup, filled by one 4-byte LDS-DMA load per wave per stage.
template <int DT, class C>
constexpr int tiled_scale_bytes() {
  return DT == kDtFp8 ? C::NW * 256 : 0;
}
// LDS of one ring (COMPACT: BMA activation rows, STAGES_C slots), and the
// launch's allocation: the larger of the rings a configuration uses.
template <int DT, class C, bool COMPACT>
constexpr int tiled_ring_bytes() {
  return (COMPACT ? C::STAGES_C : C::STAGES) *
         (((COMPACT ? C::BMA : C::BM) + C::BNR) * C::SK + tiled_scale_bytes<DT, C>());
}
template <int DT, class C>
constexpr int tiled_lds_bytes() {
  return C::BMA < C::BM && tiled_ring_bytes<DT, C, true>() > tiled_ring_bytes<DT, C, false>()
             ? tiled_ring_bytes<DT, C, true>()
             : tiled_ring_bytes<DT, C, false>();
}

// 4-byte LDS-DMA load: lane l copies 4 bytes from `src` to byte 4*l of the
// 256-byte block at `lds_dst`.
__device__ __forceinline__ void lds_dma4(const void* src, void* lds_dst) {
  __builtin_amdgcn_global_load_lds(
      src, (__attribute__((address_space(3))) void*)(lds_dst), 4, 0, 0);
}

// One tile (row block rb_id of expert e, column tile tile_n, k split ks).
// COMPACT: the row block's rows from C::BMA on are all padding, and the LDS
// ring holds C::BMA activation rows per stage in C::STAGES_C slots.
template <int DT, class C, bool GEMM1, bool COMPACT>
__device__ __forceinline__ void tiled_tile(const GemmParams& p, const int rb_id,
                                           const int tile_n, const int ks, const int e) {
  using T = TiledType<DT>;
  using Frag = typename T::Frag;
  using Acc = typename T::Acc;
  constexpr bool FP8 = DT == kDtFp8;
  constexpr bool INT8 = DT == kDtInt8;
  constexpr int ESZ = T::ESZ, FC = T::FC;
  constexpr int BM = C::BM, BNR = C::BNR, SK = C::SK;
  constexpr int STAGES = COMPACT ? C::STAGES_C : C::STAGES;
  constexpr int NW = C::NW, WN = C::WN;
  constexpr int A_BYTES = (COMPACT ? C::BMA : BM) * SK;  // activation rows in LDS
  constexpr int B_BYTES = BNR * SK;
  constexpr int SC_OFF = A_BYTES + B_BYTES;
  constexpr int STAGE = SC_OFF + tiled_scale_bytes<DT, C>();
  constexpr int NLA = BM / (C::LR * NW);   // A loads per wave per stage
  constexpr int NLB = BNR / (C::LR * NW);  // B loads per wave per stage
  constexpr int NL = NLA + NLB + (FP8 ? 1 : 0);
  constexpr int WROWS = BM / C::WM;        // rows per wave
  constexpr int WCOLS = BNR / WN;          // weight rows per wave
  constexpr int RB = WROWS / 32;           // 32-row MFMA blocks
  constexpr int CB = WCOLS / 32;           // 32-col MFMA blocks
  constexpr int KK = SK / (32 * FC);       // MFMA k steps per stage
  static_assert(NLA * C::LR * NW == BM, "A tile / waves");
  static_assert(NLB * C::LR * NW == BNR, "B tile / waves");
  static_assert(STAGES >= 2 && (STAGES - 1) * NL < 64, "stages");
  static_assert(RB >= 1 && CB >= 1 && KK >= 1, "wave tile");
  static_assert(!GEMM1 || CB % 2 == 0, "gate/up pairing");
  static_assert(tiled_ring_bytes<DT, C, COMPACT>() <= 160 * 1024, "gfx950 LDS is 160 KiB");
  // a compact ring holds whole per-wave activation load groups
  static_assert(!COMPACT || C::BMA % (NLA * C::LR) == 0, "compact ring rows");
  // fp8: one stage is one 128-wide k block of the block scales, and a tile's
  // weight rows (GEMM1: each of its gate and up halves) lie in whole 128-row
  // scale blocks or inside one
  static_assert(!FP8 || (SK == 128 && BNR % 128 == 0 && BM + 4 <= NW * 64), "fp8 tile");

  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];


  const int lane = threadIdx.x & 63;
  // wave index in an SGPR: LDS-DMA destinations (M0) then stay scalar
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int row0 = rb_id * BM;
  const int64_t row_bytes = p.kdim * ESZ;

  // Activation row feeding padded row r of the block. Pad rows (always a
  // suffix of the block: one expert per block) read a row every pad shares
  // -- token 0, or the block's first row -- so they cost L1/L2 hits only;
  // their results are never stored.
  auto act_row = [&](int r) -> int64_t {
    const int sid = p.sorted_ids[row0 + r];
    const bool ok = sid < p.numel;
    return GEMM1 ? (ok ? div_topk(p, sid) : 0) : row0 + (ok ? r : 0);
  };

  // ---- this lane's source of each LDS-DMA load: row lane/CPR, chunk lane%CPR
  const int lrow = lane / C::CPR;
  const int lchunk = lane % C::CPR;
  // all token slots first: computing a row (GEMM1 divides by topk for real
  // rows only) compiles to a branch, which would otherwise hold each load
  // back until the previous row is done
  const uint8_t* a_src[NLA];
  int a_sid[NLA];
#pragma unroll
  for (int i = 0; i < NLA; ++i) a_sid[i] = p.sorted_ids[row0 + (wave * NLA + i) * C::LR + lrow];
#pragma unroll
  for (int i = 0; i < NLA; ++i) {
    const int r = (wave * NLA + i) * C::LR + lrow;
    const bool ok = a_sid[i] < p.numel;
    const int64_t arow = GEMM1 ? (ok ? div_topk(p, a_sid[i]) : 0) : row0 + (ok ? r : 0);
    a_src[i] = p.a + arow * row_bytes + chunk_pos<C>(r, lchunk) * 16;
  }
  const uint8_t* b_src[NLB];
  const int64_t wbase = static_cast<int64_t>(e) * p.nrows_w;
#pragma unroll
  for (int i = 0; i < NLB; ++i) {
    const int j = (wave * NLB + i) * C::LR + lrow;  // tile row
    int64_t wrow;
    if constexpr (GEMM1) {
      // tile rows of wave column wc: WCOLS/2 gate rows, then the same
      // output columns' up rows
      constexpr int HALF = WCOLS / 2;
      const int wc = j / WCOLS;
      const int in = j % WCOLS;
      const int ncol = tile_n * (BNR / 2) + wc * HALF + in % HALF;
      wrow = (in >= HALF ? p.n_out : 0) + ncol;
    } else {
      wrow = static_cast<int64_t>(tile_n) * BNR + j;
    }
    b_src[i] = p.w + (wbase + wrow) * row_bytes + chunk_pos<C>(j, lchunk) * 16;
  }

  // fp8 block scales of one k block, staged with the tiles: slot s < BM is
  // padded row s's activation scale, slot BM + b the tile's b-th 128-row
  // weight scale block (GEMM1: b = 0 gate, 1 up); other slots are unused.
  // Stage kt's scale is sc_src + kt * sc_step: activation scales stored
  // k-block-major over the padded rows (a_scale_kstride > 0; a pad row
  // reads the tile's first row) step by the stride, so a wave's 64 rows
  // are one contiguous 256-byte read; row-major ones and the weight scales
  // step by one float.
  const int kblocks = static_cast<int>(p.kdim / 128);
  const float* sc_src = nullptr;
  int64_t sc_step = 1;
  if constexpr (FP8) {
    const int slot = wave * 64 + lane;
    const int64_t wblk0 = static_cast<int64_t>(e) * (p.nrows_w / 128);
    if (slot < BM) {
      if (p.a_scale_kstride > 0) {
        const bool live = p.sorted_ids[row0 + slot] < p.numel;
        sc_src = p.a_scale + row0 + (live ? slot : 0);
        sc_step = p.a_scale_kstride;
      } else {
        sc_src = p.a_scale + act_row(slot) * kblocks;
      }
    } else {
      int64_t wb = 0;
      if (slot < BM + (GEMM1 ? 2 : BNR / 128)) {
        const int b = slot - BM;
        wb = GEMM1 ? (b ? p.n_out / 128 : 0) + tile_n * (BNR / 2) / 128
                   : static_cast<int64_t>(tile_n) * (BNR / 128) + b;
      }
      sc_src = p.w_scale + (wblk0 + wb) * kblocks;
    }
  }

  // A wave whose activation-load rows are all padding (they are a suffix of
  // the block) issues none of its activation loads: those rows' LDS holds
  // stale bytes, which only the all-pad rows' (discarded) outputs see.
  const bool a_on = __builtin_amdgcn_readfirstlane(a_sid[0]) < p.numel;
  auto issue = [&](int kt, int slot, auto a_on_c) {
    const int64_t koff = static_cast<int64_t>(kt) * SK;
    uint8_t* base = lds + slot * STAGE;
    if constexpr (decltype(a_on_c)::value) {
#pragma unroll
      for (int i = 0; i < NLA; ++i)
        lds_dma16(a_src[i] + koff, base + (wave * NLA + i) * 1024);
    }
#pragma unroll
    for (int i = 0; i < NLB; ++i)
      lds_dma16(b_src[i] + koff, base + A_BYTES + (wave * NLB + i) * 1024);
    if constexpr (FP8) lds_dma4(sc_src + kt * sc_step, base + SC_OFF + wave * 256);
  };
  // With a two-slot ring (bf16 / int8) a freed slot's refill is split: the
  // activation rows right after the barrier, the weight rows during the
  // next stage's first k step, so a CU's loads of a stage are spread over
  // two k steps.
  constexpr bool SPLIT = STAGES == 2 && !FP8;
  auto issue_part = [&](int kt, int slot, auto part_c, auto a_on_c) {
    constexpr int PART = decltype(part_c)::value;
    const int64_t koff = static_cast<int64_t>(kt) * SK;
    uint8_t* base = lds + slot * STAGE;
    if constexpr (PART == 0) {
      if constexpr (decltype(a_on_c)::value) {
#pragma unroll
        for (int i = 0; i < NLA; ++i)
          lds_dma16(a_src[i] + koff, base + (wave * NLA + i) * 1024);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NLB; ++i)
        lds_dma16(b_src[i] + koff, base + A_BYTES + (wave * NLB + i) * 1024);
    }
  };

  Acc acc[RB][CB];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

  // Fragment reads: lane reads row (lane & 31) of a 32-row block, logical
  // chunks FC*(2*kk + (lane >> 5)) + c, c < FC.
  const int fr = lane & 31;
  int frag_off[KK][FC];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk)
#pragma unroll
    for (int c = 0; c < FC; ++c)
      frag_off[kk][c] = fr * SK + chunk_pos<C>(fr, FC * (2 * kk + (lane >> 5)) + c) * 16;
  const int a_base = wm * WROWS * SK;
  const int b_base = A_BYTES + wn * WCOLS * SK;

  const int KT_all = static_cast<int>(row_bytes / SK);
  const int kt0 = ks * KT_all / p.ksplit;
  const int KT = (ks + 1) * KT_all / p.ksplit - kt0;
#pragma unroll
  for (int i = 0; i < NLA; ++i) a_src[i] += static_cast<int64_t>(kt0) * SK;
#pragma unroll
  for (int i = 0; i < NLB; ++i) b_src[i] += static_cast<int64_t>(kt0) * SK;
  if constexpr (FP8) sc_src += kt0 * sc_step;
  // the first token slot of each of the wave's 32-row blocks, loaded before
  // the stage loads: the counter drains in issue order, so waiting on these
  // never waits on a stage load
  int first_sid[RB];
#pragma unroll
  for (int i = 0; i < RB; ++i) first_sid[i] = p.sorted_ids[row0 + wm * WROWS + i * 32];
  // activation row (a_scale index) of tile row rr holding slot sid
  auto act_of = [&](int rr, int sid) -> int64_t {
    const bool ok = sid < p.numel;
    return GEMM1 ? (ok ? div_topk(p, sid) : 0) : row0 + (ok ? rr : 0);
  };
#pragma unroll
  for (int s = 0; s < STAGES; ++s) {
    if (s >= KT) break;
    if (a_on) issue(s, s, std::true_type{});
    else issue(s, s, std::false_type{});
  }

  // Waits until at most `n` of this wave's later stages (LPS loads each:
  // NL, or NL - NLA without activation loads) are in flight.
  auto wait_stages = [&](int n, auto lps_c) {
    constexpr int LPS = decltype(lps_c)::value;
    if (n >= 6) wait_vmcnt<(6 * LPS < 64 ? 6 * LPS : 0)>();
    else if (n == 5) wait_vmcnt<(5 * LPS < 64 ? 5 * LPS : 0)>();
    else if (n == 4) wait_vmcnt<(4 * LPS < 64 ? 4 * LPS : 0)>();
    else if (n == 3) wait_vmcnt<(3 * LPS < 64 ? 3 * LPS : 0)>();
    else if (n == 2) wait_vmcnt<2 * LPS>();
    else if (n == 1) wait_vmcnt<LPS>();
    else wait_vmcnt<0>();
  };
  auto load_frag = [&](const uint8_t* p0, int kk) -> Frag {
    if constexpr (FC == 1) {
      return *reinterpret_cast<const Frag*>(p0 + frag_off[kk][0]);
    } else {
      const i32x4 lo = *reinterpret_cast<const i32x4*>(p0 + frag_off[kk][0]);
      const i32x4 hi = *reinterpret_cast<const i32x4*>(p0 + frag_off[kk][FC - 1]);
      return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  };
  auto read_frags = [&](int kt, int kk, Frag (&fa)[RB], Frag (&fb)[CB]) {
    const uint8_t* st = lds + (kt % STAGES) * STAGE;
#pragma unroll
    for (int i = 0; i < RB; ++i) fa[i] = load_frag(st + a_base + i * 32 * SK, kk);
#pragma unroll
    for (int j = 0; j < CB; ++j) fb[j] = load_frag(st + b_base + j * 32 * SK, kk);
  };
  // fp8: this lane's activation scale per 32-row block and the wave's weight
  // scale per 32-col block, for stage kt.
  auto read_scales = [&](int kt, float (&sa)[RB], float (&sw)[CB]) {
    const float* sc = reinterpret_cast<const float*>(lds + (kt % STAGES) * STAGE + SC_OFF);
#pragma unroll
    for (int i = 0; i < RB; ++i) sa[i] = sc[wm * WROWS + i * 32 + fr];
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      const int b = GEMM1 ? (j >= CB / 2 ? 1 : 0) : (wn * WCOLS + j * 32) / 128;
      sw[j] = sc[BM + b];
    }
  };
  // Weights are the MFMA's A operand and activations its B operand, so the
  // 32x32 accumulator is transposed: lane l holds token (l & 31) and four
  // runs of 4 consecutive output columns -> 8-byte stores in the epilogue.
  // 32-row blocks of this wave that hold at least one real row. Pad rows are
  // a suffix of the block, so the live blocks are a prefix; the main loop is
  // instantiated per live count so all-pad blocks (the tail of an expert's
  // last block) skip their MFMAs without branches inside the MFMA stream.
  int nlive = 0;
#pragma unroll
  for (int i = 0; i < RB; ++i) nlive += first_sid[i] < p.numel ? 1 : 0;

  Frag fa[2][RB], fb[2][CB];
  auto main_loop = [&](auto nlive_c, auto a_on_c) {
    constexpr int NLIVE = decltype(nlive_c)::value;
    constexpr int LPS = decltype(a_on_c)::value ? NL : NL - NLA;  // loads per stage
    const auto lps = std::integral_constant<int, LPS>{};
    const auto aon = a_on_c;
    // fp8: each stage (one k block) accumulates into tmp, which is then
    // added to acc times the block's activation x weight scale.
    Acc tmp[FP8 ? RB : 1][FP8 ? CB : 1];
    float sa_c[RB], sw_c[CB], sa_n[RB], sw_n[CB];
    auto mma = [&](int kk, const Frag (&a)[RB], const Frag (&b)[CB]) {
#pragma unroll
      for (int i = 0; i < NLIVE; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j) {
          if constexpr (FP8) {
            const Acc zero = {};
            tmp[i][j] = T::mma(b[j], a[i], kk == 0 ? zero : tmp[i][j]);
          } else {
            acc[i][j] = T::mma(b[j], a[i], acc[i][j]);
          }
        }
    };
    // Region schedule: one MFMA, then all of the next step's fragment
    // reads, then the remaining MFMAs (reads get the MFMAs' time to land).
    auto sched_step = [&]() {
      constexpr int NR = (RB + CB) * FC;
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, NLIVE * CB - 1, 0);
    };
    // ... with the weight-row loads of a split refill one between each pair
    // of the remaining MFMAs
    auto sched_step_dma = [&]() {
      constexpr int NR = (RB + CB) * FC;
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
#pragma unroll
      for (int t = 0; t < NLB; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        if (t < NLIVE * CB - 1) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
      if constexpr (NLIVE * CB - 1 > NLB)
        __builtin_amdgcn_sched_group_barrier(0x008, NLIVE * CB - 1 - NLB, 0);
    };
    auto fold = [&]() {
      if constexpr (FP8) {
#pragma unroll
        for (int i = 0; i < NLIVE; ++i)
#pragma unroll
          for (int j = 0; j < CB; ++j) {
            const float s = sa_c[i] * sw_c[j];
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] += tmp[i][j][v] * s;
          }
      }
    };
    // Software pipeline over k-step fragment sets: the fragments of the
    // next k step are read from LDS while the MFMAs of the current one run.
    // The barrier sits before the last k step of stage kt, once this wave's
    // reads of stage kt have all completed (its last fragments are in
    // registers): it publishes stage kt+1 and frees stage kt's slot, which
    // the DMA of stage kt+STAGES then refills, STAGES-1 stages ahead of its
    // use. The last stage is peeled so the loop body has no branch around
    // LDS reads.
    wait_stages(min(STAGES - 1, KT - 1), lps);
    wave_barrier_all();
    read_frags(0, 0, fa[0], fb[0]);
    if constexpr (FP8) read_scales(0, sa_c, sw_c);
    // PREV (split refills, from the second stage on): the weight rows of
    // stage kt+1, whose slot was freed at the previous barrier
    auto body = [&](int kt, auto prev_c) {
      constexpr bool PREV = decltype(prev_c)::value;
#pragma unroll
      for (int kk = 0; kk + 1 < KK; ++kk) {
        read_frags(kt, kk + 1, fa[(kk + 1) & 1], fb[(kk + 1) & 1]);
        if constexpr (PREV) {
          if (kk == 0)
            issue_part(kt + 1, (kt + 1) % STAGES, std::integral_constant<int, 1>{}, aon);
        }
        mma(kk, fa[kk & 1], fb[kk & 1]);
        if (PREV && kk == 0) sched_step_dma();
        else sched_step();
        __builtin_amdgcn_sched_barrier(0);
      }
      wait_lgkm0();
      wait_stages(min(STAGES - 2, KT - 2 - kt), lps);
      wave_barrier_all();
      if (kt + STAGES < KT) {
        if constexpr (SPLIT)
          issue_part(kt + STAGES, kt % STAGES, std::integral_constant<int, 0>{}, aon);
        else
          issue(kt + STAGES, kt % STAGES, aon);
      }
      read_frags(kt + 1, 0, fa[KK & 1], fb[KK & 1]);
      if constexpr (FP8) read_scales(kt + 1, sa_n, sw_n);
      mma(KK - 1, fa[(KK - 1) & 1], fb[(KK - 1) & 1]);
      if constexpr (FP8) {
        fold();
#pragma unroll
        for (int i = 0; i < RB; ++i) sa_c[i] = sa_n[i];
#pragma unroll
        for (int j = 0; j < CB; ++j) sw_c[j] = sw_n[j];
      }
      if constexpr (KK & 1) {
        // odd KK: the next stage's first fragments landed in set 1; move
        // them to set 0 where the next iteration expects them
#pragma unroll
        for (int i = 0; i < RB; ++i) fa[0][i] = fa[1][i];
#pragma unroll
        for (int j = 0; j < CB; ++j) fb[0][j] = fb[1][j];
      }
    };
    if constexpr (SPLIT) {
      // stages 0 and 1 were loaded whole; from stage 1 on each stage
      // finishes the refill begun at the previous barrier
      if (KT > 1) body(0, std::false_type{});
      for (int kt = 1; kt + 1 < KT; ++kt) body(kt, std::true_type{});
    } else {
      for (int kt = 0; kt + 1 < KT; ++kt) body(kt, std::false_type{});
    }
#pragma unroll
    for (int kk = 0; kk + 1 < KK; ++kk) {
      read_frags(KT - 1, kk + 1, fa[(kk + 1) & 1], fb[(kk + 1) & 1]);
      mma(kk, fa[kk & 1], fb[kk & 1]);
    }
    mma(KK - 1, fa[(KK - 1) & 1], fb[(KK - 1) & 1]);
    fold();
  };
  if (a_on)
    dispatch_count<RB>(nlive, [&](auto n) { main_loop(n, std::true_type{}); });
  else
    dispatch_count<RB>(nlive, [&](auto n) { main_loop(n, std::false_type{}); });

  // ---- epilogue: lane owns token row (lane & 31) of each 32-row block and,
  // in each 32-column block, columns 8*q + 4*(lane>>5) + {0..3}, q = 0..3
  // (accumulator registers 4q..4q+3). int8 dequantises here:
  // float(acc) * a_scale[row] * w_scale[channel].
  uint16_t* out = static_cast<uint16_t*>(p.out);
  const int csub = 4 * (lane >> 5);
  const int half = lane >> 5;
  const float* wsc = INT8 ? p.w_scale + wbase : nullptr;
  auto wscale4 = [&](int64_t wrow) -> f32x4 {
    if constexpr (INT8) return *reinterpret_cast<const f32x4*>(wsc + wrow);
    else return f32x4{1.f, 1.f, 1.f, 1.f};
  };
  auto value = [&](const Acc& a, int v, float sa, float sw) -> float {
    if constexpr (INT8) return static_cast<float>(a[v]) * sa * sw;
    else return a[v];
  };
  // per-expert fp32 bias (the bias variant); GEMM2 split-K adds it once
  const float* bias = p.bias && (GEMM1 || ks == 0) ? p.bias + wbase : nullptr;
  auto bias4 = [&](int64_t col) -> f32x4 {
    return bias ? *reinterpret_cast<const f32x4*>(bias + col) : f32x4{0.f, 0.f, 0.f, 0.f};
  };
  // A store straight from the accumulator layout touches 32 output rows per
  // instruction; the silu GEMM1 and the GEMM2 outputs instead go through
  // this wave's share of a free stage slot (stage KT-2's: no wave reads it
  // again and no refill targets it; with a single stage, after a barrier)
  // in passes of 32 rows x JP column blocks, and leave as whole row
  // segments, 16 bytes per lane. Chunks (16 bytes) of a staged row are
  // XOR-swizzled by the row so the column-major writes spread over the
  // banks.
  constexpr int REGION = (STAGE / NW) & ~15;
  const int fslot = KT >= 2 ? (KT - 2) % STAGES : 0;
  if (KT < 2) wave_barrier_all();
  uint8_t* stg = lds + fslot * STAGE + wave * REGION;
  // orders this wave's staging writes before its reads (and the reads
  // before the next pass's writes)
  auto stage_sync = [] {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  // staged bytes of lane row r, chunk c (CH chunks per row)
  auto slot_at = [&](auto ch_c, int r, int c) -> uint8_t* {
    constexpr int CH = decltype(ch_c)::value;
    return stg + r * (CH * 16) + ((c ^ (r % CH)) * 16);
  };
  // writes the staged 32 x CH-chunk block: staged row sr goes to dst(sr)
  // (a byte address; null: not stored)
  // (passes in groups of four: their staged values and row addresses --
  // a lane shuffle each -- are read before their stores, so a group costs
  // one LDS round trip instead of two per pass)
  auto drain = [&](auto ch_c, auto&& dst) {
    constexpr int CH = decltype(ch_c)::value;
    constexpr int NP = 32 / (64 / CH);
    constexpr int G = NP < 4 ? NP : 4;
    static_assert(NP % G == 0, "passes in whole groups");
    stage_sync();
#pragma unroll
    for (int k0 = 0; k0 < NP; k0 += G) {
      uint4 val[G];
      uint8_t* d[G];
#pragma unroll
      for (int kq = 0; kq < G; ++kq) {
        const int sr = (k0 + kq) * (64 / CH) + lane / CH;
        const int c = lane % CH;
        val[kq] = *reinterpret_cast<const uint4*>(slot_at(ch_c, sr, c));
        d[kq] = dst(sr);
      }
#pragma unroll
      for (int kq = 0; kq < G; ++kq) {
        const int c = lane % CH;
        if (d[kq]) *reinterpret_cast<uint4*>(d[kq] + c * 16) = val[kq];
      }
    }
    stage_sync();
  };
  // column blocks per pass for `ob`-byte outputs over `cb` column blocks
  constexpr auto pass_blocks = [](int ob, int cb) {
    int jp = cb;
    while (jp > 1 && 32 * jp * 32 * ob > REGION) jp /= 2;
    return jp;
  };
  // Every load of the epilogue is issued before its first store: the vector
  // memory counter counts stores too, so a load issued after one 32-row
  // block's stores would wait for them to complete. Per block: the token
  // slot of this lane's row, its int8 activation scale and (GEMM1 with
  // weight_on_input) its router weight; per column: the int8 weight scales
  // and the bias, loaded once for all blocks.
  int esid[RB];
  float esa[RB], egam[RB];
#pragma unroll
  for (int i = 0; i < RB; ++i) esid[i] = p.sorted_ids[row0 + wm * WROWS + i * 32 + (lane & 31)];
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    const int rr = wm * WROWS + i * 32 + (lane & 31);
    const bool ok = esid[i] < p.numel;
    esa[i] = INT8 ? p.a_scale[act_of(rr, esid[i])] : 1.f;
    egam[i] = GEMM1 && p.weight_on_input && ok ? p.topk_w[esid[i]] : 1.f;
  }
  // Column values of column block j, group g4 (one f32x4 each, gate and
  // up for GEMM1): int8 weight scales (else ones) and bias (else zeros),
  // held in registers when they fit in 32 VGPRs, else loaded where used.
  constexpr int CBS = GEMM1 ? CB / 2 : CB;
  constexpr bool HOIST = CBS * (GEMM1 ? 2 : 1) <= 2;
  struct Cols {
    f32x4 g[HOIST ? CBS : 1][4], u[HOIST && GEMM1 ? CBS : 1][4];
  };
  const f32x4 ones = {1.f, 1.f, 1.f, 1.f}, zeros = {0.f, 0.f, 0.f, 0.f};
  auto load_cols = [&](Cols& c, auto load4, int64_t col_base) {
    if constexpr (HOIST) {
#pragma unroll
      for (int j = 0; j < CBS; ++j)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int64_t col = col_base + j * 32 + csub + 8 * g4;
          c.g[j][g4] = load4(col);
          if constexpr (GEMM1) c.u[j][g4] = load4(p.n_out + col);
        }
    }
  };
  // value of column block j, group g4 (gate; up when `up`)
  auto col_of = [&](const Cols& c, auto load4, int64_t col_base, int j, int g4,
                    bool up) -> f32x4 {
    if constexpr (HOIST) {
      if constexpr (GEMM1) return up ? c.u[j][g4] : c.g[j][g4];
      else return c.g[j][g4];
    } else {
      return load4((up ? p.n_out : 0) + col_base + j * 32 + csub + 8 * g4);
    }
  };
  auto sc4 = [&](int64_t col) -> f32x4 { return wscale4(col); };
  auto no_sc4 = [&](int64_t) -> f32x4 { return ones; };
  auto b4 = [&](int64_t col) -> f32x4 { return bias4(col); };
  auto no_b4 = [&](int64_t) -> f32x4 { return zeros; };
  // GEMM1 with silu and no bias (the common case): the router-weight
  // scaling as a compile-time branch, no bias adds, pairwise conversions
  if constexpr (GEMM1) {
    if (p.act == kActSilu && bias == nullptr) {
      constexpr int JP = pass_blocks(2, CB / 2);
      constexpr std::integral_constant<int, JP * 4> ch{};
      static_assert(32 * JP * 32 * 2 <= REGION, "staging fits");
      const int col_base = tile_n * (BNR / 2) + wn * (WCOLS / 2);
      Cols sc;
      if constexpr (INT8) load_cols(sc, sc4, col_base);
      auto scale_at = [&](int j, int g4, bool up) -> f32x4 {
        if constexpr (INT8) return col_of(sc, sc4, col_base, j, g4, up);
        else return no_sc4(0);
      };
      auto emit = [&](auto scale_c) {
        constexpr bool SCALE = decltype(scale_c)::value;
#pragma unroll
        for (int i = 0; i < RB; ++i) {
          if (i >= nlive) break;  // all-pad blocks (wave-uniform)
          const int sid = esid[i];
          const float sa = esa[i];
          const float gamma = egam[i];
          const int r = lane & 31;
#pragma unroll
          for (int jp0 = 0; jp0 < CB / 2; jp0 += JP) {
#pragma unroll
            for (int jl = 0; jl < JP; ++jl) {
              const int jb = jp0 + jl;
#pragma unroll
              for (int g4 = 0; g4 < 4; ++g4) {
                const f32x4 sg = scale_at(jb, g4, false);
                const f32x4 su = scale_at(jb, g4, true);
                const Acc& ag = acc[i][jb];
                const Acc& au = acc[i][jb + CB / 2];
                const int v = 4 * g4;
                uint2 v2;
                v2.x = silu_mul_bf16x2<SCALE>(
                    value(ag, v, sa, sg[0]), value(ag, v + 1, sa, sg[1]),
                    value(au, v, sa, su[0]), value(au, v + 1, sa, su[1]), gamma);
                v2.y = silu_mul_bf16x2<SCALE>(
                    value(ag, v + 2, sa, sg[2]), value(ag, v + 3, sa, sg[3]),
                    value(au, v + 2, sa, su[2]), value(au, v + 3, sa, su[3]), gamma);
                *reinterpret_cast<uint2*>(slot_at(ch, r, jl * 4 + g4) + half * 8) = v2;
              }
            }
            drain(ch, [&](int sr) -> uint8_t* {
              if (__shfl(sid, sr, 64) >= p.numel) return nullptr;
              const int64_t orow = row0 + wm * WROWS + i * 32 + sr;
              return reinterpret_cast<uint8_t*>(out + orow * p.n_out + col_base + jp0 * 32);
            });
          }
        }
      };
      if (p.weight_on_input) emit(std::true_type{});
      else emit(std::false_type{});
      return;
    }
    // other activations and the bias variant: stores straight from the
    // accumulator layout
    const int col_base = tile_n * (BNR / 2) + wn * (WCOLS / 2);
    auto emit = [&](auto bias_c) {
      constexpr bool BIAS = decltype(bias_c)::value;
      Cols sc, bs;
      if constexpr (INT8) load_cols(sc, sc4, col_base);
      if constexpr (BIAS) load_cols(bs, b4, col_base);
      auto scale_at = [&](int j, int g4, bool up) -> f32x4 {
        if constexpr (INT8) return col_of(sc, sc4, col_base, j, g4, up);
        else return no_sc4(0);
      };
      auto bias_at = [&](int j, int g4, bool up) -> f32x4 {
        if constexpr (BIAS) return col_of(bs, b4, col_base, j, g4, up);
        else return no_b4(0);
      };
      const bool scale = p.weight_on_input != 0;
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int r = row0 + wm * WROWS + i * 32 + (lane & 31);
        if (esid[i] >= p.numel) continue;  // pad rows: never stored
        const float sa = esa[i];
        const float gamma = egam[i];
        uint16_t* orow = out + static_cast<int64_t>(r) * p.n_out;
#pragma unroll
        for (int jb = 0; jb < CB / 2; ++jb) {
          const int col0 = col_base + jb * 32 + csub;
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const f32x4 sg = scale_at(jb, g4, false);
            const f32x4 su = scale_at(jb, g4, true);
            const f32x4 bg = bias_at(jb, g4, false);
            const f32x4 bu = bias_at(jb, g4, true);
            uint32_t w0 = 0, w1 = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const uint32_t b = gemm1_epilogue(
                  value(acc[i][jb], 4 * g4 + t, sa, sg[t]) + bg[t],
                  value(acc[i][jb + CB / 2], 4 * g4 + t, sa, su[t]) + bu[t], scale,
                  gamma, p.act, p.alpha, p.limit);
              if (t < 2) w0 |= b << (16 * t);
              else w1 |= b << (16 * (t - 2));
            }
            uint2 v2;
            v2.x = w0;
            v2.y = w1;
            *reinterpret_cast<uint2*>(orow + col0 + 8 * g4) = v2;
          }
        }
      }
    };
    if (bias) emit(std::true_type{});
    else emit(std::false_type{});
  } else {
    const int col_base = tile_n * BNR + wn * WCOLS;
    auto emit = [&](auto bias_c) {
      constexpr bool BIAS = decltype(bias_c)::value;
      Cols sc, bs;
      if constexpr (INT8) load_cols(sc, sc4, col_base);
      if constexpr (BIAS) load_cols(bs, b4, col_base);
      auto scale_at = [&](int j, int g4) -> f32x4 {
        if constexpr (INT8) return col_of(sc, sc4, col_base, j, g4, false);
        else return no_sc4(0);
      };
      auto bias_at = [&](int j, int g4) -> f32x4 {
        if constexpr (BIAS) return col_of(bs, b4, col_base, j, g4, false);
        else return no_b4(0);
      };
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        if (i >= nlive) break;  // all-pad blocks (wave-uniform)
        const int sid = esid[i];
        const float sa = esa[i];
        const int r = lane & 31;
        if (p.ksplit > 1) {
          // fp32 partial sums of split ks, reduced in fixed order by moe_sum
          constexpr int JP = pass_blocks(4, CB);
          constexpr std::integral_constant<int, JP * 8> ch{};
          static_assert(32 * JP * 32 * 4 <= REGION, "staging fits");
#pragma unroll
          for (int jp0 = 0; jp0 < CB; jp0 += JP) {
#pragma unroll
            for (int jl = 0; jl < JP; ++jl) {
              const int j = jp0 + jl;
#pragma unroll
              for (int g4 = 0; g4 < 4; ++g4) {
                const f32x4 w = scale_at(j, g4);
                const f32x4 b = bias_at(j, g4);
                const int v = 4 * g4;
                *reinterpret_cast<f32x4*>(slot_at(ch, r, jl * 8 + g4 * 2 + half)) =
                    f32x4{value(acc[i][j], v, sa, w[0]) + b[0],
                          value(acc[i][j], v + 1, sa, w[1]) + b[1],
                          value(acc[i][j], v + 2, sa, w[2]) + b[2],
                          value(acc[i][j], v + 3, sa, w[3]) + b[3]};
              }
            }
            drain(ch, [&](int sr) -> uint8_t* {
              const int row_sid = __shfl(sid, sr, 64);
              if (row_sid >= p.numel) return nullptr;
              return reinterpret_cast<uint8_t*>(
                  static_cast<float*>(p.out) +
                  (static_cast<int64_t>(ks) * p.numel + row_sid) * p.n_out + col_base + jp0 * 32);
            });
          }
        } else {
          constexpr int JP = pass_blocks(2, CB);
          constexpr std::integral_constant<int, JP * 4> ch{};
          static_assert(32 * JP * 32 * 2 <= REGION, "staging fits");
#pragma unroll
          for (int jp0 = 0; jp0 < CB; jp0 += JP) {
#pragma unroll
            for (int jl = 0; jl < JP; ++jl) {
              const int j = jp0 + jl;
#pragma unroll
              for (int g4 = 0; g4 < 4; ++g4) {
                const f32x4 w = scale_at(j, g4);
                const f32x4 b = bias_at(j, g4);
                const int v = 4 * g4;
                // (no bias: no add, so the pair converts straight from
                // the accumulators)
                auto with_b = [&](float x, float bv) { return BIAS ? x + bv : x; };
                uint2 v2;
                v2.x = pack_bf16x2(with_b(value(acc[i][j], v, sa, w[0]), b[0]),
                                   with_b(value(acc[i][j], v + 1, sa, w[1]), b[1]));
                v2.y = pack_bf16x2(with_b(value(acc[i][j], v + 2, sa, w[2]), b[2]),
                                   with_b(value(acc[i][j], v + 3, sa, w[3]), b[3]));
                *reinterpret_cast<uint2*>(slot_at(ch, r, jl * 4 + g4) + half * 8) = v2;
              }
            }
            drain(ch, [&](int sr) -> uint8_t* {
              const int row_sid = __shfl(sid, sr, 64);
              if (row_sid >= p.numel) return nullptr;
              return reinterpret_cast<uint8_t*>(out + static_cast<int64_t>(row_sid) * p.n_out +
                                                col_base + jp0 * 32);
            });
          }
        }
      }
    };
    if (bias) emit(std::true_type{});
    else emit(std::false_type{});
  }
}

template <int DT, class C, bool GEMM1>
__global__ __launch_bounds__(C::NW * 64, 1) void moe_gemm_tiled_kernel(
    const GemmParams p) {
  constexpr int BM = C::BM, BNR = C::BNR;

  constexpr int N_PER_TILE = GEMM1 ? BNR / 2 : BNR;
  const int n_ct = static_cast<int>(p.n_out / N_PER_TILE);
  int rb_id, tile_n;
  if (!tile_of(blockIdx.x, gridDim.x, p.row_blocks * p.ksplit, n_ct, p.group_m,
               p.group_n, &rb_id, &tile_n))
    return;
  // split-K (GEMM2 only): the row-block index space repeats once per split
  const int ks = rb_id / p.row_blocks;
  rb_id -= ks * p.row_blocks;
  // Every word the early exits read, loaded together: none depends on
  // another, so one round trip instead of up to four (blocks past the
  // padded count hold -1 experts and pad slots, so the loads stay in the
  // buffers whatever the block).
  const int npp = p.num_post_pad[0];
  // row blocks smaller than the alignment block (eid_shift > 0): the expert
  // of the enclosing block; a block that is all padding has nothing to do
  const int e = p.expert_ids[rb_id >> p.eid_shift];
  const int sid_first = p.eid_shift > 0 ? p.sorted_ids[rb_id * BM] : 0;
  const int sid_bma = C::BMA < BM ? p.sorted_ids[rb_id * BM + (C::BMA < BM ? C::BMA : 0)] : 0;
  if (rb_id * BM >= npp) return;
  if (e < 0) return;
  if (p.eid_shift > 0 && sid_first >= p.numel) return;
  if constexpr (C::BMA < BM) {
    if (sid_bma >= p.numel) {
      tiled_tile<DT, C, GEMM1, true>(p, rb_id, tile_n, ks, e);
      return;
    }
  }
  tiled_tile<DT, C, GEMM1, false>(p, rb_id, tile_n, ks, e);
}

// Rasterization (FGS_MOE_GROUPM / FGS_MOE_GROUPN override; tuning aids read
// once): row blocks per band, or, with bands off (0), column tiles per group.
static int env_choice(const char* name, int dflt, int lo, int hi) {
  const char* s = tuning_env(name);
  const int v = s ? atoi(s) : dflt;
  return (v >= lo && v <= hi) ? v : dflt;
}
// Default (unset): bands of one row block -- the column tiles of a block
// run back to back, sharing its activation tile in L2 -- for 128-row
// blocks of layers with >= 64 experts (measured: DeepSeek fp8 M=512
// -4.4 %, Qwen3 M=256 -1.6 % and skewed -3.8 %, Qwen2 int8 M=64 -1.5 %;
// few experts, other row blocks and the half blocks of fp8 GEMM2 lose,
// Mixtral M=128 +14 %, DeepSeek M=32 +12 %, M=4096 +20 %), else none.
static int group_m_choice(int bm, const GemmParams& p) {
  static const int g = env_choice("FGS_MOE_GROUPM", -1, 0, 64);
  if (g >= 0) return g;
  return bm == 128 && p.num_experts >= 64 && p.eid_shift == 0 ? 1 : 0;
}
// Whether the GEMMs of the 256-row configuration run the 4-wave kernel
// (gemm_wide.hip): 1 (default) both, 0 neither (FGS_MOE_WIDE, a tuning
// aid; read once).
static int wide_choice() {
  static const int mode = env_choice("FGS_MOE_WIDE", 1, 0, 1);
  return mode;
}
static int group_n_choice() {
  static const int g = env_choice("FGS_MOE_GROUPN", 4, 1, 64);
  return g;
}

template <int DT, class C, bool GEMM1>
static int launch_tiled(const GemmParams& p, int row_blocks, hipStream_t stream) {
  auto kern = moe_gemm_tiled_kernel<DT, C, GEMM1>;
  constexpr int lds_bytes = tiled_lds_bytes<DT, C>();
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [&] {
    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
  });
  if (attr != hipSuccess)
    return fail(FGS_ELAUNCH, std::string("tiled GEMM LDS opt-in: ") +
                                 hipGetErrorString(attr));
  const int tiles_n = static_cast<int>(GEMM1 ? p.n_out / (C::BNR / 2) : p.n_out / C::BNR);
  GemmParams q = p;
  q.row_blocks = row_blocks;
  set_topk_magic(&q);
  q.group_m = group_m_choice(C::BM, p);
  q.group_n = group_n_choice();
  if (GEMM1 || q.ksplit < 1) q.ksplit = 1;
  const int tiles = (row_blocks * q.ksplit * tiles_n + 7) / 8 * 8;
  hipLaunchKernelGGL(kern, dim3(tiles), dim3(C::NW * 64), lds_bytes, stream, q);
  return check_launch("moe_gemm_tiled_kernel");
}

// Tile configurations (BM, BNR, WM, WN, SK, STAGES), one per rows-per-expert
// regime. Small row blocks keep padding low and still read every weight
// tile once per block; the 256-row tile has the highest MFMA intensity.
using Cfg256 = TileCfg<256, 256, 4, 2, 128, 2>;  // 8 waves of 64x128
using Cfg128 = TileCfg<128, 256, 2, 4, 128, 3>;  // 8 waves of 64x64
using Cfg64 = TileCfg<64, 256, 1, 4, 128, 4>;   // 4 waves of 64x64
using Cfg32 = TileCfg<32, 256, 1, 4, 128, 4>;   // 4 waves of 32x64
// 160-row blocks for ~100-150 rows per expert (a 256-row block would be
// half padding): 4 waves of 160x64, a 3-slot ring holding two stages of
// 256 weight rows in flight (the 256-row configurations hold one or two
// stages of 128 or 256)
using Cfg160 = TileCfg<160, 256, 1, 4, 128, 3>;
// fp8 keeps a second accumulator set per k block (the block-scale fold), so
// its 256-row configuration has 64x64 wave tiles over 128 weight rows, and
// the stage scale area costs a stage at 64 and 32 rows. Its blocks of at
// most 160 rows (~128 rows per expert: DeepSeek M=4096) run a 4-slot ring
// of 160 activation rows -- three stages in flight instead of two, GEMM1
// 1.90 -> 1.77 ms -- and fuller blocks the 3-slot ring of all 256 rows.
using Fp8Cfg256 = TileCfg<256, 128, 4, 2, 128, 3, 160, 4>;  // 8 waves of 64x64
using Fp8Cfg64 = TileCfg<64, 256, 1, 4, 128, 3>;
using Fp8Cfg32 = TileCfg<32, 256, 1, 4, 128, 3>;

static const int kTileRows[kTiledConfigs] = {Cfg256::BM, Cfg128::BM, Cfg64::BM,
                                             Cfg32::BM, Cfg160::BM};

// FGS_MOE_TILE (0..4) forces one configuration (a tuning aid; read once).
static int forced_tile() {
  static const int forced = [] {
    const char* s = tuning_env("FGS_MOE_TILE");
    if (!s) return -1;
    const int v = atoi(s);
    return (v >= 0 && v < kTiledConfigs) ? v : -1;
  }();
  return forced;
}

int tiled_config_supported(int dt, int cfg) {
  (void)dt;
  return cfg >= 0 && cfg < kTiledConfigs;
}

// Configuration by rows per expert and expert count (measured on the four
// model shapes, M from 32 to 8192):
// * from 112 rows, 256-row blocks: fewer would spill a noticeable share of
//   the experts into a second, mostly empty block that streams the
//   expert's weights again, and the 256-row kernels skip the MFMAs of their
//   all-pad 32-row blocks;
// * with many experts (>= 32) the 256-row configuration already wins from
//   48 rows (64 rows: Qwen3 -14 %, Qwen2 int8 -15 %, DeepSeek fp8 -10 %
//   against the 64-row kernel); with 8 experts (Mixtral) it loses there;
// * otherwise the 8-wave 128-row kernel from 24 rows (Mixtral M=256 -11 %,
//   Qwen2 M=256 -6 %, DeepSeek M=1024 -4 %), and for many experts also from
//   8 rows (Qwen2 M=64 -6 %, DeepSeek M=256/512 -3/-5 %, Qwen3 M=256 -7 %);
// * the 32-row kernel below that (Mixtral M=32/64, DeepSeek M=32);
// * bf16 with few experts takes the 256-row configuration from 96 rows
//   (Mixtral M=384 -1.5 %, 448 -4 %, 512 -3.5 %, 576 -10 %, 640 -3.5 %
//   against the 160-row kernel that had those rows; M=256, 64 rows, stays
//   on the 128-row kernel: +5 % on 256-row blocks).
// The 64- and 160-row configurations are no longer chosen; they stay for
// FGS_MOE_TILE.
int tiled_config_for(int dt, double rows_per_expert, int num_experts) {
  const bool many = num_experts >= 32;
  int c = 3;
  if (rows_per_expert >= 112 || (many && rows_per_expert >= 48) ||
      (dt == kDtBf16 && rows_per_expert >= 96))
    c = 0;
  else if (rows_per_expert >= 24 || (many && rows_per_expert >= 8)) c = 1;
  if (forced_tile() >= 0) c = forced_tile();
  return c;
}

int tiled_block_m(int cfg) { return kTileRows[cfg]; }

// n_out granularity the tiled kernels need: GEMM1 output cols per tile,
// GEMM2 output cols per tile (every configuration uses BNR = 256).
int tiled_n_align(bool gemm1) { return gemm1 ? 128 : 256; }

template <int DT, class C>
static int launch_cfg(bool gemm1, const GemmParams& p, int row_blocks,
                      hipStream_t stream) {
  return gemm1 ? launch_tiled<DT, C, true>(p, row_blocks, stream)
               : launch_tiled<DT, C, false>(p, row_blocks, stream);
}

void tiled_plan_request(int dt, int cfg, bool gemm1, const GemmParams& p, int row_blocks,
                        WidePlanReq* req) {
  *req = WidePlanReq{};
  if (tiled_config_supported(dt, cfg) && row_blocks > 0 && cfg == 0 && wide_choice() >= 1 &&
      wide_supported(dt, gemm1, p))
    wide_plan_request(gemm1, p, row_blocks, req);
}

int launch_gemm_tiled(int dt, int cfg, bool gemm1, const GemmParams& p,
                      int row_blocks, hipStream_t stream) {
  if (!tiled_config_supported(dt, cfg))
    return fail(FGS_EINVAL, "tiled GEMM: configuration " + std::to_string(cfg) +
                                " not available for this element type");
  if (row_blocks <= 0) return FGS_OK;
  // The 4-wave kernel runs both GEMMs of the 256-row configuration: with
  // its weight rows a stage ahead it also wins on the long GEMM2
  // contraction it used to leave to the 8-wave kernel (Mixtral, 28 KiB k
  // rows: M=512 with a k split GEMM2 0.192 -> 0.181 ms against the 160-row
  // kernel, 0.210 against the 8-wave 256-row one; M=16384 3.35 -> 3.16 ms).
  if (cfg == 0 && wide_choice() >= 1 && wide_supported(dt, gemm1, p))
    return launch_gemm_wide(dt, gemm1, p, row_blocks, stream);
  switch (dt) {
    case kDtBf16:
      switch (cfg) {
        case 0: return launch_cfg<kDtBf16, Cfg256>(gemm1, p, row_blocks, stream);
        case 1: return launch_cfg<kDtBf16, Cfg128>(gemm1, p, row_blocks, stream);
        case 2: return launch_cfg<kDtBf16, Cfg64>(gemm1, p, row_blocks, stream);
        case 4: return launch_cfg<kDtBf16, Cfg160>(gemm1, p, row_blocks, stream);
        default: return launch_cfg<kDtBf16, Cfg32>(gemm1, p, row_blocks, stream);
      }
    case kDtInt8:
      switch (cfg) {
        case 0: return launch_cfg<kDtInt8, Cfg256>(gemm1, p, row_blocks, stream);
        case 1: return launch_cfg<kDtInt8, Cfg128>(gemm1, p, row_blocks, stream);
        case 2: return launch_cfg<kDtInt8, Cfg64>(gemm1, p, row_blocks, stream);
        case 4: return launch_cfg<kDtInt8, Cfg160>(gemm1, p, row_blocks, stream);
        default: return launch_cfg<kDtInt8, Cfg32>(gemm1, p, row_blocks, stream);
      }
    case kDtFp8:
      switch (cfg) {
        case 0: return launch_cfg<kDtFp8, Fp8Cfg256>(gemm1, p, row_blocks, stream);
        case 1: return launch_cfg<kDtFp8, Cfg128>(gemm1, p, row_blocks, stream);
        case 2: return launch_cfg<kDtFp8, Fp8Cfg64>(gemm1, p, row_blocks, stream);
        case 4: return launch_cfg<kDtFp8, Cfg160>(gemm1, p, row_blocks, stream);
        default: return launch_cfg<kDtFp8, Fp8Cfg32>(gemm1, p, row_blocks, stream);
      }
  }
  return fail(FGS_EINVAL, "tiled GEMM: unknown element type");
}

}  // namespace fgs
