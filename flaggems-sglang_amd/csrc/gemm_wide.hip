// 4-wave grouped GEMM for the prefill regime (bf16, int8).
//
// Same contraction, row order and epilogues as moe_gemm_tiled_kernel
// (gemm_tiled.hip) on 256-row blocks, organised for one wave per SIMD:
//
// * a tile is 256 padded rows x 256 weight rows; wave (wm, wn) of the 2x2
//   grid computes 128 rows x 128 weight rows with 16 accumulators of
//   v_mfma_f32_32x32x16_bf16 / v_mfma_i32_32x32x32_i8 (256 AGPRs), so each
//   k step reads 8 fragments from LDS for 16 MFMAs (the 8-wave 64x128 layout
//   reads 6 for 8). Its rows are the 32-row blocks wm, wm+2, wm+4, wm+6:
//   the pad rows of a partial block (a suffix) then fall evenly on both
//   row halves, i.e. on all four SIMDs, whose all-pad blocks skip their
//   MFMAs;
// * operand tiles stream through an LDS ring of SK-byte k stages -- NS
//   activation slots, then NSB weight slots -- filled by buffer_load ... lds:
//   one buffer resource per operand (the weight resource starts at the
//   tile's expert), 32-bit row offsets per lane and the k offset in the
//   scalar offset, so a stage costs no address arithmetic. One operand has
//   three slots and goes out two stages ahead, during the first k step of
//   stage s; the other has two and goes out after stage s's barrier, each
//   load between two MFMAs (the weight rows early, or for GEMM2 on large
//   row counts the activation rows);
// * tiles are ordered for the L2 of each XCD: the live tiles are cut into 8
//   row-block-major ranges, one per XCD (about one expert in eight each),
//   walked in column groups.
#include <stdlib.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <type_traits>

#include "gemm_tiled_common.h"
#include "wide_plan.h"

namespace fgs {

template <int SK_, int NS_, int NSB_>
struct WideCfg {
  static constexpr int BM = 256;              // rows per tile (= alignment block)
  static constexpr int BNR = 256;             // weight rows per tile
  static constexpr int NW = 4;                // waves: 2 row halves x 2 weight-row halves
  static constexpr int WROWS = 128;           // rows per wave (4 interleaved 32-row blocks)
  static constexpr int WCOLS = 128;           // weight rows per wave
  static constexpr int RB = WROWS / 32;       // 32-row MFMA blocks per wave
  static constexpr int CB = WCOLS / 32;       // 32-col MFMA blocks per wave
  static constexpr int SK = SK_;              // k bytes per stage row
  static constexpr int NS = NS_;              // activation ring slots
  static constexpr int NSB = NSB_;            // weight ring slots
  static constexpr int KK = SK / 32;          // MFMA k steps per stage (32 bytes each)
  static constexpr int CPR = SK / 16;         // 16-byte chunks per stage row
  static constexpr int LR = 64 / CPR;         // rows one wave load (1 KiB) covers
  static constexpr int RPL = 256 / SK;        // stage rows per 256-byte bank line
  static constexpr int NLA = BM / (LR * NW);  // loads per wave per stage
  static constexpr int NLB = BNR / (LR * NW);
  static constexpr int NL = NLA + NLB;
  static constexpr int SLOT = BM * SK;        // bytes per operand slot
  static constexpr int B_OFF = NS * SLOT;     // the weight slots follow the activation slots
  // the operand with three slots is issued a stage earlier than the other
  static constexpr bool EARLY_A = NS > NSB;
  // a 2 KiB table per wave of what the epilogue reads (column scales /
  // bias, and per row the token slot and scales), in a slot of the
  // two-slot ring the last stage does not use
  static constexpr int TAB_BYTES = 2048;
  static constexpr int LDS_BYTES = (NS + NSB) * SLOT;
  static_assert(BM == BNR, "one slot size for both operands");
  static_assert(KK % 2 == 0, "fragment double buffer wraps at a stage boundary");
  static_assert((NS == 2 && NSB == 3) || (NS == 3 && NSB == 2),
                "the refill schedule: one operand a stage ahead");
  static_assert(NW * TAB_BYTES <= SLOT, "the epilogue table fits a slot");
  static_assert(LDS_BYTES <= 160 * 1024, "gfx950 LDS is 160 KiB");
};
using WideRing = WideCfg<128, 2, 3>;   // weight rows early
using WideRingA = WideCfg<128, 3, 2>;  // activation rows early

// Position of logical 16-byte chunk c of stage row r: RPL rows share a
// 256-byte bank line, and the XOR gives the 16 rows a fragment read serves
// at once 16 distinct bank positions.
template <class C>
__device__ __forceinline__ int wide_chunk(int r, int c) {
  return c ^ ((r / C::RPL) % C::CPR);
}

// One wave-wide buffer load into LDS: lane l copies 16 bytes from
// rsrc + voff + soff to byte 16*l of the 1 KiB block at `lds_dst` (uniform).
__device__ __forceinline__ void lds_dma16_buf(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff,
                                              int soff, void* lds_dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      rsrc, (__attribute__((address_space(3))) void*)(lds_dst), 16, voff, soff, 0, 0);
}

// gfx9 buffer resource word 3 for raw 32-bit loads.
constexpr int kBufWord3 = 0x00020000;

// The d-th tile (0-based) of an XCD's range [lo, hi) of the row-block-major
// tile numbering (tile = rball * n_ct + ct), walked over groups of gn
// columns, then row blocks, then the columns of the group: the first and
// last row blocks of a range may hold only some columns, every other row
// block all columns of each group.
__device__ __forceinline__ bool wide_walk(int lo, int hi, int n_ct, int gn, int d, int* rball,
                                          int* ct) {
  if (d < 0 || lo >= hi) return false;
  const int rb_lo = lo / n_ct, rb_hi = (hi - 1) / n_ct;
  const int c_first = lo - rb_lo * n_ct;  // first column of rb_lo in the range
  const int c_last = hi - 1 - rb_hi * n_ct;  // last column of rb_hi in the range
  for (int g0 = 0; g0 < n_ct; g0 += gn) {
    const int g1 = min(n_ct, g0 + gn);
    if (rb_lo == rb_hi) {
      const int a = max(g0, c_first), n = max(0, min(g1, c_last + 1) - a);
      if (d < n) {
        *rball = rb_lo;
        *ct = a + d;
        return true;
      }
      d -= n;
      continue;
    }
    const int a = max(g0, c_first), n0 = max(0, g1 - a);
    if (d < n0) {
      *rball = rb_lo;
      *ct = a + d;
      return true;
    }
    d -= n0;
    const int gs = g1 - g0, ni = (rb_hi - rb_lo - 1) * gs;
    if (d < ni) {
      *rball = rb_lo + 1 + d / gs;
      *ct = g0 + d % gs;
      return true;
    }
    d -= ni;
    const int n1 = max(0, min(g1, c_last + 1) - g0);
    if (d < n1) {
      *rball = rb_hi;
      *ct = g0 + d;
      return true;
    }
    d -= n1;
  }
  return false;
}

// Tail split of an XCD's walk (GEMM2, p.tail_split): its T tiles run as R =
// T / 32 full rounds on the XCD's 32 CUs; the rem = T % 32 tiles of the last
// round are each split over k into S = min(8, 32 / rem) pieces, so the last
// round holds rem * S pieces instead of rem whole tiles. Piece i of tail
// tile t writes fp32 partial sums to tail_part slot (xcd * 32 + t * S + i);
// moe_wide_tail_fixup_kernel adds a tile's pieces in order. S = 1 (no
// split) when rem is 0 or above 16; a piece keeps >= 2 stages of k (the
// two stages the prologue loads), so S <= KT_all / 2.
constexpr int kWideMaxPieces = 8;
struct WideTail {
  int T, R, rem, S;
};
__device__ __forceinline__ WideTail wide_tail(int lo, int hi, bool on, int kt_all) {
  WideTail w;
  w.T = hi - lo;
  w.R = w.T / 32;
  w.rem = w.T - 32 * w.R;
  w.S = on && w.rem > 0 ? max(1, min(min(kWideMaxPieces, 32 / w.rem), kt_all / 2)) : 1;
  return w;
}
constexpr int kWideTailSlots = 8 * 32;  // tail_part slots: 32 per XCD

// ---- tile plan. Workgroup b runs on XCD b % 8 and takes position b / 8
// of its XCD's tile range, walked in column groups (wide_walk). Tiles of a
// row block whose rows are mostly padding (an expert's last few rows) cost
// a fraction of a full tile -- measured per tile with in-kernel timestamps,
// Mixtral M=4096 GEMM1: 84 vs 117 us, GEMM2: 308-324 vs 361-386 us -- and
// with few row blocks (about one expert per XCD) the even split by count
// gave whole XCDs those cheap tiles: their CUs went idle for the last ~8 %
// of GEMM1 while the other XCDs finished full tiles. The plan, made before
// the GEMM:
//  * costs each row block at base + ceil(live / 2), live = the live 32-row
//    blocks of its first wave row (1..4);
//  * cuts the row-block-major tile sequence into 8 contiguous ranges of
//    equal cost (contiguous, so an XCD still holds about one expert in
//    eight), or of equal count when an equal-cost range would hold more
//    tiles than the launch has positions for.
// The alignment writes both GEMMs' plans from its per-expert counts when it
// runs in the same call (wide_plan.h); otherwise wide_plan_kernel writes a
// GEMM's plan from the padded order, ahead of it.
// plan[0..8]: the ranges' bounds in tile index (plan[0] = -1: no plan);
// then one claim counter per XCD, each in its own 256-byte slot. The XCDs'
// tiles still take different times (per XCD, full tiles averaged 113-121
// us in one measurement), so in GEMM1 the last kPlanClaimTail positions of
// each range are claimed instead of fixed: a workgroup at such a position
// takes the next unclaimed one from its XCD's counter (relaxed
// device-scope atomics), and once its own tail is used up it tries one
// other XCD's tail and otherwise exits. The launch gives every XCD
// positions beyond its range, so an XCD that finishes early takes over
// tiles of slower ones; every XCD's own workgroups still cover its whole
// range. Every workgroup either takes a tile or exits, and a tile computes
// the same whichever CU runs it. (Claiming every position, with the
// counters in one cache line, made GEMM1 45 % slower: the atomics
// serialise.) GEMM2 balances its last round by the tail split instead.
// Measured (Mixtral M=4096, same box, alternating runs): GEMM1 1.729 ->
// 1.680 ms (layer 2.678 -> 2.633 ms) with the plan and the claimed tails.
// Listing each XCD's full row blocks before its light ones was slower
// everywhere (a light tile then no longer reads its weight tiles while its
// expert's full tiles have them in L2), and with hundreds of row blocks
// (Qwen3 / Qwen2 at M=8192: the cheap tiles are spread over every XCD) a
// plan with claimed tails was slower (Qwen3 M=2048 GEMM1 +27 %, Qwen2 int8
// M=1024 +15 %), so only launches of at most kPlanMaxRows row blocks get
// one.
// The plan from the padded order (calls whose alignment did not write it):
// one wave, lane r costs row block r from its 32-row groups' first slots.
__global__ __launch_bounds__(kWave) void wide_plan_kernel(
    const int32_t* __restrict__ sorted_ids, const int32_t* __restrict__ num_post_pad, int numel,
    int bm, int n_ct, int cap, int base, int32_t* __restrict__ plan) {
  const int lane = threadIdx.x;
  const int rows = num_post_pad[0] / bm;
  int c = 0;
  if (rows <= kPlanMaxRows && lane < rows) {
    int sid[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) sid[j] = 32 * j < bm ? sorted_ids[lane * bm + 32 * j] : numel;
    int lb = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) lb += sid[j] < numel ? 1 : 0;
    c = wide_plan_cost(32 * lb, base);
  }
  wide_plan_write(lane, rows, c, n_ct, cap, plan);
}

int64_t wide_plan_words() { return kPlanWords + 8 * kPlanClaimStride; }

// An XCD's range [lo, hi) of the row-block-major tile index: the plan's
// (GEMM1 with few row blocks), else an even split by count.
struct WideRange {
  int lo, hi;
  bool claims;  // positions are claimed from the plan's counters
};
__device__ __forceinline__ WideRange wide_range(const GemmParams& p, int total, int xcd) {
  WideRange w;
  w.claims = false;
  if (p.plan) {
    // the three words load together (one round trip): the plan always holds
    // all nine bounds, valid or not
    const int first = __builtin_amdgcn_readfirstlane(p.plan[0]);
    const int lo = __builtin_amdgcn_readfirstlane(p.plan[xcd]);
    const int hi = __builtin_amdgcn_readfirstlane(p.plan[xcd + 1]);
    if (first >= 0) {
      w.lo = lo;
      w.hi = hi;
      w.claims = true;
      return w;
    }
  }
  w.lo = static_cast<int>(static_cast<int64_t>(total) * xcd / 8);
  w.hi = static_cast<int>(static_cast<int64_t>(total) * (xcd + 1) / 8);
  return w;
}

template <int DT, bool GEMM1, class C>
__global__ __launch_bounds__(C::NW * 64, 1) void moe_gemm_wide_kernel(const GemmParams p) {
  using T = TiledType<DT>;
  using Frag = typename T::Frag;
  using Acc = typename T::Acc;
  constexpr bool INT8 = DT == kDtInt8;
  constexpr int ESZ = T::ESZ;
  constexpr int BM = C::BM, BNR = C::BNR, WCOLS = C::WCOLS;
  constexpr int RB = C::RB, CB = C::CB, SK = C::SK, NS = C::NS, NSB = C::NSB, KK = C::KK;
  constexpr int NLA = C::NLA, NLB = C::NLB, NL = C::NL, SLOT = C::SLOT, B_OFF = C::B_OFF;
  static_assert(T::FC == 1, "one LDS chunk per fragment");

  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / 2;
  const int wn = wave % 2;
  const int64_t row_bytes = p.kdim * ESZ;
  const int npp = __builtin_amdgcn_readfirstlane(p.num_post_pad[0]);
  constexpr int N_PER_TILE = GEMM1 ? BNR / 2 : BNR;
  const int n_ct = static_cast<int>(p.n_out / N_PER_TILE);
  const int KT_all = static_cast<int>(row_bytes / SK);

  // ---- tile walk. The live tiles -- row blocks below
  // num_tokens_post_padded (times the k splits) x column tiles -- are
  // numbered row-block-major and cut into 8 equal contiguous ranges, one per
  // XCD (workgroup b runs on XCD b % 8): an XCD works on about 1/8 of the
  // row blocks, i.e. a few experts, across all columns, so each weight tile
  // is fetched into its L2 once for all the row blocks of its expert. Inside
  // a range, positions run over groups of group_n columns, then row blocks,
  // then the columns of the group. Workgroup b takes position b / 8 of its
  // XCD's walk (the hardware hands out workgroups in order as CUs free up),
  // so the tiles in flight at once share weight and activation tiles.
  const int rb_live = npp / BM;
  const int rows_all = rb_live * p.ksplit;  // row-block index space over splits
  const int total = rows_all * n_ct;
  const int xcd = blockIdx.x % 8;
  const WideRange range = wide_range(p, total, xcd);
  const WideTail tail = wide_tail(range.lo, range.hi, !GEMM1 && p.tail_split, KT_all);

  struct Tile {
    int rb, ct, e, kt0, KT, ks;
    int slot;  // tail piece: its tail_part slot; whole tile: -1
  };
  // Workgroup position pos of the XCD: a whole tile of the walk, or (tail
  // split) a k piece of one of the last round's tiles.
  auto live_tile = [&](const WideRange& rg, int pos, Tile& t) -> bool {
    int d = pos, piece = -1;
    if (tail.S > 1 && pos >= 32 * tail.R) {
      const int q = pos - 32 * tail.R;
      if (q >= tail.rem * tail.S) return false;
      d = 32 * tail.R + q / tail.S;
      piece = q % tail.S;
    }
    if (d >= rg.hi - rg.lo) return false;  // (the owner's range: a claim may be another XCD's)
    int rball, ct;
    if (!wide_walk(rg.lo, rg.hi, n_ct, p.group_n, d, &rball, &ct)) return false;
    t.ct = ct;
    t.ks = rball / rb_live;
    t.rb = rball - t.ks * rb_live;
    if (piece >= 0) {
      t.kt0 = piece * KT_all / tail.S;
      t.KT = (piece + 1) * KT_all / tail.S - t.kt0;
      t.slot = xcd * 32 + (d - 32 * tail.R) * tail.S + piece;
      t.ks = piece;  // the bias goes into piece 0's partial
    } else {
      t.kt0 = t.ks * KT_all / p.ksplit;
      t.KT = (t.ks + 1) * KT_all / p.ksplit - t.kt0;
      t.slot = -1;
    }
    return true;
  };

  // ---- per-tile DMA sources: the expert and this lane's row offsets
  struct Src {
    int e;  // expert of the weight rows
    uint32_t va[NLA], vb[NLB];
  };
  const int lrow = lane / C::CPR;   // row of a load this lane copies
  const int lchunk = lane % C::CPR;  // its physical chunk
  auto make_src = [&](const Tile& t, Src& s) {
    const int row0 = t.rb * BM;
    // all token slots first: computing a row (GEMM1 divides by topk for
    // real rows only) compiles to a branch, which would otherwise hold each
    // load back until the previous row is done
    int sid[NLA];
#pragma unroll
    for (int i = 0; i < NLA; ++i) sid[i] = p.sorted_ids[row0 + (wave * NLA + i) * C::LR + lrow];
#pragma unroll
    for (int i = 0; i < NLA; ++i) {
      const int r = (wave * NLA + i) * C::LR + lrow;
      const bool ok = sid[i] < p.numel;
      const int64_t arow = GEMM1 ? (ok ? div_topk(p, sid[i]) : 0) : row0 + (ok ? r : 0);
      s.va[i] = static_cast<uint32_t>(arow * row_bytes + wide_chunk<C>(r, lchunk) * 16);
    }
#pragma unroll
    for (int i = 0; i < NLB; ++i) {
      const int j = (wave * NLB + i) * C::LR + lrow;  // tile row
      int64_t wrow;
      if constexpr (GEMM1) {
        // wave column wc's tile rows: WCOLS/2 gate rows, then the same
        // output columns' up rows
        constexpr int HALF = WCOLS / 2;
        const int wc = j / WCOLS;
        const int in = j % WCOLS;
        wrow = (in >= HALF ? p.n_out : 0) + t.ct * (BNR / 2) + wc * HALF + in % HALF;
      } else {
        wrow = static_cast<int64_t>(t.ct) * BNR + j;
      }
      s.vb[i] = static_cast<uint32_t>(wrow * row_bytes + wide_chunk<C>(j, lchunk) * 16);
    }
  };
  // Buffer resources are built from scalars at each issue (the operands'
  // sources change between tiles), so they stay in SGPRs.
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(p.a), 0, static_cast<int>(p.a_rows * row_bytes), kBufWord3);
  const int w_bytes = static_cast<int>(p.nrows_w * row_bytes);
  // Loads of one stage (k offset kbyte) into the activation slot at byte
  // offset oa and the weight slot at ob (of the weight slots).
  auto issue = [&](const Src& s, int kbyte, int oa, int ob) {
    kbyte = __builtin_amdgcn_readfirstlane(kbyte);  // the scalar offset (uniform)
    const int e = __builtin_amdgcn_readfirstlane(s.e);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(p.w) + static_cast<int64_t>(e) * w_bytes, 0, w_bytes, kBufWord3);
    uint8_t* a_dst = lds + oa + wave * NLA * 1024;
    uint8_t* b_dst = lds + B_OFF + ob + wave * NLB * 1024;
#pragma unroll
    for (int i = 0; i < NLA; ++i) lds_dma16_buf(ra, s.va[i], kbyte, a_dst + i * 1024);
#pragma unroll
    for (int i = 0; i < NLB; ++i) lds_dma16_buf(rb, s.vb[i], kbyte, b_dst + i * 1024);
  };
  // One operand's loads of a stage: PART 0 the activation rows (into the
  // activation slot at byte offset o), 1 the weight rows (the weight slot
  // at o of the weight slots).
  auto issue_part = [&](const Src& s, int kbyte, int o, auto part_c) {
    constexpr int PART = decltype(part_c)::value;
    kbyte = __builtin_amdgcn_readfirstlane(kbyte);
    if constexpr (PART == 0) {
      uint8_t* a_dst = lds + o + wave * NLA * 1024;
#pragma unroll
      for (int i = 0; i < NLA; ++i) lds_dma16_buf(ra, s.va[i], kbyte, a_dst + i * 1024);
    } else {
      const int e = __builtin_amdgcn_readfirstlane(s.e);
      const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint8_t*>(p.w) + static_cast<int64_t>(e) * w_bytes, 0, w_bytes, kBufWord3);
      uint8_t* b_dst = lds + B_OFF + o + wave * NLB * 1024;
#pragma unroll
      for (int i = 0; i < NLB; ++i) lds_dma16_buf(rb, s.vb[i], kbyte, b_dst + i * 1024);
    }
  };

  // Fragment reads: lane reads row (lane & 31) of a 32-row block, logical
  // chunk 2*kk + (lane >> 5): the lane's offset f_off[kk] within a block,
  // the wave's blocks at a_base (block i of the wave: tile rows
  // (2i + wm) * 32) and b_base (uniform) of a slot.
  const int fr = lane & 31;
  int f_off[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) f_off[kk] = fr * SK + wide_chunk<C>(fr, 2 * kk + (lane >> 5)) * 16;
  const int a_base = wm * 32 * SK;
  const int b_base = B_OFF + wn * WCOLS * SK;

  Tile cur;
  if (GEMM1 && range.claims &&
      static_cast<int>(blockIdx.x / 8) >= range.hi - range.lo - kPlanClaimTail) {
    // a claimed position (one lane claims; the tile goes to every wave
    // through LDS, before any stage load writes it)
    int* claim_s = reinterpret_cast<int*>(lds);
    if (threadIdx.x == 0) {
      const int me = static_cast<int>(blockIdx.x / 8);
      int owner = -1, pos = 0;
      for (int k = 0; k < 2 && owner < 0; ++k) {
        // own tail first, then one other XCD's (spread by position)
        const int x = k == 0 ? xcd : (xcd + 1 + me % 7) & 7;
        const int n = p.plan[x + 1] - p.plan[x];
        const int first = max(0, n - kPlanClaimTail);
        pos = first + __hip_atomic_fetch_add(p.plan + kPlanWords + x * kPlanClaimStride, 1,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (pos < n) owner = x;
      }
      claim_s[0] = owner;
      claim_s[1] = pos;
    }
    __syncthreads();
    const int owner = __builtin_amdgcn_readfirstlane(claim_s[0]);
    const int pos = __builtin_amdgcn_readfirstlane(claim_s[1]);
    __syncthreads();
    if (owner < 0) return;
    WideRange rg;
    rg.lo = __builtin_amdgcn_readfirstlane(p.plan[owner]);
    rg.hi = __builtin_amdgcn_readfirstlane(p.plan[owner + 1]);
    rg.claims = true;
    if (!live_tile(rg, pos, cur)) return;
  } else {
    if (!live_tile(range, static_cast<int>(blockIdx.x / 8), cur)) return;
  }
  // the tile's expert loads beside its token slots (make_src), so the two
  // round trips overlap
  const int e_tile = p.expert_ids[cur.rb];
  Src src;
  make_src(cur, src);
  cur.e = __builtin_amdgcn_readfirstlane(e_tile);
  if (cur.e < 0) return;
  src.e = cur.e;
  const int row0 = cur.rb * BM;
  // the first token slot of each of the wave's 32-row blocks, loaded before
  // the stage loads: the counter drains in issue order, so waiting on these
  // never waits on a stage load
  int first_sid[RB];
#pragma unroll
  for (int i = 0; i < RB; ++i) first_sid[i] = p.sorted_ids[row0 + i * 64 + wm * 32];
  // stage s lives in activation slot s % NS and weight slot s % NSB;
  // stages 0 and 1 load first
  const int KT = cur.KT;
#pragma unroll
  for (int s = 0; s < 2; ++s) issue(src, (cur.kt0 + s) * SK, s * SLOT, s * SLOT);

  // live 32-row blocks of this wave (pad rows are a suffix of the tile, so
  // the wave's live blocks are a prefix of i)
  int nlive = 0;
#pragma unroll
  for (int i = 0; i < RB; ++i) nlive += first_sid[i] < p.numel ? 1 : 0;
  nlive = __builtin_amdgcn_readfirstlane(nlive);

  // The tile (accumulators, k loop, epilogue) is instantiated per count of
  // live 32-row blocks: all-pad blocks (the tail of an expert's last block)
  // skip their MFMAs with no branch in the MFMA stream, and no accumulator
  // crosses a control-flow join.
  auto tile_body = [&](auto nlive_c) {
    constexpr int NLIVE = decltype(nlive_c)::value;
    Acc acc[RB][CB];
    Frag fa[2][RB], fb[2][CB];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

    // (slots by byte offset: oa of the activation slots, ob of the weight
    // slots)
    auto read_frags = [&](int oa, int ob, int kk, Frag (&a)[RB], Frag (&b)[CB]) {
      const uint8_t* sta = lds + (oa + a_base) + f_off[kk];
      const uint8_t* stb = lds + (ob + b_base) + f_off[kk];
#pragma unroll
      for (int i = 0; i < RB; ++i) a[i] = *reinterpret_cast<const Frag*>(sta + i * 64 * SK);
#pragma unroll
      for (int j = 0; j < CB; ++j) b[j] = *reinterpret_cast<const Frag*>(stb + j * 32 * SK);
    };
    auto mma = [&](const Frag (&a)[RB], const Frag (&b)[CB]) {
#pragma unroll
      for (int i = 0; i < NLIVE; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j) acc[i][j] = T::mma(b[j], a[i], acc[i][j]);
    };
    // the next k step's fragment reads, one after each of the first MFMAs
    // (measured 1.3 % faster than issuing all eight after the first MFMA),
    // then ND loads one between each pair of the remaining MFMAs
    auto sched_step = [&](auto nd_c) {
      constexpr int ND = decltype(nd_c)::value;
      if constexpr (NLIVE > 0) {
#pragma unroll
        for (int t = 0; t < RB + CB; ++t) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
#pragma unroll
        for (int t = 0; t < ND; ++t) {
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
          if (t < NLIVE * CB - (RB + CB)) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
        if constexpr (NLIVE * CB > RB + CB + ND)
          __builtin_amdgcn_sched_group_barrier(0x008, NLIVE * CB - (RB + CB) - ND, 0);
      }
    };
    // after a stage barrier: one MFMA, the next k step's fragment reads,
    // then ND loads one between each pair of MFMAs, so the wave never
    // stalls on a burst of vector-memory issues
    auto sched_tail = [&](auto nd_c) {
      constexpr int ND = decltype(nd_c)::value;
      if constexpr (NLIVE > 0) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, RB + CB, 0);
#pragma unroll
        for (int t = 0; t < ND; ++t) {
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
          if (t < NLIVE * CB - 1) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
        if constexpr (NLIVE * CB - 1 > ND)
          __builtin_amdgcn_sched_group_barrier(0x008, NLIVE * CB - 1 - ND, 0);
      }
    };
    // The barrier before the last k step of stage s publishes stage s+1
    // (every wave has waited for its own loads of it) and frees stage s's
    // slots. Stage s+2, when there is one, loads its early operand (the one
    // with three slots) during the first k step of stage s, into slot
    // (s+2) % 3, free since the barrier of stage s-1, and its other operand
    // right after that barrier, into slot s % 2. A CU's 64 loads of a stage
    // are spread over two k steps, and the operand that misses L2 more often
    // (the weight rows; in GEMM2 on large row counts the activation rows,
    // gathered from an intermediate too large for the caches) is in flight
    // for seven k steps before a barrier waits for it, the other for four.
    // Slot byte offsets advance with the stage: 0, SLOT, 0, ... in the
    // two-slot ring, 0, SLOT, 2 SLOT, 0, ... in the three-slot one.
    auto next_a = [](int o) { return o == (NS - 1) * SLOT ? 0 : o + SLOT; };
    auto prev_a = [](int o) { return o == 0 ? (NS - 1) * SLOT : o - SLOT; };
    auto next_b = [](int o) { return o == (NSB - 1) * SLOT ? 0 : o + SLOT; };
    auto prev_b = [](int o) { return o == 0 ? (NSB - 1) * SLOT : o - SLOT; };
    constexpr bool EA = C::EARLY_A;
    constexpr int NLE = EA ? NLA : NLB, NLL = EA ? NLB : NLA;  // early / late loads
    auto stage = [&](int s, int oa, int ob, auto refill_c) {
      constexpr bool REFILL = decltype(refill_c)::value;
#pragma unroll
      for (int kk = 0; kk + 1 < KK; ++kk) {
        read_frags(oa, ob, kk + 1, fa[(kk + 1) & 1], fb[(kk + 1) & 1]);
        if (REFILL && kk == 0)  // three-slot ring: slot (s + 2) % 3 = (s - 1) % 3
          issue_part(src, (cur.kt0 + s + 2) * SK, EA ? prev_a(oa) : prev_b(ob),
                     std::integral_constant<int, EA ? 0 : 1>{});
        mma(fa[kk & 1], fb[kk & 1]);
        if (REFILL && kk == 0) sched_step(std::integral_constant<int, NLE>{});
        else sched_step(std::integral_constant<int, 0>{});
        __builtin_amdgcn_sched_barrier(0);
      }
      wait_lgkm0();
      // stage s+2's early loads may stay in flight
      wait_vmcnt<REFILL ? NLE : 0>();
      wave_barrier_all();
      read_frags(next_a(oa), next_b(ob), 0, fa[0], fb[0]);
      if constexpr (REFILL)
        issue_part(src, (cur.kt0 + s + 2) * SK, EA ? ob : oa,
                   std::integral_constant<int, EA ? 1 : 0>{});
      mma(fa[1], fb[1]);
      sched_tail(std::integral_constant<int, REFILL ? NLL : 0>{});
      __builtin_amdgcn_sched_barrier(0);
    };
    wait_vmcnt<NL>();
    wave_barrier_all();
    read_frags(0, 0, 0, fa[0], fb[0]);
    int s = 0, oa = 0, ob = 0;
    for (; s + 2 < KT; ++s, oa = next_a(oa), ob = next_b(ob)) stage(s, oa, ob, std::true_type{});
    for (; s + 1 < KT; ++s, oa = next_a(oa), ob = next_b(ob)) stage(s, oa, ob, std::false_type{});
    // the last stage (KT-1): oa, ob
#pragma unroll
    for (int kk = 0; kk + 1 < KK; ++kk) {
      read_frags(oa, ob, kk + 1, fa[(kk + 1) & 1], fb[(kk + 1) & 1]);
      mma(fa[kk & 1], fb[kk & 1]);
      sched_step(std::integral_constant<int, 0>{});
      __builtin_amdgcn_sched_barrier(0);
    }
    mma(fa[1], fb[1]);

    // ---- epilogue (the tiled kernel's arithmetic): lane owns token row
    // (lane & 31) of each 32-row block and, per 32-column block, columns
    // 8*q + 4*(lane>>5) + {0..3} (accumulator registers 4q..4q+3). A store
    // straight from that layout would touch 32 output rows per
    // instruction; instead each 32-row block goes through this wave's half
    // of a free slot of the three-slot ring (stage KT-2's for waves 0-1, the
    // slot stage KT would take for waves 2-3: no wave reads them again and
    // no refill targets them; other waves may still read stage KT-1's) and leaves as
    // whole row segments, 16 bytes per lane. Chunks (16 bytes) of a staged
    // row are XOR-swizzled by the row so the column-major writes spread over
    // the banks.
    {
      const int ks = cur.ks;
      const int64_t wbase = static_cast<int64_t>(cur.e) * p.nrows_w;


      const int csub = 4 * (lane >> 5);
      const int half = lane >> 5;
      const float* wsc = INT8 ? p.w_scale + wbase : nullptr;
      constexpr int R3 = EA ? 0 : B_OFF, R2 = EA ? B_OFF : 0;  // three- / two-slot ring
      const int fslot = wave < 2 ? (KT - 2) % 3 : KT % 3;
      uint8_t* stg = lds + R3 + fslot * SLOT + (wave % 2) * (SLOT / 2);
      static_assert(SLOT / 2 >= 32 * WCOLS * 4, "a 32-row fp32 block fits a wave's staging");
      auto value = [&](const Acc& a, int v, float sa, float sw) -> float {
        if constexpr (INT8) return static_cast<float>(a[v]) * sa * sw;
        else return a[v];
      };
      // orders this wave's staging writes before its reads (and the reads
      // before the next block's writes)
      auto stage_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      };
      // Everything the epilogue reads from global memory -- per row of this
      // wave's live blocks the token slot, int8 activation scale and router
      // weight; per column the int8 weight scale and bias -- is loaded
      // first and parked in the wave's LDS table: the vector memory counter
      // counts stores too, so a global load issued after one block's stores
      // would wait for them to complete. Table (floats): [0, 128) column
      // scales (GEMM1: 64 gate, 64 up), [128, 256) bias (GEMM2) or router
      // weights (GEMM1), [256, 384) token slots, [384, 512) row scales;
      // row (block i, r) at i * 32 + r.
      // (in stage KT-2's slot of the two-slot ring)
      float* tab = reinterpret_cast<float*>(lds + R2 + ((KT - 2) % 2) * SLOT + wave * C::TAB_BYTES);
      int* tsid = reinterpret_cast<int*>(tab + 256);
      const bool woi = GEMM1 && p.weight_on_input;
      static_assert(RB * 32 <= 128, "table rows");
#pragma unroll
      for (int q = 0; q < (NLIVE + 1) / 2; ++q) {
        // lanes 0-31 take block 2q, lanes 32-63 block 2q+1, row lane & 31
        const int i = 2 * q + (lane >> 5);
        if (i < NLIVE) {
          const int rr = i * 64 + wm * 32 + (lane & 31);
          const int sid = p.sorted_ids[row0 + rr];
          const bool ok = sid < p.numel;
          const int t = i * 32 + (lane & 31);
          tsid[t] = sid;
          if constexpr (INT8)
            tab[384 + t] = p.a_scale[GEMM1 ? (ok ? div_topk(p, sid) : 0) : row0 + (ok ? rr : 0)];
          if (woi) tab[128 + t] = ok ? p.topk_w[sid] : 1.f;
        }
      }
      auto row_sa = [&](int i) -> float {
        if constexpr (INT8) return tab[384 + i * 32 + (lane & 31)];
        else return 1.f;
      };
      if constexpr (GEMM1) {
        // silu, no bias (the launch guarantees both): 64 output columns per
        // wave, 128-byte staged rows (8 chunks). The router-weight scaling is
        // a compile-time branch so the common case carries no per-element
        // select.
        constexpr int CH = WCOLS / 2 / 8;  // chunks per staged row
        uint16_t* out = static_cast<uint16_t*>(p.out);
        const int col_base = cur.ct * (BNR / 2) + wn * (WCOLS / 2);
        static_assert(WCOLS / 2 == 64, "a lane per gate column");
        if constexpr (INT8) {
          tab[lane] = wsc[col_base + lane];
          tab[64 + lane] = wsc[p.n_out + col_base + lane];
        }
        stage_sync();
        auto csc4 = [&](int c) -> f32x4 {
          if constexpr (INT8) return *reinterpret_cast<const f32x4*>(tab + c);
          else return f32x4{1.f, 1.f, 1.f, 1.f};
        };
        auto emit = [&](auto scale_c) {
          constexpr bool SCALE = decltype(scale_c)::value;
#pragma unroll
          for (int i = 0; i < NLIVE; ++i) {
            const float sa = row_sa(i);
            const float gamma = SCALE ? tab[128 + i * 32 + (lane & 31)] : 1.f;
            const int r = lane & 31;
#pragma unroll
            for (int jb = 0; jb < CB / 2; ++jb) {
#pragma unroll
              for (int g4 = 0; g4 < 4; ++g4) {
                const f32x4 swg = csc4(jb * 32 + csub + 8 * g4);
                const f32x4 swu = csc4(64 + jb * 32 + csub + 8 * g4);
                const Acc& ag = acc[i][jb];
                const Acc& au = acc[i][jb + CB / 2];
                const int v = 4 * g4;
                uint2 v2;
                v2.x = silu_mul_bf16x2<SCALE>(
                    value(ag, v, sa, swg[0]), value(ag, v + 1, sa, swg[1]),
                    value(au, v, sa, swu[0]), value(au, v + 1, sa, swu[1]), gamma);
                v2.y = silu_mul_bf16x2<SCALE>(
                    value(ag, v + 2, sa, swg[2]), value(ag, v + 3, sa, swg[3]),
                    value(au, v + 2, sa, swu[2]), value(au, v + 3, sa, swu[3]), gamma);
                const int c = jb * 4 + g4;
                *reinterpret_cast<uint2*>(stg + r * (CH * 16) + ((c ^ (r % CH)) * 16) + half * 8) = v2;
              }
            }
            stage_sync();
            // 8 lanes per row, 8 rows per pass. Every row of a live 32-row
            // block is stored: a pad row has its own row in the padded
            // order, which nothing reads, so the passes need no branch and
            // their staged reads all issue ahead of the stores (one LDS
            // round trip per block instead of one per pass)
            constexpr int NP = 32 / (64 / CH);
            uint4 val[NP];
#pragma unroll
            for (int k = 0; k < NP; ++k) {
              const int sr = k * (64 / CH) + lane / CH;
              const int c = lane % CH;
              val[k] = *reinterpret_cast<const uint4*>(stg + sr * (CH * 16) + ((c ^ (sr % CH)) * 16));
            }
#pragma unroll
            for (int k = 0; k < NP; ++k) {
              const int sr = k * (64 / CH) + lane / CH;
              const int c = lane % CH;
              const int64_t orow = row0 + i * 64 + wm * 32 + sr;
              *reinterpret_cast<uint4*>(out + orow * p.n_out + col_base + c * 8) = val[k];
            }
            stage_sync();
          }
        };
        if (p.weight_on_input) emit(std::true_type{});
        else emit(std::false_type{});
      } else {
        const float* bias = p.bias && ks == 0 ? p.bias + wbase : nullptr;
        // the bias as a compile-time branch: without one the epilogue
        // issues no loads between its stores
        auto run = [&](auto bias_c) {
          constexpr bool BIAS = decltype(bias_c)::value;
          const int col_base = cur.ct * BNR + wn * WCOLS;
          static_assert(WCOLS == 128, "two columns per lane");
          if constexpr (INT8) {
            tab[lane] = wsc[col_base + lane];
            tab[64 + lane] = wsc[col_base + 64 + lane];
          }
          if constexpr (BIAS) {
            tab[128 + lane] = bias[col_base + lane];
            tab[192 + lane] = bias[col_base + 64 + lane];
          }
          stage_sync();
          auto csc4 = [&](int c) -> f32x4 {
            if constexpr (INT8) return *reinterpret_cast<const f32x4*>(tab + c);
            else return f32x4{1.f, 1.f, 1.f, 1.f};
          };
          auto cb4 = [&](int c) -> f32x4 {
            if constexpr (BIAS) return *reinterpret_cast<const f32x4*>(tab + 128 + c);
            else return f32x4{0.f, 0.f, 0.f, 0.f};
          };
#pragma unroll
          for (int i = 0; i < NLIVE; ++i) {
            const float sa = row_sa(i);
            const int r = lane & 31;
            if (p.ksplit > 1 || cur.slot >= 0) {
              // fp32 partials (k splits, tail pieces): 512-byte staged rows
              // (32 chunks), 2 rows per pass
              constexpr int CH = WCOLS * 4 / 16;
#pragma unroll
              for (int j = 0; j < CB; ++j) {
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                  const f32x4 sw = csc4(j * 32 + csub + 8 * g4);
                  const f32x4 bb = cb4(j * 32 + csub + 8 * g4);
                  const int v = 4 * g4;
                  const int c = j * 8 + g4 * 2 + half;
                  *reinterpret_cast<f32x4*>(stg + r * (CH * 16) + ((c ^ (r % CH)) * 16)) =
                      f32x4{value(acc[i][j], v, sa, sw[0]) + bb[0],
                            value(acc[i][j], v + 1, sa, sw[1]) + bb[1],
                            value(acc[i][j], v + 2, sa, sw[2]) + bb[2],
                            value(acc[i][j], v + 3, sa, sw[3]) + bb[3]};
                }
              }
              stage_sync();
              float* outf = static_cast<float*>(p.out);
              // four passes' row slots and staged values first, then their
              // stores (one LDS round trip per four passes instead of two
              // per pass; four keep the registers within budget)
              constexpr int NP = 32 / (64 / CH);
              static_assert(NP % 4 == 0, "passes in groups of four");
#pragma unroll
              for (int k0 = 0; k0 < NP; k0 += 4) {
                f32x4 vals[4];
                int sids[4];
#pragma unroll
                for (int kq = 0; kq < 4; ++kq) {
                  const int sr = (k0 + kq) * (64 / CH) + lane / CH;
                  const int c = lane % CH;
                  sids[kq] = tsid[i * 32 + sr];
                  vals[kq] = *reinterpret_cast<const f32x4*>(stg + sr * (CH * 16) + ((c ^ (sr % CH)) * 16));
                }
#pragma unroll
                for (int kq = 0; kq < 4; ++kq) {
                  const int sr = (k0 + kq) * (64 / CH) + lane / CH;
                  const int c = lane % CH;
                  const int row_sid = sids[kq];
                  const f32x4 val = vals[kq];
                  if (row_sid >= p.numel) continue;
                  float* dst;
                  if (cur.slot >= 0)  // tail piece: [slot][tile row][tile column]
                    dst = p.tail_part + (static_cast<int64_t>(cur.slot) * BM + i * 64 + wm * 32 + sr) * BNR +
                          wn * WCOLS + c * 4;
                  else
                    dst = outf + (static_cast<int64_t>(ks) * p.numel + row_sid) * p.n_out + col_base + c * 4;
                  *reinterpret_cast<f32x4*>(dst) = val;
                }
              }
              stage_sync();
            } else {
              // bf16 rows: 256-byte staged rows (16 chunks), 4 rows per pass
              constexpr int CH = WCOLS * 2 / 16;
              uint16_t* out = static_cast<uint16_t*>(p.out);
#pragma unroll
              for (int j = 0; j < CB; ++j) {
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                  const f32x4 sw = csc4(j * 32 + csub + 8 * g4);
                  const f32x4 bb = cb4(j * 32 + csub + 8 * g4);
                  const int v = 4 * g4;
                  uint2 v2;
                  // (no bias: no add, so the pair converts straight from
                  // the accumulators)
                  auto with_b = [&](float x, float b) { return BIAS ? x + b : x; };
                  v2.x = pack_bf16x2(with_b(value(acc[i][j], v, sa, sw[0]), bb[0]),
                                     with_b(value(acc[i][j], v + 1, sa, sw[1]), bb[1]));
                  v2.y = pack_bf16x2(with_b(value(acc[i][j], v + 2, sa, sw[2]), bb[2]),
                                     with_b(value(acc[i][j], v + 3, sa, sw[3]), bb[3]));
                  const int c = j * 4 + g4;
                  *reinterpret_cast<uint2*>(stg + r * (CH * 16) + ((c ^ (r % CH)) * 16) + half * 8) = v2;
                }
              }
              stage_sync();
              // four passes' row slots and staged values first, then their
              // stores (one LDS round trip per four passes instead of two
              // per pass; four keep the registers within budget)
              constexpr int NP = 32 / (64 / CH);
              static_assert(NP % 4 == 0, "passes in groups of four");
#pragma unroll
              for (int k0 = 0; k0 < NP; k0 += 4) {
                u32x4 vals[4];
                int sids[4];
#pragma unroll
                for (int kq = 0; kq < 4; ++kq) {
                  const int sr = (k0 + kq) * (64 / CH) + lane / CH;
                  const int c = lane % CH;
                  sids[kq] = tsid[i * 32 + sr];
                  vals[kq] = *reinterpret_cast<const u32x4*>(stg + sr * (CH * 16) + ((c ^ (sr % CH)) * 16));
                }
#pragma unroll
                for (int kq = 0; kq < 4; ++kq) {
                  const int c = lane % CH;
                  if (sids[kq] < p.numel)
                    *reinterpret_cast<u32x4*>(out + static_cast<int64_t>(sids[kq]) * p.n_out + col_base + c * 8) = vals[kq];
                }
              }
              stage_sync();
            }
          }
        };
        if (bias) run(std::true_type{});
        else run(std::false_type{});
      }
    }
  };
  dispatch_count<RB>(nlive, tile_body);
}

// Tail fixup of a tail-split GEMM2: 32 tile rows of one tail tile:
// y[slot, tile columns] = bf16(sum of the tile's pieces in piece order).
// Grid: 8 XCDs x 32 tail tiles x 8 blocks of 32 tile rows; 4 waves, a wave
// per row at a time (64 lanes x 4 fp32 = one 256-column partial row, so
// every piece read is one contiguous KiB).
template <int BM, int BNR, int SK, int ESZ>
__global__ __launch_bounds__(256) void moe_wide_tail_fixup_kernel(const GemmParams p) {
  static_assert(BNR == 64 * 4, "a wave covers a partial row");
  const int xcd = blockIdx.x % 8;
  const int t = (blockIdx.x / 8) % 32;
  const int rblk = blockIdx.x / (8 * 32);
  const int npp = p.num_post_pad[0];
  const int n_ct = static_cast<int>(p.n_out / BNR);
  const int total = npp / BM * n_ct;  // ksplit is 1 with a tail split
  const WideRange range = wide_range(p, total, xcd);
  const WideTail tail = wide_tail(range.lo, range.hi, true, static_cast<int>(p.kdim * ESZ / SK));
  if (tail.S < 2 || t >= tail.rem) return;
  int rb, ct;
  if (!wide_walk(range.lo, range.hi, n_ct, p.group_n, 32 * tail.R + t, &rb, &ct)) return;
  const int lane = threadIdx.x & 63;
  const int slot0 = xcd * 32 + t * tail.S;
  // a wave's 8 rows in two batches of 4, every piece of a batch's rows in
  // flight at once (the reads, not the adds, set this kernel's time)
  constexpr int RW = 4;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    int tr[RW], sid[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j) {
      tr[j] = rblk * 32 + (b * RW + j) * 4 + static_cast<int>(threadIdx.x >> 6);
      sid[j] = p.sorted_ids[rb * BM + tr[j]];
    }
    // pieces in order, ((p0 + p1) + p2) + ..., four at a time
    f32x4 acc[RW];
#pragma unroll
    for (int i0 = 0; i0 < kWideMaxPieces; i0 += 4) {
      if (i0 >= tail.S) break;
      f32x4 part[RW][4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < RW; ++j)
          part[j][i] = i0 + i < tail.S && sid[j] < p.numel
                           ? *reinterpret_cast<const f32x4*>(
                                 p.tail_part +
                                 (static_cast<int64_t>(slot0 + i0 + i) * BM + tr[j]) * BNR +
                                 lane * 4)
                           : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < RW; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (i0 + i < tail.S) acc[j] = i0 + i == 0 ? part[j][0] : acc[j] + part[j][i];
    }
#pragma unroll
    for (int j = 0; j < RW; ++j) {
      if (sid[j] >= p.numel) continue;
      uint2 v;
      v.x = pack_bf16x2(acc[j][0], acc[j][1]);
      v.y = pack_bf16x2(acc[j][2], acc[j][3]);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.out) + static_cast<int64_t>(sid[j]) * p.n_out +
                                ct * BNR + lane * 4) = v;
    }
  }
}

int64_t wide_tail_part_bytes() {
  return static_cast<int64_t>(kWideTailSlots) * WideRing::BM * WideRing::BNR * 4;
}

// Whether the 4-wave kernel covers a launch: bf16 / int8, GEMM1 with
// the silu activation and no bias (gelu and the swiglu bias variant keep the
// 8-wave kernel), k split into >= 2 stages per split, output tiles that
// divide n_out, and operands whose byte offsets fit the 32-bit buffer
// addressing.
bool wide_supported(int dt, bool gemm1, const GemmParams& p) {
  using C = WideRing;
  if (dt != kDtBf16 && dt != kDtInt8) return false;
  if (p.eid_shift != 0) return false;  // row blocks are whole alignment blocks
  if (gemm1 && (p.act != kActSilu || p.bias != nullptr)) return false;
  const int64_t esz = dt == kDtBf16 ? 2 : 1;
  const int64_t row_bytes = p.kdim * esz;
  if (row_bytes % C::SK != 0) return false;
  const int ks = std::max(1, gemm1 ? 1 : p.ksplit);
  if (row_bytes / C::SK < 2 * ks) return false;  // the prologue loads two stages
  if (p.n_out % (gemm1 ? C::BNR / 2 : C::BNR) != 0) return false;
  constexpr int64_t kMax = (int64_t{1} << 31) - 1;
  return p.a_rows > 0 && p.a_rows * row_bytes <= kMax && p.nrows_w * row_bytes <= kMax;
}

// Column-group width of the tile walk. With a plan (few row blocks: about
// one expert per XCD range) 8 for GEMM1 and 2 for GEMM2 (measured, Mixtral
// M=4096, two runs each: GEMM1 1.700 ms at 8 against 1.712 at 4, GEMM2
// 0.888 at 2 against 0.902 at 8). Without one, 4 for a GEMM1 of >= 16
// column tiles over mostly full row blocks (>= 512 rows per expert: Qwen2
// int8 M=8192 GEMM1 1.238 at 4 against 1.250 at 8), else 8 (half-full
// blocks and Qwen3's 6-tile GEMM1 are slower at 4; Qwen2 int8 M=8192 GEMM2
// 0.749 at 8 against 0.764 at 4). FGS_MOE_WIDE_GROUPN overrides it (a
// tuning aid, read once).
static int wide_group_n_choice(bool gemm1, int n_ct, double rows_per_expert, bool planned) {
  static const int g = [] {
    const char* s = tuning_env("FGS_MOE_WIDE_GROUPN");
    const int v = s ? atoi(s) : 0;
    return (v >= 1 && v <= 64) ? v : 0;
  }();
  if (g > 0) return g;
  if (planned) return gemm1 ? 8 : 2;
  return gemm1 && n_ct >= 16 && rows_per_expert >= 512 ? 4 : 8;
}

// FGS_MOE_PLAN=0 turns the GEMM1 tile plan off (a tuning aid; read once).
static bool plan_off() {
  static const bool off = [] {
    const char* v = tuning_env("FGS_MOE_PLAN");
    return v && atoi(v) == 0;
  }();
  return off;
}

// GEMM2's ring orientation: activation rows early from 512 rows per expert,
// where its gathered intermediate rows outgrow the caches (measured, same
// box, twice, GEMM2 with activation against weight rows early: Mixtral
// M=2048 / 4096 -4.2 % / -1.7 %, Qwen2 int8 M=8192 -1.3 %, Qwen3 M=8192 and
// Qwen2 int8 M=4096 level; below 512 rows weight rows early: Mixtral M=512
// by 4 %, Qwen3 M=4096 by 1.5 %, Mixtral M=1024 level). FGS_MOE_WIDE_EARLY=0
// / 1 forces weight / activation rows early (a tuning aid, read once).
static bool wide_early_a_choice(const GemmParams& p) {
  static const int forced = [] {
    const char* s = tuning_env("FGS_MOE_WIDE_EARLY");
    const int v = s ? atoi(s) : -1;
    return (v == 0 || v == 1) ? v : -1;
  }();
  if (forced >= 0) return forced == 1;
  return p.num_experts > 0 && p.numel >= 512LL * p.num_experts;
}

// A launch's normalised parameters (k split, tail split, whether it has a
// plan) and the positions per XCD its whole tiles may take: the even split
// needs total / 8; a cost-balanced plan may give an XCD up to a quarter more
// (the plan falls back to the even split beyond that).
static void wide_launch_shape(bool gemm1, const GemmParams& p, int row_blocks, GemmParams* q,
                              int64_t* cap) {
  using C = WideRing;
  *q = p;
  q->row_blocks = row_blocks;
  if (gemm1 || q->ksplit < 1) q->ksplit = 1;
  if (gemm1 || !q->tail_part) q->tail_split = 0;
  if (q->tail_split) q->ksplit = 1;
  // the plan: few row blocks, whole tiles (see wide_plan_kernel)
  if (row_blocks > kPlanMaxRows || q->ksplit > 1 || plan_off()) q->plan = nullptr;
  const int n_ct = static_cast<int>(gemm1 ? p.n_out / (C::BNR / 2) : p.n_out / C::BNR);
  const int64_t total = static_cast<int64_t>(row_blocks) * q->ksplit * n_ct;
  *cap = (total + 7) / 8;
  if (q->plan) *cap = *cap * 5 / 4 + 1;
}

void wide_plan_request(bool gemm1, const GemmParams& p, int row_blocks, WidePlanReq* req) {
  using C = WideRing;
  GemmParams q;
  int64_t cap;
  wide_launch_shape(gemm1, p, row_blocks, &q, &cap);
  *req = WidePlanReq{};
  if (!q.plan) return;
  req->plan = q.plan;
  req->n_ct = static_cast<int32_t>(gemm1 ? p.n_out / (C::BNR / 2) : p.n_out / C::BNR);
  req->cap = static_cast<int32_t>(cap);
  req->base = gemm1 ? kPlanBaseGemm1 : kPlanBaseGemm2;
}

template <int DT, bool GEMM1, class C>
static int launch_wide_t(const GemmParams& p, int row_blocks, hipStream_t stream) {
  auto kern = moe_gemm_wide_kernel<DT, GEMM1, C>;
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [&] {
    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS_BYTES);
  });
  if (attr != hipSuccess)
    return fail(FGS_ELAUNCH, std::string("wide GEMM LDS opt-in: ") + hipGetErrorString(attr));
  GemmParams q;
  int64_t cap;
  wide_launch_shape(GEMM1, p, row_blocks, &q, &cap);
  set_topk_magic(&q);
  const int n_ct_walk = static_cast<int>(GEMM1 ? p.n_out / (C::BNR / 2) : p.n_out / C::BNR);
  const double rows_per_expert =
      p.num_experts > 0 ? static_cast<double>(p.numel) / p.num_experts : 0.0;
  if (q.group_n < 1)
    q.group_n = wide_group_n_choice(GEMM1, n_ct_walk, rows_per_expert, q.plan != nullptr);
  // enough positions for the largest XCD walk the kernel can form from the
  // launched row blocks (it splits the live ones, known on the device), and
  // for the tail pieces of its last round
  const int n_ct = static_cast<int>(GEMM1 ? p.n_out / (C::BNR / 2) : p.n_out / C::BNR);
  int64_t extra = 0;  // positions past an XCD's range (claims of others' tails)
  if (q.plan) {
    extra = GEMM1 ? 32 : 0;
    if (!q.plan_ready) {
      hipLaunchKernelGGL(wide_plan_kernel, dim3(1), dim3(kWave), 0, stream, q.sorted_ids,
                         q.num_post_pad, static_cast<int>(q.numel), C::BM, n_ct,
                         static_cast<int>(cap), GEMM1 ? kPlanBaseGemm1 : kPlanBaseGemm2,
                         q.plan);
      const int rc = check_launch("wide_plan_kernel");
      if (rc) return rc;
    }
  }
  const int64_t n_pos = cap + extra + (q.tail_split ? 32 : 0);
  const int grid = static_cast<int>(8 * n_pos);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(C::NW * 64), C::LDS_BYTES, stream, q);
  int rc = check_launch("moe_gemm_wide_kernel");
  if (rc || !q.tail_split) return rc;
  hipLaunchKernelGGL((moe_wide_tail_fixup_kernel<C::BM, C::BNR, C::SK, TiledType<DT>::ESZ>),
                     dim3(8 * 32 * (C::BM / 32)), dim3(256), 0, stream, q);
  return check_launch("moe_wide_tail_fixup_kernel");
}

int launch_gemm_wide(int dt, bool gemm1, const GemmParams& p, int row_blocks,
                     hipStream_t stream) {
  if (!wide_supported(dt, gemm1, p))
    return fail(FGS_EINVAL, "wide GEMM: launch not covered by the 4-wave kernel");
  if (row_blocks <= 0) return FGS_OK;
  const bool early_a = !gemm1 && wide_early_a_choice(p);
  if (dt == kDtBf16) {
    if (gemm1) return launch_wide_t<kDtBf16, true, WideRing>(p, row_blocks, stream);
    return early_a ? launch_wide_t<kDtBf16, false, WideRingA>(p, row_blocks, stream)
                   : launch_wide_t<kDtBf16, false, WideRing>(p, row_blocks, stream);
  }
  if (gemm1) return launch_wide_t<kDtInt8, true, WideRing>(p, row_blocks, stream);
  return early_a ? launch_wide_t<kDtInt8, false, WideRingA>(p, row_blocks, stream)
                 : launch_wide_t<kDtInt8, false, WideRing>(p, row_blocks, stream);
}

}  // namespace fgs
