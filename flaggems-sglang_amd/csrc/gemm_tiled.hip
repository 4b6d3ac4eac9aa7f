// LDS-tiled grouped GEMMs of the fused-MoE path (prefill regime: many rows
// per expert, the layer is bound by MFMA throughput).
//
// A workgroup of WM x WN waves owns a BM-row block of the expert-sorted,
// padded row order (one expert per block, from moe_align_block_size) and
// BNR weight rows. Each k-step stages a BM x 128-byte activation tile and a
// BNR x 128-byte weight tile in LDS (double buffered: the next step's global
// loads are in flight while the current step's MFMAs run), and each wave
// multiplies its (BM/WM) x (BNR/WN) sub-tile with v_mfma_f32_32x32x16_bf16.
//
// GEMM1 (fused activation): the weight tile interleaves 64 gate rows and the
// 64 matching up rows per wave column, so every lane holds the gate and up
// accumulators of the same output element; the epilogue applies the
// reference's rounding points and silu (ops/fused_moe.py:205-218).
// GEMM2: plain y = a2 W2^T per padded row, scattered to its top-k slot.
#include <mutex>
#include <string>

#include "fgs_moe_kernels.h"

namespace fgs {

constexpr int kStageK = 64;  // bytes of k per stage row (32 bf16)
constexpr int kLoadRows = 16;  // rows one wave-wide 16 B/lane LDS-DMA load covers

// XOR swizzle of the four 16-byte chunks of a 64-byte LDS row. The DMA
// writes rows densely (lane l -> byte 16*l of a 1 KiB block), so rows are not
// padded; instead row r keeps logical chunk c at chunk c ^ swz(r), which puts
// the 8 rows any 8 consecutive lanes read in distinct 16-byte bank groups.
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 3; }

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Tile order. The grid is 1-D and padded to a multiple of the 8 XCDs.
// Workgroup `pid` runs on XCD pid % 8, so logical tile
// (pid % 8) * (grid / 8) + pid / 8 gives every XCD a contiguous range of
// tiles, walked in groups of kGroupN column tiles: the ~32 workgroups an
// XCD runs at once cover a few row blocks x kGroupN column tiles and share
// their activation and weight tiles through that XCD's L2.
constexpr int kGroupN = 8;

__device__ __forceinline__ bool tile_of(int pid, int grid, int n_rb, int n_ct,
                                        int* rb, int* ct) {
  const int logical = (pid % 8) * (grid / 8) + pid / 8;
  if (logical >= n_rb * n_ct) return false;
  const int span = n_rb * kGroupN;
  const int group = logical / span;
  const int idx = logical - group * span;
  const int gsize = min(kGroupN, n_ct - group * kGroupN);
  *rb = idx / gsize;
  *ct = group * kGroupN + idx % gsize;
  return true;
}

// One wave-wide LDS-DMA load: lane l copies 16 bytes from `src` (its own
// global address) to byte 16*l of the 1 KiB block at `lds_dst` (uniform).
__device__ __forceinline__ void lds_dma16(const void* src, void* lds_dst) {
  __builtin_amdgcn_global_load_lds(
      src, (__attribute__((address_space(3))) void*)(lds_dst), 16, 0, 0);
}

__device__ __forceinline__ void wave_barrier_all() { __builtin_amdgcn_s_barrier(); }

template <int BM, int BNR, int WM, int WN, int STAGES, bool GEMM1>
__global__ __launch_bounds__(WM * WN * 64, 1) void moe_gemm_tiled_bf16_kernel(
    const GemmParams p) {
  constexpr int NW = WM * WN;
  constexpr int A_BYTES = BM * kStageK;
  constexpr int B_BYTES = BNR * kStageK;
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int NLA = BM / (kLoadRows * NW);   // A loads per wave per stage
  constexpr int NLB = BNR / (kLoadRows * NW);  // B loads per wave per stage
  constexpr int NL = NLA + NLB;
  constexpr int WROWS = BM / WM;               // rows per wave
  constexpr int WCOLS = BNR / WN;              // weight rows per wave
  constexpr int RB = WROWS / 32;               // 32-row MFMA blocks
  constexpr int CB = WCOLS / 32;               // 32-col MFMA blocks
  static_assert(NLA * kLoadRows * NW == BM, "A tile / waves");
  static_assert(NLB * kLoadRows * NW == BNR, "B tile / waves");
  static_assert(STAGES >= 3 && STAGES <= 5, "stages");
  static_assert(RB >= 1 && CB >= 1, "wave tile");
  static_assert(!GEMM1 || (WCOLS % 64 == 0 && CB % 2 == 0), "gate/up pairing");

  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];

  constexpr int N_PER_TILE = GEMM1 ? BNR / 2 : BNR;
  int rb_id, tile_n;
  if (!tile_of(blockIdx.x, gridDim.x, p.row_blocks,
               static_cast<int>(p.n_out / N_PER_TILE), &rb_id, &tile_n))
    return;
  if (rb_id * BM >= p.num_post_pad[0]) return;
  const int e = p.expert_ids[rb_id];
  if (e < 0) return;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int row0 = rb_id * BM;

  // ---- this lane's source of each LDS-DMA load (row lane/4, chunk lane%4)
  const int lrow = lane >> 2;
  const int lchunk = lane & 3;
  const uint8_t* a_src[NLA];
#pragma unroll
  for (int i = 0; i < NLA; ++i) {
    const int r = (wave * NLA + i) * kLoadRows + lrow;
    const int sid = p.sorted_ids[row0 + r];
    // pad rows read token 0 / their own row: finite values, never stored
    const int64_t src = GEMM1 ? (sid < p.numel ? sid / p.topk : 0) : row0 + r;
    a_src[i] = p.a + src * p.kdim * 2 + ((lchunk ^ swz(r)) * 16);
  }
  const uint8_t* b_src[NLB];
  const int64_t wbase = static_cast<int64_t>(e) * p.nrows_w;
#pragma unroll
  for (int i = 0; i < NLB; ++i) {
    const int j = (wave * NLB + i) * kLoadRows + lrow;  // tile row
    int64_t wrow;
    if constexpr (GEMM1) {
      // rows [64q, 64q+64): q even -> gate, q odd -> up, column block q/2
      const int q = j / 64;
      wrow = (q & 1 ? p.n_out : 0) + tile_n * (BNR / 2) + (q / 2) * 64 + j % 64;
    } else {
      wrow = static_cast<int64_t>(tile_n) * BNR + j;
    }
    b_src[i] = p.w + (wbase + wrow) * p.kdim * 2 + ((lchunk ^ swz(j)) * 16);
  }

  auto issue = [&](int kt, int slot) {
    const int64_t koff = static_cast<int64_t>(kt) * kStageK;
    uint8_t* base = lds + slot * STAGE;
#pragma unroll
    for (int i = 0; i < NLA; ++i)
      lds_dma16(a_src[i] + koff, base + (wave * NLA + i) * 1024);
#pragma unroll
    for (int i = 0; i < NLB; ++i)
      lds_dma16(b_src[i] + koff, base + A_BYTES + (wave * NLB + i) * 1024);
  };

  f32x16 acc[RB][CB];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // Fragment reads: lane reads row (lane & 31) of a 32-row block, logical
  // chunk 2*kk + (lane >> 5) (16 bf16 of k per kk step).
  const int fr = lane & 31;
  int frag_off[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
    frag_off[kk] = fr * kStageK + (((2 * kk + (lane >> 5)) ^ swz(fr)) * 16);
  const int a_base = wm * WROWS * kStageK;
  const int b_base = A_BYTES + wn * WCOLS * kStageK;

  const int KT = static_cast<int>(p.kdim * 2 / kStageK);
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < KT) issue(s, s);

  // Waits until at most `n` of this wave's later stages are in flight.
  auto wait_stages = [&](int n) {
    if (n >= 3) wait_vmcnt<3 * NL>();
    else if (n == 2) wait_vmcnt<2 * NL>();
    else if (n == 1) wait_vmcnt<NL>();
    else wait_vmcnt<0>();
  };
  auto read_frags = [&](int kt, int kk, bf16x8 (&fa)[RB], bf16x8 (&fb)[CB]) {
    const uint8_t* st = lds + (kt % STAGES) * STAGE;
#pragma unroll
    for (int i = 0; i < RB; ++i)
      fa[i] = *reinterpret_cast<const bf16x8*>(st + a_base + i * 32 * kStageK +
                                               frag_off[kk]);
#pragma unroll
    for (int j = 0; j < CB; ++j)
      fb[j] = *reinterpret_cast<const bf16x8*>(st + b_base + j * 32 * kStageK +
                                               frag_off[kk]);
  };
  auto mma = [&](const bf16x8 (&fa)[RB], const bf16x8 (&fb)[CB]) {
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j) acc[i][j] = mfma32_bf16(fa[i], fb[j], acc[i][j]);
  };

  // Software pipeline: the fragments of the next half-stage are read from
  // LDS while the MFMAs of the current one run; the barrier that publishes
  // stage kt+1 (and frees slot kt-1 for the next DMA) sits between the two
  // halves of stage kt.
  bf16x8 fa0[RB], fb0[CB], fa1[RB], fb1[CB];
  wait_stages(min(STAGES - 2, KT - 1));
  wave_barrier_all();
  read_frags(0, 0, fa0, fb0);
  // (the last stage is peeled so the loop body has no branch around LDS
  // reads, which lets the compiler wait for exactly the fragments it needs)
  for (int kt = 0; kt + 1 < KT; ++kt) {
    read_frags(kt, 1, fa1, fb1);
    mma(fa0, fb0);
    wait_stages(min(STAGES - 3, KT - 2 - kt));
    wave_barrier_all();
    if (kt + STAGES - 1 < KT) issue(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
    read_frags(kt + 1, 0, fa0, fb0);
    mma(fa1, fb1);
  }
  read_frags(KT - 1, 1, fa1, fb1);
  mma(fa0, fb0);
  mma(fa1, fb1);

  // ---- epilogue: lane owns column (lane & 31) of each 32x32 block and rows
  // 8*(v>>2) + 4*(lane>>5) + (v&3).
  uint16_t* out = static_cast<uint16_t*>(p.out);
  const int ccol = lane & 31;
#pragma unroll
  for (int i = 0; i < RB; ++i) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int r = row0 + wm * WROWS + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
      const int sid = p.sorted_ids[r];
      const bool valid = sid < p.numel;
      if constexpr (GEMM1) {
        const float gamma = (p.weight_on_input && valid) ? p.topk_w[sid] : 0.f;
#pragma unroll
        for (int jb = 0; jb < CB / 2; ++jb) {
          // wave columns: [gate 64 | up 64] per 64-column group
          const int q = jb / 2;
          const int h = jb % 2;
          const float g = acc[i][q * 4 + h][v];
          const float u = acc[i][q * 4 + 2 + h][v];
          const int col = tile_n * (BNR / 2) + wn * (WCOLS / 2) + q * 64 + h * 32 + ccol;
          out[static_cast<int64_t>(r) * p.n_out + col] =
              gemm1_epilogue(g, u, p.weight_on_input && valid, gamma);
        }
      } else {
        if (valid) {
#pragma unroll
          for (int j = 0; j < CB; ++j) {
            const int col = tile_n * BNR + wn * WCOLS + j * 32 + ccol;
            out[static_cast<int64_t>(sid) * p.n_out + col] = f32_to_bf16_bits(acc[i][j][v]);
          }
        }
      }
    }
  }
}

template <int BM, int BNR, int WM, int WN, int STAGES, bool GEMM1>
static int launch_tiled(const GemmParams& p, int row_blocks, hipStream_t stream) {
  constexpr int kLds = STAGES * (BM + BNR) * kStageK;
  auto kern = moe_gemm_tiled_bf16_kernel<BM, BNR, WM, WN, STAGES, GEMM1>;
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [&] {
    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
  });
  if (attr != hipSuccess)
    return fail(FGS_ELAUNCH, std::string("tiled GEMM LDS opt-in: ") +
                                 hipGetErrorString(attr));
  const int tiles_n = static_cast<int>(GEMM1 ? p.n_out / (BNR / 2) : p.n_out / BNR);
  GemmParams q = p;
  q.row_blocks = row_blocks;
  const int tiles = (row_blocks * tiles_n + 7) / 8 * 8;
  hipLaunchKernelGGL(kern, dim3(tiles), dim3(WM * WN * 64), kLds, stream, q);
  return check_launch("moe_gemm_tiled_bf16_kernel");
}

int tiled_block_m() { return 256; }

// n_out granularity the tiled kernels need (GEMM1 output cols per tile,
// GEMM2 output cols per tile).
int tiled_n_align(bool gemm1) { return gemm1 ? 128 : 256; }

int launch_gemm_tiled(int dt, bool gemm1, const GemmParams& p, int row_blocks,
                      hipStream_t stream) {
  if (dt != kDtBf16) return fail(FGS_EUNSUPPORTED, "tiled GEMM: bf16 only");
  if (row_blocks <= 0) return FGS_OK;
  if (gemm1) return launch_tiled<256, 256, 4, 2, 4, true>(p, row_blocks, stream);
  return launch_tiled<256, 256, 4, 2, 4, false>(p, row_blocks, stream);
}

}  // namespace fgs
