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

constexpr int kTileKBytes = 128;              // k bytes per stage (64 bf16)
constexpr int kLdsRowBytes = kTileKBytes + 16;  // padded row: no bank conflicts

template <int BM, int BNR, int WM, int WN, bool GEMM1>
__global__ __launch_bounds__(WM * WN * 64, 1) void moe_gemm_tiled_bf16_kernel(
    const GemmParams p) {
  constexpr int NT = WM * WN * 64;
  constexpr int CHUNKS_ROW = kTileKBytes / 16;       // 16-byte chunks per row
  constexpr int A_CHUNKS = BM * CHUNKS_ROW / NT;     // per thread
  constexpr int B_CHUNKS = BNR * CHUNKS_ROW / NT;
  constexpr int ROWS_PER_PASS = NT / CHUNKS_ROW;
  constexpr int WROWS = BM / WM;                     // rows per wave
  constexpr int WCOLS = BNR / WN;                    // weight rows per wave
  constexpr int RB = WROWS / 32;                     // 32-row MFMA blocks
  constexpr int CB = WCOLS / 32;                     // 32-col MFMA blocks
  constexpr int A_BYTES = BM * kLdsRowBytes;
  constexpr int B_BYTES = BNR * kLdsRowBytes;
  static_assert(A_CHUNKS * NT == BM * CHUNKS_ROW, "A tile / threads");
  static_assert(B_CHUNKS * NT == BNR * CHUNKS_ROW, "B tile / threads");
  static_assert(RB >= 1 && CB >= 1, "wave tile");
  static_assert(!GEMM1 || (WCOLS % 64 == 0 && CB % 2 == 0), "gate/up pairing");

  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  // stage s: A tile at s*(A_BYTES+B_BYTES), B tile right after it
  constexpr int STAGE = A_BYTES + B_BYTES;

  const int rb_id = blockIdx.x;
  const int tile_n = blockIdx.y;
  if (rb_id * BM >= p.num_post_pad[0]) return;
  const int e = p.expert_ids[rb_id];
  if (e < 0) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int row0 = rb_id * BM;

  // ---- global source pointers of this thread's chunks
  const int chunk = tid % CHUNKS_ROW;
  const uint8_t* a_src[A_CHUNKS];
  bool a_ok[A_CHUNKS];
#pragma unroll
  for (int c = 0; c < A_CHUNKS; ++c) {
    const int r = row0 + c * ROWS_PER_PASS + tid / CHUNKS_ROW;
    const int sid = p.sorted_ids[r];
    a_ok[c] = sid < p.numel;
    const int64_t src = GEMM1 ? (a_ok[c] ? sid / p.topk : 0) : r;
    a_src[c] = p.a + src * p.kdim * 2 + chunk * 16;
  }
  const uint8_t* b_src[B_CHUNKS];
  const int64_t wbase = static_cast<int64_t>(e) * p.nrows_w;
#pragma unroll
  for (int c = 0; c < B_CHUNKS; ++c) {
    const int j = c * ROWS_PER_PASS + tid / CHUNKS_ROW;  // tile row
    int64_t wrow;
    if constexpr (GEMM1) {
      // rows [64q, 64q+64): q even -> gate, q odd -> up, column block q/2
      const int q = j / 64;
      wrow = (q & 1 ? p.n_out : 0) + tile_n * (BNR / 2) + (q / 2) * 64 + j % 64;
    } else {
      wrow = static_cast<int64_t>(tile_n) * BNR + j;
    }
    b_src[c] = p.w + (wbase + wrow) * p.kdim * 2 + chunk * 16;
  }
  const int lds_off_base = (tid / CHUNKS_ROW) * kLdsRowBytes + chunk * 16;

  u32x4 ra[A_CHUNKS], rbv[B_CHUNKS];
  auto gload = [&](int kt) {
    const int64_t koff = static_cast<int64_t>(kt) * kTileKBytes;
#pragma unroll
    for (int c = 0; c < A_CHUNKS; ++c)
      ra[c] = a_ok[c] ? *reinterpret_cast<const u32x4*>(a_src[c] + koff)
                      : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < B_CHUNKS; ++c)
      rbv[c] = *reinterpret_cast<const u32x4*>(b_src[c] + koff);
  };
  auto lstore = [&](int s) {
#pragma unroll
    for (int c = 0; c < A_CHUNKS; ++c)
      *reinterpret_cast<u32x4*>(lds + s * STAGE + lds_off_base +
                                c * ROWS_PER_PASS * kLdsRowBytes) = ra[c];
#pragma unroll
    for (int c = 0; c < B_CHUNKS; ++c)
      *reinterpret_cast<u32x4*>(lds + s * STAGE + A_BYTES + lds_off_base +
                                c * ROWS_PER_PASS * kLdsRowBytes) = rbv[c];
  };

  f32x16 acc[RB][CB];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // Fragment addressing: lane reads row (lane & 31), 16 bytes at
  // kk*32 + (lane >> 5)*16 of the 128-byte stage row.
  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * 16;
  const int a_frag = (wm * WROWS + frag_row) * kLdsRowBytes + frag_k;
  const int b_frag = (wn * WCOLS + frag_row) * kLdsRowBytes + frag_k;

  const int KT = static_cast<int>(p.kdim * 2 / kTileKBytes);
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int s = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
    for (int kk = 0; kk < kTileKBytes / 32; ++kk) {
      bf16x8 af[RB], bfr[CB];
#pragma unroll
      for (int i = 0; i < RB; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(lds + s * STAGE + a_frag +
                                                 i * 32 * kLdsRowBytes + kk * 32);
#pragma unroll
      for (int j = 0; j < CB; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(lds + s * STAGE + A_BYTES + b_frag +
                                                  j * 32 * kLdsRowBytes + kk * 32);
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j) acc[i][j] = mfma32_bf16(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < KT) lstore(s ^ 1);
    __syncthreads();
  }

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
          // wave columns: [gate 64 | up 64] per column block pair
          const int q = jb / 2;           // 64-wide column group of the wave
          const int h = jb % 2;           // 32-col half inside the group
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

template <int BM, int BNR, int WM, int WN, bool GEMM1>
static int launch_tiled(const GemmParams& p, int row_blocks, hipStream_t stream) {
  constexpr int kLds = 2 * (BM + BNR) * kLdsRowBytes;
  auto kern = moe_gemm_tiled_bf16_kernel<BM, BNR, WM, WN, GEMM1>;
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
  hipLaunchKernelGGL(kern, dim3(row_blocks, tiles_n), dim3(WM * WN * 64), kLds,
                     stream, p);
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
  if (gemm1) return launch_tiled<256, 256, 4, 2, true>(p, row_blocks, stream);
  return launch_tiled<256, 256, 4, 2, false>(p, row_blocks, stream);
}

}  // namespace fgs
