// Single-token fused MoE (bf16 weights, one token): both GEMMs in one launch.
//
// With one token the layer reads every touched expert's weights once and
// does almost no arithmetic, so its time is the weight stream plus whatever
// the stream stops for. The unfused single-token path (GEMM1 with silu, then
// GEMM2 with the top-k sum) drains the memory pipe between its two
// launches; here GEMM2's weight reads do not depend on GEMM1, so one launch
// carries both:
//
//   workgroup (slot j, chunk c of C intermediate columns):
//     phase 1  g, u = x . W13[e_j][gate / up rows of the chunk]   (MFMA)
//     phase 2  h = act(g, u) in bf16, the rounding points of the
//              unfused GEMM1 epilogue (gemm1_epilogue)
//     phase 3  part[j][c][:] = W2[e_j][:, chunk] h               (MFMA)
//
// The chunk's W2 columns (C contiguous values of each of the K rows) are
// fetched before phase 1 starts, so both GEMMs' loads are in flight
// together. A second, small kernel sums each slot's chunk partials in a
// fixed order, rounds y_j to bf16 (the row the unfused GEMM2 writes for
// slot j), and adds the slots as moe_sum does: out = bf16(sum_j gamma_j *
// y_j), product and sum rounded separately, slots in order, dropped slots
// (ids outside [0, E)) skipped. Deterministic: no atomics.
//
// Replaces, for one token, matmul_ogs (gather) + silu + matmul_ogs
// (scatter, gammas) of ops/fused_moe.py:202-231.
#include <stdlib.h>

#include <type_traits>

#include "fgs_moe_kernels.h"

namespace fgs {

namespace {

typedef __attribute__((ext_vector_type(2))) unsigned u32x2;
typedef __attribute__((ext_vector_type(4))) short i16x4;

__device__ __forceinline__ f32x4 mma_step4(const u32x4 (&a)[4], const u32x4 (&b)[4], f32x4 acc) {
#pragma unroll
  for (int v = 0; v < 4; ++v)
    acc = mfma16_bf16(__builtin_bit_cast(bf16x8, a[v]), __builtin_bit_cast(bf16x8, b[v]), acc);
  return acc;
}

}  // namespace

// C: intermediate columns per workgroup (32 or 64); KW: waves; D: phase-1
// k steps in flight per wave; B3: phase-3 tiles per load batch.
// Phase 1 has T1 = 2C/16 tiles of 16 W13 rows (gate tiles, then the
// matching up tiles); wave w multiplies tile w % T1 over k part w / T1 of
// KW / T1, 128 k (256 bytes of a row) per step: lane (ln, lg) holds row ln's
// 16-byte vectors v*64 + lg*16 (v < 4), x the same vectors in MFMA row 0
// (the same k permutation for both operands, so the dot products are exact).
// Phase 3: wave w owns W2 rows [w*K/KW, (w+1)*K/KW) in 16-row MFMA tiles,
// each tile C/32 MFMAs deep; the first batch of B3 tiles is fetched before
// phase 1, the rest in batches after it.
template <int C, int KW, int D, int B3>
__global__ __launch_bounds__(KW * 64) void moe_decode_bf16_kernel(const DecodeParams p) {
  constexpr int T1 = 2 * C / 16;
  static_assert(KW % T1 == 0, "phase 1: whole tiles per wave");
  constexpr int KP = KW / T1;  // k parts of phase 1
  // phase 3: Q MFMAs per 16-row tile, 32 deep with 16 bytes per lane
  // (C >= 32) or one 16 deep with 8 bytes per lane (C = 16)
  constexpr bool NARROW = C == 16;
  constexpr int Q = NARROW ? 1 : C / 32;
  typedef typename std::conditional<NARROW, u32x2, u32x4>::type Frag3;
  extern __shared__ __attribute__((aligned(16))) uint8_t xs[];  // x: hidden bf16

  // Workgroup b runs on XCD b % 8. The G = 64 / C chunks whose W2 columns
  // share 128-byte lines (G = 2 for C = 32, 4 for C = 16) go to one XCD, so
  // its L2 fetches each line once: unit L = j * n_chunks + c, line group
  // P = L / G, member m = L % G, b = (P / 8) * 8G + 8m + P % 8.
  constexpr int G = C >= 64 ? 1 : 64 / C;
  const int b = blockIdx.x;
  const int unit = ((b / (8 * G)) * 8 + b % 8) * G + (b / 8) % G;
  if (unit >= p.slots * p.n_chunks) return;  // grid padding
  const int j = unit / p.n_chunks;
  const int c = unit - j * p.n_chunks;
  const int e = p.ids[j];
  if (e < 0 || e >= p.num_experts) return;  // dropped slot: never read

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int ln = lane & 15;
  const int lg = lane >> 4;
  const int64_t K = p.hidden, N = p.inter;

  // ---- phase 3 addresses and its first batch of loads
  const int rows3 = static_cast<int>(K / KW);  // W2 rows of this wave
  const int tiles3 = rows3 / 16;
  const uint8_t* w2row = reinterpret_cast<const uint8_t*>(p.w2) +
                         ((static_cast<int64_t>(e) * K + wave * rows3 + ln) * N +
                          static_cast<int64_t>(c) * C + lg * (NARROW ? 4 : 8)) * 2;
  const int64_t w2_tile_bytes = 16 * N * 2;
  Frag3 wb[B3][Q];
  auto load3 = [&](int t0) {
#pragma unroll
    for (int t = 0; t < B3; ++t)
#pragma unroll
      for (int q = 0; q < Q; ++q)
        wb[t][q] = (t0 + t < tiles3)
                       ? __builtin_nontemporal_load(reinterpret_cast<const Frag3*>(
                             w2row + (t0 + t) * w2_tile_bytes + q * 64))
                       : Frag3{};
  };
  load3(0);

  // ---- phase 1: this wave's tile and k part, D steps in flight
  const int tile = wave % T1;
  const int kpart = wave / T1;
  const bool up = tile >= T1 / 2;
  const int64_t wrow = (up ? N : 0) + static_cast<int64_t>(c) * C + (tile % (T1 / 2)) * 16 + ln;
  const uint8_t* w1row = reinterpret_cast<const uint8_t*>(p.w13) +
                         ((static_cast<int64_t>(e) * 2 * N + wrow) * K) * 2 + lg * 16;
  const int steps = static_cast<int>(K / 128);
  const int s0 = kpart * steps / KP;
  const int s1 = (kpart + 1) * steps / KP;
  u32x4 bw[D][4];
  auto load1 = [&](int i, int st) {
#pragma unroll
    for (int v = 0; v < 4; ++v)
      bw[i][v] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(w1row + st * 256 + v * 64));
  };
#pragma unroll
  for (int i = 0; i < D; ++i)
    if (s0 + i < s1) load1(i, s0 + i);
  // x into LDS (every wave's MFMA row 0)
  {
    const u32x4* src = reinterpret_cast<const u32x4*>(p.x);
    for (int i = threadIdx.x; i < static_cast<int>(K / 8); i += KW * 64)
      reinterpret_cast<u32x4*>(xs)[i] = src[i];
  }
  __syncthreads();
  const bool xvalid = ln == 0;  // MFMA row 0 is the token, rows 1..15 zero
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s = s0; s < s1; s += D) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const int cur = s + i;
      if (cur < s1) {
        u32x4 xf[4];
#pragma unroll
        for (int v = 0; v < 4; ++v)
          xf[v] = xvalid ? *reinterpret_cast<const u32x4*>(xs + cur * 256 + v * 64 + lg * 16)
                         : u32x4{0, 0, 0, 0};
        acc = mma_step4(xf, bw[i], acc);
        if (cur + D < s1) load1(i, cur + D);
      }
    }
  }

  // ---- phase 2: k parts in order, then the GEMM1 epilogue
  __shared__ float red[KP][T1][16];
  __shared__ __attribute__((aligned(16))) uint16_t hbuf[C];
  if (lg == 0) red[kpart][tile][ln] = acc[0];  // row 0 of the tile
  __syncthreads();
  if (threadIdx.x < C) {
    const int n = threadIdx.x;
    const int tg = n / 16, tu = T1 / 2 + n / 16;
    float g = red[0][tg][n % 16], u = red[0][tu][n % 16];
#pragma unroll
    for (int kp = 1; kp < KP; ++kp) {
      g += red[kp][tg][n % 16];
      u += red[kp][tu][n % 16];
    }
    if (p.b13) {
      const float* b = p.b13 + static_cast<int64_t>(e) * 2 * N + static_cast<int64_t>(c) * C + n;
      g += b[0];
      u += b[N];
    }
    hbuf[n] = gemm1_epilogue(g, u, p.weight_on_input != 0, p.topk_w[j], p.act, p.alpha,
                             p.limit);
  }
  __syncthreads();

  // ---- phase 3: A operand = h in row 0 (lanes ln == 0), B = W2 tile rows
  Frag3 hf[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q)
    hf[q] = xvalid ? *reinterpret_cast<const Frag3*>(&hbuf[q * 32 + lg * (NARROW ? 4 : 8)])
                   : Frag3{};
  float* dst = p.part + (static_cast<int64_t>(j) * p.n_chunks + c) * K + wave * rows3 + ln;
  for (int t0 = 0; t0 < tiles3; t0 += B3) {
    f32x4 y[B3];
#pragma unroll
    for (int t = 0; t < B3; ++t) {
      y[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        if constexpr (NARROW)
          y[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
              __builtin_bit_cast(i16x4, hf[q]), __builtin_bit_cast(i16x4, wb[t][q]), y[t], 0, 0,
              0);
        else
          y[t] = mfma16_bf16(__builtin_bit_cast(bf16x8, hf[q]),
                             __builtin_bit_cast(bf16x8, wb[t][q]), y[t]);
      }
    }
    if (t0 + B3 < tiles3) load3(t0 + B3);
    if (lg == 0) {
#pragma unroll
      for (int t = 0; t < B3; ++t)
        if (t0 + t < tiles3) dst[(t0 + t) * 16] = y[t][0];
    }
  }
}

// out[k] = bf16(sum_j gamma_j * bf16(sum_c part[j][c][k] + b2[e_j][k])).
// A workgroup owns 32 columns: thread (r, kq) holds columns 4*kq .. +3 for
// row r = j * CP + cp (slot j, chunks c = cp, cp + CP, ... in order, CP =
// the chunk parts that fit 32 rows); the parts meet in LDS in order, then
// the slots are added in order as moe_sum adds them (product and sum
// rounded separately). gamma_j = 1 with the router weight on the input;
// dropped slots (ids outside [0, E)) add nothing.
__global__ __launch_bounds__(256) void moe_decode_reduce_kernel(const DecodeParams p) {
  const int kq = threadIdx.x & 7;
  const int r = threadIdx.x >> 3;  // 0 .. 31
  const int cp_n = max(1, 32 / p.slots);
  const int j = r / cp_n;
  const int cp = r - j * cp_n;
  const int64_t K = p.hidden;
  const int64_t k = static_cast<int64_t>(blockIdx.x) * 32 + kq * 4;
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  if (j < p.slots) {
    const int e = p.ids[j];
    if (e >= 0 && e < p.num_experts) {
      const float* src = p.part + static_cast<int64_t>(j) * p.n_chunks * K + k;
      int cc = cp;
      for (; cc + 3 * cp_n < p.n_chunks; cc += 4 * cp_n) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(src + cc * K);
        const f32x4 b = *reinterpret_cast<const f32x4*>(src + (cc + cp_n) * K);
        const f32x4 c2 = *reinterpret_cast<const f32x4*>(src + (cc + 2 * cp_n) * K);
        const f32x4 d = *reinterpret_cast<const f32x4*>(src + (cc + 3 * cp_n) * K);
        s += a;
        s += b;
        s += c2;
        s += d;
      }
      for (; cc < p.n_chunks; cc += cp_n) s += *reinterpret_cast<const f32x4*>(src + cc * K);
    }
  }
  __shared__ f32x4 sred[32][8];
  sred[r][kq] = s;
  __syncthreads();
  if (r != 0) return;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int jj = 0; jj < p.slots; ++jj) {
    const int e = p.ids[jj];
    if (e < 0 || e >= p.num_experts) continue;
    f32x4 y = sred[jj * cp_n][kq];
    for (int q = 1; q < cp_n; ++q) y += sred[jj * cp_n + q][kq];
    const float gamma = p.weight_on_input ? 1.f : p.topk_w[jj];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = y[i];
      if (p.b2) v += p.b2[static_cast<int64_t>(e) * K + k + i];
      v = bf16_bits_to_f32(f32_to_bf16_bits(v));
      acc[i] = __fadd_rn(acc[i], __fmul_rn(gamma, v));
    }
  }
  uint2 o;
  o.x = pack_bf16x2(acc[0], acc[1]);
  o.y = pack_bf16x2(acc[2], acc[3]);
  *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.out) + k) = o;
}

// FGS_MOE_F1CHUNK forces the chunk width (16, 32, 64; a tuning aid).
static int forced_chunk() {
  static const int v = [] {
    const char* s = getenv("FGS_MOE_F1CHUNK");
    const int x = s ? atoi(s) : 0;
    return (x == 16 || x == 32 || x == 64) ? x : 0;
  }();
  return v;
}

int decode_chunk(int64_t hidden, int64_t inter, int slots) {
  (void)hidden;
  const int f = forced_chunk();
  if (f && inter % f == 0) return f;
  // 32 columns per workgroup unless that gives more than 512 workgroups
  // 32 columns per workgroup; 16 when that leaves CUs idle (fewer than 256
  // workgroups), 64 when it gives more than 512
  const int64_t wgs32 = static_cast<int64_t>(slots) * (inter / 32);
  if (wgs32 < 256 && inter % 16 == 0) return 16;
  if (inter % 64 == 0 && wgs32 > 512) return 64;
  return 32;
}

// FGS_MOE_F1CFG picks the fused kernel's (waves, steps in flight) for
// tuning: 0 = (8, 4), 1 = (16, 2), 2 = (16, 3), 3 = (8, 2) (read once).
static int f1_cfg() {
  static const int v = [] {
    const char* s = getenv("FGS_MOE_F1CFG");
    const int x = s ? atoi(s) : 0;
    return (x >= 0 && x <= 3) ? x : 0;
  }();
  return v;
}

template <int C, int KW, int D>
static void launch_f1(const DecodeParams& p, hipStream_t stream) {
  constexpr int B3 = C == 16 ? 128 / KW : 128 / KW / (C / 32);  // tiles per phase-3 batch
  constexpr int G = C >= 64 ? 1 : 64 / C;  // chunks per 128-byte W2 line
  const int units = p.slots * p.n_chunks;
  const dim3 grid(static_cast<unsigned>((units + 8 * G - 1) / (8 * G) * (8 * G)));
  hipLaunchKernelGGL((moe_decode_bf16_kernel<C, KW, D, B3>), grid,
                     dim3(KW * 64), p.hidden * 2, stream, p);
}

int launch_decode_fused(const DecodeParams& p, hipStream_t stream) {
  if (p.slots < 1 || p.slots > kDecodeMaxSlots)
    return fail(FGS_EUNSUPPORTED, "single-token fused path: topk out of range");
  if (p.hidden % 256 != 0 || p.hidden > kDecodeMaxHidden || p.inter % p.chunk != 0 ||
      p.n_chunks != p.inter / p.chunk)
    return fail(FGS_EINVAL, "single-token fused path: bad shape");
  const int cfg = f1_cfg();
  if (p.chunk == 16) {
    if (cfg == 1) launch_f1<16, 16, 2>(p, stream);
    else launch_f1<16, 8, 4>(p, stream);
  } else if (p.chunk == 32) {
    if (cfg == 1) launch_f1<32, 16, 2>(p, stream);
    else if (cfg == 2) launch_f1<32, 16, 3>(p, stream);
    else if (cfg == 3) launch_f1<32, 8, 2>(p, stream);
    else launch_f1<32, 8, 4>(p, stream);
  } else if (p.chunk == 64) {
    if (cfg == 1) launch_f1<64, 16, 2>(p, stream);
    else if (cfg == 2) launch_f1<64, 16, 3>(p, stream);
    else launch_f1<64, 8, 4>(p, stream);
  } else {
    return fail(FGS_EINVAL, "single-token fused path: chunk must be 16, 32 or 64");
  }
  return check_launch("moe_decode_bf16_kernel");
}

int launch_decode_reduce(const DecodeParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(moe_decode_reduce_kernel, dim3(static_cast<unsigned>(p.hidden / 32)),
                     dim3(256), 0, stream, p);
  return check_launch("moe_decode_reduce_kernel");
}

}  // namespace fgs
