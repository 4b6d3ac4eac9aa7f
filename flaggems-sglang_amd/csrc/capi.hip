// C ABI of libfgs_moe.so (declared in include/fgs_moe.h): host-side
// validation, the kernel schedule of one fused-MoE call, the workspace
// layout and the launch sequence. No device allocation, no synchronisation.
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <array>
#include <mutex>
#include <string>
#include <vector>

#include "fgs_moe_kernels.h"

namespace fgs {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

const char* tuning_env(const char* name) {
  static const bool on = [] {
    const char* v = getenv("FGS_MOE_TUNING");
    return v && strcmp(v, "1") == 0;
  }();
  return on ? getenv(name) : nullptr;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return fail(FGS_ELAUNCH, std::string(what) + ": " + hipGetErrorString(err));
  return FGS_OK;
}

static hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

static int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

constexpr int kMaxExperts = 1024;
constexpr int kKnownFlags = FGS_FLAG_ROUTER_WEIGHT_ON_INPUT | FGS_FLAG_ACT_GELU |
                            FGS_FLAG_SEPARATE_QUANT |
                            FGS_FLAG_FORCE_DECODE | FGS_FLAG_FORCE_PREFILL |
                            FGS_FLAG_SEPARATE_SUM | FGS_FLAG_FOLD_SUM |
                            FGS_FLAG_TILE_MASK;

static int max_padded_of(int64_t numel, int e, int block) {
  return static_cast<int>(numel + static_cast<int64_t>(e) * (block - 1));
}

// ------------------------------------------------------------- schedule ---
struct Plan {
  int dt;
  int block_m;     // alignment block = rows per GEMM row block
  int mt;          // 16-row MFMA tiles per row block (streaming kernels)
  int kw1, kw2;    // waves splitting the contraction of GEMM1 / GEMM2
  bool tiled;      // LDS-tiled MFMA kernels (prefill) instead of streaming
  int tile_cfg;    // tiled kernel configuration
  int tile_cfg2;   // GEMM2's configuration (rows per block <= block_m)
  int eid_shift2;  // log2(block_m / GEMM2 block rows)
  int ksplit2;     // GEMM2 k splits (tiled only; > 1 -> fp32 partials)
  bool tail2;      // GEMM2 on the 4-wave kernel with its last round's tiles
                   // split over k (partials in the workspace, fixed up)
  bool direct;     // one token, streaming: slots index the GEMM rows directly
                   // (no alignment; distinct experts per token)
  bool direct_sum; // ... and GEMM2 folds the top-k sum (no moe_sum)
  int kwd;         // waves of the folded GEMM2
  bool pair2;      // ... two slots per MFMA (moe_gemm2_pair_kernel)
  bool qfold1;     // one token, fp8 / int8: GEMM1 quantises x itself
  bool qfold;      // one token, fp8 / int8: GEMM2 quantises the GEMM1 output rows
                   // itself (no quantiser launch between the GEMMs)
  int64_t max_padded, n_blocks, n_launch;
  // workspace layout (byte offsets)
  int64_t o_sorted, o_eids, o_npp, o_alg, o_a2, o_xq, o_xs, o_a2q, o_a2s, o_y, o_tail,
      o_xst, o_rids, o_rw, o_plan, o_plan2,
      total;
};

// k splits for the tiled GEMM2: its grid (row blocks x hidden/256 column
// tiles) is often a few waves of 256 workgroups, and a partial last wave
// idles most CUs for a whole tile. Pick the smallest split (<= 4, keeping
// >= 8 LDS stages of 128 bytes of k per split) whose expected grid fills
// >= 90 % of its last wave, else the best one. Row blocks are estimated for
// balanced routing: numel / B plus half a padded block per touched expert.
constexpr int kNumCUs = 256;  // MI355X

static int pick_ksplit(int64_t numel, int e, int bm, int64_t hidden,
                       int64_t k_bytes, bool one_block_per_expert = false) {
  const double blocks = one_block_per_expert
                            ? static_cast<double>(std::min<int64_t>(e, numel))
                            : static_cast<double>(numel) / bm +
                                  0.5 * static_cast<double>(std::min<int64_t>(e, numel));
  const double wgs = blocks * static_cast<double>(hidden / 256);
  int best = 1;
  double best_eff = 0.0;
  for (int s = 1; s <= 4; ++s) {
    if (k_bytes / 128 < 8 * s) break;
    const double waves = wgs * s / kNumCUs;
    const double eff = waves / std::ceil(waves);
    if (eff >= 0.9) return s;
    if (eff > best_eff + 1e-9) {
      best_eff = eff;
      best = s;
    }
  }
  return best;
}

// FGS_MOE_DIRECT selects the single-token schedule (a tuning aid; read
// once): 0 aligned rows, 1 direct rows with GEMM2 folding the top-k sum
// for bf16 / int8 outputs of >= 192 column tiles (the default), 2 direct
// rows with moe_sum, 3 direct rows, always folded.
static int direct_choice() {
  static const int d = [] {
    const char* v = tuning_env("FGS_MOE_DIRECT");
    const int x = v ? atoi(v) : 1;
    return (x >= 0 && x <= 3) ? x : 1;
  }();
  return d;
}

// FGS_MOE_KSPLIT (1..4) forces the tiled GEMM2's k split (a tuning aid;
// read once).
static int forced_ksplit() {
  static const int k = [] {
    const char* v = tuning_env("FGS_MOE_KSPLIT");
    const int x = v ? atoi(v) : 0;
    return (x >= 1 && x <= 4) ? x : 0;
  }();
  return k;
}

// FGS_MOE_TAIL (0 off, 1 default) switches the tail split of the 4-wave
// GEMM2 (a tuning aid; read once).
static int tail_choice() {
  static const int t = [] {
    const char* v = tuning_env("FGS_MOE_TAIL");
    const int x = v ? atoi(v) : 1;
    return (x == 0 || x == 1) ? x : 1;
  }();
  return t;
}

// FGS_MOE_PAIR (0 never, 1 always, unset: by output width) runs the folded
// single-token GEMM2 with two slots per MFMA (a tuning aid; read once).
static int pair_choice() {
  static const int f = [] {
    const char* v = tuning_env("FGS_MOE_PAIR");
    if (!v) return -1;
    return atoi(v) == 1 ? 1 : atoi(v) == 0 ? 0 : -1;
  }();
  return f;
}

// FGS_MOE_QFOLD switches the single-token GEMMs' on-the-fly activation
// quantisation: 0 off, 1 default, and for int8 2 x only (GEMM1), 3 the GEMM1
// output rows only (GEMM2), 4 both (a tuning aid; read once).
static int qfold_choice() {
  static const int q = [] {
    const char* v = tuning_env("FGS_MOE_QFOLD");
    if (!v) return 1;
    const int c = atoi(v);
    return c >= 0 && c <= 4 ? c : 1;
  }();
  return q;
}

// Waves splitting a streaming GEMM's contraction: the most (a power of two
// up to cap) that leave each wave at least min_steps k steps.
static int pick_kw(int64_t kdim, int step, int cap, int min_steps) {
  const int64_t steps = kdim / step;
  int kw = 1;
  while (kw * 2 <= cap && steps / (kw * 2) >= min_steps) kw *= 2;
  return kw;
}

static int make_plan(int64_t m, int64_t hidden, int64_t inter, int e, int topk,
                     int qmode, int flags, Plan* pl) {
  const int64_t numel = m * topk;
  Plan p{};
  p.dt = qmode == FGS_QMODE_FP8_BLOCK ? kDtFp8
         : qmode == FGS_QMODE_INT8_CHANNEL ? kDtInt8 : kDtBf16;
  const double rows_per_expert = static_cast<double>(numel) / e;
  p.mt = rows_per_expert <= 16 ? 1 : rows_per_expert <= 32 ? 2 : 4;
  p.block_m = 16 * p.mt;
  // LDS-tiled kernels (deep DMA pipeline) or the streaming kernels (weights
  // straight into registers), by the rows per expert at which the tiled
  // kernels' pipeline fill pays off, measured per element type and
  // contraction length (kmin: the shorter of the two GEMMs' k rows in
  // bytes), both schedules forced on the same box:
  // * fp8 from 3 rows per expert (DeepSeek: streaming -6 % at 2 rows,
  //   level at 3, tiled -1 % at 4);
  // * a short k row (< 2 KiB, Qwen3) from 16 (streaming -10 % at 12 rows,
  //   +4 % with skewed routing; tiled -9 % at 16);
  // * a long one (>= 8 KiB, Mixtral) from 12 (streaming -9 % at 8 rows,
  //   tiled -6 % at 12);
  // * else (Qwen2 int8) from 8 (streaming -11 % at 6 rows, level at 8,
  //   tiled -8 % at 12).
  // One token always streams (its direct-row schedule); shapes the tiled
  // kernels do not cover always stream.
  const int64_t esz = p.dt == kDtBf16 ? 2 : 1;
  const bool tiled_ok = inter % tiled_n_align(true) == 0 &&
                        hidden % tiled_n_align(false) == 0;
  const int forced_cfg = ((flags & FGS_FLAG_TILE_MASK) >> 12) - 1;
  const int64_t kmin = std::min(hidden, inter) * esz;
  double tiled_from = 8.0;
  if (p.dt == kDtFp8) tiled_from = 3.0;
  else if (kmin < 2048) tiled_from = 16.0;
  else if (kmin >= 8192) tiled_from = 12.0;
  const bool many_rows = m >= 2 && rows_per_expert >= tiled_from;
  p.tiled = tiled_ok && !(flags & FGS_FLAG_FORCE_DECODE) &&
            ((flags & FGS_FLAG_FORCE_PREFILL) || forced_cfg >= 0 || many_rows);
  p.ksplit2 = 1;
  if (p.tiled) {
    p.tile_cfg = forced_cfg >= 0 ? forced_cfg : tiled_config_for(p.dt, rows_per_expert, e);
    p.block_m = tiled_block_m(p.tile_cfg);
    // fp8 GEMM2 runs its 128-row kernel on 256-row blocks (as two halves,
    // the all-pad ones skipped): the 256-row fp8 tile spans only 128 weight
    // rows, so GEMM2 would re-read each activation tile for twice as many
    // column tiles
    p.tile_cfg2 = p.tile_cfg;
    p.eid_shift2 = 0;
    if (p.dt == kDtFp8 && p.tile_cfg == 0 && forced_cfg < 0) {
      p.tile_cfg2 = 1;
      p.eid_shift2 = 1;
    }
    // (the 160-row configuration, when forced, runs below 160 rows per
    // expert: about one block per touched expert)
    p.ksplit2 = pick_ksplit(numel, e, tiled_block_m(p.tile_cfg2), hidden, inter * esz,
                            p.tile_cfg2 == 4 && rows_per_expert < 160);
    // a forced split still keeps >= 8 LDS stages of k per split
    if (forced_ksplit() > 0 && inter * esz / 128 >= 8 * forced_ksplit())
      p.ksplit2 = forced_ksplit();
    // GEMM2 of 256-row blocks (bf16 / int8) over 1 to 8 rounds of the CUs:
    // the 4-wave kernel, whole tiles except the last round's, which are
    // split over k (instead of splitting every tile: fp32 partials of a few
    // tiles, not of all). Measured: the 4-wave kernel runs a 256 x 256 x 64
    // stage in ~1.78 us against the 8-wave kernel's ~2.1 us on the dense
    // Mixtral GEMM2, but left alone its tiles fill 2.25 rounds.
    const int64_t rows_est = numel / 256 + std::min<int64_t>(e, numel);
    const int64_t tiles_est = rows_est * (hidden / 256);
    p.tail2 = tail_choice() && p.tile_cfg2 == 0 && p.dt != kDtFp8 && forced_ksplit() == 0 &&
              tiles_est >= kNumCUs && tiles_est <= 8 * kNumCUs;
    if (p.tail2) p.ksplit2 = 1;
  }
  const int step = stream_step_k(p.dt);
  // GEMM1 on up to 4 waves; GEMM2 on as many as leave each wave 5 steps,
  // at least 2. Measured (same box, 3 x 20 flushed calls, twice): GEMM2 on
  // 2 waves instead of 8 -- Qwen2 int8 M=16 -13 %, DeepSeek fp8 M=8 -10 %,
  // Qwen3 M=16 -2.5 % (2 to 16 steps per wave); Mixtral's 112 steps level
  // at 4 and 8; GEMM1 on 2 or 1 waves is slower for Mixtral and Qwen3.
  p.kw1 = pick_kw(hidden, step, 4, 1);
  const int steps2 = static_cast<int>(inter / step);
  p.kw2 = std::max(std::min(2, steps2), pick_kw(inter, step, 8, 5));
  // One token: its top-k slots go to distinct experts, so the streaming
  // GEMMs take slot j as row tile j (expert topk_ids[j]) and the alignment
  // is skipped; GEMM2 also folds the weighted top-k sum when the output
  // spans enough column tiles (one workgroup each) to fill the chip.
  const int dc = direct_choice();
  p.direct = !p.tiled && m == 1 && dc != 0;
  // (measured, 3 x 20 flushed calls, twice: folding on one workgroup per 16
  // columns wins from 192 of them -- Qwen2 int8 -3 %, Mixtral -1.5 %,
  // DeepSeek fp8 -4 % -- and loses for Qwen3's 128, +3 %; see below for the
  // paired form)
  // One fp8 token: the GEMMs quantise their activation rows (x, the GEMM1
  // output) themselves, with the group quantiser's arithmetic. Measured
  // (DeepSeek fp8 M=1, 3 x 50 flushed calls): 88.4 -> 83.0 us. int8's
  // per-token scale needs each row's amax before any of it is quantised:
  // every wave reduces its row first (after issuing its first weight loads).
  // Measured (Qwen2 int8 M=1, 3 x 50 flushed calls, twice): 54.2 us with
  // both quantisers, 52.7 with GEMM2 quantising the GEMM1 output rows, 56.2
  // with GEMM1 quantising x (its 1280 workgroups each reduce the row), 54.4
  // with both -- so int8 folds the GEMM2 side only.
  const int qc = qfold_choice();
  const bool qa_ok = p.direct && topk <= kQaMaxSlots && !(flags & FGS_FLAG_SEPARATE_QUANT);
  if (p.dt == kDtFp8) {
    p.qfold = p.qfold1 = qa_ok && qc != 0;
  } else if (p.dt == kDtInt8) {
    p.qfold1 = qa_ok && (qc == 2 || qc == 4);
    p.qfold = qa_ok && (qc == 1 || qc == 3 || qc == 4);
  }
  // Folding needs about 192 workgroups: one per 16 output columns, or with
  // two slots per MFMA one per 8 (moe_gemm2_pair_kernel; it quantises two
  // rows per step, so it is the slower one where 16-column workgroups
  // suffice: Qwen2 int8 M=1 +5 %, DeepSeek fp8 +9 %, Mixtral +2 %; Qwen3's
  // 128 sixteen-column tiles fold only paired: 24.7 us against 27.3 for
  // GEMM2 + moe_sum and 28.0 for the one-slot fold)
  // one fp8 token's GEMM1 (k rows of 56+ steps, quantised on the fly) on
  // 8 waves: DeepSeek fp8 M=1 67.0 -> 65.9 us; 8 waves lose elsewhere
  // (Qwen3 / Qwen2 int8 / Mixtral M=1 +7..10 %, M=8..16 +3..18 %)
  if (p.direct && p.dt == kDtFp8 && hidden / step >= 48) p.kw1 = pick_kw(hidden, step, 8, 1);
  const int pairs = (topk + 1) / 2;
  const bool pair_ok = pairs <= 16 && hidden % 8 == 0;
  const bool fold_wide = hidden / 16 >= 192;
  const bool fold_pair = !fold_wide && hidden / 8 >= 192 && pair_ok;
  p.direct_sum = p.direct && !(flags & FGS_FLAG_SEPARATE_SUM) &&
                 ((flags & FGS_FLAG_FOLD_SUM) || dc == 3 ||
                  (dc == 1 && (fold_wide || fold_pair)));
  // the folded GEMM2's waves: 8 while its grid (one workgroup per 16
  // output columns) stays resident in one round at 16 waves per CU
  // (measured against 16 and 4: Mixtral M=1 110.6 -> 106.9 us, Qwen2 int8
  // 52.2 -> 51.7, DeepSeek fp8 level with 8, 4 is 7-14 % slower)
  const int64_t wgs = hidden / 16;
  p.kwd = wgs * 8 <= kNumCUs * 16 ? 8 : 4;
  // paired: (topk + 1) / 2 pairs, each on the most waves (<= 16 in all)
  // that keep 3 k steps per wave
  const int pc = pair_choice();
  p.pair2 = p.direct_sum && pair_ok && (pc == 1 || (pc == -1 && !fold_wide));
  if (p.pair2) {
    int wps = 1;
    while (pairs * wps * 2 <= 16 && steps2 / (wps * 2) >= 3) wps *= 2;
    p.kwd = 4;
    while (p.kwd < pairs * wps) p.kwd *= 2;
  }
  p.max_padded = max_padded_of(numel, e, p.block_m);
  p.n_blocks = p.max_padded / p.block_m;
  // Blocks that can hold rows: each touched expert pads at most one partial
  // block, so sum_e ceil(cnt_e / B) <= numel / B + min(E, numel). The GEMMs
  // launch only these (the rest of the expert_ids buffer is -1 anyway).
  p.n_launch = std::min<int64_t>(p.n_blocks,
                                 numel / p.block_m + std::min<int64_t>(e, numel));

  int64_t o = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = o;
    o = align_up(o + bytes, 256);
    return at;
  };
  p.o_sorted = take(p.max_padded * 4);
  p.o_eids = take(std::max<int64_t>(p.n_blocks, 1) * 4);
  p.o_npp = take(4);
  const int64_t alg = align_scratch_bytes(numel, e);
  p.o_alg = alg > 0 ? take(alg) : -1;
  p.o_a2 = take(p.max_padded * inter * 2);
  p.o_xq = p.o_xs = p.o_a2q = p.o_a2s = p.o_xst = -1;
  if (p.dt != kDtBf16) {
    p.o_xq = take(m * hidden * esz);
    p.o_xs = take(p.dt == kDtFp8 ? m * (hidden / 128) * 4 : m * 4);
    p.o_a2q = take(p.max_padded * inter * esz);
    p.o_a2s = take(p.dt == kDtFp8 ? p.max_padded * (inter / 128) * 4
                                  : p.max_padded * 4);
  }
  p.o_y = take(p.ksplit2 > 1 ? p.ksplit2 * numel * hidden * 4 : numel * hidden * 2);
  p.o_tail = p.tail2 ? take(wide_tail_part_bytes()) : -1;
  // fp8 on 256-row blocks: x's group scales gathered into the padded row
  // order, k-block-major, so a GEMM1 wave reads its 64 rows' scales of a k
  // block as one 256-byte run instead of 64 lines (measured, DeepSeek
  // M=4096: GEMM1 2.02 -> 1.86 ms for a ~10 us gather; at M <= 512 the
  // gather costs what it saves)
  if (p.tiled && p.dt == kDtFp8 && p.tile_cfg == 0)
    p.o_xst = take((hidden / 128) * p.max_padded * 4);
  // the 4-wave kernel's tile plan (256-row configuration; GEMM1, then GEMM2)
  p.o_plan = p.o_plan2 = -1;
  if (p.tiled && p.tile_cfg == 0 && p.dt != kDtFp8) {
    p.o_plan = take(4 * wide_plan_words());   // GEMM1's tile plan
    p.o_plan2 = take(4 * wide_plan_words());  // GEMM2's
  }
  // a call on the routing tuple: each flat slot's expert id and gate scale
  p.o_rids = take(numel * 4);
  p.o_rw = take(numel * 4);
  p.total = o;
  *pl = p;
  return FGS_OK;
}

static int validate(int64_t m, int64_t hidden, int64_t inter, int e, int topk,
                    int qmode, int flags, int64_t ws_bytes, bool check_ws) {
  if (m < 0) return fail(FGS_EINVAL, "m must be >= 0");
  if (hidden <= 0 || inter <= 0)
    return fail(FGS_EINVAL, "hidden and inter must be > 0");
  if (e < 1 || e > kMaxExperts)
    return fail(FGS_EINVAL, "num_experts must be in [1, 1024]");
  if (topk < 1 || topk > e)
    return fail(FGS_EINVAL, "topk must be in [1, num_experts]");
  if (qmode != FGS_QMODE_BF16 && qmode != FGS_QMODE_FP8_BLOCK &&
      qmode != FGS_QMODE_INT8_CHANNEL)
    return fail(FGS_EINVAL, "unknown qmode");
  if (flags & ~kKnownFlags) return fail(FGS_EINVAL, "unknown flag bits");
  if ((flags & FGS_FLAG_SEPARATE_SUM) && (flags & FGS_FLAG_FOLD_SUM))
    return fail(FGS_EINVAL, "FGS_FLAG_SEPARATE_SUM and FGS_FLAG_FOLD_SUM exclude each other");
  if ((flags & FGS_FLAG_FORCE_DECODE) &&
      (flags & (FGS_FLAG_FORCE_PREFILL | FGS_FLAG_TILE_MASK)))
    return fail(FGS_EINVAL, "FORCE_DECODE excludes FORCE_PREFILL / TILE");
  if (((flags & FGS_FLAG_TILE_MASK) >> 12) > kTiledConfigs)
    return fail(FGS_EINVAL, "unknown FGS_FLAG_TILE configuration");
  const int64_t numel = m * topk;
  // padded slots (alignment blocks of up to 256 rows) must fit int32 ids
  if (numel + static_cast<int64_t>(e) * 256 >= (int64_t(1) << 31))
    return fail(FGS_EUNSUPPORTED, "m * topk too large for int32 slot ids");
  const int dt = qmode == FGS_QMODE_FP8_BLOCK ? kDtFp8
                 : qmode == FGS_QMODE_INT8_CHANNEL ? kDtInt8 : kDtBf16;
  const int forced_cfg = ((flags & FGS_FLAG_TILE_MASK) >> 12) - 1;
  if (forced_cfg >= 0 && !tiled_config_supported(dt, forced_cfg))
    return fail(FGS_EUNSUPPORTED, "FGS_FLAG_TILE configuration " +
                                      std::to_string(forced_cfg) +
                                      " is not available for this qmode");
  const int step = stream_step_k(dt);
  if (hidden % step != 0 || inter % step != 0)
    return fail(FGS_EUNSUPPORTED, "hidden and inter must be multiples of " +
                                      std::to_string(step));
  if ((inter / 16) > 65535 || (hidden / 16) > 65535)
    return fail(FGS_EUNSUPPORTED, "hidden / inter too large");
  if (check_ws) {
    Plan p;
    make_plan(m, hidden, inter, e, topk, qmode, flags, &p);
    if (ws_bytes < p.total)
      return fail(FGS_EINVAL, "workspace too small: need " +
                                  std::to_string(p.total) + " bytes");
  }
  return FGS_OK;
}

// ------------------------------------------------------ stage profiler ---
// Per-thread record of HIP events around the stages of each fused call.
struct StageProfiler {
  int on = 0;  // 0 off, 1 every boundary, 2 the boundaries of stages 2..4,
               // 3 those of stage 2 (GEMM1) only
  std::vector<int> modes;  // the mode of each recorded call
  std::vector<std::array<hipEvent_t, FGS_PROFILE_STAGES + 1>> calls;
  std::vector<std::array<hipEvent_t, FGS_PROFILE_STAGES + 1>> pool;
  std::array<hipEvent_t, FGS_PROFILE_STAGES + 1>* cur = nullptr;

  ~StageProfiler() {
    for (auto* v : {&calls, &pool})
      for (auto& a : *v)
        for (hipEvent_t e : a) (void)hipEventDestroy(e);
  }
  // Starts a call record; returns false (profiling silently off) on failure.
  bool begin() {
    cur = nullptr;
    if (!on) return false;
    std::array<hipEvent_t, FGS_PROFILE_STAGES + 1> ev;
    if (!pool.empty()) {
      ev = pool.back();
      pool.pop_back();
    } else {
      for (auto& e : ev)
        if (hipEventCreate(&e) != hipSuccess) return false;
    }
    calls.push_back(ev);
    modes.push_back(on);
    cur = &calls.back();
    return true;
  }
  void mark(int i, hipStream_t s) {
    if (cur && (on == 1 || (on == 2 && i >= 2 && i <= 5) || (on == 3 && (i == 2 || i == 3))))
      (void)hipEventRecord((*cur)[i], s);
  }
};
static thread_local StageProfiler g_prof;

// ------------------------------------------------------- fused pipeline ---
struct FusedArgs {
  int qmode;
  const void* x;
  const void* w13;
  const void* w2;
  const float* w13_scale;
  const float* w2_scale;
  const float* topk_weights;
  const int32_t* topk_ids;
  int64_t m, hidden, inter;
  int e, topk, flags;
  void* ws;
  int64_t ws_bytes;
  void* out;
  hipStream_t stream;
  // bias variant: fp32 biases, swiglu(alpha, limit) activation
  const float* b13 = nullptr;
  const float* b2 = nullptr;
  bool swiglu = false;
  float alpha = 1.f, limit = 0.f;
  // stage events off for this call (the allocation-free entry point: event
  // creation is a runtime allocation)
  bool no_profile = false;
  // routing tuple input (gate_scal, gather_indx.src_indx, expt_hist) in
  // place of topk_weights / topk_ids
  const float* gate_scal = nullptr;
  const int32_t* gather_src = nullptr;
  const int32_t* expt_hist = nullptr;
};

static int run_fused(const FusedArgs& a) {
  int rc = validate(a.m, a.hidden, a.inter, a.e, a.topk, a.qmode, a.flags,
                    a.ws_bytes, true);
  if (rc) return rc;
  if (a.m == 0) return FGS_OK;  // nothing to read or write
  const bool routed = a.gather_src != nullptr;
  if (!a.x || !a.w13 || !a.w2 || !a.out || !a.ws ||
      (routed ? (!a.gate_scal || !a.expt_hist) : (!a.topk_weights || !a.topk_ids)))
    return fail(FGS_EINVAL, "null pointer argument");
  if (a.qmode != FGS_QMODE_BF16 && (!a.w13_scale || !a.w2_scale))
    return fail(FGS_EINVAL, "quantised mode needs w13_scale and w2_scale");
  if (reinterpret_cast<uintptr_t>(a.x) % 16 || reinterpret_cast<uintptr_t>(a.w13) % 16 ||
      reinterpret_cast<uintptr_t>(a.w2) % 16 || reinterpret_cast<uintptr_t>(a.out) % 16 ||
      reinterpret_cast<uintptr_t>(a.b13) % 16 || reinterpret_cast<uintptr_t>(a.b2) % 16 ||
      reinterpret_cast<uintptr_t>(a.ws) % 256)
    return fail(FGS_EINVAL, "tensors must be 16-byte aligned (workspace 256)");

  Plan p;
  make_plan(a.m, a.hidden, a.inter, a.e, a.topk, a.qmode, a.flags, &p);
  uint8_t* ws = static_cast<uint8_t*>(a.ws);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + p.o_sorted);
  int32_t* eids = reinterpret_cast<int32_t*>(ws + p.o_eids);
  int32_t* npp = reinterpret_cast<int32_t*>(ws + p.o_npp);
  uint16_t* a2 = reinterpret_cast<uint16_t*>(ws + p.o_a2);
  uint16_t* y = reinterpret_cast<uint16_t*>(ws + p.o_y);
  const int64_t numel = a.m * a.topk;
  // the per-slot routing every later stage reads
  const float* topk_w = a.topk_weights;
  const int32_t* topk_ids = a.topk_ids;

  if (a.no_profile) g_prof.cur = nullptr;
  else g_prof.begin();
  g_prof.mark(0, a.stream);
  int32_t* rids = reinterpret_cast<int32_t*>(ws + p.o_rids);
  const int32_t* route_hist = nullptr;
  float* rw = p.o_rw >= 0 ? reinterpret_cast<float*>(ws + p.o_rw) : nullptr;
  if (routed && p.direct) {
    // one token: its gathered order is its slots' ascending expert order,
    // so GEMM rows are gathered positions, weighted by gate_scal as it
    // stands; GEMM1 finds each position's expert from the histogram and
    // records it (rids) for GEMM2 and the top-k sum -- no extra launch
    topk_w = a.gate_scal;
    topk_ids = rids;
    route_hist = a.expt_hist;
  } else if (routed) {
    // the routing tuple's gathered order is the alignment's order: one
    // launch (below) gives the padded order and each slot's expert and
    // gate scale
    topk_w = rw;
    topk_ids = rids;
  }

  // operands of the two GEMMs (the quantised copies are written below)
  const bool on_input = (a.flags & FGS_FLAG_ROUTER_WEIGHT_ON_INPUT) != 0;
  const uint8_t* act = static_cast<const uint8_t*>(a.x);
  const float* act_scale = nullptr;
  if (p.qfold1) {
    // GEMM1 quantises x itself
  } else if (p.dt == kDtFp8) {
    act = ws + p.o_xq;
    act_scale = reinterpret_cast<const float*>(ws + (p.o_xst >= 0 ? p.o_xst : p.o_xs));
  } else if (p.dt == kDtInt8) {
    act = ws + p.o_xq;
    act_scale = reinterpret_cast<const float*>(ws + p.o_xs);
  }
  const uint8_t* act2 = reinterpret_cast<const uint8_t*>(a2);
  const float* act2_scale = nullptr;
  if (!p.qfold && p.dt != kDtBf16) {
    act2 = ws + p.o_a2q;
    act2_scale = reinterpret_cast<const float*>(ws + p.o_a2s);
  }

  GemmParams g1{};
  g1.a = act;
  g1.a_scale = act_scale;
  g1.w = static_cast<const uint8_t*>(a.w13);
  g1.w_scale = a.w13_scale;
  g1.sorted_ids = sorted;
  g1.expert_ids = eids;
  g1.num_post_pad = npp;
  g1.topk_w = topk_w;
  g1.out = a2;
  g1.kdim = a.hidden;
  g1.n_out = a.inter;
  g1.nrows_w = 2 * a.inter;
  g1.numel = numel;
  g1.topk = a.topk;
  g1.weight_on_input = on_input;
  g1.act = a.swiglu ? kActSwiglu : (a.flags & FGS_FLAG_ACT_GELU) ? kActGelu : kActSilu;
  g1.alpha = a.alpha;
  g1.limit = a.limit;
  g1.bias = a.b13;
  g1.a_rows = a.m;
  g1.num_experts = a.e;
  g1.a_scale_kstride = p.o_xst >= 0 ? p.max_padded : 0;
  g1.plan = p.o_plan >= 0 ? reinterpret_cast<int32_t*>(ws + p.o_plan) : nullptr;
  if (p.direct) {
    // slot j is row tile j; a2 holds the compact slot rows
    g1.direct_ids = topk_ids;
    g1.route_hist = route_hist;
    g1.route_ids = rids;
  }
  if (p.qfold1) g1.a_src = static_cast<const uint16_t*>(a.x);

  GemmParams g2 = g1;
  g2.route_hist = nullptr;
  g2.a = act2;
  g2.a_scale = act2_scale;
  g2.w = static_cast<const uint8_t*>(a.w2);
  g2.w_scale = a.w2_scale;
  g2.bias = a.b2;
  g2.out = y;
  g2.kdim = a.inter;
  g2.n_out = a.hidden;
  g2.nrows_w = a.hidden;
  g2.ksplit = p.ksplit2;
  g2.tail_split = p.tail2 ? 1 : 0;
  g2.tail_part = p.tail2 ? reinterpret_cast<float*>(ws + p.o_tail) : nullptr;
  g2.a_rows = p.max_padded;
  g2.eid_shift = p.tiled ? p.eid_shift2 : 0;
  g2.a_src = p.qfold ? a2 : nullptr;
  g2.a_scale_kstride = p.tiled && p.dt == kDtFp8 ? p.max_padded : 0;
  g2.plan = p.o_plan2 >= 0 ? reinterpret_cast<int32_t*>(ws + p.o_plan2) : nullptr;
  const int rows1 = static_cast<int>(p.n_launch);
  const int rows2 = static_cast<int>(p.n_launch << p.eid_shift2);

  if (routed && !p.direct) {
    rc = launch_routing_order(a.gate_scal, a.gather_src, a.expt_hist, numel, a.e, p.block_m,
                              p.max_padded, sorted, eids, npp, rids, rw, a.stream);
    if (rc) return rc;
  } else if (!p.direct) {
    // the alignment also writes the 4-wave GEMMs' tile plans (their launches
    // then skip the plan kernel)
    WidePlanReq req[2] = {};
    if (p.tiled) {
      tiled_plan_request(p.dt, p.tile_cfg, true, g1, rows1, &req[0]);
      tiled_plan_request(p.dt, p.tile_cfg2, false, g2, rows2, &req[1]);
    }
    bool planned = false;
    rc = launch_align(topk_ids, numel, a.e, p.block_m, sorted, eids, npp,
                      p.max_padded, a.stream,
                      p.o_alg >= 0 ? reinterpret_cast<int32_t*>(ws + p.o_alg) : nullptr,
                      req, &planned);
    if (rc) return rc;
    g1.plan_ready = planned && req[0].plan ? 1 : 0;
    g2.plan_ready = planned && req[1].plan ? 1 : 0;
  }
  g_prof.mark(1, a.stream);

  if (p.dt == kDtFp8 && !p.qfold1) {
    rc = launch_quant_fp8_group(a.x, ws + p.o_xq,
                                reinterpret_cast<float*>(ws + p.o_xs), a.m,
                                a.hidden, 128, a.stream);
    if (rc) return rc;
    if (p.o_xst >= 0) {
      float* xst = reinterpret_cast<float*>(ws + p.o_xst);
      rc = launch_scale_gather(reinterpret_cast<const float*>(ws + p.o_xs),
                               static_cast<int>(a.hidden / 128), sorted, npp, numel,
                               a.topk, p.block_m, p.max_padded, xst, a.stream);
      if (rc) return rc;
    }
  } else if (p.dt == kDtInt8 && !p.qfold1) {
    rc = launch_quant_int8_token(a.x, reinterpret_cast<int8_t*>(ws + p.o_xq),
                                 reinterpret_cast<float*>(ws + p.o_xs), a.m,
                                 a.hidden, a.stream);
    if (rc) return rc;
  }

  g_prof.mark(2, a.stream);
  rc = p.tiled ? launch_gemm_tiled(p.dt, p.tile_cfg, true, g1, rows1, a.stream)
               : launch_gemm_stream(p.dt, true, g1, p.mt, p.kw1,
                                    static_cast<int>(p.direct ? numel : p.n_launch),
                                    a.stream);
  if (rc) return rc;
  g_prof.mark(3, a.stream);

  // direct rows: the compact slot rows; else only the padded rows in use
  // (num_tokens_post_padded, on the device)
  const int64_t a2_rows = p.direct ? numel : p.max_padded;
  const int32_t* a2_npp = p.direct ? nullptr : npp;
  const int32_t* a2_sorted = p.direct ? nullptr : sorted;
  if (p.qfold) {
    // GEMM2 quantises the a2 slot rows itself
  } else if (p.dt == kDtFp8) {
    // tiled: the scales k-block-major over the padded rows (see o_xst)
    rc = launch_quant_fp8_group(a2, ws + p.o_a2q,
                                reinterpret_cast<float*>(ws + p.o_a2s),
                                a2_rows, a.inter, 128, a.stream, a2_npp, a2_sorted, numel,
                                p.tiled ? p.max_padded : 0);
    if (rc) return rc;
  } else if (p.dt == kDtInt8) {
    rc = launch_quant_int8_token(a2, reinterpret_cast<int8_t*>(ws + p.o_a2q),
                                 reinterpret_cast<float*>(ws + p.o_a2s),
                                 a2_rows, a.inter, a.stream, a2_npp, a2_sorted, numel);
    if (rc) return rc;
  }

  g_prof.mark(4, a.stream);
  if (p.direct_sum) {
    // out = the weighted top-k sum, straight from GEMM2
    g2.out = a.out;
    rc = p.pair2 ? launch_gemm2_pair(p.dt, g2, p.kwd, a.stream)
                 : launch_gemm2_direct(p.dt, g2, p.kwd, a.stream);
    if (rc) return rc;
    g_prof.mark(5, a.stream);
    g_prof.mark(6, a.stream);
    return FGS_OK;
  }
  rc = p.tiled ? launch_gemm_tiled(p.dt, p.tile_cfg2, false, g2, rows2, a.stream)
               : launch_gemm_stream(p.dt, false, g2, p.mt, p.kw2,
                                    static_cast<int>(p.direct ? numel : p.n_launch),
                                    a.stream);
  if (rc) return rc;
  g_prof.mark(5, a.stream);

  if (p.ksplit2 > 1)
    rc = launch_moe_sum_partials(reinterpret_cast<const float*>(y), p.ksplit2,
                                 a.out, a.m, a.topk, a.hidden, topk_ids, a.e,
                                 on_input ? nullptr : topk_w, a.stream);
  else
    rc = launch_moe_sum_routed(y, a.out, a.m, a.topk, a.hidden, topk_ids,
                               a.e, on_input ? nullptr : topk_w,
                               a.stream);
  g_prof.mark(6, a.stream);
  return rc;
}

// ------------------------------------------ allocation-free entry point ---
// The workspace of fgs_moe_fused_bf16_noalloc: a file-scope device array,
// one per GPU, held from library load until the process ends. Host code
// never uses the array's name as an address (in host code it is only a
// stand-in for the device symbol): each device's address comes from
// hipGetSymbolAddress, taken once per device with that device current.
static __device__ __align__(256) uint8_t scratch[FGS_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;

// Address of this device's `scratch` (nullptr with the error set on failure).
static void* device_scratch() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(FGS_ELAUNCH, std::string("no-alloc scratch: hipGetDevice: ") + hipGetErrorString(e));
    return nullptr;
  }
  static std::mutex mu;
  static void* ptrs[kMaxDevices] = {};
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      fail(FGS_ELAUNCH, std::string("no-alloc scratch: hipGetSymbolAddress: ") +
                            hipGetErrorString(e));
      return nullptr;
    }
    ptrs[dev] = p;
  }
  return ptrs[dev];
}

}  // namespace fgs

using namespace fgs;

extern "C" {

const char* fgs_moe_version(void) { return "fgs_moe 0.1.0 gfx950"; }

const char* fgs_moe_last_error(void) { return g_last_error.c_str(); }

int64_t fgs_moe_align_max_padded(int64_t numel, int32_t num_experts,
                                 int32_t block_size) {
  if (numel < 0 || num_experts < 1 || block_size < 1) return -1;
  return numel + static_cast<int64_t>(num_experts) * (block_size - 1);
}

int64_t fgs_moe_align_scratch_bytes(int64_t numel, int32_t num_experts) {
  if (numel < 0 || num_experts < 1 || num_experts > kMaxExperts) return -1;
  return align_scratch_bytes(numel, num_experts);
}

int32_t fgs_moe_align_block_size(const int32_t* topk_ids, int64_t numel,
                                 int32_t num_experts, int32_t block_size,
                                 int32_t* sorted_ids, int32_t* expert_ids,
                                 int32_t* num_post_pad, int64_t max_padded,
                                 void* scratch, int64_t scratch_bytes,
                                 void* stream) {
  if (numel < 0) return fail(FGS_EINVAL, "numel must be >= 0");
  if (num_experts < 1 || num_experts > kMaxExperts)
    return fail(FGS_EINVAL, "num_experts must be in [1, 1024]");
  if (block_size < 1 || block_size > 4096)
    return fail(FGS_EINVAL, "block_size must be in [1, 4096]");
  const int64_t need = numel + static_cast<int64_t>(num_experts) * (block_size - 1);
  if (max_padded < need)
    return fail(FGS_EINVAL, "max_padded must be >= numel + E*(block_size-1) = " +
                                std::to_string(need));
  if (max_padded >= (int64_t(1) << 31))
    return fail(FGS_EUNSUPPORTED, "max_padded must fit in int32");
  if ((numel > 0 && !topk_ids) || !sorted_ids || !expert_ids || !num_post_pad)
    return fail(FGS_EINVAL, "null pointer argument");
  // the multi-workgroup path only with enough scratch (else one workgroup)
  const int64_t need_scratch = align_scratch_bytes(numel, num_experts);
  int32_t* sc = (scratch && need_scratch > 0 && scratch_bytes >= need_scratch)
                    ? static_cast<int32_t*>(scratch) : nullptr;
  return launch_align(topk_ids, numel, num_experts, block_size, sorted_ids,
                      expert_ids, num_post_pad, max_padded, as_stream(stream), sc);
}

int64_t fgs_moe_routing_max_tiles(int64_t numel, int32_t num_experts) {
  if (numel < 0 || num_experts < 1 || num_experts > kRoutingMaxExperts) return -1;
  return routing_max_tiles(numel, num_experts);
}

int64_t fgs_moe_routing_workspace_bytes(int64_t numel, int32_t num_experts) {
  if (numel < 0 || num_experts < 1 || num_experts > kRoutingMaxExperts) return -1;
  return routing_workspace_bytes(numel, num_experts);
}

int32_t fgs_moe_topk_to_routing(const float* topk_weights, const int32_t* topk_ids,
                                int64_t m, int32_t topk, int32_t num_experts,
                                float* gate_scal, int32_t* topk_indx, int32_t* gate_indx,
                                int32_t* hist, int32_t* token_offs_raw,
                                int32_t* token_offs_pad, int32_t* block_pid_map,
                                int64_t max_tiles, void* workspace, int64_t ws_bytes,
                                void* stream) {
  if (m < 0 || topk < 1) return fail(FGS_EINVAL, "m >= 0 and topk >= 1 required");
  if (num_experts < 1 || num_experts > kRoutingMaxExperts)
    return fail(FGS_EINVAL, "num_experts must be in [1, " +
                                std::to_string(kRoutingMaxExperts) + "]");
  const int64_t numel = m * topk;
  if (numel >= (int64_t(1) << 31) / 2)
    return fail(FGS_EUNSUPPORTED, "m * topk too large for int32 indices");
  if (max_tiles < routing_max_tiles(numel, num_experts))
    return fail(FGS_EINVAL, "max_tiles must be >= fgs_moe_routing_max_tiles() = " +
                                std::to_string(routing_max_tiles(numel, num_experts)));
  if (ws_bytes < routing_workspace_bytes(numel, num_experts))
    return fail(FGS_EINVAL, "workspace too small: need " +
                                std::to_string(routing_workspace_bytes(numel, num_experts)) +
                                " bytes");
  if ((numel > 0 && (!topk_weights || !topk_ids || !gate_scal || !topk_indx || !gate_indx)) ||
      !hist || !token_offs_raw || !token_offs_pad || !block_pid_map || !workspace)
    return fail(FGS_EINVAL, "null pointer argument");
  if (reinterpret_cast<uintptr_t>(workspace) % 256)
    return fail(FGS_EINVAL, "workspace must be 256-byte aligned");
  return launch_topk_to_routing(topk_weights, topk_ids, m, topk, num_experts, gate_scal,
                                topk_indx, gate_indx, hist, token_offs_raw, token_offs_pad,
                                block_pid_map, max_tiles, workspace, as_stream(stream));
}

int32_t fgs_moe_silu_and_mul(const void* in, void* out, int64_t rows,
                             int64_t n, void* stream) {
  if (rows < 0 || n <= 0) return fail(FGS_EINVAL, "rows >= 0 and n > 0 required");
  if (n % 8) return fail(FGS_EUNSUPPORTED, "n must be a multiple of 8");
  if (rows > 0 && (!in || !out)) return fail(FGS_EINVAL, "null pointer argument");
  if (reinterpret_cast<uintptr_t>(in) % 16 || reinterpret_cast<uintptr_t>(out) % 16)
    return fail(FGS_EINVAL, "tensors must be 16-byte aligned");
  return launch_silu_and_mul(in, out, rows, n, as_stream(stream));
}

int32_t fgs_moe_sum(const void* in, void* out, int64_t m, int32_t topk,
                    int64_t k, void* stream) {
  if (m < 0 || topk < 1 || k <= 0)
    return fail(FGS_EINVAL, "m >= 0, topk >= 1 and k > 0 required");
  if (k % 8) return fail(FGS_EUNSUPPORTED, "k must be a multiple of 8");
  if (m > 0 && (!in || !out)) return fail(FGS_EINVAL, "null pointer argument");
  if (reinterpret_cast<uintptr_t>(in) % 16 || reinterpret_cast<uintptr_t>(out) % 16)
    return fail(FGS_EINVAL, "tensors must be 16-byte aligned");
  return launch_moe_sum(in, out, m, topk, k, as_stream(stream));
}

int32_t fgs_moe_topk_gating(const void* logits, int32_t logits_bf16, int64_t m,
                            int32_t num_experts, int32_t topk, int32_t scoring,
                            int32_t renormalize, float* topk_weights,
                            int32_t* topk_ids, void* stream) {
  if (m < 0) return fail(FGS_EINVAL, "m must be >= 0");
  if (num_experts < 1 || num_experts > 1024)
    return fail(FGS_EINVAL, "num_experts must be in [1, 1024]");
  if (topk < 1 || topk > num_experts || topk > 64)
    return fail(FGS_EINVAL, "topk must be in [1, min(num_experts, 64)]");
  if (scoring != FGS_SCORING_SOFTMAX && scoring != FGS_SCORING_SIGMOID)
    return fail(FGS_EINVAL, "unknown scoring function");
  if (m > 0 && (!logits || !topk_weights || !topk_ids))
    return fail(FGS_EINVAL, "null pointer argument");
  return launch_topk_gating(logits, logits_bf16 != 0, m, num_experts, topk,
                            scoring == FGS_SCORING_SIGMOID, renormalize != 0,
                            topk_weights, topk_ids, as_stream(stream));
}

int32_t fgs_moe_quant_fp8_group(const void* x, void* q, float* scales,
                                int64_t rows, int64_t cols, int32_t group,
                                void* stream) {
  if (rows < 0 || cols <= 0) return fail(FGS_EINVAL, "rows >= 0 and cols > 0 required");
  if (group < 8 || group > 512 || (group & (group - 1)) || cols % group)
    return fail(FGS_EUNSUPPORTED,
                "group must be a power of two in [8, 512] dividing cols");
  if (rows > 0 && (!x || !q || !scales))
    return fail(FGS_EINVAL, "null pointer argument");
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(q) % 8)
    return fail(FGS_EINVAL, "x must be 16-byte and q 8-byte aligned");
  return launch_quant_fp8_group(x, q, scales, rows, cols, group,
                                as_stream(stream));
}

int32_t fgs_moe_quant_int8_token(const void* x, int8_t* q, float* scales,
                                 int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols <= 0) return fail(FGS_EINVAL, "rows >= 0 and cols > 0 required");
  if (cols % 8) return fail(FGS_EUNSUPPORTED, "cols must be a multiple of 8");
  if (rows > 0 && (!x || !q || !scales))
    return fail(FGS_EINVAL, "null pointer argument");
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(q) % 8)
    return fail(FGS_EINVAL, "x must be 16-byte and q 8-byte aligned");
  return launch_quant_int8_token(x, q, scales, rows, cols, as_stream(stream));
}

int64_t fgs_moe_workspace_bytes(int64_t m, int64_t hidden, int64_t inter,
                                int32_t num_experts, int32_t topk,
                                int32_t qmode, int32_t flags) {
  if (validate(m, hidden, inter, num_experts, topk, qmode, flags, 0, false))
    return -1;
  Plan p;
  make_plan(m, hidden, inter, num_experts, topk, qmode, flags, &p);
  return p.total;
}

int32_t fgs_moe_schedule(int64_t m, int64_t hidden, int64_t inter, int32_t num_experts,
                         int32_t topk, int32_t qmode, int32_t flags, char* buf,
                         int32_t len) {
  int rc = validate(m, hidden, inter, num_experts, topk, qmode, flags, 0, false);
  if (rc) return rc;
  if (!buf || len < 1) return fail(FGS_EINVAL, "buf must hold at least one byte");
  Plan p;
  make_plan(m, hidden, inter, num_experts, topk, qmode, flags, &p);
  std::string s;
  if (p.direct) {
    s = p.direct_sum ? (p.pair2 ? "direct_sum pair" : "direct_sum") : "direct";
    if (p.qfold || p.qfold1)
      s += p.qfold && p.qfold1 ? " qfold" : p.qfold1 ? " qfold_x" : " qfold_a2";
  } else if (!p.tiled) {
    s = "stream mt=" + std::to_string(p.mt);
  } else {
    s = "tiled cfg=" + std::to_string(p.tile_cfg) + " cfg2=" + std::to_string(p.tile_cfg2);
    if (p.ksplit2 > 1) s += " ksplit2=" + std::to_string(p.ksplit2);
    if (p.tail2) s += " tail2";
  }
  const size_t n = std::min(s.size(), static_cast<size_t>(len - 1));
  memcpy(buf, s.data(), n);
  buf[n] = 0;
  return FGS_OK;
}

int32_t fgs_moe_validate(int64_t m, int64_t hidden, int64_t inter,
                         int32_t num_experts, int32_t topk, int32_t qmode,
                         int32_t flags, int64_t ws_bytes) {
  return validate(m, hidden, inter, num_experts, topk, qmode, flags, ws_bytes,
                  true);
}

int32_t fgs_moe_profile_enable(int32_t on) {
  if (on < 0 || on > 3) return fail(FGS_EINVAL, "profile mode must be 0, 1, 2 or 3");
  g_prof.on = on;
  return FGS_OK;
}

int32_t fgs_moe_profile_read(float* stage_ms, int32_t n_stages) {
  if (!stage_ms || n_stages < 1 || n_stages > FGS_PROFILE_STAGES)
    return fail(FGS_EINVAL, "stage_ms must hold 1..FGS_PROFILE_STAGES floats");
  for (int i = 0; i < n_stages; ++i) stage_ms[i] = 0.f;
  const int n = static_cast<int>(g_prof.calls.size());
  for (int c = 0; c < n; ++c) {
    auto& ev = g_prof.calls[c];
    // stages whose two boundaries this call recorded (pooled events keep
    // older recordings, which must not be mixed in)
    const int mode = g_prof.modes[c];
    const int lo = mode == 1 ? 0 : 2;
    const int hi = mode == 1 ? FGS_PROFILE_STAGES : mode == 2 ? 5 : 3;
    if (hipEventSynchronize(ev[hi]) != hipSuccess)
      return fail(FGS_ELAUNCH, "profile: event synchronisation failed");
    for (int i = lo; i < n_stages && i < hi; ++i) {
      float ms = 0.f;
      if (hipEventElapsedTime(&ms, ev[i], ev[i + 1]) == hipSuccess)
        stage_ms[i] += ms;
    }
    g_prof.pool.push_back(ev);
  }
  g_prof.calls.clear();
  g_prof.modes.clear();
  g_prof.cur = nullptr;
  if (n > 0)
    for (int i = 0; i < n_stages; ++i) stage_ms[i] /= n;
  return n;
}

int32_t fgs_moe_fused_bf16(const void* x, const void* w13, const void* w2,
                           const float* topk_weights, const int32_t* topk_ids,
                           int64_t m, int64_t hidden, int64_t inter,
                           int32_t num_experts, int32_t topk, int32_t flags,
                           void* workspace, int64_t ws_bytes, void* out,
                           void* stream) {
  FusedArgs a{FGS_QMODE_BF16, x,      w13,    w2,          nullptr,
              nullptr,        topk_weights, topk_ids, m,      hidden,
              inter,          num_experts,  topk,     flags,  workspace,
              ws_bytes,       out,          as_stream(stream)};
  return run_fused(a);
}

int32_t fgs_moe_fused_bf16_noalloc(const void* x, const void* w13, const void* w2,
                                   const float* topk_weights, const int32_t* topk_ids,
                                   int64_t m, int64_t hidden, int64_t inter,
                                   int32_t num_experts, int32_t topk, int32_t flags,
                                   void* out, void* stream) {
  int rc = validate(m, hidden, inter, num_experts, topk, FGS_QMODE_BF16, flags, 0, false);
  if (rc) return rc;
  Plan p;
  make_plan(m, hidden, inter, num_experts, topk, FGS_QMODE_BF16, flags, &p);
  if (p.total > FGS_NOALLOC_SCRATCH_BYTES)
    return fail(FGS_EUNSUPPORTED,
                "fgs_moe_fused_bf16_noalloc: this problem needs " + std::to_string(p.total) +
                    " bytes of workspace, more than the " +
                    std::to_string(static_cast<int64_t>(FGS_NOALLOC_SCRATCH_BYTES)) +
                    "-byte device scratch (use fgs_moe_fused_bf16 with a workspace)");
  if (m == 0) return FGS_OK;
  // the scratch is the current device's: a stream of another device would
  // run on memory it cannot use
  if (stream) {
    int cur = -1, sdev = -1;
    if (hipGetDevice(&cur) != hipSuccess ||
        hipStreamGetDevice(as_stream(stream), &sdev) != hipSuccess)
      return fail(FGS_ELAUNCH, "fgs_moe_fused_bf16_noalloc: cannot query the stream's device");
    if (sdev != cur)
      return fail(FGS_EINVAL, "fgs_moe_fused_bf16_noalloc: the stream belongs to device " +
                                  std::to_string(sdev) + ", the current device is " +
                                  std::to_string(cur));
  }
  void* ws = device_scratch();
  if (!ws) return FGS_ELAUNCH;
  FusedArgs a{FGS_QMODE_BF16, x,      w13,    w2,          nullptr,
              nullptr,        topk_weights, topk_ids, m,      hidden,
              inter,          num_experts,  topk,     flags,  ws,
              FGS_NOALLOC_SCRATCH_BYTES, out, as_stream(stream)};
  a.no_profile = true;
  return run_fused(a);
}

int32_t fgs_moe_fused_bf16_bias(const void* x, const void* w13, const float* b13,
                                const void* w2, const float* b2,
                                const float* topk_weights, const int32_t* topk_ids,
                                int64_t m, int64_t hidden, int64_t inter,
                                int32_t num_experts, int32_t topk, int32_t flags,
                                float alpha, float limit, void* workspace,
                                int64_t ws_bytes, void* out, void* stream) {
  if (flags & FGS_FLAG_ACT_GELU)
    return fail(FGS_EUNSUPPORTED, "the bias variant's activation is swiglu only");
  if (m > 0 && (!b13 || !b2))
    return fail(FGS_EINVAL, "bias variant needs both b13 and b2");
  if (!(alpha == alpha) || !(limit == limit))
    return fail(FGS_EINVAL, "alpha and limit must not be NaN");
  FusedArgs a{FGS_QMODE_BF16, x,      w13,    w2,          nullptr,
              nullptr,        topk_weights, topk_ids, m,      hidden,
              inter,          num_experts,  topk,     flags,  workspace,
              ws_bytes,       out,          as_stream(stream)};
  a.b13 = b13;
  a.b2 = b2;
  a.swiglu = true;
  a.alpha = alpha;
  a.limit = limit;
  return run_fused(a);
}

int32_t fgs_moe_fused_quant_bias(int32_t qmode, const void* x, const void* w13,
                                 const float* b13, const void* w2, const float* b2,
                                 const float* w13_scale, const float* w2_scale,
                                 const float* topk_weights, const int32_t* topk_ids,
                                 int64_t m, int64_t hidden, int64_t inter,
                                 int32_t num_experts, int32_t topk, int32_t flags,
                                 float alpha, float limit, void* workspace,
                                 int64_t ws_bytes, void* out, void* stream) {
  if (qmode != FGS_QMODE_FP8_BLOCK && qmode != FGS_QMODE_INT8_CHANNEL)
    return fail(FGS_EINVAL, "quantised bias variant: qmode must be fp8 block or int8 channel");
  if (flags & FGS_FLAG_ACT_GELU)
    return fail(FGS_EUNSUPPORTED, "the bias variant's activation is swiglu only");
  if (m > 0 && (!b13 || !b2))
    return fail(FGS_EINVAL, "bias variant needs both b13 and b2");
  if (!(alpha == alpha) || !(limit == limit))
    return fail(FGS_EINVAL, "alpha and limit must not be NaN");
  FusedArgs a{qmode,     x,            w13,      w2, w13_scale, w2_scale, topk_weights,
              topk_ids,  m,            hidden,   inter, num_experts, topk, flags,
              workspace, ws_bytes,     out,      as_stream(stream)};
  a.b13 = b13;
  a.b2 = b2;
  a.swiglu = true;
  a.alpha = alpha;
  a.limit = limit;
  return run_fused(a);
}

int32_t fgs_moe_fused_fp8_block(const void* x, const void* w13,
                                const void* w2, const float* w13_scale,
                                const float* w2_scale, int32_t block_n,
                                int32_t block_k, const float* topk_weights,
                                const int32_t* topk_ids, int64_t m,
                                int64_t hidden, int64_t inter,
                                int32_t num_experts, int32_t topk,
                                int32_t flags, void* workspace,
                                int64_t ws_bytes, void* out, void* stream) {
  if (block_n != 128 || block_k != 128)
    return fail(FGS_EUNSUPPORTED, "fp8 block scales must be 128x128");
  FusedArgs a{FGS_QMODE_FP8_BLOCK, x,     w13,      w2,       w13_scale,
              w2_scale,            topk_weights, topk_ids, m,  hidden,
              inter,               num_experts,  topk,     flags, workspace,
              ws_bytes,            out,          as_stream(stream)};
  return run_fused(a);
}

int32_t fgs_moe_fused_int8_channel(const void* x, const void* w13,
                                   const void* w2, const float* w13_scale,
                                   const float* w2_scale,
                                   const float* topk_weights,
                                   const int32_t* topk_ids, int64_t m,
                                   int64_t hidden, int64_t inter,
                                   int32_t num_experts, int32_t topk,
                                   int32_t flags, void* workspace,
                                   int64_t ws_bytes, void* out, void* stream) {
  FusedArgs a{FGS_QMODE_INT8_CHANNEL, x,     w13,      w2,       w13_scale,
              w2_scale,               topk_weights, topk_ids, m,  hidden,
              inter,                  num_experts,  topk,     flags, workspace,
              ws_bytes,               out,          as_stream(stream)};
  return run_fused(a);
}

int32_t fgs_moe_fused_routed(int32_t qmode, const void* x, const void* w13, const void* w2,
                             const float* w13_scale, const float* w2_scale, const float* b13,
                             const float* b2, float alpha, float limit,
                             const float* gate_scal, const int32_t* gather_src,
                             const int32_t* expt_hist, int64_t m, int64_t hidden,
                             int64_t inter, int32_t num_experts, int32_t topk, int32_t flags,
                             void* workspace, int64_t ws_bytes, void* out, void* stream) {
  const bool bias = b13 != nullptr || b2 != nullptr;
  if (bias && (!b13 || !b2)) return fail(FGS_EINVAL, "bias variant needs both b13 and b2");
  if (bias && (flags & FGS_FLAG_ACT_GELU))
    return fail(FGS_EUNSUPPORTED, "the bias variant's activation is swiglu only");
  if (bias && (!(alpha == alpha) || !(limit == limit)))
    return fail(FGS_EINVAL, "alpha and limit must not be NaN");
  if (m > 0 && (!gate_scal || !gather_src || !expt_hist))
    return fail(FGS_EINVAL, "null pointer argument");
  FusedArgs a{qmode,     x,        w13,      w2,    w13_scale,   w2_scale, nullptr,
              nullptr,   m,        hidden,   inter, num_experts, topk,     flags,
              workspace, ws_bytes, out,      as_stream(stream)};
  a.gate_scal = gate_scal;
  a.gather_src = gather_src;
  a.expt_hist = expt_hist;
  if (bias) {
    a.b13 = b13;
    a.b2 = b2;
    a.swiglu = true;
    a.alpha = alpha;
    a.limit = limit;
  }
  return run_fused(a);
}

int32_t fgs_moe_routing_to_topk(const float* gate_scal, const int32_t* gather_src,
                                const int32_t* expt_hist, int64_t m, int32_t topk,
                                int32_t num_experts, float* topk_weights, int32_t* topk_ids,
                                void* stream) {
  if (m < 0 || topk < 1) return fail(FGS_EINVAL, "m >= 0 and topk >= 1 required");
  if (num_experts < 1 || num_experts > kMaxExperts)
    return fail(FGS_EINVAL, "num_experts must be in [1, 1024]");
  const int64_t numel = m * topk;
  if (numel >= (int64_t(1) << 31))
    return fail(FGS_EUNSUPPORTED, "m * topk too large for int32 indices");
  if (numel == 0) return FGS_OK;
  if (!gate_scal || !gather_src || !expt_hist || !topk_weights || !topk_ids)
    return fail(FGS_EINVAL, "null pointer argument");
  return launch_routing_order(gate_scal, gather_src, expt_hist, numel, num_experts, 1, numel,
                              nullptr, nullptr, nullptr, topk_ids, topk_weights,
                              as_stream(stream));
}

}  // extern "C"
