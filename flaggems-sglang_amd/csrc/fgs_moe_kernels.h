// Internal interface between the C-ABI layer (capi.hip) and the kernel
// translation units. Nothing here is exported from libfgs_moe.so.
#pragma once

#include "fgs_common.h"
#include "wide_plan.h"

namespace fgs {

enum : int { kDtBf16 = 0, kDtFp8 = 1, kDtInt8 = 2 };

// One grouped GEMM over the expert-sorted, block-padded row order.
//   GEMM1: a = activations [m, kdim] gathered by token = sorted_id / topk,
//          w = w13 [E, 2*n_out, kdim], out = a2 bf16 [rows_pad, n_out].
//   GEMM2: a = a2 [rows_pad, kdim] (row = padded position),
//          w = w2 [E, n_out, kdim], out = per-slot y bf16 [numel, n_out].
constexpr int kQaMaxSlots = 64;  // on-the-fly quantisation: slots per call

struct GemmParams {
  const uint8_t* a;
  const float* a_scale;   // fp8: [rows, kdim/128]; int8: [rows]; else null
  const uint8_t* w;
  const float* w_scale;   // fp8: [E, nrows_w/128, kdim/128]; int8: [E, nrows_w]
  const int32_t* sorted_ids;
  const int32_t* expert_ids;
  const int32_t* num_post_pad;
  const float* topk_w;    // [numel]
  void* out;
  int64_t kdim;
  int64_t n_out;
  int64_t nrows_w;
  int64_t numel;
  int32_t topk;
  // slot / topk as (t + ((slot - t) >> topk_sh1)) >> topk_sh2, t = the high
  // word of topk_magic * slot (set by the 4-wave kernel's launch)
  uint32_t topk_magic;
  int32_t topk_sh1, topk_sh2;
  int32_t weight_on_input;
  int32_t row_blocks;     // row blocks of the launch (tiled kernels)
  int32_t group_m;        // row blocks per rasterization band (tiled; 0: off)
  int32_t group_n;        // column tiles per rasterization group (tiled)
  int32_t ksplit;         // GEMM2 k splits; > 1: out is fp32 [ksplit][numel][n_out]
  int32_t act;            // GEMM1 activation (kActSilu / kActGelu / kActSwiglu)
  float alpha, limit;     // swiglu parameters
  const float* bias;      // fp32 per expert: GEMM1 [E, 2N] (gate | up), GEMM2 [E, K]; or null
  int64_t a_rows;         // rows of `a` (GEMM1: tokens; GEMM2: padded rows)
  int32_t eid_shift;      // tiled: row block rb belongs to alignment block rb >> eid_shift
  const int32_t* direct_ids;  // streaming, one token: topk_ids ([numel] slots) in
                              // place of the alignment; null: aligned rows
  int32_t num_experts;        // experts of the layer (with direct_ids: the
                              // valid ids are [0, num_experts))
  int32_t tail_split;         // 4-wave GEMM2: split the last round's tiles over
                              // k into pieces (partials in tail_part, fixed up
                              // into out); needs ksplit 1
  float* tail_part;           // wide_tail_part_bytes() of fp32 partials
  const uint16_t* a_src;      // direct rows, fp8 (at most kQaMaxSlots
                              // slots): the bf16 activation
                              // rows ([a_rows, kdim]) the kernel quantises
                              // itself (a and a_scale unused); null: off
  int64_t a_scale_kstride;    // tiled fp8: > 0 -> a_scale is k-block-major
                              // over the padded rows, a_scale[kb * stride +
                              // padded row]; 0 -> [rows][kblocks]
  int32_t* plan;              // 4-wave kernel: workspace for its tile plan
                              // (wide_plan_words ints; null: no plan, the
                              // tiles are split over the XCDs by count)
  int32_t plan_ready;         // 1: the alignment has written that plan (for
                              // this launch's tiled_plan_request), so the
                              // launch skips the plan kernel
  const int32_t* route_hist;  // direct rows of a call on the routing tuple
                              // (GEMM1): row j is gathered position j, its
                              // expert found from this histogram
                              // (routed_expert_of) in place of direct_ids[j]
                              // and recorded in route_ids[j] for GEMM2 and
                              // the top-k sum; null: off
  int32_t* route_ids;
};

// Router gating (scores -> top-k -> renormalise), one wave per token;
// num_experts <= 1024, topk <= min(num_experts, 64).
int launch_topk_gating(const void* logits, bool bf16_in, int64_t m,
                       int num_experts, int topk, bool sigmoid,
                       bool renormalize, float* w_out, int32_t* id_out,
                       hipStream_t stream);

size_t align_smem_bytes(int num_experts);
// Scratch (int32 per chunk and expert) the multi-workgroup alignment uses for
// `numel` slots; 0 when the single-workgroup kernel runs.
int64_t align_scratch_bytes(int64_t numel, int num_experts);
// With `scratch` (align_scratch_bytes of it) large inputs run on many
// workgroups; without it, one workgroup. Same output either way.
// `plans` (two requests, or null): the 4-wave GEMMs' tile plans, written
// from the per-expert counts by the same launch; *planned says whether they
// were (not on the single-wave path for at most 64 slots).
int launch_align(const int32_t* ids, int64_t numel, int num_experts,
                 int block_size, int32_t* sorted_ids, int32_t* expert_ids,
                 int32_t* num_post_pad, int64_t max_padded, hipStream_t stream,
                 int32_t* scratch = nullptr, const WidePlanReq* plans = nullptr,
                 bool* planned = nullptr);

// Routing-format conversion (routing.hip): the triton_kernels routing tuple
// of _standard_topk_to_triton_kernels, block metadata for block_m in
// {16, 32, 64, 128}. num_experts <= 1022.
constexpr int kRoutingMaxExperts = 1022;
int64_t routing_max_tiles(int64_t numel, int num_experts);
int64_t routing_workspace_bytes(int64_t numel, int num_experts);
int launch_topk_to_routing(const float* weights, const int32_t* ids, int64_t m, int topk,
                           int num_experts, float* gate_scal, int32_t* topk_indx,
                           int32_t* gate_indx, int32_t* hist, int32_t* token_offs_raw,
                           int32_t* token_offs_pad, int32_t* block_pid_map,
                           int64_t max_tiles, void* workspace, hipStream_t stream);

// The routing tuple -> the alignment's padded order (sorted_ids non-null:
// sorted_ids [max_padded], expert_ids [max_padded / block], num_post_pad)
// and / or per flat slot its expert id and gate scale (ids_out non-null:
// ids_out, w_out [numel]); num_experts <= 1024. See routing.hip.
int launch_routing_order(const float* gate_scal, const int32_t* src, const int32_t* hist,
                         int64_t numel, int num_experts, int block, int64_t max_padded,
                         int32_t* sorted_ids, int32_t* expert_ids, int32_t* num_post_pad,
                         int32_t* ids_out, float* w_out, hipStream_t stream);

int launch_silu_and_mul(const void* in, void* out, int64_t rows, int64_t n,
                        hipStream_t stream);
int launch_moe_sum(const void* in, void* out, int64_t m, int topk, int64_t k,
                   hipStream_t stream);
int launch_moe_sum_routed(const void* in, void* out, int64_t m, int topk,
                          int64_t k, const int32_t* ids, int num_experts,
                          const float* weights, hipStream_t stream);
// Same reduction over fp32 split-K partials [nsplit][m*topk][k]: each slot's
// y = bf16(sum_s part[s]) (splits in order), then the weighted top-k sum.
int launch_moe_sum_partials(const float* part, int nsplit, void* out, int64_t m,
                            int topk, int64_t k, const int32_t* ids,
                            int num_experts, const float* weights,
                            hipStream_t stream);
// Activation quantisers; with `rows_dev` given only rows < *rows_dev (a
// device-side count such as num_tokens_post_padded) are processed, and with
// `sorted_ids` given the pad rows (sorted_ids[r] >= numel) are skipped.
// The int8 quantiser holds a row in a wave's registers up to
// 512 * kInt8QuantMaxVec columns; wider rows take a workgroup each.
constexpr int kInt8QuantMaxVec = 16;
// With scale_kstride > 0 the scales are stored k-block-major:
// scales[g * scale_kstride + row].
int launch_quant_fp8_group(const void* x, void* q, float* scales, int64_t rows,
                           int64_t cols, int group, hipStream_t stream,
                           const int32_t* rows_dev = nullptr,
                           const int32_t* sorted_ids = nullptr, int64_t numel = 0,
                           int64_t scale_kstride = 0);
// Per-token group scales xs [tokens][kblocks] -> k-block-major scales of
// the padded row order (out[kb * max_padded + r], rows below
// num_tokens_post_padded; a pad row gets its block's first row's scales).
int launch_scale_gather(const float* xs, int kblocks, const int32_t* sorted_ids,
                        const int32_t* num_post_pad, int64_t numel, int topk, int block,
                        int64_t max_padded, float* out, hipStream_t stream);
int launch_quant_int8_token(const void* x, int8_t* q, float* scales,
                            int64_t rows, int64_t cols, hipStream_t stream,
                            const int32_t* rows_dev = nullptr,
                            const int32_t* sorted_ids = nullptr, int64_t numel = 0);

// k elements per pipeline step of the streaming kernels (kdim must be a
// multiple of it).
int stream_step_k(int dt);
int launch_gemm_stream(int dt, bool gemm1, const GemmParams& p, int mt, int kw,
                       int row_blocks, hipStream_t stream);
// GEMM2 of one token with the top-k sum folded in (p.direct_ids set, p.out
// the bf16 [1, n_out] output); kw in {4, 8, 16}. With p.a_src (fp8, at
// most 64 slots) the slot rows are quantised on the fly.
int launch_gemm2_direct(int dt, const GemmParams& p, int kw, hipStream_t stream);
// The same with two slots per MFMA (8 output columns per workgroup, twice
// the workgroups); needs (numel + 1) / 2 <= kw and n_out % 8 == 0.
int launch_gemm2_pair(int dt, const GemmParams& p, int kw, hipStream_t stream);

// LDS-tiled MFMA kernels (bf16, fp8, int8): configuration per element type
// and rows-per-expert regime, its row block, n_out granularity, launch.
constexpr int kTiledConfigs = 5;  // row blocks 256, 128, 64, 32, 160
int tiled_config_supported(int dt, int cfg);
int tiled_config_for(int dt, double rows_per_expert, int num_experts);
int tiled_block_m(int cfg);
int tiled_n_align(bool gemm1);
int launch_gemm_tiled(int dt, int cfg, bool gemm1, const GemmParams& p,
                      int row_blocks, hipStream_t stream);
// The tile plan the launch of launch_gemm_tiled(dt, cfg, gemm1, p,
// row_blocks, ...) would make (the 4-wave kernel with a plan), for the
// alignment to write in its place; req->plan null: none.
void tiled_plan_request(int dt, int cfg, bool gemm1, const GemmParams& p, int row_blocks,
                        WidePlanReq* req);

// 4-wave kernel of the 256-row configuration (bf16, int8): whether it
// covers a launch, and the launch.
bool wide_supported(int dt, bool gemm1, const GemmParams& p);
// fp32 partial bytes the 4-wave GEMM2's tail split needs (fixed: 32 tiles
// per XCD of 256 x 256).
int64_t wide_tail_part_bytes();
int launch_gemm_wide(int dt, bool gemm1, const GemmParams& p, int row_blocks,
                     hipStream_t stream);
// The plan request of a launch_gemm_wide launch (req->plan null: no plan).
void wide_plan_request(bool gemm1, const GemmParams& p, int row_blocks, WidePlanReq* req);
// Ints of tile-plan workspace the 4-wave GEMM1 uses (gemm_wide.hip).
int64_t wide_plan_words();

}  // namespace fgs
