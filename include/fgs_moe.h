/*
 * fgs_moe.h -- C ABI of the MI355X (gfx950) fused-MoE library `libfgs_moe.so`.
 *
 * The library replaces the fused-MoE operator path of FlagGems-sglang
 * (reference: src/flaggems_sglang/ops/fused_moe.py). The reference has no
 * native FFI of its own -- its Python entry points launch Triton JIT kernels
 * and call `triton_kernels.matmul_ogs`. Each entry point below names the
 * reference function (file:line) whose work it takes over; the Python host
 * layer (flaggems_sglang.ops.fused_moe) binds them with ctypes.
 *
 * Conventions
 *   - Plain pointers to device memory and plain integer sizes. bf16 tensors
 *     are passed as `void*` (IEEE bfloat16, little endian); fp8 tensors are
 *     OCP e4m3fn bytes (max 448); int8 tensors are two's complement.
 *   - `stream` is a `hipStream_t` passed as `void*` (NULL = legacy stream).
 *   - Every launching entry point is asynchronous and stream ordered. The
 *     library never allocates or frees device memory and never synchronises;
 *     scratch memory comes in through the caller's `workspace` argument,
 *     sized with fgs_moe_workspace_bytes().
 *   - All arguments are validated on the host before any launch. Return
 *     codes: FGS_OK (0); FGS_EINVAL (-1) invalid argument; FGS_EUNSUPPORTED
 *     (-2) valid but unsupported combination; FGS_ELAUNCH (-3) HIP error.
 *     fgs_moe_last_error() returns the message of the calling thread's last
 *     failure.
 *   - Thread-safe and re-entrant: no mutable globals besides the
 *     thread-local error string and device properties cached once.
 */
#ifndef FGS_MOE_H_
#define FGS_MOE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FGS_OK 0
#define FGS_EINVAL (-1)
#define FGS_EUNSUPPORTED (-2)
#define FGS_ELAUNCH (-3)

/* Quantisation modes (`qmode` arguments). */
#define FGS_QMODE_BF16 0        /* bf16 weights and activations               */
#define FGS_QMODE_FP8_BLOCK 1   /* e4m3fn w8a8, 128x128 weight blocks, 1x128  */
#define FGS_QMODE_INT8_CHANNEL 2 /* int8 w8a8, per-channel w, per-token a     */

/* `flags` bits of the fused entry points. */
#define FGS_FLAG_ROUTER_WEIGHT_ON_INPUT 0x1 /* gammas on GEMM1 output rows */
/* GEMM1 activation gelu(gate) * up (exact erf gelu, sgl_kernel's
 * gelu_and_mul, ops/fused_moe.py:219-220) instead of silu(gate) * up */
#define FGS_FLAG_ACT_GELU 0x2
#define FGS_FLAG_FORCE_DECODE 0x100         /* schedule: streaming kernels  */
#define FGS_FLAG_FORCE_PREFILL 0x200        /* schedule: LDS-tiled kernels  */
/* schedule: the weighted top-k sum runs as its own kernel (moe_sum); a
 * one-token call otherwise folds it into GEMM2 when that is faster */
#define FGS_FLAG_SEPARATE_SUM 0x400
/* schedule: a one-token call folds the weighted top-k sum into GEMM2 */
#define FGS_FLAG_FOLD_SUM 0x800
/* schedule: a one-token fp8 / int8 call quantises its activations with the
 * separate quantiser kernels; by default (top-k <= 64) its GEMMs quantise
 * their bf16 activation rows themselves (fp8: x and the GEMM1 output; int8:
 * the GEMM1 output, per-token scales), with the quantisers' arithmetic, so
 * both give the same bytes and scales */
#define FGS_FLAG_SEPARATE_QUANT 0x8
/* schedule: LDS-tiled kernels with row-block configuration c (0: 256 rows,
 * 1: 128, 2: 64, 3: 32, 4: 160) instead of the rows-per-expert choice */
#define FGS_FLAG_TILE(c) ((((c) + 1) & 0x7) << 12)
#define FGS_FLAG_TILE_MASK 0x7000

/* Library version string, e.g. "fgs_moe 0.1.0 gfx950". */
const char* fgs_moe_version(void);

/* Message of the calling thread's most recent failed call ("" if none). */
const char* fgs_moe_last_error(void);

/* Size of the padded sorted-id buffer the alignment writes:
 * numel + num_experts * (block_size - 1). Returns -1 on invalid input. */
int64_t fgs_moe_align_max_padded(int64_t numel, int32_t num_experts,
                                 int32_t block_size);

/* moe_align_block_size: expert-grouped, block-padded routing order.
 * Replaces the routing conversion of _standard_topk_to_triton_kernels
 * (ops/fused_moe.py:119-146: stable argsort :134, histogram :137-139).
 *   topk_ids     int32 [numel] (numel = M * topk), expert id per slot.
 *   sorted_ids   int32 [max_padded]: for each expert e in ascending order,
 *                the flat slot indices i with topk_ids[i] == e in ascending
 *                i (stable), then pad entries = numel up to a multiple of
 *                block_size; entries past the padded total are numel too.
 *   expert_ids   int32 [max_padded / block_size]: expert of each block,
 *                -1 past the padded total.
 *   num_post_pad int32 [1]: padded total.
 * Slots whose id is outside [0, num_experts) are dropped (not routed).
 * Bit-exact and deterministic (no atomics decide any order).
 * scratch: device memory of fgs_moe_align_scratch_bytes() bytes (or null /
 * too small: the computation then runs on one workgroup, slower for large
 * numel); the result is identical either way. */
int32_t fgs_moe_align_block_size(const int32_t* topk_ids, int64_t numel,
                                 int32_t num_experts, int32_t block_size,
                                 int32_t* sorted_ids, int32_t* expert_ids,
                                 int32_t* num_post_pad, int64_t max_padded,
                                 void* scratch, int64_t scratch_bytes,
                                 void* stream);

/* Scratch bytes fgs_moe_align_block_size uses for numel slots (0: none
 * needed), or -1 for invalid arguments. No reference counterpart (the
 * reference's conversion runs as torch ops, ops/fused_moe.py:130-139). */
int64_t fgs_moe_align_scratch_bytes(int64_t numel, int32_t num_experts);

/* Routing-format conversion: (topk_weights, topk_ids) -> the routing tuple
 * of triton_kernels that _standard_topk_to_triton_kernels builds
 * (ops/fused_moe.py:119-146), computed on the GPU:
 *   gate_scal  f32 [numel], topk_indx int32 [numel], gate_indx int32 [numel]:
 *              the reference's per-token ascending id sort (:130-131), the
 *              stable argsort of the flattened ids (:134), its inverse
 *              (:135) and the gathered weights (:136);
 *   hist       int32 [E] (:137-139, ids outside [0, E) not counted);
 *   token_offs_raw int32 [E + 1], token_offs_pad int32 [4][E + 1] and
 *   block_pid_map int32 [4][max_tiles]: the tables of triton_kernels'
 *              compute_expt_data_torch (:140) for block_m = 16, 32, 64, 128
 *              (row i of the [4][...] arrays): exclusive sums of hist and of
 *              ceil(hist / block_m) (the latter in tiles), and per tile
 *              (b << 16) | e for expert e's b-th tile, -1 past the last.
 * numel = m * topk; num_experts <= 1022; max_tiles >=
 * fgs_moe_routing_max_tiles(numel, E) (compute_expt_data_torch's bound);
 * workspace: fgs_moe_routing_workspace_bytes(numel, E) bytes, 256-aligned.
 * Slots whose id is outside [0, E) (not routed here) sort behind expert
 * E-1, in slot order, where no expert's token_offs_raw range reaches them
 * (the reference's argsort would put negative ids ahead of expert 0; its
 * callers never pass any). Deterministic (no atomics). */
int64_t fgs_moe_routing_max_tiles(int64_t numel, int32_t num_experts);
int64_t fgs_moe_routing_workspace_bytes(int64_t numel, int32_t num_experts);
int32_t fgs_moe_topk_to_routing(const float* topk_weights, const int32_t* topk_ids,
                                int64_t m, int32_t topk, int32_t num_experts,
                                float* gate_scal, int32_t* topk_indx, int32_t* gate_indx,
                                int32_t* hist, int32_t* token_offs_raw,
                                int32_t* token_offs_pad, int32_t* block_pid_map,
                                int64_t max_tiles, void* workspace, int64_t ws_bytes,
                                void* stream);

/* The inverse conversion: the routing tuple -> per-slot (topk_weights,
 * topk_ids) in the row-sorted slot order of the tuple's flat indices (each
 * token's slots by ascending expert id, ops/fused_moe.py:130). Expert e owns
 * the gathered positions [token_offs_raw[e], token_offs_raw[e + 1]) of
 * gather_src, with token_offs_raw the exclusive sums of expt_hist -- the
 * ranges matmul_ogs reads (ops/fused_moe.py:205-231); slots at positions
 * past the histogram's total get id -1 (dropped). For v = gather_src[p]:
 * topk_ids[v] = that expert, topk_weights[v] = gate_scal[p].
 *   gate_scal f32 [m*topk], gather_src int32 [m*topk] (gather_indx.src_indx,
 *   a permutation of [0, m*topk)), expt_hist int32 [num_experts];
 *   num_experts <= 1024. Counts are clamped to the slots that exist;
 *   gather_src entries outside [0, m*topk) are skipped. */
int32_t fgs_moe_routing_to_topk(const float* gate_scal, const int32_t* gather_src,
                                const int32_t* expt_hist, int64_t m, int32_t topk,
                                int32_t num_experts, float* topk_weights, int32_t* topk_ids,
                                void* stream);

/* silu_and_mul: out[r, c] = bf16(silu(f32(in[r, c])) * f32(in[r, n + c])).
 * in bf16 [rows, 2n], out bf16 [rows, n].
 * Replaces _silu_and_mul_triton / _silu_and_mul_kernel
 * (ops/fused_moe.py:44-63, 88-116). */
int32_t fgs_moe_silu_and_mul(const void* in, void* out, int64_t rows,
                             int64_t n, void* stream);

/* moe_sum: out[t, c] = bf16(sum_j f32(in[t, j, c])), in bf16 [m, topk, k],
 * out bf16 [m, k]. Replaces the top-k reduction that matmul_ogs performs
 * with `scatter_indx` (ops/fused_moe.py:224-231). */
int32_t fgs_moe_sum(const void* in, void* out, int64_t m, int32_t topk,
                    int64_t k, void* stream);

/* Router gating: scores -> top-k -> optional renormalisation, producing
 * the (topk_weights, topk_ids) the fused entry points consume. Replaces the
 * torch routing of the reference's tests (tests/test_fused_moe.py:37-41:
 * softmax, topk, renormalise) that feeds _standard_topk_to_triton_kernels
 * (ops/fused_moe.py:119-146); sigmoid scoring for DeepSeek-style routers.
 *   logits  f32 or bf16 (logits_bf16 != 0) [m, num_experts], num_experts <= 1024
 *   topk_weights f32 [m, topk], topk_ids int32 [m, topk], topk <= 64
 * Experts are ranked by logit (descending; equal logits: lower id first) and
 * written in rank order; weights are the scores, divided by their top-k sum
 * when renormalize != 0. */
#define FGS_SCORING_SOFTMAX 0
#define FGS_SCORING_SIGMOID 1
int32_t fgs_moe_topk_gating(const void* logits, int32_t logits_bf16, int64_t m,
                            int32_t num_experts, int32_t topk, int32_t scoring,
                            int32_t renormalize, float* topk_weights,
                            int32_t* topk_ids, void* stream);

/* Dynamic per-(row, group) fp8 quantisation: x bf16 [rows, cols],
 * q e4m3fn [rows, cols], scales f32 [rows, cols / group] with
 * scale = max(amax, 1e-10) / 448 and q = e4m3fn(clamp(x / scale, +-448)).
 * group: a power of two in [8, 512] dividing cols.
 * No reference counterpart (the reference asserts fp8 off,
 * ops/fused_moe.py:170-172); needed by the fp8 w8a8 path. */
int32_t fgs_moe_quant_fp8_group(const void* x, void* q, float* scales,
                                int64_t rows, int64_t cols, int32_t group,
                                void* stream);

/* Dynamic per-row int8 quantisation: scale = max(amax, 1e-10) / 127,
 * q = clamp(rne(x / scale), -127, 127). x bf16 [rows, cols], q int8,
 * scales f32 [rows]; cols a multiple of 8.
 * No reference counterpart (ops/fused_moe.py:173-175 asserts per-channel
 * quant off); needed by the int8 w8a8 path. */
int32_t fgs_moe_quant_int8_token(const void* x, int8_t* q, float* scales,
                                 int64_t rows, int64_t cols, void* stream);

/* Workspace bytes one fused call needs for the given problem.
 * m tokens, hidden K, inter N (per-expert intermediate), num_experts E,
 * topk, qmode, flags (schedule bits matter). Returns -1 on invalid input. */
int64_t fgs_moe_workspace_bytes(int64_t m, int64_t hidden, int64_t inter,
                                int32_t num_experts, int32_t topk,
                                int32_t qmode, int32_t flags);

/* The schedule a fused call of this problem runs, as a short text into
 * buf (NUL-terminated, truncated to len - 1 bytes):
 * "direct" / "direct_sum" (one token, two streaming GEMMs, the top-k sum
 * separate / folded into GEMM2), "stream mt=T" (streaming GEMMs over the
 * aligned rows) or "tiled cfg=A cfg2=B [ksplit2=S] [tail2]" (LDS-tiled
 * GEMMs). Host-only. No counterpart in the reference (a diagnostic for
 * benchmarks and tests). */
int32_t fgs_moe_schedule(int64_t m, int64_t hidden, int64_t inter, int32_t num_experts,
                         int32_t topk, int32_t qmode, int32_t flags, char* buf,
                         int32_t len);

/* Host-only validation of a problem (no device access). Returns FGS_OK or
 * the status and message the fused entry point would return. */
int32_t fgs_moe_validate(int64_t m, int64_t hidden, int64_t inter,
                         int32_t num_experts, int32_t topk, int32_t qmode,
                         int32_t flags, int64_t ws_bytes);

/* Fused MoE, bf16. Replaces triton_kernel_fused_experts
 * (ops/fused_moe.py:149-232): routing conversion, GEMM1 (matmul_ogs with
 * gather, :205-212), silu_and_mul (:214-218), GEMM2 with top-k gammas and
 * scatter-reduce (:224-231).
 *   x            bf16 [m, hidden]
 *   w13          bf16 [E, 2*inter, hidden]  (gate rows 0..inter-1, then up)
 *   w2           bf16 [E, hidden, inter]
 *   topk_weights f32  [m, topk]
 *   topk_ids     int32 [m, topk]
 *   out          bf16 [m, hidden]
 *   out = sum_j w[t,j] * (silu(x W13g^T) * (x W13u^T)) W2^T  per token.
 * With FGS_FLAG_ROUTER_WEIGHT_ON_INPUT the gamma scales the GEMM1 output
 * rows (before the activation) and GEMM2 is unweighted
 * (ops/fused_moe.py:202-203). */
int32_t fgs_moe_fused_bf16(const void* x, const void* w13, const void* w2,
                           const float* topk_weights, const int32_t* topk_ids,
                           int64_t m, int64_t hidden, int64_t inter,
                           int32_t num_experts, int32_t topk, int32_t flags,
                           void* workspace, int64_t ws_bytes, void* out,
                           void* stream);

/* Allocation-free variant of fgs_moe_fused_bf16. No counterpart in the
 * reference: it is for callers that cannot allocate device memory -- code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc. Same arguments, kernels and results as fgs_moe_fused_bf16,
 * without the workspace: the library's own device scratch array of
 * FGS_NOALLOC_SCRATCH_BYTES per GPU (held from library load until the
 * process ends) stands in for it, and the call makes no hipMalloc / hipFree
 * or other allocating runtime call (stage profiling is off for it).
 * Problems whose workspace (fgs_moe_workspace_bytes) exceeds the scratch
 * return FGS_EUNSUPPORTED with a message naming the size, before any
 * launch. Every call on a GPU shares that GPU's scratch, which keeps the
 * last call's contents (no part of it needs to start at zero): calls that
 * overlap on one GPU -- on different streams, or from different threads
 * without ordering -- race. The scratch is the current device's: a stream
 * of another device is refused (FGS_EINVAL). Under HIP graph capture, make
 * one eager call on the device first: the first call on a device takes the
 * scratch address and sets kernel attributes, which must not happen inside
 * a capture; the captured launches use no memset and allocate nothing. */
#define FGS_NOALLOC_SCRATCH_BYTES (64ll << 20)
int32_t fgs_moe_fused_bf16_noalloc(const void* x, const void* w13, const void* w2,
                                   const float* topk_weights, const int32_t* topk_ids,
                                   int64_t m, int64_t hidden, int64_t inter,
                                   int32_t num_experts, int32_t topk, int32_t flags,
                                   void* out, void* stream);

/* Fused MoE with biases and the swiglu activation, bf16. Replaces
 * triton_kernel_fused_experts_with_bias (ops/fused_moe.py:235-325):
 * GEMM1 with bias b1 and swiglu fused (matmul_ogs(..., bias=b1,
 * fused_activation=swiglu, :303-313)), GEMM2 with bias b2 (:315-323), top-k
 * gammas and sum.
 *   w13 bf16 [E, 2*inter, hidden] (gate rows 0..inter-1, then linear rows:
 *       the reference's interleaved columns de-interleaved once by the caller)
 *   b13 f32 [E, 2*inter] (same row order), b2 f32 [E, hidden]
 *   a = bf16(g * sigmoid(alpha*g) * (u + 1)) with g = x W13g^T + b13g,
 *   u = x W13u^T + b13u and, for limit > 0, g = min(g, limit),
 *   u = clamp(u, -limit, limit); y = bf16(a W2^T + b2); out = bf16(sum_j w_j y_j).
 *   With FGS_FLAG_ROUTER_WEIGHT_ON_INPUT: a = bf16(w_j * swiglu) and
 *   out = bf16(sum_j y_j) (matmul_ogs scales its fused activation's output).
 * FGS_FLAG_ACT_GELU is rejected (the reference raises for non-silu,
 * :280-283). */
int32_t fgs_moe_fused_bf16_bias(const void* x, const void* w13, const float* b13,
                                const void* w2, const float* b2,
                                const float* topk_weights, const int32_t* topk_ids,
                                int64_t m, int64_t hidden, int64_t inter,
                                int32_t num_experts, int32_t topk, int32_t flags,
                                float alpha, float limit, void* workspace,
                                int64_t ws_bytes, void* out, void* stream);

/* The same with quantised weights: the precision configs the reference
 * threads into its two matmul_ogs calls (w1_pcg / w2_pcg,
 * ops/fused_moe.py:296-301, 303-324) carrying this build's w8a8 formats.
 *   qmode FGS_QMODE_FP8_BLOCK: w13 / w2 e4m3fn with the 128x128 block
 *       scales of fgs_moe_fused_fp8_block (activations quantised per 1x128
 *       group inside the call);
 *   qmode FGS_QMODE_INT8_CHANNEL: w13 / w2 int8 with the per-output-row
 *       scales of fgs_moe_fused_int8_channel (activations per token).
 * Biases, swiglu, gammas and the sum as fgs_moe_fused_bf16_bias; the
 * biases add to the dequantised GEMM outputs. */
int32_t fgs_moe_fused_quant_bias(int32_t qmode, const void* x, const void* w13,
                                 const float* b13, const void* w2, const float* b2,
                                 const float* w13_scale, const float* w2_scale,
                                 const float* topk_weights, const int32_t* topk_ids,
                                 int64_t m, int64_t hidden, int64_t inter,
                                 int32_t num_experts, int32_t topk, int32_t flags,
                                 float alpha, float limit, void* workspace,
                                 int64_t ws_bytes, void* out, void* stream);

/* Fused MoE on the reference's routing tuple instead of (topk_weights,
 * topk_ids): the inputs triton_kernel_fused_experts
 * (ops/fused_moe.py:149-232) and triton_kernel_fused_experts_with_bias
 * (:235-325) hand to matmul_ogs -- routing_data.gate_scal, gather_indx.src_indx
 * and routing_data.expt_hist. The tuple's gathered order is used as the
 * GEMMs' expert-sorted order directly (one kernel builds the block-padded
 * rows and each slot's expert id and gate scale; no top-k reconstruction, no
 * second alignment), with the slot conventions of fgs_moe_routing_to_topk.
 * qmode and scales as fgs_moe_fused_bf16 / _fp8_block / _int8_channel; b13
 * and b2 both null (silu, or gelu with FGS_FLAG_ACT_GELU) or both set (the
 * bias variant: swiglu(alpha, limit) as fgs_moe_fused_bf16_bias). Same
 * workspace (fgs_moe_workspace_bytes) and output as those entry points on
 * the equivalent (topk_weights, topk_ids). */
int32_t fgs_moe_fused_routed(int32_t qmode, const void* x, const void* w13, const void* w2,
                             const float* w13_scale, const float* w2_scale, const float* b13,
                             const float* b2, float alpha, float limit,
                             const float* gate_scal, const int32_t* gather_src,
                             const int32_t* expt_hist, int64_t m, int64_t hidden,
                             int64_t inter, int32_t num_experts, int32_t topk, int32_t flags,
                             void* workspace, int64_t ws_bytes, void* out, void* stream);

/* Fused MoE, fp8 w8a8 with block scales (block_n = block_k = 128).
 *   w13 e4m3fn [E, 2*inter, hidden], w13_scale f32 [E, 2*inter/128, hidden/128]
 *   w2  e4m3fn [E, hidden, inter],   w2_scale  f32 [E, hidden/128, inter/128]
 * Activations (x and the GEMM1 output) are quantised dynamically per 1x128
 * group inside the call. No reference counterpart: the reference rejects
 * use_fp8_w8a8 / w*_scale / block_shape (ops/fused_moe.py:170-185). */
int32_t fgs_moe_fused_fp8_block(const void* x, const void* w13,
                                const void* w2, const float* w13_scale,
                                const float* w2_scale, int32_t block_n,
                                int32_t block_k, const float* topk_weights,
                                const int32_t* topk_ids, int64_t m,
                                int64_t hidden, int64_t inter,
                                int32_t num_experts, int32_t topk,
                                int32_t flags, void* workspace,
                                int64_t ws_bytes, void* out, void* stream);

/* Fused MoE, int8 w8a8 with per-output-channel weight scales.
 *   w13 int8 [E, 2*inter, hidden], w13_scale f32 [E, 2*inter]
 *   w2  int8 [E, hidden, inter],   w2_scale  f32 [E, hidden]
 * Activations are quantised dynamically per token (row) inside the call.
 * No reference counterpart (per_channel_quant asserted off,
 * ops/fused_moe.py:173-175). */
int32_t fgs_moe_fused_int8_channel(const void* x, const void* w13,
                                   const void* w2, const float* w13_scale,
                                   const float* w2_scale,
                                   const float* topk_weights,
                                   const int32_t* topk_ids, int64_t m,
                                   int64_t hidden, int64_t inter,
                                   int32_t num_experts, int32_t topk,
                                   int32_t flags, void* workspace,
                                   int64_t ws_bytes, void* out, void* stream);

/* Stage timing for benchmarks. No reference counterpart (the reference
 * times the whole op with triton.testing.do_bench,
 * benchmark/performance_utils.py:365-377). While enabled on the calling
 * thread, every fused call records HIP events on its stream between its
 * stages: 0 alignment, 1 activation quantisation, 2 GEMM1 (+activation),
 * 3 GEMM2-input quantisation, 4 GEMM2, 5 top-k sum. Stages a mode does not
 * run read ~0. on = 1 records every stage boundary; on = 2 only those of
 * stages 2..4 (GEMM1 through GEMM2), so a timed run carries three fewer
 * events per call; on = 3 only GEMM1's two (the other stages then read
 * 0); on = 0 stops. */
#define FGS_PROFILE_STAGES 6
int32_t fgs_moe_profile_enable(int32_t on);

/* Waits for the recorded events, writes the mean milliseconds of each stage
 * over the calls recorded since the last read into stage_ms[0..n_stages),
 * clears the record and returns the number of calls averaged (or < 0). */
int32_t fgs_moe_profile_read(float* stage_ms, int32_t n_stages);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* FGS_MOE_H_ */
