/*
 * CPU restatement of moe_align_block_size -- TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this; the product path never does.
 *
 * Follows the reference's routing conversion
 * (src/flaggems_sglang/ops/fused_moe.py:133-139): the expert-grouped order is
 * the stable argsort of the flattened expert ids (:134) and the per-expert
 * counts are its histogram (:137-139). Restated as a stable counting sort,
 * then padded per expert to a multiple of the block size with the sentinel
 * `numel` (the block layout the grouped GEMMs consume).
 */
#include <stdint.h>
#include <stdlib.h>

/* Returns 0 on success, -1 on invalid arguments. */
int oracle_align(const int32_t* ids, int64_t numel, int32_t num_experts,
                 int32_t block_size, int32_t* sorted_ids, int32_t* expert_ids,
                 int32_t* num_post_pad, int64_t max_padded) {
  if (numel < 0 || num_experts < 1 || block_size < 1) return -1;
  if (max_padded < numel + (int64_t)num_experts * (block_size - 1)) return -1;
  int64_t* cnt = (int64_t*)calloc((size_t)num_experts, sizeof(int64_t));
  int64_t* off = (int64_t*)calloc((size_t)num_experts + 1, sizeof(int64_t));
  int64_t* cur = (int64_t*)calloc((size_t)num_experts, sizeof(int64_t));
  if (!cnt || !off || !cur) {
    free(cnt); free(off); free(cur);
    return -1;
  }
  /* histogram (ids outside [0, E) are not routed) */
  for (int64_t i = 0; i < numel; ++i)
    if (ids[i] >= 0 && ids[i] < num_experts) cnt[ids[i]]++;
  /* padded exclusive prefix sum */
  for (int e = 0; e < num_experts; ++e) {
    int64_t padded = (cnt[e] + block_size - 1) / block_size * block_size;
    off[e + 1] = off[e] + padded;
  }
  for (int64_t p = 0; p < max_padded; ++p) sorted_ids[p] = (int32_t)numel;
  /* stable scatter: ascending slot index within each expert */
  for (int64_t i = 0; i < numel; ++i) {
    int e = ids[i];
    if (e < 0 || e >= num_experts) continue;
    sorted_ids[off[e] + cur[e]++] = (int32_t)i;
  }
  int64_t nblocks = max_padded / block_size;
  for (int64_t b = 0; b < nblocks; ++b) expert_ids[b] = -1;
  for (int e = 0; e < num_experts; ++e)
    for (int64_t b = off[e] / block_size; b < off[e + 1] / block_size; ++b)
      expert_ids[b] = e;
  *num_post_pad = (int32_t)off[num_experts];
  free(cnt); free(off); free(cur);
  return 0;
}
