// ck_internal.h - launch helpers shared between the translation units of
// libcascade_hip.so (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "stage1_wide.h"

namespace ck {

// fa_stage1.hip: validates and launches stage-1 exactly as ck_fa_fp32_stage1.
// With combine == false and more than one split, the split partials stay in
// the workspace -- part_o fp32 [splits][num_tokens * num_heads][128] followed
// by part_lse fp32 [splits][num_tokens * num_heads] -- and out/lse are not
// written; with one split out/lse are written as usual. *splits_used reports
// the split count of the plan.
int stage1_launch(const void *q, const void *k, const void *v, const int32_t *block_table, int64_t bt_cols,
                  const int64_t *q_seqlens, const int64_t *kv_seqlens, const int32_t *q_start, int64_t batch,
                  int64_t q_len_uniform, int64_t max_q_len, int64_t num_tokens, int64_t num_heads,
                  int64_t kv_heads, int64_t head_dim, int64_t num_blocks, int64_t block_size, float scale,
                  int64_t kv_cap, int64_t num_splits, float *out, float *lse, void *workspace,
                  int64_t workspace_bytes, bool combine, hipStream_t stream, int64_t *splits_used);

// fa_stage1.hip: the stage-1 role of the fused cascade kernel (suffix_decode.hip)
// for B decode queries flattened into one request: 128-row units over splits of
// the prefix, about `target` units. stage1_fused_plan sizes it (units, splits,
// workspace bytes for the partials); stage1_fused_args validates the operands
// and fills the kernel arguments (with one split, out/lse receive the result).
void stage1_fused_plan(int64_t batch, int64_t num_heads, int64_t kv_heads, int64_t kv_cap, int64_t target,
                       int64_t *units, int64_t *splits, int64_t *ws_bytes);
int stage1_fused_args(const void *q, const void *k, const void *v, const int32_t *block_table, int64_t bt_cols,
                      const int64_t *kv_seqlen, int64_t batch, int64_t num_heads, int64_t kv_heads,
                      int64_t num_blocks, float scale, int64_t kv_cap, int64_t target, float *out, float *lse,
                      void *workspace, int64_t workspace_bytes, s1::Stage1Args *a, int64_t *units,
                      int64_t *splits_used);

// suffix_decode.hip: sequences per launch of the suffix stream kernel, its
// chunk count and the workspace one launch group needs.
int64_t suffix_group_batch(int64_t kv_cap);
int64_t suffix_default_chunks(int64_t num_heads, int64_t kv_heads);
int64_t suffix_group_ws_bytes(int64_t nb, int64_t num_heads, int64_t kv_heads, int64_t chunks);

// Stage-1 result the cascade epilogue folds in, for query token b (row b * H + h).
struct Stage1Result {
    const float *o;    // splits > 1: [splits][rows][128] partials; else [rows][128]
    const float *lse;  // splits > 1: [splits][rows]; else [rows * 8] (padded)
    int64_t rows;      // batch * num_heads
    int splits;
};

// Chunks per kv head group of the fused cascade kernel: a pair per fused
// workgroup (one workgroup per CU), one for each of its two roles.
int64_t suffix_fused_chunks(int64_t num_heads, int64_t kv_heads);

// Suffix kernels for sequences [b0, b0 + nb) of a batch (nb <= suffix_group_batch).
// With fixup, out/lse receive the final suffix result (ck_suffix_decode); with
// a stage-1 result instead (cascade), whole sequences go to out/lse (bf16 /
// fp32 scratch indexed from b0) and the cascade epilogue writes the merged
// result of every sequence of the group to final_out/final_lse. With `fused`
// (stage-1 arguments from stage1_fused_args, fused_units units) one fused
// kernel runs the stage-1 units and the suffix chunks side by side instead.
int suffix_launch_group(const void *q, const void *k, const void *v, const int32_t *block_table, int64_t bt_cols,
                        const int64_t *kv_seqlens, int64_t b0, int64_t nb, int64_t num_heads, int64_t kv_heads,
                        int64_t num_blocks, int64_t kv_layout, float scale, int64_t kv_cap, int64_t chunks,
                        void *out, float *lse, void *group_ws, const Stage1Result *cascade, void *final_out,
                        float *final_lse, hipStream_t stream, const s1::Stage1Args *fused = nullptr,
                        int64_t fused_units = 0);

}  // namespace ck
