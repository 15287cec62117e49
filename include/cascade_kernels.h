/*
 * cascade_kernels.h - C ABI of the MI355X (gfx950) cascade-decode operator set.
 *
 * Every entry point takes raw device pointers, POD sizes/strides and a
 * hipStream_t passed as `void *stream`, enqueues its kernels on that stream
 * and returns without synchronising. Return value: 0 on success, a negative
 * CK_E* code for a rejected argument (nothing is launched), or a positive
 * hipError_t from the launch. Callers own every buffer, including the
 * workspaces whose sizes the *_plan functions report. No entry point
 * allocates or frees device memory. Pointers the kernels move 16 bytes at a
 * time per lane (q, K/V pools, O rows, the padded stage-1 LSE, workspaces)
 * must be 16-byte aligned, bf16 results and the GEMM workspace (written or
 * read 8 bytes at a time) 8-byte aligned and compact LSE arrays 4-byte
 * aligned; a misaligned pointer is refused with CK_E_INVALID_ARG before any
 * launch.
 *
 * Reference interfaces replaced (paths relative to the reference root,
 * ascend-kernel/csrc/ops/ abbreviated OPS/):
 *   ck_lse_merge          <- device entry lse_merge(o1, o2, lse1, lse2, out,
 *                            totalRows, dim, o1IsF32, outIsF32, lseStride1,
 *                            lseStride2), OPS/lse_merge/op_kernel/kernel_lse_merge.cpp:343-346,
 *                            launched from OPS/lse_merge/op_host/lse_merge.cpp:67-68
 *   ck_fa_fp32_stage1     <- device entry fa_fp32_stage1(q, k, v, mask, blockTables, o,
 *                            actualQseqlen, actualKvseqlen, s/p/oTemp/oUpdate workspaces,
 *                            tiling, lse), OPS/fa_fp32_stage1/op_kernel/kernel_fa_fp32_stage1.cpp:848-863,
 *                            launched from OPS/fa_fp32_stage1/op_host/fa_fp32_stage1.cpp:325-327
 *   ck_suffix_decode      <- the stage-2 suffix attention the reference takes from the
 *                            closed CANN op npu_fused_infer_attention_score_v2
 *                            (call sites ascend-kernel/README.md:186-197,
 *                            OPS/fa_fp32_stage1/test/run_merge_probe.py:173-179)
 *   ck_f3_gateup_epilogue <- device entry f3_gateup_epilogue(a, b, workspace, d, m, nHalf,
 *                            k, mode, dStride), OPS/f3_floor/op_kernel/kernel_f3_floor.cpp:319-321,
 *                            launched from OPS/f3_floor/op_host/f3_floor.cpp:123
 *   ck_cascade_decode     <- the caller-side cascade the reference documents
 *                            (ascend-kernel/README.md:160-201: fa_fp32_stage1
 *                            flattened, FIA v2 per suffix, lse_merge) as one call
 *   ck_add_rms_norm_stats <- device entries add_rms_norm_stats_{bf16,fp16}(x1, x2, gamma,
 *                            beta, xOut, rstd, y, mRows, kDim, mode, eps, kInv, hasBeta,
 *                            batchStats, pairSum), launched from
 *                            OPS/add_rms_norm_stats/op_host/add_rms_norm_stats.cpp:130-138
 */
#ifndef CASCADE_KERNELS_H
#define CASCADE_KERNELS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error codes (negative; positive values are hipError_t) ---------------- */
#define CK_OK 0
#define CK_E_INVALID_ARG (-1)   /* a size, stride or mode is outside the supported domain */
#define CK_E_NULL_PTR (-2)      /* a required pointer is NULL */
#define CK_E_WORKSPACE (-3)     /* workspace missing or smaller than the plan requires */
#define CK_E_UNSUPPORTED (-4)   /* shape supported by the API but not by a built kernel */
#define CK_E_SCRATCH_LIMIT (-5) /* more workspace than ck_cascade_decode_noalloc's scratch holds */

/* Human-readable text for a code returned by any ck_* function. */
const char *ck_error_string(int code);

/* ---- element type tags ------------------------------------------------------ */
#define CK_DTYPE_BF16 0
#define CK_DTYPE_F32 1
#define CK_DTYPE_F16 2

/* ---- paged K/V pool layouts (block size 128, head dim 128) ----------------- */
#define CK_KV_NHD 0   /* [num_blocks, 128 tokens, kv_heads, 128]: the stage-1 pool  */
#define CK_KV_BNSD 1  /* [num_blocks, kv_heads, 128 tokens, 128]: the reference's
                         stage-2 pool (ascend-kernel/README.md:182-183)           */

/* ============================================================================
 * LSE merge of two partial attention results, per row r (fp32 arithmetic):
 *   m = max(l1, l2); w1 = exp(l1 - m); w2 = exp(l2 - m); s = w1 + w2
 *   out[r, :] = (o1[r, :] * w1 + o2[r, :] * w2) * (1 / s)
 *   lse_out[r] = m + log(s)                         (when lse_out != NULL)
 * One side at -inf contributes weight 0 (out equals the other side exactly).
 * Both sides at -inf: out = 0 and lse_out = -inf.
 *   o1, o2      [rows, dim], dtype o1_dtype / o2_dtype (CK_DTYPE_*)
 *   lse1, lse2  fp32; row r's value is lse[r * lse_stride] (1 = compact,
 *               8 = the padded layout ck_fa_fp32_stage1 writes)
 *   out         [rows, dim], dtype out_dtype
 *   lse_out     fp32 [rows] or NULL
 * Domain: rows >= 0, dim > 0 and dim % 16 == 0, strides in [1, 64].
 * Replaces OPS/lse_merge/op_kernel/kernel_lse_merge.cpp:343-346 (o2 fp32 and
 * lse_out are additions; the reference takes o2 bf16 only and has no lse_out).
 * ========================================================================== */
int ck_lse_merge(const void *o1, int o1_dtype, const void *o2, int o2_dtype,
                 const float *lse1, int64_t lse1_stride, const float *lse2, int64_t lse2_stride,
                 void *out, int out_dtype, float *lse_out, int64_t rows, int64_t dim,
                 void *stream);

/* ============================================================================
 * Stage-1 paged flash attention over a shared prefix (no mask, GQA).
 *   q            bf16 [num_tokens, num_heads, 128]; request b owns tokens
 *                [q_start(b), q_start(b) + q_len(b))
 *   k, v         bf16 [num_blocks, 128, kv_heads, 128] (token-major pages)
 *   block_table  int32 [batch, bt_cols]; logical kv token j of request b is
 *                k[block_table[b * bt_cols + j / 128], j % 128, kv_head, :]
 *   kv_seqlens   int64 [batch] on the device (read by the kernel)
 *   q_seqlens    int64 [batch] on the device; read only when q_len_uniform == 0
 *   q_start      int32 [batch] on the device; read only when q_len_uniform == 0
 *   q_len_uniform  > 0: every request has this q length, q_start(b) = b * q_len_uniform
 *                  = 0: per-request q_seqlens / q_start
 *   max_q_len    upper bound of q_len(b) (equals q_len_uniform when that is > 0)
 *   kv_cap       upper bound of kv_seqlens(b), <= bt_cols * 128; tokens beyond
 *                min(kv_seqlens(b), bt_cols * 128) are never read
 *   scale        softmax scale, finite and > 0 (the reference fixes 1/sqrt(128),
 *                OPS/fa_fp32_stage1/design.md:73); CK_E_INVALID_ARG otherwise
 *   out          fp32 [num_tokens, num_heads, 128] = softmax(q k^T * scale) v
 *   lse          fp32 [num_tokens * num_heads * 8]; row (t * num_heads + h)
 *                holds 8 identical copies of log(sum exp(q k^T * scale))
 *   workspace    device buffer of ck_fa_fp32_stage1_plan's workspace_bytes
 *                (may be NULL when that is 0)
 * P = exp(S - rowmax) is rounded to bf16 (RNE) before the PV product and the
 * row sums use the unrounded fp32 values, as
 * third_party/catlass/.../block_epilogue_online_softmax_no_mask.hpp:487-594 does.
 * Replaces OPS/fa_fp32_stage1/op_kernel/kernel_fa_fp32_stage1.cpp:848-863.
 * ========================================================================== */
int ck_fa_fp32_stage1_plan(int64_t batch, int64_t max_q_len, int64_t num_heads, int64_t kv_heads,
                           int64_t head_dim, int64_t kv_cap, int64_t *num_splits,
                           int64_t *workspace_bytes);

int ck_fa_fp32_stage1(const void *q, const void *k, const void *v, const int32_t *block_table,
                      int64_t bt_cols, const int64_t *q_seqlens, const int64_t *kv_seqlens,
                      const int32_t *q_start, int64_t batch, int64_t q_len_uniform,
                      int64_t max_q_len, int64_t num_tokens, int64_t num_heads, int64_t kv_heads,
                      int64_t head_dim, int64_t num_blocks, int64_t block_size, float scale,
                      int64_t kv_cap, int64_t num_splits, float *out, float *lse,
                      void *workspace, int64_t workspace_bytes, void *stream);

/* ============================================================================
 * Per-sequence paged decode attention over each sequence's own suffix
 * (one query token per sequence, GQA; P at fp32 precision).
 *   q            bf16 [batch, num_heads, 128]
 *   k, v         bf16 paged pool in layout kv_layout: CK_KV_NHD
 *                [num_blocks, 128, kv_heads, 128] or CK_KV_BNSD
 *                [num_blocks, kv_heads, 128, 128] (same results)
 *   block_table  int32 [batch, bt_cols]; kv_seqlens int64 [batch] on the device
 *   out          bf16 [batch, num_heads, 128]
 *   lse          fp32 [batch * num_heads] (compact); a sequence with kv length 0
 *                gets out = 0 and lse = -inf (an empty suffix)
 *   kv_cap       upper bound of kv_seqlens(b), <= bt_cols * 128
 *   num_splits   workgroups per kv head group that share the list of 64-token
 *                windows (<= 0: the plan's count, as many as are resident at
 *                once); the plan sizes the workspace for it. A GQA group of
 *                more than 8 query heads per kv head is split into the fewest
 *                equal groups of at most 8, each streamed as its own kv head
 *                group (the K/V pages are then read once per group).
 * Same softmax arithmetic as ck_fa_fp32_stage1 (fp32 accumulation).
 * Replaces the closed CANN op npu_fused_infer_attention_score_v2 used as
 * stage 2 (ascend-kernel/README.md:186-197).
 * ========================================================================== */
int ck_suffix_decode_plan(int64_t batch, int64_t num_heads, int64_t kv_heads, int64_t head_dim,
                          int64_t kv_cap, int64_t *num_splits, int64_t *workspace_bytes);

int ck_suffix_decode(const void *q, const void *k, const void *v, const int32_t *block_table,
                     int64_t bt_cols, const int64_t *kv_seqlens, int64_t batch, int64_t num_heads,
                     int64_t kv_heads, int64_t head_dim, int64_t num_blocks, int64_t block_size,
                     int64_t kv_layout, float scale, int64_t kv_cap, int64_t num_splits, void *out, float *lse,
                     void *workspace, int64_t workspace_bytes, void *stream);

/* ============================================================================
 * Fused cascade decode of B single-token queries that share one prefix.
 *   q                 bf16 [batch, num_heads, 128]
 *   prefix_k/v        bf16 [prefix_num_blocks, 128, kv_heads, 128]
 *   prefix_block_table int32 [1, prefix_bt_cols]; prefix_kv_seqlen int64 [1]
 *                     on the device (the shared prefix length)
 *   suffix_k/v        bf16 suffix pool in layout suffix_kv_layout (CK_KV_NHD,
 *                     or CK_KV_BNSD [suffix_num_blocks, kv_heads, 128, 128]);
 *                     an NHD suffix pool may be the prefix pool itself
 *   suffix_block_table int32 [batch, suffix_bt_cols]; suffix_kv_seqlens int64
 *                     [batch] on the device (0 = empty suffix)
 *   out               bf16 [batch, num_heads, 128]: attention of each query over
 *                     prefix + its own suffix
 *   lse_out           fp32 [batch * num_heads]: the merged log-sum-exp
 *   prefix_cap / suffix_cap  bounds of the kv lengths, <= bt_cols * 128
 * Arithmetic: stage-1 as ck_fa_fp32_stage1 (bf16 P into the PV product),
 * suffix as ck_suffix_decode (fp32 P), merge as ck_lse_merge with lse_out;
 * the stage-1 split partials and cut-suffix partials are folded in fp32
 * without an intermediate bf16 or fp32 output pass.
 * Replaces the composition fa_fp32_stage1 -> FIA v2 -> lse_merge of
 * ascend-kernel/README.md:160-201.
 * ========================================================================== */
int ck_cascade_decode_plan(int64_t batch, int64_t num_heads, int64_t kv_heads, int64_t head_dim,
                           int64_t prefix_cap, int64_t suffix_cap, int64_t *workspace_bytes);

int ck_cascade_decode(const void *q, const void *prefix_k, const void *prefix_v,
                      const int32_t *prefix_block_table, int64_t prefix_bt_cols,
                      const int64_t *prefix_kv_seqlen, int64_t prefix_num_blocks, const void *suffix_k,
                      const void *suffix_v, const int32_t *suffix_block_table, int64_t suffix_bt_cols,
                      const int64_t *suffix_kv_seqlens, int64_t suffix_num_blocks,
                      int64_t suffix_kv_layout, int64_t batch,
                      int64_t num_heads, int64_t kv_heads, int64_t head_dim, int64_t block_size,
                      float scale, int64_t prefix_cap, int64_t suffix_cap, void *out, float *lse_out,
                      void *workspace, int64_t workspace_bytes, void *stream);

/* ============================================================================
 * ck_cascade_decode without a workspace argument, for callers that cannot
 * allocate (code under HIP-graph capture, serving loops that forbid
 * allocation). No counterpart in the reference. Arguments and results are
 * those of ck_cascade_decode; the workspace is a device array inside this
 * library, 32 MiB per GPU (CK_CASCADE_NOALLOC_SCRATCH_BYTES), held by every GPU
 * the library runs on until the process ends. A shape whose
 * ck_cascade_decode_plan exceeds it is refused with CK_E_SCRATCH_LIMIT before
 * anything is launched. The call allocates and frees nothing. All calls on one
 * GPU share its array: calls that overlap on one GPU (other streams, other
 * threads) race and must be serialised by the caller.
 * ========================================================================== */
#define CK_CASCADE_NOALLOC_SCRATCH_BYTES (32ll << 20)

int ck_cascade_decode_noalloc(const void *q, const void *prefix_k, const void *prefix_v,
                              const int32_t *prefix_block_table, int64_t prefix_bt_cols,
                              const int64_t *prefix_kv_seqlen, int64_t prefix_num_blocks, const void *suffix_k,
                              const void *suffix_v, const int32_t *suffix_block_table, int64_t suffix_bt_cols,
                              const int64_t *suffix_kv_seqlens, int64_t suffix_num_blocks,
                              int64_t suffix_kv_layout, int64_t batch,
                              int64_t num_heads, int64_t kv_heads, int64_t head_dim, int64_t block_size,
                              float scale, int64_t prefix_cap, int64_t suffix_cap, void *out, float *lse_out,
                              void *stream);

/* ============================================================================
 * gate_up GEMM with the epilogue ladder of OPS/f3_floor (bf16, fp32 accumulate).
 *   a          bf16 [m, k] row-major (activations)
 *   b          bf16 [2 * n_half, k] row-major (nn.Linear weight: gate rows
 *              0..n_half-1, up rows n_half..2*n_half-1)
 *   workspace  bf16 [m, 2 * n_half] = C = a b^T (RNE), written by modes
 *              0, 2, 4, 5, 7, 8; read by mode 3; untouched by mode 1
 *   d          bf16 [m, n_half] with row stride d_stride (elements)
 *   mode 0: d = C[:, :n_half]            mode 1: d = silu(g) * u, fused: g and u
 *   mode 2: C only                                are the fp32 accumulators
 *   mode 3: d = workspace[:, :n_half]    mode 4: d = C[:, n_half:]
 *   mode 5: d = C[:, :n_half]            mode 7: C only (d not written)
 *   mode 8: C, and d = 0
 * Domain: m >= 1, k >= 64 and k % 16 == 0, n_half % 128 == 0,
 * d_stride >= n_half and d_stride % 4 == 0; a and b 16-byte aligned, d and
 * workspace 8-byte aligned (CK_E_INVALID_ARG otherwise). silu(x) = x / (1 + exp(-x)).
 * Replaces OPS/f3_floor/op_kernel/kernel_f3_floor.cpp:319-321.
 * ========================================================================== */
int ck_f3_gateup_epilogue(const void *a, const void *b, void *workspace, void *d, int64_t m,
                          int64_t n_half, int64_t k, int64_t mode, int64_t d_stride, void *stream);

/* ============================================================================
 * Residual add + RMSNorm statistics (+ apply): the norm stage of the
 * reference's F2 fusion study (OPS/add_rms_norm_stats/design.md:37-62). Per
 * row r of the [m_rows, k_dim] inputs, with rd() = rounding to the data dtype:
 *   mode 0: x_out = rd(x1 + x2);  rstd = 1 / sqrt(mean_k(x_out^2) + eps)
 *   mode 1: rstd from x1 (the already rounded residual);
 *           y = rd(rd(x1 * rstd) * gamma + beta)          (beta NULL = no bias)
 *   mode 2: rstd of rd(x1 + x2) only
 *   x1, x2, x_out, y  [m_rows, k_dim] contiguous, dtype CK_DTYPE_BF16 or CK_DTYPE_F16
 *   gamma, beta       [k_dim], same dtype (mode 1)
 *   rstd              fp32 [ceil(m_rows / 8) * 8]; rows >= m_rows are written 0
 * x2 is not read in mode 1; x_out is written in mode 0 only, y in mode 1 only.
 * The statistics and the apply products are evaluated in fp64 and every rd()
 * goes fp64 -> fp32 -> dtype (RNE twice), as the reference's fp64 model casts
 * (OPS/add_rms_norm_stats/test/add_rms_norm_stats_ref.py:139-156).
 * Domain: 0 < k_dim <= 5120, k_dim % 16 == 0, m_rows >= 0, eps > 0 and finite,
 * mode in {0, 1, 2}.
 * Replaces the device entries add_rms_norm_stats_{bf16,fp16} of
 * OPS/add_rms_norm_stats/op_kernel/kernel_add_rms_norm_stats.cpp:453.
 * ========================================================================== */
int ck_add_rms_norm_stats(const void *x1, const void *x2, const void *gamma, const void *beta,
                          void *x_out, float *rstd, void *y, int64_t m_rows, int64_t k_dim,
                          int dtype, int64_t mode, double eps, void *stream);

/* ============================================================================
 * Health counter of the bounded waits inside the suffix and fused cascade
 * kernels (ck_suffix_decode, ck_cascade_decode, ck_cascade_decode_noalloc).
 * Their waves wait on each other only through LDS counters whose waits are
 * bounded (a hang is never possible); a wait that runs out means a broken
 * invariant and wrong results, and is counted on the device. *count receives
 * the number counted on the current device since the library was loaded or
 * last reset; reset != 0 sets it back to 0. Synchronous: call it after the
 * kernels of interest have completed (e.g. after hipDeviceSynchronize).
 * No counterpart in the reference (its waits are hardware pipe flags).
 * ========================================================================== */
int ck_wait_giveups(uint64_t *count, int reset);

/* ============================================================================
 * Benchmark-only probes of the measured ceilings the roofline fractions are
 * quoted against (no production path calls them). They take the measurement
 * role of the reference's benchmark-only bandwidth probe
 * (OPS/bw_probe/design.md:1-30); the code and access patterns are this
 * library's own.
 *   ck_bw_probe  variant 0: stream-read `bytes` from src (each lane folds its
 *                16-byte loads into one word of `sink`, sink_bytes >=
 *                CK_PROBE_SINK_BYTES); variant 1: copy `bytes` from src to dst.
 *                bytes % 16 == 0; src, dst 16-byte aligned.
 *   ck_mfma_probe  iterations (1 .. 2^24) rounds of 16 independent
 *                v_mfma_f32_32x32x16_bf16 per wave on register operands, two
 *                waves per SIMD; *flops receives the work launched (set before
 *                the kernel runs; time it with events on `stream`); sink as above.
 * ========================================================================== */
#define CK_PROBE_SINK_BYTES (2ll << 20)

int ck_bw_probe(const void *src, void *dst, int64_t bytes, int variant, void *sink, int64_t sink_bytes,
                void *stream);

int ck_mfma_probe(int64_t iterations, void *sink, int64_t sink_bytes, double *flops, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* CASCADE_KERNELS_H */
