// fa_stage1.hip - stage-1 shared-prefix paged flash attention on gfx950 MFMA.
//
// Semantics (reference: ascend-kernel/csrc/ops/fa_fp32_stage1 and the CATLASS
// FAI blocks it instantiates; fp64 model in its test/fa_fp32_ref.py:82-126):
//   for every query row (token t, head h) of request b, kv head g = h / (H/KVH):
//     S = (q k^T) * scale                      fp32, scale = 1/sqrt(128)
//     online softmax over kv tiles: m = running max, dm = exp(m_old - m),
//       p = exp(S - m), P = bf16_RNE(p) feeds PV, l = dm*l + rowsum(p) (fp32, unrounded)
//     O = acc / l (fp32 out), LSE = ln(l) + m, written as 8 identical fp32 per row
//   kv token j of request b is page block_table[b][j / 128], row j % 128
//   (CATLASS block_mmad_fai_qk_normal.hpp:157-169; row stride = bt_cols,
//   op_host/fa_fp32_stage1.cpp:238).
//
// MI355X design (not a translation of the AIC/AIV pipeline):
// * Work item = (request b, kv head g, m-tile of query rows, kv split).
//   Query rows of one kv head are token-major (row r -> token r / group,
//   head g*group + r % group), so the GQA group and every query of the request
//   that shares the prefix ride in the same MFMA tile: the flattened cascade
//   form (one request, q_len = batch) reads each prefix page once per m-tile.
// * Every wave owns 32 query rows and all tokens of them, so a row has one
//   online-softmax state over the whole split and P is rounded on the row's
//   own running maximum (moved once per 64-token tile; for kv <= 64 that is
//   the row maximum the reference rounds on). Two kernels run the same body
//   (stage1_wide.h):
//   - stage1_narrow_kernel (m-tile of 128 rows): 4 waves with at most 256
//     registers each and a 3-slot K/V ring, the body the fused cascade kernel
//     runs as its stage-1 role.
//   - stage1_wide_kernel (m-tile of 256 rows, when a request has more than 128
//     rows per kv head and enough kv to fill the chip): 8 waves, two per SIMD;
//     every 64-token K/V tile in LDS feeds 256 rows, and one wave of a SIMD
//     issues MFMAs while the other waits on reads or runs its softmax.
//   K/V tiles land by buffer->LDS DMA (buffer_load_dwordx4 ... lds, 16 B per
//   lane, one buffer resource per tile; no staging registers, no vector address
//   arithmetic); the split's page ids are read once into LDS, so no
//   load in the loop depends on another load. Q stays in registers as MFMA
//   operands for the whole kv loop.
// * S^T = K Q^T on v_mfma_f32_32x32x16_bf16 (A = K rows from LDS, B = Q); the
//   accumulator layout puts one query row per lane, so row max / row sum need a
//   single cross-half exchange. P^T leaves the accumulator directly as the B
//   operand of O^T += V^T P^T; the V^T operand comes from the untransposed V
//   tile through ds_read_b64_tr_b16, two reads per fragment, whose token order
//   (0-3, 8-11 | 4-7, 12-15 per 16) is the accumulator's own.
// * K and V rows are XOR-swizzled at 16-byte granularity by choosing which
//   global chunk each DMA lane fetches: chunk c of token t sits at c ^ swz(t),
//   swz(t) = the 4-bit rotation ((t & 3) << 2) | ((t >> 2) & 3). Over 16
//   consecutive tokens swz is a bijection (fragment reads: 16 rows, one chunk,
//   16 distinct bank groups), and over 4 consecutive tokens it differs in bits
//   2-3 (transpose reads: 4 rows x 4 chunks of one 64-byte group land in 16
//   distinct bank groups). Both read kinds are bank-conflict free.
// * Softmax runs in the log2 domain (p = exp2(s * scale * log2(e) - m), one
//   FMA and one exp2 per score); LSE is converted back to natural log.
// * The epilogue re-lays O out as whole rows through the idle rings, so each
//   global store writes two contiguous 512-byte rows.
// * Split-KV fills the chip when batch*kv_heads*m-tiles is small; partial
//   (O, LSE) pairs are folded by an N-way LSE merge (stage1_combine_kernel).
// * Block order is XCD-aware: the m-tiles that read the same kv pages are
//   placed on the same XCD so the later reads hit that XCD's L2.
#include <cmath>

#include "ck_common.h"
#include "ck_internal.h"
#include "stage1_wide.h"

namespace ck {
namespace {

using namespace s1;

__global__ __launch_bounds__(kWW * 64) void stage1_wide_kernel(Stage1Args a) {
    extern __shared__ __attribute__((aligned(16))) char smem_raw[];
    stage1_wide_body<kWW, kWSlots>(a, (CK_LDS char *)smem_raw, blockIdx.x, gridDim.x, threadIdx.x, WgBarrier{});
}

// 128-row m-tiles: the same whole-row body on 4 waves with a 3-slot ring (the
// stage-1 role of the fused cascade kernel, as a kernel of its own)
constexpr int kNLds = wide_lds_bytes<3>();
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void stage1_narrow_kernel(Stage1Args a) {
    extern __shared__ __attribute__((aligned(16))) char smem_raw[];
    stage1_wide_body<4, 3>(a, (CK_LDS char *)smem_raw, blockIdx.x, gridDim.x, threadIdx.x, WgBarrier{});
}

// N-way LSE merge of split partials: 32 threads per row, 4 dims each. One
// pass with an online maximum, 8 splits per rescale step; the first 16 splits'
// partials are fetched together (one memory round trip at the usual split
// counts), later ones 8 at a time.
__global__ __launch_bounds__(256) void stage1_combine_kernel(const float *part_o, const float *part_lse,
                                                             int num_splits, int64_t rows,
                                                             float *out, float *lse) {
    constexpr int kBatch = 8;   // splits folded per rescale step
    constexpr int kPreS = 16;   // splits loaded up front: one memory round trip up to 16 splits
    const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int d4 = threadIdx.x & 31;
    if (row >= rows) return;
    float m = -INFINITY, wsum = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    // split s0 + j of a batch: its LSE (-inf past the last split) and O (a clamped,
    // in-bounds index whose weight is 0)
    auto load = [&](int s0, float *ls, float4 *o) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int s = s0 + j < num_splits ? s0 + j : num_splits - 1;
            ls[j] = s0 + j < num_splits ? part_lse[(int64_t)s * rows + row] : -INFINITY;
            o[j] = *reinterpret_cast<const float4 *>(part_o + ((int64_t)s * rows + row) * kD + 4 * d4);
        }
    };
    auto fold = [&](const float *ls, const float4 *o) __attribute__((always_inline)) {
        float mb = m;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) mb = fmaxf(mb, ls[j]);
        const float mu = mb == -INFINITY ? 0.f : mb;
        const float r = exp2_fast((m - mu) * kLog2e);  // 0 while nothing has been seen
        acc.x *= r; acc.y *= r; acc.z *= r; acc.w *= r;
        wsum *= r;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const float wgt = exp2_fast((ls[j] - mu) * kLog2e);
            acc.x = fmaf(wgt, o[j].x, acc.x);
            acc.y = fmaf(wgt, o[j].y, acc.y);
            acc.z = fmaf(wgt, o[j].z, acc.z);
            acc.w = fmaf(wgt, o[j].w, acc.w);
            wsum += wgt;
        }
        m = mb;
    };
    {
        float ls[kPreS];
        float4 o[kPreS];
#pragma unroll
        for (int s0 = 0; s0 < kPreS; s0 += kBatch) load(s0, ls + s0, o + s0);
#pragma unroll
        for (int s0 = 0; s0 < kPreS; s0 += kBatch)
            if (s0 < num_splits) fold(ls + s0, o + s0);
    }
    for (int s0 = kPreS; s0 < num_splits; s0 += kBatch) {
        float ls[kBatch];
        float4 o[kBatch];
        load(s0, ls, o);
        fold(ls, o);
    }
    const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
    *reinterpret_cast<float4 *>(out + row * kD + 4 * d4) =
        make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
    if (d4 < 2) {
        const float lv = wsum > 0.f ? m + __logf(wsum) : -INFINITY;
        *reinterpret_cast<float4 *>(lse + row * 8 + 4 * d4) = make_float4(lv, lv, lv, lv);
    }
}

int64_t ceil_div(int64_t x, int64_t y) { return (x + y - 1) / y; }

struct Plan {
    int64_t roww, mtiles, splits, split_len, ws_bytes;
};

int make_plan(int64_t batch, int64_t max_q_len, int64_t num_heads, int64_t kv_heads, int64_t kv_cap,
              int64_t forced_splits, Plan *p) {
    const int64_t group = num_heads / kv_heads;
    // 256-row workgroups (8 waves) once a request's rows for one kv head fill
    // more than 128 and the 256-row grid still holds at least one workgroup per
    // CU with >= 1024 tokens per split; 128-row workgroups (4 waves) otherwise
    const int64_t rows = max_q_len * group;
    p->roww = 1;
    if (rows > 128 && batch * kv_heads * ceil_div(rows, 256) * ceil_div(kv_cap, 1024) >= 256) p->roww = 2;
    p->mtiles = ceil_div(rows, 128 * p->roww);
    const int64_t base = batch * kv_heads * p->mtiles;
    int64_t s = forced_splits;
    if (s <= 0) {
        // Aim for one workgroup per CU with at least 512 kv tokens per split: a
        // shorter split spends more on its partial (O, LSE) write than on kv reads.
        const int64_t target = 256;
        s = 1;
        if (base < target) s = ceil_div(target, base);
        const int64_t max_s = ceil_div(kv_cap, 512);
        if (s > max_s) s = max_s;
        if (s < 1) s = 1;
    }
    const int64_t cap = kv_cap > 0 ? kv_cap : 1;
    const int64_t min_s = ceil_div(cap, (int64_t)kMaxSplitPages * kPage);
    if (s < min_s) s = min_s;
    // splits start on page boundaries and hold at most kMaxSplitPages pages
    int64_t split_len = ceil_div(ceil_div(cap, s), kPage) * kPage;
    s = ceil_div(cap, split_len);
    p->splits = s;
    p->split_len = split_len;
    p->ws_bytes = s > 1 ? s * batch * max_q_len * num_heads * (kD + 1) * (int64_t)sizeof(float) : 0;
    return CK_OK;
}

int check_dims(int64_t batch, int64_t max_q_len, int64_t num_heads, int64_t kv_heads, int64_t head_dim,
               int64_t kv_cap) {
    if (batch < 0 || max_q_len < 0 || kv_cap < 0) return CK_E_INVALID_ARG;
    if (head_dim != kD) return CK_E_UNSUPPORTED;
    if (kv_heads <= 0 || num_heads <= 0 || num_heads % kv_heads != 0) return CK_E_INVALID_ARG;
    if (kv_cap > (int64_t)1 << 30 || max_q_len * (num_heads / kv_heads) > (int64_t)1 << 30)
        return CK_E_INVALID_ARG;
    return CK_OK;
}

}  // namespace
}  // namespace ck

using namespace ck;

extern "C" int ck_fa_fp32_stage1_plan(int64_t batch, int64_t max_q_len, int64_t num_heads,
                                      int64_t kv_heads, int64_t head_dim, int64_t kv_cap,
                                      int64_t *num_splits, int64_t *workspace_bytes) {
    int rc = check_dims(batch, max_q_len, num_heads, kv_heads, head_dim, kv_cap);
    if (rc != CK_OK) return rc;
    if (!num_splits || !workspace_bytes) return CK_E_NULL_PTR;
    Plan p;
    make_plan(batch, max_q_len, num_heads, kv_heads, kv_cap, 0, &p);
    *num_splits = p.splits;
    *workspace_bytes = p.ws_bytes;
    return CK_OK;
}

int ck::stage1_launch(const void *q, const void *k, const void *v, const int32_t *block_table, int64_t bt_cols,
                      const int64_t *q_seqlens, const int64_t *kv_seqlens, const int32_t *q_start, int64_t batch,
                      int64_t q_len_uniform, int64_t max_q_len, int64_t num_tokens, int64_t num_heads,
                      int64_t kv_heads, int64_t head_dim, int64_t num_blocks, int64_t block_size, float scale,
                      int64_t kv_cap, int64_t num_splits, float *out, float *lse, void *workspace,
                      int64_t workspace_bytes, bool combine, hipStream_t s, int64_t *splits_used) {
    if (splits_used) *splits_used = 1;
    int rc = check_dims(batch, max_q_len, num_heads, kv_heads, head_dim, kv_cap);
    if (rc != CK_OK) return rc;
    if (block_size != kPage) return CK_E_UNSUPPORTED;
    if (q_len_uniform < 0 || num_tokens < 0 || bt_cols < 0 || num_blocks < 0) return CK_E_INVALID_ARG;
    if (q_len_uniform > 0 && (max_q_len != q_len_uniform || num_tokens != batch * q_len_uniform))
        return CK_E_INVALID_ARG;
    if (kv_cap > bt_cols * kPage) return CK_E_INVALID_ARG;
    // the row max is taken on the unscaled scores, which needs scale > 0
    if (!(scale > 0.f) || !std::isfinite(scale)) return CK_E_INVALID_ARG;
    if (batch == 0 || num_tokens == 0 || max_q_len == 0) return CK_OK;
    if (!q || !k || !v || !block_table || !kv_seqlens || !out || !lse) return CK_E_NULL_PTR;
    if (q_len_uniform == 0 && (!q_seqlens || !q_start)) return CK_E_NULL_PTR;
    // q/k/v rows, O rows and the padded LSE (4 copies per store) move 16 bytes per lane
    if (!aligned_to(q, 16) || !aligned_to(k, 16) || !aligned_to(v, 16) || !aligned_to(out, 16) ||
        !aligned_to(lse, 16) || !aligned_to(workspace, 16))
        return CK_E_INVALID_ARG;
    if (num_tokens * num_heads > ((int64_t)1 << 31)) return CK_E_INVALID_ARG;

    Plan p;
    make_plan(batch, max_q_len, num_heads, kv_heads, kv_cap, num_splits, &p);
    if (splits_used) *splits_used = p.splits;
    const int64_t need = p.splits > 1 ? p.splits * num_tokens * num_heads * (kD + 1) * (int64_t)sizeof(float) : 0;
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return CK_E_WORKSPACE;

    Stage1Args a;
    a.q = static_cast<const uint16_t *>(q);
    a.k = static_cast<const uint16_t *>(k);
    a.v = static_cast<const uint16_t *>(v);
    a.bt = block_table;
    a.q_seqlens = q_seqlens;
    a.kv_seqlens = kv_seqlens;
    a.q_start = q_start;
    a.out = out;
    a.lse = lse;
    a.num_rows = num_tokens * num_heads;
    a.part_o = p.splits > 1 ? static_cast<float *>(workspace) : nullptr;
    a.part_lse = p.splits > 1 ? a.part_o + p.splits * a.num_rows * kD : nullptr;
    a.bt_cols = bt_cols;
    a.num_blocks = num_blocks;
    a.batch = (int)batch;
    a.q_len_uniform = (int)q_len_uniform;
    a.num_heads = (int)num_heads;
    a.kv_heads = (int)kv_heads;
    a.group = (int)(num_heads / kv_heads);
    a.kv_cap = (int)kv_cap;
    a.split_len = (int)p.split_len;
    a.num_splits = (int)p.splits;
    a.mtiles = (int)p.mtiles;
    a.scale_log2 = scale * kLog2e;

    const int64_t grid = batch * kv_heads * p.mtiles * p.splits;
    if (grid <= 0 || grid > 0x7FFFFFFF) return CK_E_INVALID_ARG;
    if (p.roww == 2) {
        static std::atomic<uint64_t> lds_set_w{0};
        rc = ensure_dynamic_lds(reinterpret_cast<const void *>(&stage1_wide_kernel), kWLds, lds_set_w);
        if (rc != CK_OK) return rc;
        hipLaunchKernelGGL(stage1_wide_kernel, dim3((unsigned)grid), dim3(kWW * 64), kWLds, s, a);
    } else {
        static std::atomic<uint64_t> lds_set1{0};
        rc = ensure_dynamic_lds(reinterpret_cast<const void *>(&stage1_narrow_kernel), kNLds, lds_set1);
        if (rc != CK_OK) return rc;
        hipLaunchKernelGGL(stage1_narrow_kernel, dim3((unsigned)grid), dim3(256), kNLds, s, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return static_cast<int>(e);
    if (p.splits > 1 && combine) {
        const int64_t rows = a.num_rows;
        hipLaunchKernelGGL(stage1_combine_kernel, dim3((unsigned)ceil_div(rows, 8)), dim3(256), 0, s,
                           (const float *)a.part_o, (const float *)a.part_lse, (int)p.splits, rows, out, lse);
        CK_RETURN_LAUNCH();
    }
    return CK_OK;
}

// Plan of the stage-1 role of the fused cascade kernel: the B flattened queries
// of one request as 128-row units (the body on 4 waves), over page-aligned
// splits of the prefix, about `target` units in all.
void ck::stage1_fused_plan(int64_t batch, int64_t num_heads, int64_t kv_heads, int64_t kv_cap, int64_t target,
                           int64_t *units, int64_t *splits, int64_t *ws_bytes) {
    const int64_t rows = batch * (num_heads / kv_heads);
    const int64_t mtiles = ceil_div(rows, 128);
    const int64_t base = kv_heads * mtiles;
    const int64_t cap = kv_cap > 0 ? kv_cap : 1;
    int64_t s = (target + base / 2) / base;
    if (s < 1) s = 1;
    if (s > ceil_div(cap, kPage)) s = ceil_div(cap, kPage);
    const int64_t min_s = ceil_div(cap, (int64_t)kMaxSplitPages * kPage);
    if (s < min_s) s = min_s;
    const int64_t split_len = ceil_div(ceil_div(cap, s), kPage) * kPage;
    s = ceil_div(cap, split_len);
    *units = base * s;
    *splits = s;
    *ws_bytes = s > 1 ? s * batch * num_heads * (kD + 1) * (int64_t)sizeof(float) : 0;
}

int ck::stage1_fused_args(const void *q, const void *k, const void *v, const int32_t *block_table, int64_t bt_cols,
                          const int64_t *kv_seqlen, int64_t batch, int64_t num_heads, int64_t kv_heads,
                          int64_t num_blocks, float scale, int64_t kv_cap, int64_t target, float *out, float *lse,
                          void *workspace, int64_t workspace_bytes, s1::Stage1Args *a, int64_t *units,
                          int64_t *splits_used) {
    int rc = check_dims(1, batch, num_heads, kv_heads, kD, kv_cap);
    if (rc != CK_OK) return rc;
    if (kv_cap > bt_cols * kPage || bt_cols < 0 || num_blocks < 0) return CK_E_INVALID_ARG;
    if (!(scale > 0.f) || !std::isfinite(scale)) return CK_E_INVALID_ARG;
    if (batch * num_heads > ((int64_t)1 << 31)) return CK_E_INVALID_ARG;
    int64_t n = 0, s = 1, need = 0;
    stage1_fused_plan(batch, num_heads, kv_heads, kv_cap, target, &n, &s, &need);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return CK_E_WORKSPACE;
    const int64_t split_len = ceil_div(ceil_div(kv_cap > 0 ? kv_cap : 1, s), kPage) * kPage;
    a->q = static_cast<const uint16_t *>(q);
    a->k = static_cast<const uint16_t *>(k);
    a->v = static_cast<const uint16_t *>(v);
    a->bt = block_table;
    a->q_seqlens = nullptr;
    a->kv_seqlens = kv_seqlen;
    a->q_start = nullptr;
    a->out = out;
    a->lse = lse;
    a->num_rows = batch * num_heads;
    a->part_o = s > 1 ? static_cast<float *>(workspace) : nullptr;
    a->part_lse = s > 1 ? a->part_o + s * a->num_rows * kD : nullptr;
    a->bt_cols = bt_cols;
    a->num_blocks = num_blocks;
    a->batch = 1;
    a->q_len_uniform = (int)batch;
    a->num_heads = (int)num_heads;
    a->kv_heads = (int)kv_heads;
    a->group = (int)(num_heads / kv_heads);
    a->kv_cap = (int)kv_cap;
    a->split_len = (int)split_len;
    a->num_splits = (int)s;
    a->mtiles = (int)ceil_div(batch * (num_heads / kv_heads), 128);
    a->scale_log2 = scale * kLog2e;
    *units = n;
    *splits_used = s;
    return CK_OK;
}

extern "C" int ck_fa_fp32_stage1(const void *q, const void *k, const void *v, const int32_t *block_table,
                                 int64_t bt_cols, const int64_t *q_seqlens, const int64_t *kv_seqlens,
                                 const int32_t *q_start, int64_t batch, int64_t q_len_uniform,
                                 int64_t max_q_len, int64_t num_tokens, int64_t num_heads,
                                 int64_t kv_heads, int64_t head_dim, int64_t num_blocks,
                                 int64_t block_size, float scale, int64_t kv_cap, int64_t num_splits,
                                 float *out, float *lse, void *workspace, int64_t workspace_bytes,
                                 void *stream) {
    return stage1_launch(q, k, v, block_table, bt_cols, q_seqlens, kv_seqlens, q_start, batch, q_len_uniform,
                         max_q_len, num_tokens, num_heads, kv_heads, head_dim, num_blocks, block_size, scale,
                         kv_cap, num_splits, out, lse, workspace, workspace_bytes, true,
                         reinterpret_cast<hipStream_t>(stream), nullptr);
}
