// cascade.hip - fused cascade decode: stage-1 over the shared prefix, the
// per-sequence suffix attention and their LSE merge as one ABI call.
//
// Role: the caller-side composition the reference documents
// (ascend-kernel/README.md:160-201: fa_fp32_stage1 in the flattened form,
// CANN FIA v2 over each suffix, lse_merge) as a single entry point.
//
// Kernels (all on the caller's stream):
//   1. stage-1 (fa_stage1.hip) on the B decode queries flattened into one
//      request of q_len = B; its split partials stay in the workspace (no
//      separate combine pass);
//   2. the suffix stream kernel (suffix_decode.hip), whole-sequence results to
//      workspace scratch, cut sequences as fp32 partials;
//   3. the cascade epilogue: per (sequence, kv head) it folds the stage-1
//      partials and the suffix partials and merges the two results into the
//      final bf16 O and the merged LSE.
// When the batch fits one launch group and stage-1 is small enough to hide
// beside the suffix stream, 1 and 2 are one fused kernel (suffix_decode.hip):
// two launches in all; otherwise three. Either way fewer than the five of the
// composed ops (stage-1, combine, suffix, fix-up, merge), and neither partial
// result makes an extra round trip through HBM.
//
// ck_cascade_decode_noalloc is the same call for callers that cannot allocate
// (code under HIP-graph capture, serving loops that forbid allocation): its
// workspace is `scratch`, a file-scope device array of kScratchBytes that
// every GPU the library runs on holds until the process ends. Host code never
// passes the array's name to a kernel (on the host it is only a stand-in
// symbol): the device address comes from hipGetSymbolAddress, looked up once
// per device with that device current. Calls on one GPU share its array, so
// calls that overlap on one GPU race. Nothing in it has to start at zero:
// every workspace word a kernel reads was written earlier in the same call.
#include <atomic>

#include "ck_common.h"
#include "ck_internal.h"

// The no-allocation entry point's workspace (32 MiB: the cascade at BASELINE
// config 2 plans 19.6 MB, config 5 23.3 MB).
constexpr int64_t kScratchBytes = CK_CASCADE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

constexpr int64_t kD = 128;
constexpr int64_t kAlign = 256;

int64_t align_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// The fused kernel (stage-1 units and suffix chunks side by side) pays off while
// stage-1 is no larger than the suffix side can hide; a prefix whose MFMA work
// (kv heads x query rows of a kv head x prefix tokens) exceeds this runs the
// kernels one after another, stage-1 with all its waves.
constexpr int64_t kFusedMaxS1Work = (int64_t)1 << 26;
constexpr int64_t kFusedUnits = 256;  // stage-1 units of the fused kernel (one per CU)

struct CascadeLayout {
    bool fused;
    int64_t s1_units;     // fused: stage-1 units
    int64_t s1_splits;
    int64_t s1_bytes;     // stage-1 partials, or the final O1 [R][128] + padded LSE1 [R * 8]
    int64_t chunks;
    int64_t group_batch;  // sequences per suffix launch group
    int64_t sfx_bytes;    // suffix group workspace
    int64_t whole_bytes;  // bf16 O2 [nb][H][128] + fp32 LSE2 [nb * H] of one group
    int64_t total;
};

int cascade_layout(int64_t batch, int64_t num_heads, int64_t kv_heads, int64_t head_dim, int64_t prefix_cap,
                   int64_t suffix_cap, CascadeLayout *L) {
    if (batch < 0 || batch > 0x7FFFFFFF || prefix_cap < 0 || suffix_cap < 0) return CK_E_INVALID_ARG;
    if (head_dim != kD) return CK_E_UNSUPPORTED;
    if (kv_heads <= 0 || num_heads <= 0 || num_heads % kv_heads != 0) return CK_E_INVALID_ARG;
    if (num_heads > (1 << 16)) return CK_E_INVALID_ARG;
    if (prefix_cap > ((int64_t)1 << 30) || suffix_cap > ((int64_t)1 << 30)) return CK_E_INVALID_ARG;
    const int64_t rows = batch * num_heads;
    const int64_t per = ck::suffix_group_batch(suffix_cap);
    L->group_batch = batch < per ? batch : per;
    L->fused = batch > 0 && batch <= per && kv_heads * (rows / kv_heads) * prefix_cap <= kFusedMaxS1Work;
    int64_t s1 = 1, s1_ws = 0;
    L->s1_units = 0;
    if (L->fused) {
        ck::stage1_fused_plan(batch, num_heads, kv_heads, prefix_cap, kFusedUnits, &L->s1_units, &s1, &s1_ws);
    } else if (batch > 0) {
        int rc = ck_fa_fp32_stage1_plan(1, batch, num_heads, kv_heads, head_dim, prefix_cap, &s1, &s1_ws);
        if (rc != CK_OK) return rc;
    }
    L->s1_splits = s1;
    const int64_t final_bytes = rows * (kD + 8) * (int64_t)sizeof(float);
    L->s1_bytes = align_up(s1 > 1 ? s1_ws : final_bytes);
    L->chunks = L->fused ? ck::suffix_fused_chunks(num_heads, kv_heads) : ck::suffix_default_chunks(num_heads, kv_heads);
    L->sfx_bytes = align_up(ck::suffix_group_ws_bytes(L->group_batch, num_heads, kv_heads, L->chunks));
    L->whole_bytes = align_up(L->group_batch * num_heads * (kD * 2 + 4));
    L->total = batch > 0 ? L->s1_bytes + L->sfx_bytes + L->whole_bytes : 0;
    return CK_OK;
}

}  // namespace

extern "C" int ck_cascade_decode_plan(int64_t batch, int64_t num_heads, int64_t kv_heads, int64_t head_dim,
                                      int64_t prefix_cap, int64_t suffix_cap, int64_t *workspace_bytes) {
    if (!workspace_bytes) return CK_E_NULL_PTR;
    CascadeLayout L;
    int rc = cascade_layout(batch, num_heads, kv_heads, head_dim, prefix_cap, suffix_cap, &L);
    if (rc != CK_OK) return rc;
    *workspace_bytes = L.total;
    return CK_OK;
}

extern "C" int ck_cascade_decode(const void *q, const void *prefix_k, const void *prefix_v,
                                 const int32_t *prefix_block_table, int64_t prefix_bt_cols,
                                 const int64_t *prefix_kv_seqlen, int64_t prefix_num_blocks, const void *suffix_k,
                                 const void *suffix_v, const int32_t *suffix_block_table, int64_t suffix_bt_cols,
                                 const int64_t *suffix_kv_seqlens, int64_t suffix_num_blocks,
                                 int64_t suffix_kv_layout, int64_t batch,
                                 int64_t num_heads, int64_t kv_heads, int64_t head_dim, int64_t block_size,
                                 float scale, int64_t prefix_cap, int64_t suffix_cap, void *out, float *lse_out,
                                 void *workspace, int64_t workspace_bytes, void *stream) {
    CascadeLayout L;
    int rc = cascade_layout(batch, num_heads, kv_heads, head_dim, prefix_cap, suffix_cap, &L);
    if (rc != CK_OK) return rc;
    if (block_size != 128) return CK_E_UNSUPPORTED;
    if (suffix_kv_layout != CK_KV_NHD && suffix_kv_layout != CK_KV_BNSD) return CK_E_INVALID_ARG;
    if (prefix_bt_cols < 0 || suffix_bt_cols < 0 || prefix_num_blocks < 0 || suffix_num_blocks < 0)
        return CK_E_INVALID_ARG;
    if (prefix_cap > prefix_bt_cols * 128 || suffix_cap > suffix_bt_cols * 128) return CK_E_INVALID_ARG;
    if (batch == 0) return CK_OK;
    if (!q || !prefix_k || !prefix_v || !prefix_block_table || !prefix_kv_seqlen || !suffix_k || !suffix_v ||
        !suffix_block_table || !suffix_kv_seqlens || !out || !lse_out)
        return CK_E_NULL_PTR;
    using ck::aligned_to;
    if (!aligned_to(q, 16) || !aligned_to(prefix_k, 16) || !aligned_to(prefix_v, 16) ||
        !aligned_to(suffix_k, 16) || !aligned_to(suffix_v, 16) || !aligned_to(out, 8) || !aligned_to(lse_out, 4) ||
        !aligned_to(workspace, 16))
        return CK_E_INVALID_ARG;
    if (batch * num_heads > ((int64_t)1 << 31)) return CK_E_INVALID_ARG;
    if (workspace == nullptr || workspace_bytes < L.total) return CK_E_WORKSPACE;

    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    char *ws = static_cast<char *>(workspace);
    char *s1_region = ws;
    char *sfx_region = ws + L.s1_bytes;
    char *whole_region = sfx_region + L.sfx_bytes;
    const int64_t rows = batch * num_heads;

    // 1. stage-1 over the shared prefix, the B queries as one request (q_len = B):
    //    its own launch, or the stage-1 role of the fused kernel
    float *o1 = reinterpret_cast<float *>(s1_region);
    float *l1 = o1 + rows * kD;
    int64_t s1 = 1, units = 0;
    ck::s1::Stage1Args fa;
    if (L.fused) {
        rc = ck::stage1_fused_args(q, prefix_k, prefix_v, prefix_block_table, prefix_bt_cols, prefix_kv_seqlen, batch,
                                   num_heads, kv_heads, prefix_num_blocks, scale, prefix_cap, kFusedUnits, o1, l1,
                                   s1_region, L.s1_bytes, &fa, &units, &s1);
    } else {
        rc = ck::stage1_launch(q, prefix_k, prefix_v, prefix_block_table, prefix_bt_cols, nullptr, prefix_kv_seqlen,
                               nullptr, 1, batch, batch, batch, num_heads, kv_heads, head_dim, prefix_num_blocks,
                               block_size, scale, prefix_cap, L.s1_splits, o1, l1, s1_region, L.s1_bytes, false, st,
                               &s1);
    }
    if (rc != CK_OK) return rc;
    ck::Stage1Result r1;
    r1.rows = rows;
    r1.splits = (int)s1;
    r1.o = reinterpret_cast<const float *>(s1_region);
    r1.lse = s1 > 1 ? r1.o + s1 * rows * kD : l1;

    // 2 + 3. suffix and the merged result, per launch group of sequences
    uint16_t *o2 = reinterpret_cast<uint16_t *>(whole_region);
    float *l2 = reinterpret_cast<float *>(whole_region + L.group_batch * num_heads * kD * 2);
    for (int64_t b0 = 0; b0 < batch; b0 += L.group_batch) {
        const int64_t nb = batch - b0 < L.group_batch ? batch - b0 : L.group_batch;
        rc = ck::suffix_launch_group(q, suffix_k, suffix_v, suffix_block_table, suffix_bt_cols, suffix_kv_seqlens,
                                     b0, nb, num_heads, kv_heads, suffix_num_blocks, suffix_kv_layout, scale,
                                     suffix_cap, L.chunks,
                                     o2, l2, sfx_region, &r1, out, lse_out, st, L.fused ? &fa : nullptr, units);
        if (rc != CK_OK) return rc;
    }
    return CK_OK;
}

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch[kMaxDevices];

// Device address of `scratch` on the current device, looked up on the first
// call per device and kept (every GPU holds its own copy at its own address).
int scratch_address(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return static_cast<int>(e);
    if (dev < 0 || dev >= kMaxDevices) return CK_E_UNSUPPORTED;
    void *p = g_scratch[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return static_cast<int>(e);
        if (p == nullptr) return static_cast<int>(hipErrorInvalidSymbol);
        g_scratch[dev].store(p, std::memory_order_release);
    }
    *out = p;
    return CK_OK;
}

}  // namespace

extern "C" int ck_cascade_decode_noalloc(const void *q, const void *prefix_k, const void *prefix_v,
                                         const int32_t *prefix_block_table, int64_t prefix_bt_cols,
                                         const int64_t *prefix_kv_seqlen, int64_t prefix_num_blocks,
                                         const void *suffix_k, const void *suffix_v,
                                         const int32_t *suffix_block_table, int64_t suffix_bt_cols,
                                         const int64_t *suffix_kv_seqlens, int64_t suffix_num_blocks,
                                         int64_t suffix_kv_layout, int64_t batch, int64_t num_heads,
                                         int64_t kv_heads, int64_t head_dim, int64_t block_size, float scale,
                                         int64_t prefix_cap, int64_t suffix_cap, void *out, float *lse_out,
                                         void *stream) {
    CascadeLayout L;
    int rc = cascade_layout(batch, num_heads, kv_heads, head_dim, prefix_cap, suffix_cap, &L);
    if (rc != CK_OK) return rc;
    if (L.total > kScratchBytes) return CK_E_SCRATCH_LIMIT;
    void *ws = nullptr;
    if (L.total > 0) {
        rc = scratch_address(&ws);
        if (rc != CK_OK) return rc;
    }
    return ck_cascade_decode(q, prefix_k, prefix_v, prefix_block_table, prefix_bt_cols, prefix_kv_seqlen,
                             prefix_num_blocks, suffix_k, suffix_v, suffix_block_table, suffix_bt_cols,
                             suffix_kv_seqlens, suffix_num_blocks, suffix_kv_layout, batch, num_heads, kv_heads,
                             head_dim, block_size, scale, prefix_cap, suffix_cap, out, lse_out, ws,
                             L.total > 0 ? kScratchBytes : 0, stream);
}
