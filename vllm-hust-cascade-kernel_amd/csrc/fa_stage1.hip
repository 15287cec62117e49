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
// * Work item = (request b, kv head g, m-tile of 128 query rows, kv split).
//   Query rows of one kv head are token-major (row r -> token r / group,
//   head g*group + r % group), so the GQA group and every query of the request
//   that shares the prefix ride in the same MFMA tile: the flattened cascade
//   form (one request, q_len = batch) reads each prefix page once per m-tile.
// * One workgroup = 4 waves x 32 query rows. K and V^T tiles of 64 tokens are
//   staged through double-buffered LDS (2 x 32 KB); each wave keeps its Q rows
//   as MFMA operands in registers for the whole kv loop.
// * S^T = K Q^T on v_mfma_f32_32x32x16_bf16 (A = K rows from LDS, B = Q); the
//   accumulator layout puts one query row per lane, so row max / row sum need a
//   single cross-half exchange. P^T leaves the accumulator directly as the B
//   operand of O^T += V^T P^T; the MFMA's k order (tokens 0-3,8-11 | 4-7,12-15
//   per 16) is matched by storing V^T in LDS with that token permutation.
// * V is transposed in registers (4 tokens x 8 dims per thread) on its way to
//   LDS; K and V^T rows are XOR-swizzled at 16-byte granularity so the MFMA
//   fragment reads are bank-conflict free.
// * Softmax runs in the log2 domain (exp2 on the hardware unit, S pre-scaled by
//   scale*log2(e)); LSE is converted back to natural log.
// * Split-KV fills the chip when batch*kv_heads*m-tiles is small; partial
//   (O, LSE) pairs are folded by an N-way LSE merge (ck_stage1_combine).
// * Block order is XCD-aware: the m-tiles that read the same kv pages are
//   placed on the same XCD so the second read hits that XCD's L2.
#include "ck_common.h"

namespace ck {
namespace {

constexpr int kD = 128;          // head dim (op contract)
constexpr int kPage = 128;       // paged block size (op contract)
constexpr int kTileN = 64;       // kv tokens per tile
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
constexpr int kRows = 32 * kWaves;  // query rows per workgroup
constexpr int kKTileBytes = kTileN * kD * 2;  // 16 KB
constexpr int kVTileBytes = kD * kTileN * 2;  // 16 KB
constexpr int kBufBytes = kKTileBytes + kVTileBytes;

struct Stage1Args {
    const uint16_t *q;
    const uint16_t *k;
    const uint16_t *v;
    const int32_t *bt;
    const int64_t *q_seqlens;
    const int64_t *kv_seqlens;
    const int32_t *q_start;
    float *out;
    float *lse;
    float *part_o;
    float *part_lse;
    int64_t bt_cols;
    int64_t num_blocks;
    int64_t num_rows;  // num_tokens * num_heads
    int batch;
    int q_len_uniform;
    int num_heads;
    int kv_heads;
    int group;
    int kv_cap;
    int split_len;
    int num_splits;
    int mtiles;
    float scale_log2;
};

__device__ __forceinline__ bf16x8 lds_read16(const char *p) {
    return *reinterpret_cast<const bf16x8 *>(p);
}

__device__ __forceinline__ bf16x8 pack_p(const f32x16 &s, int base) {
    uint4 w;
    w.x = pack_bf16x2(s[base + 0], s[base + 1]);
    w.y = pack_bf16x2(s[base + 2], s[base + 3]);
    w.z = pack_bf16x2(s[base + 4], s[base + 5]);
    w.w = pack_bf16x2(s[base + 6], s[base + 7]);
    return __builtin_bit_cast(bf16x8, w);
}

// Byte offset of K[token][16-byte chunk c] in a K tile.
__device__ __forceinline__ int k_off(int tok, int c) { return tok * (kD * 2) + ((c ^ (tok & 15)) << 4); }

// Byte offset of the 16-byte chunk ch (token positions 8ch..8ch+7) of V^T row dim.
__device__ __forceinline__ int vt_off(int dim, int ch) {
    return dim * (kTileN * 2) + ((ch ^ ((dim ^ (dim >> 3)) & 7)) << 4);
}

__global__ __launch_bounds__(kThreads) void stage1_kernel(Stage1Args a) {
    __shared__ __attribute__((aligned(16))) char smem[2 * kBufBytes];

    const int tid = threadIdx.x;
    const int wid = tid >> 6;
    const int lane = tid & 63;
    const int hh = lane >> 5;

    uint32_t w = xcd_remap(blockIdx.x, gridDim.x);
    const int mt = w % a.mtiles;
    w /= a.mtiles;
    const int sp = w % a.num_splits;
    w /= a.num_splits;
    const int g = w % a.kv_heads;
    const int b = w / a.kv_heads;

    int qlen, qs;
    if (a.q_len_uniform > 0) {
        qlen = a.q_len_uniform;
        qs = b * qlen;
    } else {
        qlen = (int)a.q_seqlens[b];
        qs = a.q_start[b];
    }
    const int rows_b = qlen * a.group;
    const int row0 = mt * kRows;
    if (row0 >= rows_b) return;  // uniform over the workgroup

    int64_t kvl = a.kv_seqlens[b];
    const int64_t kv_lim = a.bt_cols * kPage;
    if (kvl > kv_lim) kvl = kv_lim;
    if (kvl > a.kv_cap) kvl = a.kv_cap;
    if (kvl < 0) kvl = 0;
    const int kv_lo = sp * a.split_len;
    int kv_hi = kv_lo + a.split_len;
    if (kv_hi > (int)kvl) kv_hi = (int)kvl;
    const int ntiles = kv_hi > kv_lo ? (kv_hi - kv_lo + kTileN - 1) / kTileN : 0;

    const int wrow0 = row0 + wid * 32;
    const bool wave_active = wrow0 < rows_b;
    const int r = wrow0 + (lane & 31);
    const bool row_valid = r < rows_b;
    const int t_local = r / a.group;
    const int h = g * a.group + (r - t_local * a.group);
    const int64_t qrow = (int64_t)(qs + t_local) * a.num_heads + h;

    // Q as the B operand of S^T = K Q^T: lane holds dims 16kk + 8hh .. +8.
    bf16x8 qf[8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
        if (row_valid) {
            qf[kk] = *reinterpret_cast<const bf16x8 *>(a.q + qrow * kD + 16 * kk + 8 * hh);
        } else {
            qf[kk] = __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
        }
    }

    // ---- tile staging: global -> registers -> LDS --------------------------------
    constexpr int KU = (kTileN * kD / 8) / kThreads;  // 16-byte K chunks per thread
    constexpr int VU = (kTileN / 4 * kD / 8) / kThreads;  // (4 tokens x 8 dims) V units per thread
    uint4 kreg[KU];
    uint4 vreg[VU][4];
    const int64_t head_stride = (int64_t)a.kv_heads * kD;

    auto load_tile = [&](int i) {
        const int j0 = kv_lo + i * kTileN;
        const int nvalid = min(kTileN, kv_hi - j0);
        const int page = a.bt[(int64_t)b * a.bt_cols + (j0 / kPage)];
        const bool pvalid = page >= 0 && (int64_t)page < a.num_blocks;
        const int64_t tok0 = (int64_t)page * kPage + (j0 % kPage);
        const uint4 zero = make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const int ci = tid + kThreads * u;
            const int tt = ci >> 4, c = ci & 15;
            kreg[u] = (pvalid && tt < nvalid)
                          ? *reinterpret_cast<const uint4 *>(a.k + (tok0 + tt) * head_stride + g * kD + c * 8)
                          : zero;
        }
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            const int ui = tid + kThreads * u;
            const int qd = ui >> 4, c = ui & 15;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int tt = qd * 4 + j;
                vreg[u][j] = (pvalid && tt < nvalid)
                                 ? *reinterpret_cast<const uint4 *>(a.v + (tok0 + tt) * head_stride + g * kD + c * 8)
                                 : zero;
            }
        }
    };

    auto store_tile = [&](int buf) {
        char *kb = smem + buf * kBufBytes;
        char *vb = kb + kKTileBytes;
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const int ci = tid + kThreads * u;
            const int tt = ci >> 4, c = ci & 15;
            *reinterpret_cast<uint4 *>(kb + k_off(tt, c)) = kreg[u];
        }
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            const int ui = tid + kThreads * u;
            const int qd = ui >> 4, c = ui & 15;
            // token quad qd -> permuted position quad inside its 16-token group
            const int qg = qd & 3;
            const int p = (qd >> 2) * 16 + ((((qg & 1) << 1) | (qg >> 1)) << 2);
            const uint32_t *t0 = reinterpret_cast<const uint32_t *>(&vreg[u][0]);
            const uint32_t *t1 = reinterpret_cast<const uint32_t *>(&vreg[u][1]);
            const uint32_t *t2 = reinterpret_cast<const uint32_t *>(&vreg[u][2]);
            const uint32_t *t3 = reinterpret_cast<const uint32_t *>(&vreg[u][3]);
#pragma unroll
            for (int jw = 0; jw < 4; ++jw) {
                // dims 2jw (low halves) and 2jw+1 (high halves) of tokens 0..3
                const uint2 lo = make_uint2((t0[jw] & 0xFFFFu) | (t1[jw] << 16),
                                            (t2[jw] & 0xFFFFu) | (t3[jw] << 16));
                const uint2 hi = make_uint2((t0[jw] >> 16) | (t1[jw] & 0xFFFF0000u),
                                            (t2[jw] >> 16) | (t3[jw] & 0xFFFF0000u));
                const int d0 = c * 8 + 2 * jw;
                const int ch = p >> 3, half = (p & 7) * 2;
                *reinterpret_cast<uint2 *>(vb + vt_off(d0, ch) + half) = lo;
                *reinterpret_cast<uint2 *>(vb + vt_off(d0 + 1, ch) + half) = hi;
            }
        }
    };

    // ---- online softmax state (one query row per lane, halves agree) ---------------
    f32x16 oacc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[db][i] = 0.f;
    float m_run = -INFINITY;
    float l_run = 0.f;

    if (ntiles > 0) {
        load_tile(0);
        store_tile(0);
    }
    __syncthreads();
    if (ntiles > 1) load_tile(1);

    for (int i = 0; i < ntiles; ++i) {
        if (wave_active) {
            const char *kb = smem + (i & 1) * kBufBytes;
            const char *vb = kb + kKTileBytes;
            const int nvalid = min(kTileN, kv_hi - (kv_lo + i * kTileN));
            f32x16 sacc[2];
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
#pragma unroll
                for (int e = 0; e < 16; ++e) sacc[tb][e] = 0.f;
                const int tok = tb * 32 + (lane & 31);
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                    const bf16x8 kf = lds_read16(kb + k_off(tok, 2 * kk + hh));
                    sacc[tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], sacc[tb], 0, 0, 0);
                }
            }
            // scale, mask, row max
            float smax = -INFINITY;
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int tok = tb * 32 + (e & 3) + 8 * (e >> 2) + 4 * hh;
                    float s = sacc[tb][e] * a.scale_log2;
                    s = tok < nvalid ? s : -INFINITY;
                    sacc[tb][e] = s;
                    smax = fmaxf(smax, s);
                }
            smax = fmaxf(smax, __shfl_xor(smax, 32));
            const float m_new = fmaxf(m_run, smax);
            const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
            const float dm = exp2_fast(m_run - m_use);
            float ls = 0.f;
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float p = exp2_fast(sacc[tb][e] - m_use);
                    sacc[tb][e] = p;
                    ls += p;
                }
            ls += __shfl_xor(ls, 32);
            l_run = l_run * dm + ls;
            m_run = m_new;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int e = 0; e < 16; ++e) oacc[db][e] *= dm;
            // O^T += V^T P^T over 4 k-steps of 16 tokens
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const bf16x8 pb = pack_p(sacc[s >> 1], (s & 1) * 8);
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const int dim = db * 32 + (lane & 31);
                    const bf16x8 vf = lds_read16(vb + vt_off(dim, 2 * s + hh));
                    oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb, oacc[db], 0, 0, 0);
                }
            }
        }
        if (i + 1 < ntiles) store_tile((i + 1) & 1);
        __syncthreads();
        if (i + 2 < ntiles) load_tile(i + 2);
    }

    if (!row_valid) return;
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
    const float lse_v = l_run > 0.f ? (m_run + __log2f(l_run)) * kLn2 : -INFINITY;
    float *dst;
    if (a.num_splits == 1) {
        dst = a.out + qrow * kD;
        const float4 lv = make_float4(lse_v, lse_v, lse_v, lse_v);
        *reinterpret_cast<float4 *>(a.lse + qrow * 8 + 4 * hh) = lv;
    } else {
        const int64_t prow = (int64_t)sp * a.num_rows + qrow;
        dst = a.part_o + prow * kD;
        if (hh == 0) a.part_lse[prow] = lse_v;
    }
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float4 o = make_float4(oacc[db][4 * c + 0] * inv, oacc[db][4 * c + 1] * inv,
                                         oacc[db][4 * c + 2] * inv, oacc[db][4 * c + 3] * inv);
            *reinterpret_cast<float4 *>(dst + db * 32 + 8 * c + 4 * hh) = o;
        }
}

// N-way LSE merge of split partials: 32 threads per row, 4 dims each.
__global__ __launch_bounds__(256) void stage1_combine_kernel(const float *part_o, const float *part_lse,
                                                             int num_splits, int64_t rows,
                                                             float *out, float *lse) {
    const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int d4 = threadIdx.x & 31;
    if (row >= rows) return;
    float m = -INFINITY;
    for (int s = 0; s < num_splits; ++s) m = fmaxf(m, part_lse[(int64_t)s * rows + row]);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float wsum = 0.f;
    if (m != -INFINITY) {
        for (int s = 0; s < num_splits; ++s) {
            const float ls = part_lse[(int64_t)s * rows + row];
            const float wgt = exp2_fast((ls - m) * kLog2e);
            if (wgt == 0.f) continue;
            const float4 o = *reinterpret_cast<const float4 *>(part_o + ((int64_t)s * rows + row) * kD + 4 * d4);
            acc.x += wgt * o.x;
            acc.y += wgt * o.y;
            acc.z += wgt * o.z;
            acc.w += wgt * o.w;
            wsum += wgt;
        }
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
    int64_t mtiles, splits, split_len, ws_bytes;
};

int make_plan(int64_t batch, int64_t max_q_len, int64_t num_heads, int64_t kv_heads, int64_t kv_cap,
              int64_t forced_splits, Plan *p) {
    const int64_t group = num_heads / kv_heads;
    p->mtiles = ceil_div(max_q_len * group, kRows);
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
    int64_t split_len = ceil_div(ceil_div(kv_cap > 0 ? kv_cap : 1, s), kTileN) * kTileN;
    s = ceil_div(kv_cap > 0 ? kv_cap : 1, split_len);
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

extern "C" int ck_fa_fp32_stage1(const void *q, const void *k, const void *v, const int32_t *block_table,
                                 int64_t bt_cols, const int64_t *q_seqlens, const int64_t *kv_seqlens,
                                 const int32_t *q_start, int64_t batch, int64_t q_len_uniform,
                                 int64_t max_q_len, int64_t num_tokens, int64_t num_heads,
                                 int64_t kv_heads, int64_t head_dim, int64_t num_blocks,
                                 int64_t block_size, float scale, int64_t kv_cap, int64_t num_splits,
                                 float *out, float *lse, void *workspace, int64_t workspace_bytes,
                                 void *stream) {
    int rc = check_dims(batch, max_q_len, num_heads, kv_heads, head_dim, kv_cap);
    if (rc != CK_OK) return rc;
    if (block_size != kPage) return CK_E_UNSUPPORTED;
    if (q_len_uniform < 0 || num_tokens < 0 || bt_cols < 0 || num_blocks < 0) return CK_E_INVALID_ARG;
    if (q_len_uniform > 0 && (max_q_len != q_len_uniform || num_tokens != batch * q_len_uniform))
        return CK_E_INVALID_ARG;
    if (kv_cap > bt_cols * kPage) return CK_E_INVALID_ARG;
    if (batch == 0 || num_tokens == 0 || max_q_len == 0) return CK_OK;
    if (!q || !k || !v || !block_table || !kv_seqlens || !out || !lse) return CK_E_NULL_PTR;
    if (q_len_uniform == 0 && (!q_seqlens || !q_start)) return CK_E_NULL_PTR;
    if (num_tokens * num_heads > ((int64_t)1 << 31)) return CK_E_INVALID_ARG;

    Plan p;
    make_plan(batch, max_q_len, num_heads, kv_heads, kv_cap, num_splits, &p);
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
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(stage1_kernel, dim3((unsigned)grid), dim3(kThreads), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return static_cast<int>(e);
    if (p.splits > 1) {
        const int64_t rows = a.num_rows;
        hipLaunchKernelGGL(stage1_combine_kernel, dim3((unsigned)ceil_div(rows, 8)), dim3(256), 0, s,
                           (const float *)a.part_o, (const float *)a.part_lse, (int)p.splits, rows, out, lse);
        CK_RETURN_LAUNCH();
    }
    return CK_OK;
}
