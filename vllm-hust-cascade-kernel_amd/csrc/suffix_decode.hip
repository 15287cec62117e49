// suffix_decode.hip - per-sequence paged decode attention over each sequence's
// own suffix pages (cascade stage 2) on gfx950, without MFMA.
//
// Role: replaces the closed CANN op npu_fused_infer_attention_score_v2 the
// reference calls for stage 2 (ascend-kernel/README.md:186-197): one query
// token per sequence, GQA, paged K/V, bf16 O plus a compact fp32 LSE that
// lse_merge folds into the stage-1 result. An empty suffix (kv length 0)
// yields O = 0, LSE = -inf, which the merge treats as weight 0.
//
// Arithmetic: S = q k^T * scale in fp32, online softmax in the log2 domain,
// fp32 P and fp32 accumulation (no bf16 rounding of P: there is no matrix
// core here to feed), O = acc / l, LSE = ln(l) + max.
//
// MI355X design: memory-bound (one pass over each sequence's suffix K/V,
// 4-8 query heads per kv head => 4-8 flop/byte). A workgroup = one (sequence,
// kv head, kv split); its 4 waves x 4 token slots x 16 lanes read 16 tokens per
// step, each token row of 256 B by 16 lanes (16 B per lane, fully coalesced).
// Scores need a 16-lane sum per (token, head): done with DPP row rotations
// (no LDS). Each slot keeps its own running (max, sum, acc) so the hot loop has
// no cross-slot traffic; slots merge with two xor-shuffles and the 4 waves
// through LDS once at the end. The next step's K/V loads are issued before the
// current step's math (register double buffering) to keep HBM requests in
// flight. Long suffixes are split over several workgroups; only sequences with
// more than one split pay a partial write and the follow-up merge kernel.
#include "ck_common.h"

namespace ck {
namespace {

constexpr int kD = 128;
constexpr int kPage = 128;
constexpr int kThreads = 256;
constexpr int kUnroll = 4;                      // tokens per slot per step
constexpr int kStepTokens = 16 * kUnroll;       // tokens per workgroup step

struct SuffixArgs {
    const uint16_t *q;
    const uint16_t *k;
    const uint16_t *v;
    const int32_t *bt;
    const int64_t *kv_seqlens;
    uint16_t *out;
    float *lse;
    float *part_o;
    float *part_lse;
    int64_t bt_cols;
    int64_t num_blocks;
    int batch;
    int num_heads;
    int kv_heads;
    int kv_cap;
    int split_len;
    int num_splits;
    float scale_log2;
};

// Sum over the 16 lanes of a DPP row; every lane of the row receives the total.
__device__ __forceinline__ float row16_sum(float x) {
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xF, 0xF, false));  // row_ror:8
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x124, 0xF, 0xF, false));  // row_ror:4
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x122, 0xF, 0xF, false));  // row_ror:2
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x121, 0xF, 0xF, false));  // row_ror:1
    return x;
}

__device__ __forceinline__ int64_t seq_kv(const SuffixArgs &a, int b) {
    int64_t kvl = a.kv_seqlens[b];
    const int64_t lim = a.bt_cols * kPage;
    if (kvl > lim) kvl = lim;
    if (kvl > a.kv_cap) kvl = a.kv_cap;
    return kvl < 0 ? 0 : kvl;
}

template <int G>
__global__ __launch_bounds__(kThreads) void suffix_kernel(SuffixArgs a) {
    __shared__ float sm_acc[4][G][kD];
    __shared__ float sm_m[4][G];
    __shared__ float sm_l[4][G];

    uint32_t w = xcd_remap(blockIdx.x, gridDim.x);
    const int sp = w % a.num_splits;
    w /= a.num_splits;
    const int g = w % a.kv_heads;
    const int b = w / a.kv_heads;

    const int64_t kvl = seq_kv(a, b);
    const int nsplit_b = (int)((kvl + a.split_len - 1) / a.split_len);
    if (sp >= (nsplit_b > 1 ? nsplit_b : 1)) return;  // uniform over the workgroup
    const int kv_lo = sp * a.split_len;
    const int kv_hi = (int)((int64_t)(kv_lo + a.split_len) < kvl ? kv_lo + a.split_len : kvl);

    const int tid = threadIdx.x;
    const int wid = tid >> 6;
    const int lane = tid & 63;
    const int slot = lane >> 4;
    const int c = lane & 15;

    // q for this lane's 8 dims, all G heads, pre-scaled into the log2 domain.
    float qv[G][8];
#pragma unroll
    for (int hq = 0; hq < G; ++hq) {
        const uint4 w4 = *reinterpret_cast<const uint4 *>(
            a.q + ((int64_t)b * a.num_heads + g * G + hq) * kD + 8 * c);
        qv[hq][0] = bf16_lo(w4.x) * a.scale_log2; qv[hq][1] = bf16_hi(w4.x) * a.scale_log2;
        qv[hq][2] = bf16_lo(w4.y) * a.scale_log2; qv[hq][3] = bf16_hi(w4.y) * a.scale_log2;
        qv[hq][4] = bf16_lo(w4.z) * a.scale_log2; qv[hq][5] = bf16_hi(w4.z) * a.scale_log2;
        qv[hq][6] = bf16_lo(w4.w) * a.scale_log2; qv[hq][7] = bf16_hi(w4.w) * a.scale_log2;
    }
    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int hq = 0; hq < G; ++hq) {
        m[hq] = -INFINITY;
        l[hq] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[hq][i] = 0.f;
    }

    const int64_t head_stride = (int64_t)a.kv_heads * kD;
    const int32_t *bt_row = a.bt + (int64_t)b * a.bt_cols;
    // Two register buffers with compile-time names (a runtime-indexed register
    // array would be demoted to scratch memory).
    uint4 kA[kUnroll], vA[kUnroll], kB[kUnroll], vB[kUnroll];

    auto load_step = [&](int base, uint4 (&kr)[kUnroll], uint4 (&vr)[kUnroll]) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int tok = base + u * 16 + wid * 4 + slot;
            uint4 kk = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
            if (tok < kv_hi) {
                const int page = bt_row[tok / kPage];
                if (page >= 0 && (int64_t)page < a.num_blocks) {
                    const int64_t off = ((int64_t)page * kPage + (tok % kPage)) * head_stride + g * kD + 8 * c;
                    kk = *reinterpret_cast<const uint4 *>(a.k + off);
                    vv = *reinterpret_cast<const uint4 *>(a.v + off);
                }
            }
            kr[u] = kk;
            vr[u] = vv;
        }
    };

    auto compute_step = [&](int base, const uint4 (&kr)[kUnroll], const uint4 (&vr)[kUnroll]) {
        float kf[kUnroll][8];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint4 kk = kr[u];
            kf[u][0] = bf16_lo(kk.x); kf[u][1] = bf16_hi(kk.x);
            kf[u][2] = bf16_lo(kk.y); kf[u][3] = bf16_hi(kk.y);
            kf[u][4] = bf16_lo(kk.z); kf[u][5] = bf16_hi(kk.z);
            kf[u][6] = bf16_lo(kk.w); kf[u][7] = bf16_hi(kk.w);
        }
#pragma unroll
        for (int hq = 0; hq < G; ++hq) {
            float s[kUnroll];
            float smax = -INFINITY;
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                float d = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) d = fmaf(qv[hq][i], kf[u][i], d);
                d = row16_sum(d);
                const int tok = base + u * 16 + wid * 4 + slot;
                s[u] = tok < kv_hi ? d : -INFINITY;
                smax = fmaxf(smax, s[u]);
            }
            const float m_new = fmaxf(m[hq], smax);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            const float dm = exp2_fast(m[hq] - m_use);
            float ps = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[hq][i] *= dm;
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const float p = exp2_fast(s[u] - m_use);
                ps += p;
                const uint4 vv = vr[u];
                acc[hq][0] = fmaf(p, bf16_lo(vv.x), acc[hq][0]);
                acc[hq][1] = fmaf(p, bf16_hi(vv.x), acc[hq][1]);
                acc[hq][2] = fmaf(p, bf16_lo(vv.y), acc[hq][2]);
                acc[hq][3] = fmaf(p, bf16_hi(vv.y), acc[hq][3]);
                acc[hq][4] = fmaf(p, bf16_lo(vv.z), acc[hq][4]);
                acc[hq][5] = fmaf(p, bf16_hi(vv.z), acc[hq][5]);
                acc[hq][6] = fmaf(p, bf16_lo(vv.w), acc[hq][6]);
                acc[hq][7] = fmaf(p, bf16_hi(vv.w), acc[hq][7]);
            }
            l[hq] = l[hq] * dm + ps;
            m[hq] = m_new;
        }
    };

    const int nsteps = kv_hi > kv_lo ? (kv_hi - kv_lo + kStepTokens - 1) / kStepTokens : 0;
    if (nsteps > 0) load_step(kv_lo, kA, vA);
    for (int st = 0; st < nsteps; st += 2) {
        const int base = kv_lo + st * kStepTokens;
        if (st + 1 < nsteps) load_step(base + kStepTokens, kB, vB);
        compute_step(base, kA, vA);
        if (st + 1 < nsteps) {
            if (st + 2 < nsteps) load_step(base + 2 * kStepTokens, kA, vA);
            compute_step(base + kStepTokens, kB, vB);
        }
    }

    // merge the 4 slots of the wave (lanes c, c+16, c+32, c+48 hold the same dims)
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
#pragma unroll
        for (int hq = 0; hq < G; ++hq) {
            const float mo = __shfl_xor(m[hq], off);
            const float lo = __shfl_xor(l[hq], off);
            const float mn = fmaxf(m[hq], mo);
            const float mu = mn == -INFINITY ? 0.f : mn;
            const float fa = exp2_fast(m[hq] - mu), fb = exp2_fast(mo - mu);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float ao = __shfl_xor(acc[hq][i], off);
                acc[hq][i] = acc[hq][i] * fa + ao * fb;
            }
            l[hq] = l[hq] * fa + lo * fb;
            m[hq] = mn;
        }
    }
    if (slot == 0) {
#pragma unroll
        for (int hq = 0; hq < G; ++hq) {
#pragma unroll
            for (int i = 0; i < 8; ++i) sm_acc[wid][hq][8 * c + i] = acc[hq][i];
            if (c == 0) {
                sm_m[wid][hq] = m[hq];
                sm_l[wid][hq] = l[hq];
            }
        }
    }
    __syncthreads();

    const bool single = nsplit_b <= 1;
    for (int idx = tid; idx < G * 16; idx += kThreads) {
        const int hq = idx >> 4, cc = idx & 15;
        float mn = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) mn = fmaxf(mn, sm_m[ww][hq]);
        const float mu = mn == -INFINITY ? 0.f : mn;
        float lt = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
            const float f = exp2_fast(sm_m[ww][hq] - mu);
            lt += sm_l[ww][hq] * f;
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] += sm_acc[ww][hq][8 * cc + i] * f;
        }
        const float inv = lt > 0.f ? 1.0f / lt : 0.f;
        const float lse_v = lt > 0.f ? (mn + __log2f(lt)) * kLn2 : -INFINITY;
        const int64_t row = (int64_t)b * a.num_heads + g * G + hq;
        if (single) {
            uint4 ow;
            ow.x = pack_bf16x2(o[0] * inv, o[1] * inv);
            ow.y = pack_bf16x2(o[2] * inv, o[3] * inv);
            ow.z = pack_bf16x2(o[4] * inv, o[5] * inv);
            ow.w = pack_bf16x2(o[6] * inv, o[7] * inv);
            *reinterpret_cast<uint4 *>(a.out + row * kD + 8 * cc) = ow;
            if (cc == 0) a.lse[row] = lse_v;
        } else {
            const int64_t prow = (int64_t)sp * a.batch * a.num_heads + row;
            float4 *dst = reinterpret_cast<float4 *>(a.part_o + prow * kD + 8 * cc);
            dst[0] = make_float4(o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv);
            dst[1] = make_float4(o[4] * inv, o[5] * inv, o[6] * inv, o[7] * inv);
            if (cc == 0) a.part_lse[prow] = lse_v;
        }
    }
}

// Folds the split partials of sequences with more than one split.
__global__ __launch_bounds__(256) void suffix_combine_kernel(SuffixArgs a) {
    const int64_t rows = (int64_t)a.batch * a.num_heads;
    const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int d4 = threadIdx.x & 31;
    if (row >= rows) return;
    const int b = (int)(row / a.num_heads);
    const int64_t kvl = seq_kv(a, b);
    const int ns = (int)((kvl + a.split_len - 1) / a.split_len);
    if (ns <= 1) return;
    float mx = -INFINITY;
    for (int s = 0; s < ns; ++s) mx = fmaxf(mx, a.part_lse[(int64_t)s * rows + row]);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float wsum = 0.f;
    if (mx != -INFINITY) {
        for (int s = 0; s < ns; ++s) {
            const float wgt = exp2_fast((a.part_lse[(int64_t)s * rows + row] - mx) * kLog2e);
            if (wgt == 0.f) continue;
            const float4 o = *reinterpret_cast<const float4 *>(a.part_o + ((int64_t)s * rows + row) * kD + 4 * d4);
            acc.x += wgt * o.x;
            acc.y += wgt * o.y;
            acc.z += wgt * o.z;
            acc.w += wgt * o.w;
            wsum += wgt;
        }
    }
    const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
    uint2 ow = make_uint2(pack_bf16x2(acc.x * inv, acc.y * inv), pack_bf16x2(acc.z * inv, acc.w * inv));
    *reinterpret_cast<uint2 *>(a.out + row * kD + 4 * d4) = ow;
    if (d4 == 0) a.lse[row] = wsum > 0.f ? mx + __logf(wsum) : -INFINITY;
}

int64_t ceil_div(int64_t x, int64_t y) { return (x + y - 1) / y; }

void suffix_plan(int64_t batch, int64_t kv_heads, int64_t kv_cap, int64_t forced, int64_t *splits,
                 int64_t *split_len) {
    const int64_t cap = kv_cap > 0 ? kv_cap : 1;
    const int64_t base = batch * kv_heads > 0 ? batch * kv_heads : 1;
    int64_t len;
    if (forced > 0) {
        len = ceil_div(ceil_div(cap, forced), kStepTokens) * kStepTokens;
    } else {
        // 512-token splits: a long suffix is spread over several workgroups while
        // short ones keep a single split (no partial round trip). Shorter splits
        // when the whole grid would not cover the CUs; longer ones when empty
        // split slots would dominate the launch.
        len = 512;
        while (len > kStepTokens && base * ceil_div(cap, len) < 512 && ceil_div(cap, len) < ceil_div(cap, kStepTokens))
            len /= 2;
        while (base * ceil_div(cap, len) > 65536) len *= 2;
    }
    *split_len = len;
    *splits = ceil_div(cap, len);
}

int check_suffix_dims(int64_t batch, int64_t num_heads, int64_t kv_heads, int64_t head_dim, int64_t kv_cap) {
    if (batch < 0 || kv_cap < 0) return CK_E_INVALID_ARG;
    if (head_dim != kD) return CK_E_UNSUPPORTED;
    if (kv_heads <= 0 || num_heads <= 0 || num_heads % kv_heads != 0) return CK_E_INVALID_ARG;
    const int64_t group = num_heads / kv_heads;
    if (group > 8) return CK_E_UNSUPPORTED;
    if (kv_cap > (int64_t)1 << 30) return CK_E_INVALID_ARG;
    return CK_OK;
}

}  // namespace
}  // namespace ck

using namespace ck;

extern "C" int ck_suffix_decode_plan(int64_t batch, int64_t num_heads, int64_t kv_heads, int64_t head_dim,
                                     int64_t kv_cap, int64_t *num_splits, int64_t *workspace_bytes) {
    int rc = check_suffix_dims(batch, num_heads, kv_heads, head_dim, kv_cap);
    if (rc != CK_OK) return rc;
    if (!num_splits || !workspace_bytes) return CK_E_NULL_PTR;
    int64_t s, len;
    suffix_plan(batch, kv_heads, kv_cap, 0, &s, &len);
    *num_splits = s;
    *workspace_bytes = s > 1 ? s * batch * num_heads * (kD + 1) * (int64_t)sizeof(float) : 0;
    return CK_OK;
}

extern "C" int ck_suffix_decode(const void *q, const void *k, const void *v, const int32_t *block_table,
                                int64_t bt_cols, const int64_t *kv_seqlens, int64_t batch, int64_t num_heads,
                                int64_t kv_heads, int64_t head_dim, int64_t num_blocks, int64_t block_size,
                                float scale, int64_t kv_cap, int64_t num_splits, void *out, float *lse,
                                void *workspace, int64_t workspace_bytes, void *stream) {
    int rc = check_suffix_dims(batch, num_heads, kv_heads, head_dim, kv_cap);
    if (rc != CK_OK) return rc;
    if (block_size != kPage) return CK_E_UNSUPPORTED;
    if (bt_cols < 0 || num_blocks < 0 || kv_cap > bt_cols * kPage) return CK_E_INVALID_ARG;
    if (batch == 0) return CK_OK;
    if (!q || !k || !v || !block_table || !kv_seqlens || !out || !lse) return CK_E_NULL_PTR;
    int64_t s, len;
    suffix_plan(batch, kv_heads, kv_cap, num_splits, &s, &len);
    const int64_t need = s > 1 ? s * batch * num_heads * (kD + 1) * (int64_t)sizeof(float) : 0;
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return CK_E_WORKSPACE;

    SuffixArgs a;
    a.q = static_cast<const uint16_t *>(q);
    a.k = static_cast<const uint16_t *>(k);
    a.v = static_cast<const uint16_t *>(v);
    a.bt = block_table;
    a.kv_seqlens = kv_seqlens;
    a.out = static_cast<uint16_t *>(out);
    a.lse = lse;
    a.part_o = s > 1 ? static_cast<float *>(workspace) : nullptr;
    a.part_lse = s > 1 ? a.part_o + s * batch * num_heads * kD : nullptr;
    a.bt_cols = bt_cols;
    a.num_blocks = num_blocks;
    a.batch = (int)batch;
    a.num_heads = (int)num_heads;
    a.kv_heads = (int)kv_heads;
    a.kv_cap = (int)kv_cap;
    a.split_len = (int)len;
    a.num_splits = (int)s;
    a.scale_log2 = scale * kLog2e;

    const int64_t grid = batch * kv_heads * s;
    if (grid > 0x7FFFFFFF) return CK_E_INVALID_ARG;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int group = (int)(num_heads / kv_heads);
    switch (group) {
        case 1: hipLaunchKernelGGL(suffix_kernel<1>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
        case 2: hipLaunchKernelGGL(suffix_kernel<2>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
        case 3: hipLaunchKernelGGL(suffix_kernel<3>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
        case 4: hipLaunchKernelGGL(suffix_kernel<4>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
        case 5: hipLaunchKernelGGL(suffix_kernel<5>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
        case 6: hipLaunchKernelGGL(suffix_kernel<6>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
        case 7: hipLaunchKernelGGL(suffix_kernel<7>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
        default: hipLaunchKernelGGL(suffix_kernel<8>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return static_cast<int>(e);
    if (s > 1) {
        const int64_t rows = batch * num_heads;
        hipLaunchKernelGGL(suffix_combine_kernel, dim3((unsigned)ceil_div(rows, 8)), dim3(256), 0, st, a);
        CK_RETURN_LAUNCH();
    }
    return CK_OK;
}
