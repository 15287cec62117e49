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
// MI355X design: memory-bound streaming with a persistent, token-balanced grid.
// * Suffix lengths vary widely (geometric in the benchmark), and a workgroup
//   pays several microseconds of start-up (lengths, page ids, first DMA round
//   trip) before its first byte of K/V. So instead of one workgroup per
//   (sequence, split), workgroup (kv head g, chunk c) takes the c-th 1/P of the
//   concatenation of all sequences' tokens for head g, crossing sequence
//   boundaries; every workgroup moves the same number of bytes and starts once.
//   Prefix sums of the (device-side) lengths are computed per workgroup in LDS.
// * K and V rows stream through a 4-stage LDS ring (64 tokens = 32 KB per
//   stage) by global->LDS DMA, continuously across sequence boundaries; a
//   sequence's q rows ride along with its first stage. Page ids are fetched
//   with scalar loads (lgkmcnt), so looking one up never drains the DMA ring.
// * Each of the 8 waves (2 per SIMD) consumes 8 tokens of a stage as 4 token
//   slots x 16 lanes x 8 dims; q.k uses the packed bf16 dot product
//   (v_dot2_f32_bf16), the 16-lane sum uses DPP row rotations, V is unpacked
//   once per token for all query heads of the group. At the end of a sequence
//   segment the slots merge with two xor-shuffles and the 8 waves through the
//   just-consumed ring stage.
// * A segment that is a whole sequence writes bf16 O and the LSE directly; a
//   sequence cut by a chunk boundary leaves fp32 partials that a small fix-up
//   kernel folds (it also writes O = 0, LSE = -inf for empty suffixes).
#include "ck_common.h"

namespace ck {
namespace {

constexpr int kD = 128;
constexpr int kPage = 128;
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kStageTokens = 64;
constexpr int kStages = 4;
constexpr int kTileBytes = kStageTokens * kD * 2;  // 16 KB of K (and of V) per stage
constexpr int kMaxGroup = 8;
constexpr int kQBytes = kMaxGroup * kD * 2;        // q rows of one (sequence, kv head)
constexpr int kStageBytes = 2 * kTileBytes + kQBytes;
constexpr int kMaxBatch = 2048;                    // sequences per launch (prefix sums in LDS)
constexpr int kDmaPerStage = 2 * (kTileBytes / 1024) / kWaves;  // K/V DMAs per wave per stage (4)
constexpr int kLdsBytes = kStages * kStageBytes + (kMaxBatch + 1 + 15) * 4 + 64;

struct SuffixArgs {
    const uint16_t *q;
    const uint16_t *k;
    const uint16_t *v;
    const int32_t *bt;
    const int64_t *kv_seqlens;
    uint16_t *out;
    float *lse;
    float *part_o;    // [kv_heads][chunks][2][G][kD]
    float *part_lse;  // [kv_heads][chunks][2][G]
    int32_t *cu_out;  // [batch + 1] prefix sums, written by workgroup 0
    int64_t bt_cols;
    int64_t num_blocks;
    int batch;
    int num_heads;
    int kv_heads;
    int kv_cap;
    int chunks;  // workgroups per kv head
    float scale_log2;
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Sum over the 16 lanes of a DPP row; every lane of the row receives the total.
__device__ __forceinline__ float row16_sum(float x) {
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xF, 0xF, false));  // row_ror:8
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x124, 0xF, 0xF, false));  // row_ror:4
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x122, 0xF, 0xF, false));  // row_ror:2
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x121, 0xF, 0xF, false));  // row_ror:1
    return x;
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                           false);
}

// q.k over this lane's 8 dims (4 packed bf16 pairs each), fp32 accumulate.
__device__ __forceinline__ float dot8(const uint4 &k, const uint4 &q) {
    float d = dot2(k.x, q.x, 0.f);
    d = dot2(k.y, q.y, d);
    d = dot2(k.z, q.z, d);
    return dot2(k.w, q.w, d);
}

// Scalar (SMEM) load of one int: waits on lgkmcnt only, never on the vector
// memory counter the DMA ring uses.
__device__ __forceinline__ int sload_i32(const int32_t *p) {
    int v;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
    return v;
}

__device__ __forceinline__ void wait_stages(int outstanding) {
    if (outstanding >= 2) wait_vmcnt<2 * kDmaPerStage>();
    else if (outstanding == 1) wait_vmcnt<kDmaPerStage>();
    else wait_vmcnt<0>();
}

__device__ __forceinline__ int64_t clamp_len(const SuffixArgs &a, int64_t kvl) {
    const int64_t lim = a.bt_cols * kPage;
    if (kvl > lim) kvl = lim;
    if (kvl > a.kv_cap) kvl = a.kv_cap;
    if (a.num_blocks <= 0) kvl = 0;
    return kvl < 0 ? 0 : kvl;
}

// Walk over the stages of a workgroup's token range [r0, r1): a stage is a
// 64-token aligned window of one sequence; consecutive stages cross sequences.
struct Cursor {
    int b;      // sequence
    int jst;    // sequence-local first token of the stage window (multiple of 64)
    int sj0;    // sequence-local start of this workgroup's segment of b
    int sj1;    // sequence-local end of the segment
    bool valid;
};

__device__ __forceinline__ void cursor_seg(Cursor &cur, const CK_LDS int *cu, int64_t r0, int64_t r1) {
    const int base = cu[cur.b];
    cur.sj0 = (int)((r0 > base ? r0 : base) - base);
    const int64_t e = cu[cur.b + 1];
    cur.sj1 = (int)((r1 < e ? r1 : e) - base);
    cur.jst = (cur.sj0 / kStageTokens) * kStageTokens;
}

__device__ __forceinline__ void cursor_next(Cursor &cur, const CK_LDS int *cu, int batch, int64_t r0, int64_t r1) {
    cur.jst += kStageTokens;
    if (cur.jst < cur.sj1) return;
    int b = cur.b + 1;
    while (b < batch && cu[b + 1] == cu[b]) ++b;  // empty sequences have no stages
    if (b >= batch || cu[b] >= r1) {
        cur.valid = false;
        return;
    }
    cur.b = b;
    cursor_seg(cur, cu, r0, r1);
}

template <int G>
__global__ __launch_bounds__(kThreads) void suffix_stream_kernel(SuffixArgs a) {
    extern __shared__ __attribute__((aligned(16))) char smem_raw[];
    CK_LDS char *smem = (CK_LDS char *)smem_raw;
    CK_LDS int *cu = (CK_LDS int *)(smem + kStages * kStageBytes);  // [batch + 1]
    CK_LDS int *wtot = cu + kMaxBatch + 1;                            // [kWaves] scan scratch
    CK_LDS int *slot_ok = wtot + kWaves;                              // [kStages] page validity

    const int tid = threadIdx.x;
    const int wid = tid >> 6;
    const int lane = tid & 63;
    const int slot = lane >> 4;
    const int c = lane & 15;
    const int g = blockIdx.x % a.kv_heads;
    const int chunk = blockIdx.x / a.kv_heads;

    // ---- prefix sums of the clamped lengths (4 per thread, block scan) ------------
    int lv[4];
    int local = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = 4 * tid + j;
        lv[j] = i < a.batch ? (int)clamp_len(a, a.kv_seqlens[i]) : 0;
        local += lv[j];
    }
    int x = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off);
        if (lane >= off) x += y;
    }
    if (lane == 63) wtot[wid] = x;
    __syncthreads();
    int wave_off = 0;
    for (int ww = 0; ww < wid; ++ww) wave_off += wtot[ww];
    int run = wave_off + x - local;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = 4 * tid + j;
        run += lv[j];
        if (i < a.batch) cu[i + 1] = run;
    }
    if (tid == 0) cu[0] = 0;
    __syncthreads();
    if (blockIdx.x == 0)
        for (int i = tid; i <= a.batch; i += kThreads) a.cu_out[i] = cu[i];

    const int64_t T = cu[a.batch];
    const int64_t r0 = (int64_t)chunk * T / a.chunks;
    const int64_t r1 = (int64_t)(chunk + 1) * T / a.chunks;
    if (r0 >= r1) return;  // uniform over the workgroup

    // first sequence: largest b with cu[b] <= r0 (then cu[b + 1] > r0)
    int lo = 0, hi = a.batch;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (cu[mid] <= r0) lo = mid;
        else hi = mid - 1;
    }
    Cursor ic;
    ic.b = lo;
    ic.valid = true;
    cursor_seg(ic, cu, r0, r1);
    Cursor cc = ic;

    const int64_t head_stride = (int64_t)a.kv_heads * kD;
    auto issue = [&](const Cursor &cur, int n) {
        CK_LDS char *kb = smem + (n % kStages) * kStageBytes;
        CK_LDS char *vb = kb + kTileBytes;
        CK_LDS char *qb = vb + kTileBytes;
        int page = sload_i32(a.bt + (int64_t)cur.b * a.bt_cols + cur.jst / kPage);
        const bool ok = page >= 0 && (int64_t)page < a.num_blocks;
        if (tid == 0) slot_ok[n % kStages] = ok ? 1 : 0;
        if (!ok) page = 0;  // keep the per-wave DMA count exact; rows are zeroed at use
        const int64_t tok0 = (int64_t)page * kPage + (cur.jst % kPage);
#pragma unroll
        for (int j = 0; j < kDmaPerStage / 2; ++j) {
            const int blk = wid * (kDmaPerStage / 2) + j;  // 4 token rows per DMA
            const int tt = blk * 4 + (lane >> 4);
            const int64_t off = (tok0 + tt) * head_stride + g * kD + (lane & 15) * 8;
            dma16(a.k + off, kb + blk * 1024);
            dma16(a.v + off, vb + blk * 1024);
        }
        // the sequence's q rows (G x 256 B, contiguous) with its first stage
        if (cur.jst == (cur.sj0 / kStageTokens) * kStageTokens && wid * 64 < G * 16) {
            if (lane < G * 16 - wid * 64)
                dma16(a.q + ((int64_t)cur.b * a.num_heads + g * G) * kD + (wid * 64 + lane) * 8, qb + wid * 1024);
        }
    };

    int n_issued = 0;
    for (int k = 0; k < kStages - 1 && ic.valid; ++k) {
        issue(ic, n_issued++);
        cursor_next(ic, cu, a.batch, r0, r1);
    }

    uint4 qp[G];
    float m[G], l[G], acc[G][8];
    int n_done = 0;
    while (cc.valid) {
        wait_stages(n_issued - n_done - 1);
        __syncthreads();
        const int st = n_done % kStages;
        CK_LDS char *kb = smem + st * kStageBytes;
        CK_LDS char *vb = kb + kTileBytes;
        CK_LDS char *qb = vb + kTileBytes;
        const int tlo = (cc.sj0 > cc.jst ? cc.sj0 : cc.jst) - cc.jst;
        const int thi = (cc.sj1 < cc.jst + kStageTokens ? cc.sj1 : cc.jst + kStageTokens) - cc.jst;
        const bool first = cc.jst == (cc.sj0 / kStageTokens) * kStageTokens;
        const bool last = cc.jst + kStageTokens >= cc.sj1;
        const bool page_ok = slot_ok[st] != 0;
        if (tlo > 0 || thi < kStageTokens || !page_ok) {
            // rows outside this segment (or of an invalid page) may hold anything:
            // zero them so 0 * V cannot produce a NaN
            for (int idx = tid; idx < kStageTokens * 16; idx += kThreads) {
                const int tt = idx >> 4, cc16 = idx & 15;
                if (!page_ok || tt < tlo || tt >= thi) {
                    *reinterpret_cast<CK_LDS u32x4 *>(kb + tt * 256 + cc16 * 16) = u32x4{0, 0, 0, 0};
                    *reinterpret_cast<CK_LDS u32x4 *>(vb + tt * 256 + cc16 * 16) = u32x4{0, 0, 0, 0};
                }
            }
            __syncthreads();
        }
        if (ic.valid) {
            issue(ic, n_issued++);
            cursor_next(ic, cu, a.batch, r0, r1);
        }
        if (first) {
#pragma unroll
            for (int hq = 0; hq < G; ++hq) {
                const u32x4 qq = *reinterpret_cast<const CK_LDS u32x4 *>(qb + hq * 256 + c * 16);
                const uint32_t q0 = qq[0], q1 = qq[1], q2 = qq[2], q3 = qq[3];
                qp[hq] = make_uint4(q0, q1, q2, q3);
                m[hq] = -INFINITY;
                l[hq] = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[hq][e] = 0.f;
            }
        }

        // this wave: tokens 8*wid + 4u + slot, u = 0..1
        const int tbase = 8 * wid;
        if (tbase < thi && tbase + 8 > tlo) {
            uint4 kr[2];
            float vf[2][8];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int tt = tbase + 4 * u + slot;
                const u32x4 kk = *reinterpret_cast<const CK_LDS u32x4 *>(kb + tt * 256 + c * 16);
                const u32x4 vv = *reinterpret_cast<const CK_LDS u32x4 *>(vb + tt * 256 + c * 16);
                const uint32_t k0 = kk[0], k1 = kk[1], k2 = kk[2], k3 = kk[3];
                const uint32_t v0 = vv[0], v1 = vv[1], v2 = vv[2], v3 = vv[3];
                kr[u] = make_uint4(k0, k1, k2, k3);
                vf[u][0] = bf16_lo(v0); vf[u][1] = bf16_hi(v0);
                vf[u][2] = bf16_lo(v1); vf[u][3] = bf16_hi(v1);
                vf[u][4] = bf16_lo(v2); vf[u][5] = bf16_hi(v2);
                vf[u][6] = bf16_lo(v3); vf[u][7] = bf16_hi(v3);
            }
#pragma unroll
            for (int hq = 0; hq < G; ++hq) {
                float s[2];
                float smax = -INFINITY;
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int tt = tbase + 4 * u + slot;
                    const float d = row16_sum(dot8(kr[u], qp[hq])) * a.scale_log2;
                    s[u] = (tt >= tlo && tt < thi) ? d : -INFINITY;
                    smax = fmaxf(smax, s[u]);
                }
                const float m_new = fmaxf(m[hq], smax);
                const float m_use = m_new == -INFINITY ? 0.f : m_new;
                const float dm = exp2_fast(m[hq] - m_use);
                float ps = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[hq][e] *= dm;
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const float p = exp2_fast(s[u] - m_use);
                    ps += p;
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[hq][e] = fmaf(p, vf[u][e], acc[hq][e]);
                }
                l[hq] = l[hq] * dm + ps;
                m[hq] = m_new;
            }
        }

        if (last) {
            // ---- finalize the segment: 4 slots (shuffles) then 8 waves (LDS) ----
#pragma unroll
            for (int off = 16; off <= 32; off <<= 1) {
#pragma unroll
                for (int hq = 0; hq < G; ++hq) {
                    const float mo = __shfl_xor(m[hq], off);
                    const float lo2 = __shfl_xor(l[hq], off);
                    const float mn = fmaxf(m[hq], mo);
                    const float mu = mn == -INFINITY ? 0.f : mn;
                    const float fa = exp2_fast(m[hq] - mu), fb = exp2_fast(mo - mu);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float ao = __shfl_xor(acc[hq][e], off);
                        acc[hq][e] = acc[hq][e] * fa + ao * fb;
                    }
                    l[hq] = l[hq] * fa + lo2 * fb;
                    m[hq] = mn;
                }
            }
            __syncthreads();  // every wave is done with this stage's K/V (q is in registers)
            CK_LDS float *xacc = (CK_LDS float *)kb;            // [kWaves][G][kD], spans K, V and q areas
            CK_LDS float *xm = xacc + kWaves * G * kD;          // [kWaves][G]
            CK_LDS float *xl = xm + kWaves * G;                 // [kWaves][G]
            if (slot == 0) {
#pragma unroll
                for (int hq = 0; hq < G; ++hq) {
                    *reinterpret_cast<CK_LDS f32x4 *>(xacc + (wid * G + hq) * kD + 8 * c) =
                        f32x4{acc[hq][0], acc[hq][1], acc[hq][2], acc[hq][3]};
                    *reinterpret_cast<CK_LDS f32x4 *>(xacc + (wid * G + hq) * kD + 8 * c + 4) =
                        f32x4{acc[hq][4], acc[hq][5], acc[hq][6], acc[hq][7]};
                    if (c == 0) {
                        xm[wid * G + hq] = m[hq];
                        xl[wid * G + hq] = l[hq];
                    }
                }
            }
            __syncthreads();
            const int b = cc.b;
            const bool head_part = (int64_t)cu[b] < r0;
            const bool tail_part = (int64_t)cu[b + 1] > r1;
            for (int idx = tid; idx < G * 16; idx += kThreads) {
                const int hq = idx >> 4, cc8 = idx & 15;
                float mn = -INFINITY;
#pragma unroll
                for (int ww = 0; ww < kWaves; ++ww) mn = fmaxf(mn, xm[ww * G + hq]);
                const float mu = mn == -INFINITY ? 0.f : mn;
                float lt = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ww = 0; ww < kWaves; ++ww) {
                    const float f = exp2_fast(xm[ww * G + hq] - mu);
                    lt += xl[ww * G + hq] * f;
                    const f32x4 a0 = *reinterpret_cast<const CK_LDS f32x4 *>(xacc + (ww * G + hq) * kD + 8 * cc8);
                    const f32x4 a1 = *reinterpret_cast<const CK_LDS f32x4 *>(xacc + (ww * G + hq) * kD + 8 * cc8 + 4);
                    o[0] += a0[0] * f; o[1] += a0[1] * f; o[2] += a0[2] * f; o[3] += a0[3] * f;
                    o[4] += a1[0] * f; o[5] += a1[1] * f; o[6] += a1[2] * f; o[7] += a1[3] * f;
                }
                const float inv = lt > 0.f ? 1.0f / lt : 0.f;
                const float lse_v = lt > 0.f ? (mn + __log2f(lt)) * kLn2 : -INFINITY;
                if (!head_part && !tail_part) {
                    const int64_t row = (int64_t)b * a.num_heads + g * G + hq;
                    uint4 ow;
                    ow.x = pack_bf16x2(o[0] * inv, o[1] * inv);
                    ow.y = pack_bf16x2(o[2] * inv, o[3] * inv);
                    ow.z = pack_bf16x2(o[4] * inv, o[5] * inv);
                    ow.w = pack_bf16x2(o[6] * inv, o[7] * inv);
                    *reinterpret_cast<uint4 *>(a.out + row * kD + 8 * cc8) = ow;
                    if (cc8 == 0) a.lse[row] = lse_v;
                } else {
                    const int64_t pidx = (((int64_t)g * a.chunks + chunk) * 2 + (head_part ? 0 : 1)) * G + hq;
                    float4 *dst = reinterpret_cast<float4 *>(a.part_o + pidx * kD + 8 * cc8);
                    dst[0] = make_float4(o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv);
                    dst[1] = make_float4(o[4] * inv, o[5] * inv, o[6] * inv, o[7] * inv);
                    if (cc8 == 0) a.part_lse[pidx] = lse_v;
                }
            }
        }
        ++n_done;
        cursor_next(cc, cu, a.batch, r0, r1);
    }
}

// Chunk that owns stream position p: chunk c covers [c*T/P, (c+1)*T/P).
__device__ __forceinline__ int owner_chunk(int64_t p, int64_t T, int P) {
    return (int)(((p + 1) * P - 1) / T);
}

// One workgroup per (sequence, kv head): empty suffixes get O = 0, LSE = -inf;
// a sequence cut by chunk boundaries gets its partials folded; others return.
template <int G>
__global__ __launch_bounds__(256) void suffix_fixup_kernel(SuffixArgs a) {
    const int b = blockIdx.x / a.kv_heads;
    const int g = blockIdx.x % a.kv_heads;
    const int hq = threadIdx.x >> 5;
    const int d4 = threadIdx.x & 31;
    if (hq >= G) return;
    const int64_t beg = a.cu_out[b], end = a.cu_out[b + 1], T = a.cu_out[a.batch];
    const int64_t row = (int64_t)b * a.num_heads + g * G + hq;
    if (end == beg) {
        *reinterpret_cast<uint2 *>(a.out + row * kD + 4 * d4) = make_uint2(0, 0);
        if (d4 == 0) a.lse[row] = -INFINITY;
        return;
    }
    const int ca = owner_chunk(beg, T, a.chunks);
    const int cb = owner_chunk(end - 1, T, a.chunks);
    if (ca == cb) return;  // written by the stream kernel
    auto pidx = [&](int ch, int sl) { return (((int64_t)g * a.chunks + ch) * 2 + sl) * G + hq; };
    float mx = a.part_lse[pidx(ca, 1)];
    for (int ch = ca + 1; ch <= cb; ++ch)
        if ((int64_t)ch * T / a.chunks != (int64_t)(ch + 1) * T / a.chunks) mx = fmaxf(mx, a.part_lse[pidx(ch, 0)]);
    const float mu = mx == -INFINITY ? 0.f : mx;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float wsum = 0.f;
    for (int ch = ca; ch <= cb; ++ch) {
        // chunks with an empty range (T < P) processed nothing
        if ((int64_t)ch * T / a.chunks == (int64_t)(ch + 1) * T / a.chunks) continue;
        const int64_t p = pidx(ch, ch == ca ? 1 : 0);
        const float wgt = exp2_fast((a.part_lse[p] - mu) * kLog2e);
        const float4 o = *reinterpret_cast<const float4 *>(a.part_o + p * kD + 4 * d4);
        acc.x = fmaf(wgt, o.x, acc.x);
        acc.y = fmaf(wgt, o.y, acc.y);
        acc.z = fmaf(wgt, o.z, acc.z);
        acc.w = fmaf(wgt, o.w, acc.w);
        wsum += wgt;
    }
    const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
    *reinterpret_cast<uint2 *>(a.out + row * kD + 4 * d4) =
        make_uint2(pack_bf16x2(acc.x * inv, acc.y * inv), pack_bf16x2(acc.z * inv, acc.w * inv));
    if (d4 == 0) a.lse[row] = wsum > 0.f ? mx + __logf(wsum) : -INFINITY;
}

int64_t ceil_div(int64_t x, int64_t y) { return (x + y - 1) / y; }

// Workgroups per kv head: about one workgroup per CU over the whole grid.
int64_t suffix_chunks(int64_t kv_heads, int64_t forced) {
    if (forced > 0) return forced;
    const int64_t p = 256 / kv_heads;
    return p > 0 ? p : 1;
}

int64_t suffix_ws_bytes(int64_t batch, int64_t num_heads, int64_t kv_heads, int64_t chunks) {
    const int64_t group = num_heads / kv_heads;
    const int64_t nb = batch < kMaxBatch ? batch : kMaxBatch;
    const int64_t parts = kv_heads * chunks * 2 * group;
    return parts * (kD + 1) * (int64_t)sizeof(float) + (nb + 1) * (int64_t)sizeof(int32_t) + 256;
}

template <int G>
int launch_suffix(const SuffixArgs &a, hipStream_t st) {
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&suffix_stream_kernel<G>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
        if (e != hipSuccess) return static_cast<int>(e);
        attr_set = true;
    }
    static_assert((kWaves * G * kD + 2 * kWaves * G) * 4 <= kStageBytes, "exchange fits in a stage");
    hipLaunchKernelGGL(suffix_stream_kernel<G>, dim3((unsigned)(a.kv_heads * a.chunks)), dim3(kThreads), kLdsBytes,
                       st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return static_cast<int>(e);
    hipLaunchKernelGGL(suffix_fixup_kernel<G>, dim3((unsigned)(a.batch * a.kv_heads)), dim3(256), 0, st, a);
    CK_RETURN_LAUNCH();
}

int check_suffix_dims(int64_t batch, int64_t num_heads, int64_t kv_heads, int64_t head_dim, int64_t kv_cap) {
    if (batch < 0 || kv_cap < 0) return CK_E_INVALID_ARG;
    if (head_dim != kD) return CK_E_UNSUPPORTED;
    if (kv_heads <= 0 || num_heads <= 0 || num_heads % kv_heads != 0) return CK_E_INVALID_ARG;
    const int64_t group = num_heads / kv_heads;
    if (group > kMaxGroup) return CK_E_UNSUPPORTED;
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
    const int64_t chunks = suffix_chunks(kv_heads, 0);
    *num_splits = chunks;
    *workspace_bytes = batch > 0 ? suffix_ws_bytes(batch, num_heads, kv_heads, chunks) : 0;
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
    const int64_t chunks = suffix_chunks(kv_heads, num_splits);
    if (kv_heads * chunks > 0x7FFFFFFF || chunks > (1 << 20)) return CK_E_INVALID_ARG;
    const int64_t need = suffix_ws_bytes(batch, num_heads, kv_heads, chunks);
    if (workspace == nullptr || workspace_bytes < need) return CK_E_WORKSPACE;
    const int64_t group = num_heads / kv_heads;
    const int64_t parts = kv_heads * chunks * 2 * group;

    SuffixArgs a;
    a.k = static_cast<const uint16_t *>(k);
    a.v = static_cast<const uint16_t *>(v);
    a.part_o = static_cast<float *>(workspace);
    a.part_lse = a.part_o + parts * kD;
    a.cu_out = reinterpret_cast<int32_t *>(a.part_lse + parts);
    a.bt_cols = bt_cols;
    a.num_blocks = num_blocks;
    a.num_heads = (int)num_heads;
    a.kv_heads = (int)kv_heads;
    a.kv_cap = (int)kv_cap;
    a.chunks = (int)chunks;
    a.scale_log2 = scale * kLog2e;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    // sequences are processed in launches of at most kMaxBatch (prefix sums in
    // LDS), fewer when the token total could overflow the 32-bit sums
    int64_t per_launch = kMaxBatch;
    const int64_t cap = kv_cap > 0 ? kv_cap : 1;
    if (per_launch > 0x7FFFFFFF / cap) per_launch = 0x7FFFFFFF / cap;
    if (per_launch < 1) per_launch = 1;
    for (int64_t b0 = 0; b0 < batch; b0 += per_launch) {
        const int64_t nb = batch - b0 < per_launch ? batch - b0 : per_launch;
        a.q = static_cast<const uint16_t *>(q) + b0 * num_heads * kD;
        a.bt = block_table + b0 * bt_cols;
        a.kv_seqlens = kv_seqlens + b0;
        a.out = static_cast<uint16_t *>(out) + b0 * num_heads * kD;
        a.lse = lse + b0 * num_heads;
        a.batch = (int)nb;
        switch (group) {
            case 1: rc = launch_suffix<1>(a, st); break;
            case 2: rc = launch_suffix<2>(a, st); break;
            case 3: rc = launch_suffix<3>(a, st); break;
            case 4: rc = launch_suffix<4>(a, st); break;
            case 5: rc = launch_suffix<5>(a, st); break;
            case 6: rc = launch_suffix<6>(a, st); break;
            case 7: rc = launch_suffix<7>(a, st); break;
            default: rc = launch_suffix<8>(a, st); break;
        }
        if (rc != CK_OK) return rc;
    }
    return CK_OK;
}
