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
// MI355X design: memory-bound streaming with a persistent, balanced grid.
// * Suffix lengths vary widely (geometric in the benchmark), and a workgroup
//   pays several microseconds of start-up (lengths, page ids, first DMA round
//   trip) before its first byte of K/V. So the work is cut into windows of 64
//   tokens of one sequence (the last window of a sequence may be short), and
//   workgroup (kv head g, chunk c) takes the c-th 1/P of the list of all
//   windows, crossing sequence boundaries: every workgroup streams the same
//   number of windows and starts once. Window and length prefix sums are built
//   per workgroup in LDS from the device-side lengths.
// * Two paged K/V layouts: NHD [blocks, 128, kv_heads, 128] (the stage-1 pool)
//   and BNSD [blocks, kv_heads, 128, 128] (the layout the reference's stage-2
//   op reads, ascend-kernel/README.md:182-183), so a BNSD pool needs no
//   transposing copy. A page, a token and a kv head are three strides; each
//   DMA moves four 256-byte token rows of one kv head either way.
// * K and V rows stream through a 2-stage LDS ring (one window, 32 KB, per
//   stage) by global->LDS DMA, continuously across sequence boundaries. The
//   ring, prefix sums and scratch take about 78 KB, so two workgroups share a
//   CU (16 waves): while one waits on its stage the other computes, which
//   hides more latency than a deeper ring in one workgroup per CU. A stage's
//   DMA group also carries a block-table entry kStages - 1 windows ahead (so
//   page ids never wait on memory inside the loop) and, on the first window of
//   a sequence, its q rows. Each wave counts its own vector-memory
//   operations (DMAs and output stores) and waits for exactly one stage. Half
//   the waves issue the next group right after the stage barrier and half after
//   their compute, so the DMA issue of one half overlaps the other's arithmetic.
// * Scores: lane (t, c) of wave w holds token 8w + t, dims 8c..8c+7 and
//   64+8c..64+8c+7; q.k is eight packed bf16 dot products (v_dot2_f32_bf16,
//   two chains) and a 3-step DPP sum over the token's 8 lanes.
// * Softmax: the running max is uniform over the wave and moves only when a
//   score exceeds it by more than 2^kTau (a wave-uniform branch), so rescaling
//   is rare; any reference point gives the same O and LSE.
// * Values: lane l accumulates dims 2l, 2l+1 of every query head over all of
//   the wave's tokens; the token weights reach the lanes as LDS broadcasts.
//   Closing a sequence therefore needs only a cross-wave merge through the
//   just-consumed ring stage.
// * A segment that is a whole sequence writes bf16 O and the LSE directly; a
//   sequence cut by a chunk boundary leaves fp32 partials that a small fix-up
//   kernel folds (it also writes O = 0, LSE = -inf for empty suffixes).
#include "ck_common.h"
#include "ck_internal.h"

namespace ck {
namespace {

constexpr int kD = 128;
constexpr int kPage = 128;
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kWin = 64;                           // tokens per window (= per ring stage)
constexpr int kStages = 2;
constexpr int kTileBytes = kWin * kD * 2;          // 16 KB of K (and of V) per stage
constexpr int kMaxGroup = 8;
constexpr int kQBytes = kMaxGroup * kD * 2;        // q rows of one (sequence, kv head)
constexpr int kStageBytes = 2 * kTileBytes + kQBytes;
constexpr int kMaxBatch = 1024;                    // sequences per launch (prefix sums in LDS)
constexpr int kBlocksPerCu = 2;                    // resident workgroups per CU the grid is sized for
constexpr int kPgRing = 8;                         // block-table entries in flight
constexpr int kKvDmaPerWave = 2 * (kTileBytes / 1024) / kWaves;  // 4
constexpr float kTau = 8.0f;                       // log2 headroom before the running max moves

// LDS layout (bytes)
constexpr int kCwOff = kStages * kStageBytes;                 // int cw[kMaxBatch + 1]: window prefix sums
constexpr int kLenOff = kCwOff + ((kMaxBatch + 1) * 4 + 15) / 16 * 16;  // int len[kMaxBatch]
constexpr int kWtotOff = kLenOff + kMaxBatch * 4;             // int wtot[kWaves] scan scratch
constexpr int kPgOff = kWtotOff + kWaves * 4;                 // int pgring[kPgRing]
constexpr int kPwOff = kPgOff + kPgRing * 4;                  // float pw[kWaves][8][kMaxGroup]
constexpr int kLdsBytes = kPwOff + kWaves * 8 * kMaxGroup * 4;
static_assert(kPwOff % 16 == 0, "p broadcast rows are read 16 bytes at a time");
static_assert(kLdsBytes * kBlocksPerCu <= 160 * 1024, "kBlocksPerCu workgroups share the CU's LDS");

struct SuffixArgs {
    const uint16_t *q;
    const uint16_t *k;
    const uint16_t *v;
    const int32_t *bt;
    const int64_t *kv_seqlens;
    uint16_t *out;
    float *lse;
    float *part_o;    // [kv head groups][chunks][2][G][kD]
    float *part_lse;  // [kv head groups][chunks][2][G]
    int32_t *cw_out;  // [batch + 1] window prefix sums, written by workgroup 0
    int64_t bt_cols;
    int64_t num_blocks;
    int64_t page_stride;  // elements between pages (both layouts: 128 * kv_heads * 128)
    int64_t tok_stride;   // between tokens of a page: kv_heads * 128 (NHD) or 128 (BNSD)
    int64_t head_off;     // between kv heads:          128 (NHD) or 128 * 128 (BNSD)
    int batch;
    int num_heads;
    int kv_heads;  // kv head groups of the grid: physical kv heads x kv_sub
    int kv_sub;    // query-head groups per physical kv head (group = kv_sub x G)
    int kv_cap;
    int chunks;  // workgroups per kv head group
    float scale_log2;
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Every control used below (quad_perm, row_half_mirror, row_ror) reads a lane of
// the same 16-lane row, so bound_ctrl never applies; setting it lets the
// compiler fold the move into the consuming add (v_add_f32_dpp).
#define CK_DPP(x, ctrl) __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), ctrl, 0xF, 0xF, true))

// op(x[l], x[l ^ 16]) and op(x[l], x[l ^ 32]) through v_permlane16_swap /
// v_permlane32_swap: swapping x with itself leaves x[l] in one result and the
// partner lane's x in the other (a VALU exchange, no LDS round trip).
__device__ __forceinline__ float max_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over each aligned group of 8 lanes; every lane of the group gets the total.
__device__ __forceinline__ float sum8(float x) {
    x += CK_DPP(x, 0xB1);   // quad_perm [1,0,3,2]
    x += CK_DPP(x, 0x4E);   // quad_perm [2,3,0,1]
    x += CK_DPP(x, 0x141);  // row_half_mirror: the other quad of the 8
    return x;
}
// Reduce a value that is constant within each 8-lane group over the 8 groups.
__device__ __forceinline__ float max_groups(float x) {
    x = fmaxf(x, CK_DPP(x, 0x128));  // row_ror:8, the other group of the 16-lane row
    return max_xor32(max_xor16(x));
}
__device__ __forceinline__ float sum_groups(float x) {
    x += CK_DPP(x, 0x128);
    return sum_xor32(sum_xor16(x));
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                           false);
}

__device__ __forceinline__ int64_t clamp_len(const SuffixArgs &a, int64_t kvl) {
    const int64_t lim = a.bt_cols * kPage;
    if (kvl > lim) kvl = lim;
    if (kvl > a.kv_cap) kvl = a.kv_cap;
    if (a.num_blocks <= 0) kvl = 0;
    return kvl < 0 ? 0 : kvl;
}

// Walk over the windows of a workgroup's window range [w0, w1) of the list of
// all windows; consecutive windows cross sequences. Values are wave-uniform.
struct Cursor {
    int b;       // sequence
    int k;       // window index inside the sequence (tokens 64k ..)
    int kfirst;  // first window of this workgroup's segment of b
    int kend;    // one past the segment's last window
    bool valid;
};

__device__ __forceinline__ void cursor_seg(Cursor &cur, const CK_LDS int *cw, int w0, int w1) {
    const int base = cw[cur.b];
    cur.k = (w0 > base ? w0 : base) - base;
    const int e = cw[cur.b + 1];
    cur.kend = (w1 < e ? w1 : e) - base;
    cur.kfirst = cur.k;
}

__device__ __forceinline__ void cursor_next(Cursor &cur, const CK_LDS int *cw, int batch, int w0, int w1) {
    if (!cur.valid) return;
    if (++cur.k < cur.kend) return;
    int b = cur.b + 1;
    while (b < batch && cw[b + 1] == cw[b]) ++b;  // empty sequences have no windows
    if (b >= batch || cw[b] >= w1) {
        cur.valid = false;
        return;
    }
    cur.b = b;
    cursor_seg(cur, cw, w0, w1);
}

template <int G>
__global__ __launch_bounds__(kThreads) void suffix_stream_kernel(SuffixArgs a) {
    extern __shared__ __attribute__((aligned(16))) char smem_raw[];
    CK_LDS char *smem = (CK_LDS char *)smem_raw;
    CK_LDS int *cw = (CK_LDS int *)(smem + kCwOff);
    CK_LDS int *len = (CK_LDS int *)(smem + kLenOff);
    CK_LDS int *wtot = (CK_LDS int *)(smem + kWtotOff);
    CK_LDS int *pgring = (CK_LDS int *)(smem + kPgOff);
    constexpr int kPwRow = (G + 3) / 4 * 4;  // floats per token in the broadcast rows
    constexpr int kQWaves = (G * 16 + 63) / 64;  // waves whose lanes carry the q rows

    const int tid = threadIdx.x;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int t = lane >> 3;  // token slot of this lane in the wave's 8 tokens
    const int c = lane & 7;   // column pair: dims 8c.. and 64+8c..
    const int g = blockIdx.x % a.kv_heads;  // kv head group: query heads g * G .. + G
    const int chunk = blockIdx.x / a.kv_heads;
    const int gk = g / a.kv_sub;            // the physical kv head they read
    CK_LDS float *pw = (CK_LDS float *)(smem + kPwOff) + wid * 8 * kPwRow;

    // ---- lengths and window prefix sums (4 sequences per thread, block scan) ------
    int lv[4];
    int local = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = 4 * tid + j;
        const int ln = i < a.batch ? (int)clamp_len(a, a.kv_seqlens[i]) : 0;
        if (i < a.batch) len[i] = ln;
        lv[j] = (ln + kWin - 1) / kWin;
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
        if (i < a.batch) cw[i + 1] = run;
    }
    if (tid == 0) cw[0] = 0;
    __syncthreads();
    if (blockIdx.x == 0)
        for (int i = tid; i <= a.batch; i += kThreads) a.cw_out[i] = cw[i];

    const int W = cw[a.batch];
    const int w0 = (int)((int64_t)chunk * W / a.chunks);
    const int w1 = (int)((int64_t)(chunk + 1) * W / a.chunks);
    if (w0 >= w1) return;  // uniform over the workgroup

    // first sequence: largest b with cw[b] <= w0 (then cw[b + 1] > w0)
    int lo = 0, hi = a.batch;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (cw[mid] <= w0) lo = mid;
        else hi = mid - 1;
    }
    Cursor cc;
    cc.b = lo;
    cc.valid = true;
    cursor_seg(cc, cw, w0, w1);

    // page ids of the first kStages - 1 windows; later ones travel with the ring
    Cursor pc = cc;
    for (int j = 0; j < kStages - 1; ++j) {
        if (pc.valid && tid == j) pgring[j] = a.bt[(int64_t)pc.b * a.bt_cols + pc.k * kWin / kPage];
        cursor_next(pc, cw, a.batch, w0, w1);
    }
    __syncthreads();

    int tot = 0;  // vector-memory operations this wave has issued (wave-uniform)
    // DMA group of window n (cursor cur): the block-table entry of window n + 3
    // (cursor pcur; wave 0), the window's K and V rows, and on the first window
    // of a segment the sequence's q rows.
    auto issue = [&](const Cursor &cur, const Cursor &pcur, int n) {
        CK_LDS char *kb = smem + (n % kStages) * kStageBytes;
        CK_LDS char *vb = kb + kTileBytes;
        CK_LDS char *qb = vb + kTileBytes;
        if (wid == 0) {
            const int32_t *psrc = pcur.valid ? a.bt + (int64_t)pcur.b * a.bt_cols + pcur.k * kWin / kPage : a.bt;
            if (lane == 0) dma4(psrc, pgring + (n + kStages - 1) % kPgRing);
            ++tot;
        }
        int page = pgring[n % kPgRing];
        if (page < 0 || (int64_t)page >= a.num_blocks) page = 0;  // rows ignored at use
        const int64_t pbase = (int64_t)page * a.page_stride + (int64_t)gk * a.head_off + (lane & 15) * 8;
        const int t0 = (cur.k * kWin) % kPage + (lane >> 4);
#pragma unroll
        for (int j = 0; j < kKvDmaPerWave / 2; ++j) {
            const int blk = wid * (kKvDmaPerWave / 2) + j;  // 4 token rows per DMA
            const int64_t off = pbase + (int64_t)(t0 + blk * 4) * a.tok_stride;
            dma16(a.k + off, kb + blk * 1024);
            dma16(a.v + off, vb + blk * 1024);
        }
        tot += kKvDmaPerWave;
        if (cur.k == cur.kfirst && wid < kQWaves) {
            if (wid * 64 + lane < G * 16)
                dma16(a.q + ((int64_t)cur.b * a.num_heads + g * G) * kD + (wid * 64 + lane) * 8, qb + wid * 1024);
            ++tot;
        }
    };

    // tot right after issuing each group still in flight (oldest first)
    int gend[kStages - 1];
#pragma unroll
    for (int j = 0; j < kStages - 1; ++j) gend[j] = 0;
    auto shift_gend = [&]() {
#pragma unroll
        for (int j = 0; j + 1 < kStages - 1; ++j) gend[j] = gend[j + 1];
        gend[kStages - 2] = tot;
    };
    Cursor ic = cc;
    for (int j = 0; j < kStages - 1; ++j) {
        if (ic.valid) issue(ic, pc, j);
        shift_gend();
        cursor_next(ic, cw, a.batch, w0, w1);
        cursor_next(pc, cw, a.batch, w0, w1);
    }
    // after the prologue gend[] holds groups 0 .. kStages - 2

    uint32_t qr[G][8];
    float m[G], mu[G], thr[G], l[G], acc[G][2];  // mu = m, or 0 while m = -inf
    int n_done = 0;
    while (cc.valid) {
        // everything issued after this window's group may stay in flight
        const int after = __builtin_amdgcn_readfirstlane(tot - gend[0]);
        if constexpr (kStages == 2) {
            // only the previous segment close's two stores (waves wid < G) can
            // follow the group of this window: two compares, not a 21-way switch
            if (after >= 2) wait_vmcnt<2>();
            else if (after == 1) wait_vmcnt<1>();
            else wait_vmcnt<0>();
        } else {
            wait_vmcnt_dyn(after);
        }
        __syncthreads();
        const int st = n_done % kStages;
        // the next group goes into the stage consumed last iteration; half the
        // waves issue before computing and half after, so the address unit
        // drains one half's DMAs while the other half computes
        const bool early = wid < kWaves / 2;
        if (early && ic.valid) issue(ic, pc, n_done + kStages - 1);

        CK_LDS char *kb = smem + st * kStageBytes;
        CK_LDS char *vb = kb + kTileBytes;
        CK_LDS char *qb = vb + kTileBytes;
        const int b = cc.b;
        const int thi = min(kWin, len[b] - cc.k * kWin);  // tokens of this window
        const bool first = cc.k == cc.kfirst;
        const bool last = cc.k + 1 == cc.kend;
        const int praw = pgring[n_done % kPgRing];
        const bool page_ok = praw >= 0 && (int64_t)praw < a.num_blocks;
        if (first) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const u32x4 q0 = *reinterpret_cast<const CK_LDS u32x4 *>(qb + h * 256 + c * 16);
                const u32x4 q1 = *reinterpret_cast<const CK_LDS u32x4 *>(qb + h * 256 + 128 + c * 16);
                qr[h][0] = q0[0]; qr[h][1] = q0[1]; qr[h][2] = q0[2]; qr[h][3] = q0[3];
                qr[h][4] = q1[0]; qr[h][5] = q1[1]; qr[h][6] = q1[2]; qr[h][7] = q1[3];
                m[h] = -INFINITY;
                mu[h] = 0.f;
                thr[h] = -INFINITY;
                l[h] = 0.f;
                acc[h][0] = 0.f;
                acc[h][1] = 0.f;
            }
        }

        // this wave's tokens 8 * wid + [0, t1)
        const int t1 = min(8, thi - 8 * wid);
        if (t1 > 0) {
            const int tt = 8 * wid + t;
            const u32x4 k0 = *reinterpret_cast<const CK_LDS u32x4 *>(kb + tt * 256 + c * 16);
            const u32x4 k1 = *reinterpret_cast<const CK_LDS u32x4 *>(kb + tt * 256 + 128 + c * 16);
            const uint32_t kr[8] = {k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
            const bool tok_ok = t < t1;
            float s[G];
            bool trig = false;
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float d0 = dot2(kr[0], qr[h][0], 0.f);
                float d1 = dot2(kr[4], qr[h][4], 0.f);
#pragma unroll
                for (int e = 1; e < 4; ++e) {
                    d0 = dot2(kr[e], qr[h][e], d0);
                    d1 = dot2(kr[4 + e], qr[h][4 + e], d1);
                }
                float d = sum8(d0 + d1);
                d = page_ok ? d : 0.f;  // an invalid page reads as zero rows
                s[h] = tok_ok ? d * a.scale_log2 : -INFINITY;
                trig |= s[h] > thr[h];
            }
            if (__builtin_amdgcn_ballot_w64(trig)) {
                // some score passed its head's headroom: move the reference maxima
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    const float m_new = fmaxf(m[h], max_groups(s[h]));
                    if (m_new > m[h]) {
                        const float f = exp2_fast(m[h] - m_new);  // 0 from -inf
                        acc[h][0] *= f;
                        acc[h][1] *= f;
                        l[h] *= f;
                        m[h] = m_new;
                        mu[h] = m_new;  // > -inf here
                        thr[h] = m_new + kTau;
                    }
                }
            }
            float p[kPwRow];
#pragma unroll
            for (int h = 0; h < kPwRow; ++h) p[h] = 0.f;
#pragma unroll
            for (int h = 0; h < G; ++h) {
                p[h] = exp2_fast(s[h] - mu[h]);  // 0 for masked tokens
                l[h] += p[h];
            }
            if (c == 0) {
#pragma unroll
                for (int h4 = 0; h4 < kPwRow; h4 += 4)
                    *reinterpret_cast<CK_LDS f32x4 *>(pw + t * kPwRow + h4) =
                        f32x4{p[h4], p[h4 + 1], p[h4 + 2], p[h4 + 3]};
            }
            if (page_ok) {
                // acc[h][dims 2*lane, 2*lane + 1] += p[token][h] * V[token]
                auto pv_token = [&](int j) {
                    const uint32_t vv =
                        *reinterpret_cast<const CK_LDS uint32_t *>(vb + (8 * wid + j) * 256 + lane * 4);
                    const float v0 = bf16_lo(vv), v1 = bf16_hi(vv);
#pragma unroll
                    for (int h4 = 0; h4 < kPwRow; h4 += 4) {
                        const f32x4 pv = *reinterpret_cast<const CK_LDS f32x4 *>(pw + j * kPwRow + h4);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            if (h4 + e < G) {
                                acc[h4 + e][0] = fmaf(pv[e], v0, acc[h4 + e][0]);
                                acc[h4 + e][1] = fmaf(pv[e], v1, acc[h4 + e][1]);
                            }
                        }
                    }
                };
                if (t1 == 8) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) pv_token(j);
                } else {
                    for (int j = 0; j < t1; ++j) pv_token(j);
                }
            }
        }

        if (!early && ic.valid) issue(ic, pc, n_done + kStages - 1);
        shift_gend();
        cursor_next(ic, cw, a.batch, w0, w1);
        cursor_next(pc, cw, a.batch, w0, w1);

        if (last) {
            // ---- close the segment: per-wave sums, then the 8 waves through LDS ----
#pragma unroll
            for (int h = 0; h < G; ++h) l[h] = sum_groups(l[h]);  // token-slot partials
            __syncthreads();  // every wave is done with this stage (q is in registers)
            CK_LDS float *xacc = (CK_LDS float *)kb;    // [kWaves][G][kD]
            CK_LDS float *xm = xacc + kWaves * G * kD;  // [kWaves][G]
            CK_LDS float *xl = xm + kWaves * G;         // [kWaves][G]
#pragma unroll
            for (int h = 0; h < G; ++h)
                *reinterpret_cast<CK_LDS f32x2 *>(xacc + (wid * G + h) * kD + 2 * lane) = f32x2{acc[h][0], acc[h][1]};
            if (lane == 0) {
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    xm[wid * G + h] = m[h];
                    xl[wid * G + h] = l[h];
                }
            }
            __syncthreads();
            if (wid < G) {
                const int h = wid;
                float mx = -INFINITY;
#pragma unroll
                for (int ww = 0; ww < kWaves; ++ww) mx = fmaxf(mx, xm[ww * G + h]);
                const float mu = mx == -INFINITY ? 0.f : mx;
                float lt = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
                for (int ww = 0; ww < kWaves; ++ww) {
                    const float f = exp2_fast(xm[ww * G + h] - mu);
                    lt = fmaf(xl[ww * G + h], f, lt);
                    const f32x2 xa = *reinterpret_cast<const CK_LDS f32x2 *>(xacc + (ww * G + h) * kD + 2 * lane);
                    o0 = fmaf(xa[0], f, o0);
                    o1 = fmaf(xa[1], f, o1);
                }
                const float inv = lt > 0.f ? 1.0f / lt : 0.f;
                const float lse_v = lt > 0.f ? (mx + __log2f(lt)) * kLn2 : -INFINITY;
                const bool head_part = cw[b] < w0;
                const bool tail_part = cw[b + 1] > w1;
                if (!head_part && !tail_part) {
                    const int64_t row = (int64_t)b * a.num_heads + g * G + h;
                    *reinterpret_cast<uint32_t *>(a.out + row * kD + 2 * lane) = pack_bf16x2(o0 * inv, o1 * inv);
                    if (lane == 0) a.lse[row] = lse_v;
                } else {
                    const int64_t pidx = (((int64_t)g * a.chunks + chunk) * 2 + (head_part ? 0 : 1)) * G + h;
                    *reinterpret_cast<float2 *>(a.part_o + pidx * kD + 2 * lane) = make_float2(o0 * inv, o1 * inv);
                    if (lane == 0) a.part_lse[pidx] = lse_v;
                }
                tot += 2;  // one O store and one LSE store
            }
        }
        ++n_done;
        cursor_next(cc, cw, a.batch, w0, w1);
    }
}

// Chunk that owns window p: chunk c covers windows [c*W/P, (c+1)*W/P).
__device__ __forceinline__ int owner_chunk(int64_t p, int64_t W, int P) {
    return (int)(((p + 1) * P - 1) / W);
}

// Folds the partials of one query head of a sequence cut by chunk boundaries
// (chunks ca < cb): the tail slot (1) of chunk ca and the head slot (0) of every
// later chunk that holds windows, weighted by exp(lse - max). The first kPre
// chunks' partials are loaded before any is used, so the usual 2-4 chunk case
// costs one memory round trip; longer runs continue in a loop. The arithmetic
// (max over all, then a weighted sum in chunk order) does not depend on kPre.
template <int G>
__device__ __forceinline__ void fold_cut(const float *part_o, const float *part_lse, int g, int chunks, int hq,
                                         int d4, int ca, int cb, int64_t W, float4 &o_out, float &lse_out) {
    constexpr int kPre = 4;
    auto pidx = [&](int ch, int sl) { return (((int64_t)g * chunks + ch) * 2 + sl) * G + hq; };
    // a chunk with no windows (W < P) wrote nothing
    auto empty_chunk = [&](int ch) { return (int64_t)ch * W / chunks == (int64_t)(ch + 1) * W / chunks; };
    float pl[kPre];
    float4 po[kPre];
    bool ok[kPre];
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
        const int ch = min(ca + j, cb);  // clamped: every load is in bounds
        ok[j] = ca + j <= cb && (j == 0 || !empty_chunk(ch));
        const int64_t p = pidx(ch, j == 0 ? 1 : 0);
        pl[j] = part_lse[p];
        po[j] = *reinterpret_cast<const float4 *>(part_o + p * kD + 4 * d4);
    }
    float mx = pl[0];
#pragma unroll
    for (int j = 1; j < kPre; ++j)
        if (ok[j]) mx = fmaxf(mx, pl[j]);
    for (int ch = ca + kPre; ch <= cb; ++ch)
        if (!empty_chunk(ch)) mx = fmaxf(mx, part_lse[pidx(ch, 0)]);
    const float mu = mx == -INFINITY ? 0.f : mx;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float wsum = 0.f;
    auto add = [&](float l, const float4 &o) {
        const float wgt = exp2_fast((l - mu) * kLog2e);
        acc.x = fmaf(wgt, o.x, acc.x);
        acc.y = fmaf(wgt, o.y, acc.y);
        acc.z = fmaf(wgt, o.z, acc.z);
        acc.w = fmaf(wgt, o.w, acc.w);
        wsum += wgt;
    };
#pragma unroll
    for (int j = 0; j < kPre; ++j)
        if (ok[j]) add(pl[j], po[j]);
    for (int ch = ca + kPre; ch <= cb; ++ch) {
        if (empty_chunk(ch)) continue;
        const int64_t p = pidx(ch, 0);
        add(part_lse[p], *reinterpret_cast<const float4 *>(part_o + p * kD + 4 * d4));
    }
    const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
    o_out = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
    lse_out = wsum > 0.f ? mx + __logf(wsum) : -INFINITY;
}

// One workgroup of 32 G threads per (sequence, kv head): empty suffixes get
// O = 0, LSE = -inf; a sequence cut by chunk boundaries gets its partials
// folded; others return.
template <int G>
__global__ __launch_bounds__(kMaxGroup * 32) void suffix_fixup_kernel(SuffixArgs a) {
    const int b = blockIdx.x / a.kv_heads;
    const int g = blockIdx.x % a.kv_heads;
    const int hq = threadIdx.x >> 5;
    const int d4 = threadIdx.x & 31;
    const int64_t beg = a.cw_out[b], end = a.cw_out[b + 1], W = a.cw_out[a.batch];
    const int64_t row = (int64_t)b * a.num_heads + g * G + hq;
    if (end == beg) {
        *reinterpret_cast<uint2 *>(a.out + row * kD + 4 * d4) = make_uint2(0, 0);
        if (d4 == 0) a.lse[row] = -INFINITY;
        return;
    }
    const int ca = owner_chunk(beg, W, a.chunks);
    const int cb = owner_chunk(end - 1, W, a.chunks);
    if (ca == cb) return;  // written by the stream kernel
    float4 o;
    float l;
    fold_cut<G>(a.part_o, a.part_lse, g, a.chunks, hq, d4, ca, cb, W, o, l);
    *reinterpret_cast<uint2 *>(a.out + row * kD + 4 * d4) =
        make_uint2(pack_bf16x2(o.x, o.y), pack_bf16x2(o.z, o.w));
    if (d4 == 0) a.lse[row] = l;
}

// Cascade epilogue (fused cascade decode): one workgroup of 32 G threads per
// (sequence, kv head), 32 threads x 4 dims per query head. Folds the stage-1
// split partials of the sequence's query token, the suffix result (whole, split
// partials or empty) and merges the two with the lse_merge arithmetic
//   m = max(l1, l2); w1 = exp(l1 - m); w2 = exp(l2 - m)
//   out = (o1 w1 + o2 w2) * (1 / (w1 + w2)),  lse = m + log(w1 + w2)
// (ascend-kernel/csrc/ops/lse_merge/op_kernel/kernel_lse_merge.cpp:237-289);
// a side at -inf has weight 0, both at -inf give out = 0, lse = -inf.
// Latency, not bytes, bounds it, so the loads go out in dependency order: the
// window prefix sums, then every stage-1 partial of the row (up to kPreS
// splits), then the suffix result those sums locate; the arithmetic waits once.
struct EpilogueArgs {
    Stage1Result s1;
    const uint16_t *o2;     // bf16 [nb][H][kD] whole-sequence suffix results
    const float *lse2;      // [nb * H]
    const float *part_o;    // suffix partials [kv head groups][chunks][2][G][kD]
    const float *part_lse;  // [kv head groups][chunks][2][G]
    const int32_t *cw;      // [nb + 1] window prefix sums of the group
    uint16_t *out;          // bf16 [batch][H][kD]
    float *lse_out;         // [batch * H]
    int64_t b0;
    int nb;
    int num_heads;
    int kv_heads;  // kv head groups, as in SuffixArgs
    int chunks;
};

template <int G>
__global__ __launch_bounds__(kMaxGroup * 32) void cascade_epilogue_kernel(EpilogueArgs e) {
    constexpr int kBatch = 8;   // splits folded per rescale step
    constexpr int kPreS = 16;   // splits loaded up front
    const int bl = blockIdx.x / e.kv_heads;
    const int g = blockIdx.x % e.kv_heads;
    const int hq = threadIdx.x >> 5;
    const int d4 = threadIdx.x & 31;
    const int h = g * G + hq;
    const int64_t row = (e.b0 + bl) * e.num_heads + h;
    const int splits = e.s1.splits;

    const int64_t beg = e.cw[bl], end = e.cw[bl + 1], W = e.cw[e.nb];

    // ---- stage-1 loads: the first kPreS splits of this query row ------------------
    float ls[kPreS];
    float4 os[kPreS];
    if (splits <= 1) {
        os[0] = *reinterpret_cast<const float4 *>(e.s1.o + row * kD + 4 * d4);
        ls[0] = e.s1.lse[row * 8];
    } else {
#pragma unroll
        for (int j = 0; j < kPreS; ++j) {
            const int s = j < splits ? j : splits - 1;
            ls[j] = e.s1.lse[(int64_t)s * e.s1.rows + row];
            os[j] = *reinterpret_cast<const float4 *>(e.s1.o + ((int64_t)s * e.s1.rows + row) * kD + 4 * d4);
        }
    }

    // ---- suffix: empty, whole (bf16 result) or cut by chunk boundaries ------------
    float l2 = -INFINITY;
    float4 o2 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (end > beg) {
        const int ca = owner_chunk(beg, W, e.chunks);
        const int cb = owner_chunk(end - 1, W, e.chunks);
        if (ca == cb) {
            const int64_t r2 = (int64_t)bl * e.num_heads + h;
            const uint2 w = *reinterpret_cast<const uint2 *>(e.o2 + r2 * kD + 4 * d4);
            o2 = make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
            l2 = e.lse2[r2];
        } else {
            fold_cut<G>(e.part_o, e.part_lse, g, e.chunks, hq, d4, ca, cb, W, o2, l2);
        }
    }

    // ---- stage 1: fold the split partials (online, kBatch splits per step) --------
    float l1;
    float4 o1;
    if (splits <= 1) {
        o1 = os[0];
        l1 = ls[0];
    } else {
        float m = -INFINITY, wsum = 0.f;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        auto step = [&](const float *lb, const float4 *ob, int s0) {
            float mb = m;
#pragma unroll
            for (int j = 0; j < kBatch; ++j)
                if (s0 + j < splits) mb = fmaxf(mb, lb[j]);
            const float mu = mb == -INFINITY ? 0.f : mb;
            const float r = exp2_fast((m - mu) * kLog2e);
            acc.x *= r; acc.y *= r; acc.z *= r; acc.w *= r;
            wsum *= r;
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const float wgt = s0 + j < splits ? exp2_fast((lb[j] - mu) * kLog2e) : 0.f;
                acc.x = fmaf(wgt, ob[j].x, acc.x);
                acc.y = fmaf(wgt, ob[j].y, acc.y);
                acc.z = fmaf(wgt, ob[j].z, acc.z);
                acc.w = fmaf(wgt, ob[j].w, acc.w);
                wsum += wgt;
            }
            m = mb;
        };
#pragma unroll
        for (int s0 = 0; s0 < kPreS; s0 += kBatch)
            if (s0 < splits) step(ls + s0, os + s0, s0);
        for (int s0 = kPreS; s0 < splits; s0 += kBatch) {
            float lb[kBatch];
            float4 ob[kBatch];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const int s = s0 + j < splits ? s0 + j : splits - 1;
                lb[j] = e.s1.lse[(int64_t)s * e.s1.rows + row];
                ob[j] = *reinterpret_cast<const float4 *>(e.s1.o + ((int64_t)s * e.s1.rows + row) * kD + 4 * d4);
            }
            step(lb, ob, s0);
        }
        const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
        o1 = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
        l1 = wsum > 0.f ? m + __logf(wsum) : -INFINITY;
    }

    // ---- merge --------------------------------------------------------------------
    const float m = fmaxf(l1, l2);
    uint2 ow = make_uint2(0, 0);
    float lse_v = -INFINITY;
    if (m != -INFINITY) {
        const float w1 = expf(l1 - m), w2 = expf(l2 - m);
        const float s = w1 + w2;
        const float sinv = 1.0f / s;
        auto mix = [&](float x1, float x2) {
            const float t1 = (w1 == 0.f) ? 0.f : x1 * w1;
            const float t2 = (w2 == 0.f) ? 0.f : x2 * w2;
            return (t1 + t2) * sinv;
        };
        ow = make_uint2(pack_bf16x2(mix(o1.x, o2.x), mix(o1.y, o2.y)), pack_bf16x2(mix(o1.z, o2.z), mix(o1.w, o2.w)));
        lse_v = m + logf(s);
    }
    *reinterpret_cast<uint2 *>(e.out + row * kD + 4 * d4) = ow;
    if (d4 == 0) e.lse_out[row] = lse_v;
}

int64_t ceil_div(int64_t x, int64_t y) { return (x + y - 1) / y; }

// partial (O, LSE) slots: 2 per (query head, chunk) -- the same count for any
// split of the heads into kv head groups
int64_t group_parts(int64_t num_heads, int64_t chunks) { return num_heads * chunks * 2; }

template <int G>
int launch_suffix(const SuffixArgs &a, bool fixup, const EpilogueArgs *epi, hipStream_t st) {
    static std::atomic<uint64_t> lds_set{0};
    int rc = ensure_dynamic_lds(reinterpret_cast<const void *>(&suffix_stream_kernel<G>), kLdsBytes, lds_set);
    if (rc != CK_OK) return rc;
    static_assert((kWaves * G * kD + 2 * kWaves * G) * 4 <= kStageBytes, "exchange fits in a stage");
    hipLaunchKernelGGL(suffix_stream_kernel<G>, dim3((unsigned)(a.kv_heads * a.chunks)), dim3(kThreads), kLdsBytes,
                       st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return static_cast<int>(e);
    if (fixup)
        hipLaunchKernelGGL(suffix_fixup_kernel<G>, dim3((unsigned)(a.batch * a.kv_heads)), dim3(32 * G), 0, st, a);
    if (epi)
        hipLaunchKernelGGL(cascade_epilogue_kernel<G>, dim3((unsigned)(a.batch * a.kv_heads)), dim3(32 * G), 0, st,
                           *epi);
    CK_RETURN_LAUNCH();
}

int check_suffix_dims(int64_t batch, int64_t num_heads, int64_t kv_heads, int64_t head_dim, int64_t kv_cap) {
    if (batch < 0 || kv_cap < 0) return CK_E_INVALID_ARG;
    if (head_dim != kD) return CK_E_UNSUPPORTED;
    if (kv_heads <= 0 || num_heads <= 0 || num_heads % kv_heads != 0) return CK_E_INVALID_ARG;
    if (num_heads > (1 << 16)) return CK_E_INVALID_ARG;
    if (kv_cap > (int64_t)1 << 30) return CK_E_INVALID_ARG;
    return CK_OK;
}

}  // namespace

// Query-head groups per kv head: a GQA group of more than kMaxGroup heads is
// split into the fewest equal groups of at most kMaxGroup heads. Each group is
// streamed as if it had its own kv head (the kernel reads the shared physical
// head), so the kernels keep their per-head registers bounded for any group.
int64_t suffix_sub_groups(int64_t num_heads, int64_t kv_heads) {
    const int64_t group = num_heads / kv_heads;
    for (int64_t n = (group + kMaxGroup - 1) / kMaxGroup; n < group; ++n)
        if (group % n == 0) return n;
    return group;
}

// Sequences per stream-kernel launch: the window/length prefix sums live in
// LDS (kMaxBatch entries) and must stay below 2^31 tokens.
int64_t suffix_group_batch(int64_t kv_cap) {
    int64_t n = kMaxBatch;
    const int64_t cap = kv_cap > 0 ? kv_cap : 1;
    if (n > 0x7FFFFFFF / cap) n = 0x7FFFFFFF / cap;
    return n < 1 ? 1 : n;
}

// Workgroups per kv head group: the grid holds as many workgroups as can be resident
// at once. Up to 5 query heads per kv head the stream kernel fits in 128 VGPRs
// and kBlocksPerCu workgroups share a CU; 6-8 heads need more registers (the
// per-head accumulators) and run one per CU, where a grid twice that size
// would queue half its workgroups behind the first half.
int64_t suffix_default_chunks(int64_t num_heads, int64_t kv_heads) {
    const int64_t groups = kv_heads * suffix_sub_groups(num_heads, kv_heads);
    const int64_t per_cu = num_heads / groups <= 5 ? kBlocksPerCu : 1;
    const int64_t p = per_cu * 256 / groups;
    return p > 0 ? p : 1;
}

int64_t suffix_group_ws_bytes(int64_t nb, int64_t num_heads, int64_t kv_heads, int64_t chunks) {
    const int64_t parts = group_parts(num_heads, chunks);
    return parts * (kD + 1) * (int64_t)sizeof(float) + (nb + 1) * (int64_t)sizeof(int32_t) + 256;
}

int suffix_launch_group(const void *q, const void *k, const void *v, const int32_t *block_table, int64_t bt_cols,
                        const int64_t *kv_seqlens, int64_t b0, int64_t nb, int64_t num_heads, int64_t kv_heads,
                        int64_t num_blocks, int64_t kv_layout, float scale, int64_t kv_cap, int64_t chunks,
                        void *out, float *lse, void *group_ws, const Stage1Result *cascade, void *final_out,
                        float *final_lse, hipStream_t stream) {
    const int64_t sub = suffix_sub_groups(num_heads, kv_heads);
    const int64_t G = num_heads / kv_heads / sub;  // query heads per workgroup
    const int64_t parts = group_parts(num_heads, chunks);
    SuffixArgs a;
    a.q = static_cast<const uint16_t *>(q) + b0 * num_heads * kD;
    a.k = static_cast<const uint16_t *>(k);
    a.v = static_cast<const uint16_t *>(v);
    a.bt = block_table + b0 * bt_cols;
    a.kv_seqlens = kv_seqlens + b0;
    a.out = static_cast<uint16_t *>(out);
    a.lse = lse;
    a.part_o = static_cast<float *>(group_ws);
    a.part_lse = a.part_o + parts * kD;
    a.cw_out = reinterpret_cast<int32_t *>(a.part_lse + parts);
    a.bt_cols = bt_cols;
    a.num_blocks = num_blocks;
    a.page_stride = (int64_t)kPage * kv_heads * kD;
    a.tok_stride = kv_layout == CK_KV_BNSD ? kD : kv_heads * kD;
    a.head_off = kv_layout == CK_KV_BNSD ? (int64_t)kPage * kD : kD;
    a.batch = (int)nb;
    a.num_heads = (int)num_heads;
    a.kv_heads = (int)(kv_heads * sub);
    a.kv_sub = (int)sub;
    a.kv_cap = (int)kv_cap;
    a.chunks = (int)chunks;
    a.scale_log2 = scale * kLog2e;
    EpilogueArgs e;
    if (cascade) {
        e.s1 = *cascade;
        e.o2 = a.out;
        e.lse2 = a.lse;
        e.part_o = a.part_o;
        e.part_lse = a.part_lse;
        e.cw = a.cw_out;
        e.out = static_cast<uint16_t *>(final_out);
        e.lse_out = final_lse;
        e.b0 = b0;
        e.nb = (int)nb;
        e.num_heads = (int)num_heads;
        e.kv_heads = a.kv_heads;
        e.chunks = (int)chunks;
    }
    const bool fixup = cascade == nullptr;
    const EpilogueArgs *ep = cascade ? &e : nullptr;
    switch (G) {
        case 1: return launch_suffix<1>(a, fixup, ep, stream);
        case 2: return launch_suffix<2>(a, fixup, ep, stream);
        case 3: return launch_suffix<3>(a, fixup, ep, stream);
        case 4: return launch_suffix<4>(a, fixup, ep, stream);
        case 5: return launch_suffix<5>(a, fixup, ep, stream);
        case 6: return launch_suffix<6>(a, fixup, ep, stream);
        case 7: return launch_suffix<7>(a, fixup, ep, stream);
        default: return launch_suffix<8>(a, fixup, ep, stream);
    }
}

}  // namespace ck

using namespace ck;

extern "C" int ck_suffix_decode_plan(int64_t batch, int64_t num_heads, int64_t kv_heads, int64_t head_dim,
                                     int64_t kv_cap, int64_t *num_splits, int64_t *workspace_bytes) {
    int rc = check_suffix_dims(batch, num_heads, kv_heads, head_dim, kv_cap);
    if (rc != CK_OK) return rc;
    if (!num_splits || !workspace_bytes) return CK_E_NULL_PTR;
    const int64_t chunks = suffix_default_chunks(num_heads, kv_heads);
    const int64_t nb = batch < suffix_group_batch(kv_cap) ? batch : suffix_group_batch(kv_cap);
    *num_splits = chunks;
    *workspace_bytes = batch > 0 ? suffix_group_ws_bytes(nb, num_heads, kv_heads, chunks) : 0;
    return CK_OK;
}

extern "C" int ck_suffix_decode(const void *q, const void *k, const void *v, const int32_t *block_table,
                                int64_t bt_cols, const int64_t *kv_seqlens, int64_t batch, int64_t num_heads,
                                int64_t kv_heads, int64_t head_dim, int64_t num_blocks, int64_t block_size,
                                int64_t kv_layout, float scale, int64_t kv_cap, int64_t num_splits, void *out,
                                float *lse, void *workspace, int64_t workspace_bytes, void *stream) {
    int rc = check_suffix_dims(batch, num_heads, kv_heads, head_dim, kv_cap);
    if (rc != CK_OK) return rc;
    if (block_size != kPage) return CK_E_UNSUPPORTED;
    if (kv_layout != CK_KV_NHD && kv_layout != CK_KV_BNSD) return CK_E_INVALID_ARG;
    if (bt_cols < 0 || num_blocks < 0 || kv_cap > bt_cols * kPage) return CK_E_INVALID_ARG;
    if (batch == 0) return CK_OK;
    if (!q || !k || !v || !block_table || !kv_seqlens || !out || !lse) return CK_E_NULL_PTR;
    // q/k/v rows and the workspace partials move up to 16 bytes per lane; the
    // fix-up kernel stores bf16 O four elements (8 bytes) at a time
    if (!aligned_to(q, 16) || !aligned_to(k, 16) || !aligned_to(v, 16) || !aligned_to(out, 8) ||
        !aligned_to(lse, 4) || !aligned_to(workspace, 16))
        return CK_E_INVALID_ARG;
    const int64_t chunks = num_splits > 0 ? num_splits : suffix_default_chunks(num_heads, kv_heads);
    if (kv_heads * suffix_sub_groups(num_heads, kv_heads) * chunks > 0x7FFFFFFF || chunks > (1 << 20))
        return CK_E_INVALID_ARG;
    const int64_t per_launch = suffix_group_batch(kv_cap);
    const int64_t nbmax = batch < per_launch ? batch : per_launch;
    if (workspace == nullptr || workspace_bytes < suffix_group_ws_bytes(nbmax, num_heads, kv_heads, chunks))
        return CK_E_WORKSPACE;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    for (int64_t b0 = 0; b0 < batch; b0 += per_launch) {
        const int64_t nb = batch - b0 < per_launch ? batch - b0 : per_launch;
        rc = suffix_launch_group(q, k, v, block_table, bt_cols, kv_seqlens, b0, nb, num_heads, kv_heads,
                                 num_blocks, kv_layout, scale, kv_cap, chunks, static_cast<uint16_t *>(out) + b0 * num_heads * kD,
                                 lse + b0 * num_heads, workspace, nullptr, nullptr, nullptr, st);
        if (rc != CK_OK) return rc;
    }
    return CK_OK;
}
