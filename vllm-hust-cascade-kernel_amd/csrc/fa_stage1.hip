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
// * One workgroup = 128 query rows x one kv split, run by 8 waves: wave w owns
//   query rows 32*(w%4) .. +32 and token half w/4 of every 64-token tile, with
//   its own online-softmax state; the two halves merge through LDS at the end.
//   Two waves per SIMD let one wave's softmax VALU overlap the other's MFMAs.
//   K and V tiles stream into a 4-slot LDS ring (4 x 32 KB) by global->LDS DMA
//   (global_load_lds, 16 B per lane): no staging registers. Tiles go in pairs:
//   a pair is computed while the next pair lands, with one barrier, one
//   running-max update and at most one O rescale per pair (the rescale, 64
//   multiplies per lane, is the largest VALU item of a tile). The split's page
//   ids are read once into LDS, so no load in the loop depends on another
//   load. Each wave keeps its Q rows as MFMA operands in registers for the
//   whole kv loop.
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
//   distinct bank groups). Both read kinds are bank-conflict free; the plain
//   t & 15 swizzle leaves the transpose reads 4-way conflicted.
// * Softmax runs in the log2 domain (p = exp2(s * scale * log2(e) - m), one
//   FMA and one exp2 per score); LSE is converted back to natural log.
// * The epilogue merges the two token halves through LDS and re-lays O out as
//   whole rows, so each global store writes two contiguous 512-byte rows
//   (lane-per-row stores of the accumulator layout scatter 32-byte pieces and
//   run at a fraction of the write bandwidth).
// * Split-KV fills the chip when batch*kv_heads*m-tiles is small; partial
//   (O, LSE) pairs are folded by an N-way LSE merge (stage1_combine_kernel).
// * Block order is XCD-aware: the m-tiles that read the same kv pages are
//   placed on the same XCD so the second read hits that XCD's L2.
#include <cmath>

#include "ck_common.h"
#include "ck_internal.h"

namespace ck {
namespace {

constexpr int kD = 128;          // head dim (op contract)
constexpr int kPage = 128;       // paged block size (op contract)
constexpr int kTileN = 64;       // kv tokens per tile
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;
constexpr int kRows = 128;          // query rows per workgroup (4 row blocks x 2 token halves)
constexpr int kStages = 4;          // LDS ring depth
constexpr int kTileBytes = kTileN * kD * 2;   // 16 KB for K, the same for V
constexpr int kStageBytes = 2 * kTileBytes;
constexpr int kMaxSplitPages = 256;           // page ids held in LDS per split
constexpr int kLdsBytes = kStages * kStageBytes + kMaxSplitPages * 4;
constexpr int kDmaPerTile = 2 * (kTileBytes / 1024) / kWaves;  // 16-B-per-lane DMAs per wave per tile (4)

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

__device__ __forceinline__ bf16x8 pack_p(const f32x16 &s, int base) {
    uint4 w;
    w.x = pack_bf16x2(s[base + 0], s[base + 1]);
    w.y = pack_bf16x2(s[base + 2], s[base + 3]);
    w.z = pack_bf16x2(s[base + 4], s[base + 5]);
    w.w = pack_bf16x2(s[base + 6], s[base + 7]);
    return __builtin_bit_cast(bf16x8, w);
}

// Byte offset of row tok, 16-byte chunk c inside a K or V tile (XOR swizzle).
__device__ __forceinline__ int tile_swz(int tok) { return ((tok & 3) << 2) | ((tok >> 2) & 3); }
__device__ __forceinline__ int tile_off(int tok, int c) { return tok * (kD * 2) + ((c ^ tile_swz(tok)) << 4); }

__global__ __launch_bounds__(kThreads) void stage1_kernel(Stage1Args a) {
    extern __shared__ __attribute__((aligned(16))) char smem_raw[];
    CK_LDS char *smem = (CK_LDS char *)smem_raw;
    CK_LDS int *s_pages = (CK_LDS int *)(smem + kStages * kStageBytes);

    const int tid = threadIdx.x;
    const int wid = tid >> 6;
    const int lane = tid & 63;
    const int hh = lane >> 5;
    const int rb = wid & 3;   // row block
    const int th = wid >> 2;  // token half of each tile

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

    const int wrow0 = row0 + rb * 32;
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
    // Page ids are read for the split's whole page range inside the table row,
    // whatever the kv length (only those below it are used), so they, Q and the
    // kv length are fetched together in one round trip.
    const int kv_lo = sp * a.split_len;  // a multiple of kPage
    {
        const int pg0 = kv_lo / kPage;
        const int64_t avail = a.bt_cols - pg0;
        const int pg_n = (int)min((int64_t)(a.split_len / kPage), avail > 0 ? avail : (int64_t)0);
        for (int pi = tid; pi < pg_n; pi += kThreads) {
            const int page = a.bt[(int64_t)b * a.bt_cols + pg0 + pi];
            s_pages[pi] = (page >= 0 && (int64_t)page < a.num_blocks) ? page : -1;
        }
    }
    int64_t kvl = a.kv_seqlens[b];
    const int64_t kv_lim = a.bt_cols * kPage;
    if (kvl > kv_lim) kvl = kv_lim;
    if (kvl > a.kv_cap) kvl = a.kv_cap;
    if (kvl < 0 || a.num_blocks <= 0) kvl = 0;  // no pool: nothing to attend to
    int kv_hi = kv_lo + a.split_len;
    if (kv_hi > (int)kvl) kv_hi = (int)kvl;
    const int ntiles = kv_hi > kv_lo ? (kv_hi - kv_lo + kTileN - 1) / kTileN : 0;

    // Q and page ids must be resident before the DMA ring starts: the compiler
    // does not count the inline-asm DMAs, so a wait it deferred into the loop
    // would also drain every tile in flight.
    wait_vmcnt<0>();
    __syncthreads();  // s_pages visible

    const int64_t head_stride = (int64_t)a.kv_heads * kD;
    // DMA lane geometry: one wave instruction moves 4 token rows (1 KB); lane ->
    // token 4*blk + lane/16 and LDS chunk lane%16, which holds global chunk
    // (lane%16) ^ tile_swz(token).
    const int dma_tt = lane >> 4;
    const int dma_pc = lane & 15;

    auto issue_tile = [&](int i) {
        const int j0 = kv_lo + i * kTileN;
        // an invalid page is zero-filled at wait time; its DMAs still go out (from
        // page 0) so every wave keeps exactly kDmaPerTile operations per tile and
        // the vmcnt-based waits stay exact
        const int raw_page = s_pages[(j0 - kv_lo) / kPage];
        const int page = raw_page < 0 ? 0 : raw_page;
        CK_LDS char *kb = smem + (i % kStages) * kStageBytes;
        CK_LDS char *vb = kb + kTileBytes;
        const int64_t tok0 = (int64_t)page * kPage + (j0 % kPage);
#pragma unroll
        for (int j = 0; j < kDmaPerTile / 2; ++j) {
            const int blk = wid * (kDmaPerTile / 2) + j;
            const int tt = blk * 4 + dma_tt;
            const int c = dma_pc ^ tile_swz(tt);
            const int64_t off = (tok0 + tt) * head_stride + g * kD + c * 8;
            dma16(a.k + off, kb + blk * 1024);
            dma16(a.v + off, vb + blk * 1024);
        }
    };

    // ---- online softmax state (one query row per lane, halves agree) ---------------
    f32x16 oacc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[db][i] = 0.f;
    float m_run = -INFINITY;
    float l_part = 0.f;  // row sum over the tokens of this lane half

    // Tiles go in pairs: one barrier, one max update and at most one O rescale
    // per 128 kv tokens (64 per wave). Pair p (tiles 2p, 2p + 1) is computed
    // while pair p + 1 lands; the ring's four slots hold exactly those two pairs.
    static_assert(kStages == 4, "two pairs of tiles in the ring");
    for (int i = 0; i < 2 && i < ntiles; ++i) issue_tile(i);

    // per-lane LDS offsets (loop invariant): K fragment rows of this token half,
    // and the V^T transpose-read addresses. Transpose reads: lane group
    // G = lane/16 covers dims 16*(G%2) + 0..15 of each 32-dim block and the
    // token quad 4*(G/2); its source lane s addresses token s/4, dims 4*(s%4)..+3.
    const int ktok = th * 32 + (lane & 31);
    const int trG = (lane >> 4) & 3;
    const int tr_row = (lane & 15) >> 2;
    const int tr_e4 = lane & 3;

    // S^T for this wave's token half of the tile in `slot`; tokens past nvalid -> -inf
    auto qk_tile = [&](int slot, int nvalid, f32x16 &sacc) {
        const CK_LDS char *kb = smem + slot * kStageBytes;
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[e] = 0.f;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            const bf16x8 kf = *reinterpret_cast<const CK_LDS bf16x8 *>(kb + tile_off(ktok, 2 * kk + hh));
            sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], sacc, 0, 0, 0);
        }
        if (nvalid < kTileN) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int tok = th * 32 + (e & 3) + 8 * (e >> 2) + 4 * hh;
                if (tok >= nvalid) sacc[e] = -INFINITY;
            }
        }
    };
    // O^T += V^T P^T over this half's 2 k-steps of 16 tokens of the tile in `slot`
    auto pv_tile = [&](int slot, const f32x16 &pacc) {
        const CK_LDS char *vb = smem + slot * kStageBytes + kTileBytes;
#pragma unroll
        for (int ss = 0; ss < 2; ++ss) {
            const int s = 2 * th + ss;
            const bf16x8 pb = pack_p(pacc, ss * 8);
            const int t1 = 16 * s + 4 * (trG >> 1) + tr_row;  // first read; second is t1 + 8
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const int d = 32 * db + 16 * (trG & 1) + 4 * tr_e4;  // 4 dims this lane addresses
                const int c = d >> 3, half = (d & 7) * 2;
                const uint2 lo = lds_read_tr16(vb + tile_off(t1, c) + half);
                const uint2 hi = lds_read_tr16(vb + tile_off(t1 + 8, c) + half);
                const bf16x8 vf = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
                oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb, oacc[db], 0, 0, 0);
            }
        }
    };

    for (int i = 0; i < ntiles; i += 2) {
        const bool two = i + 1 < ntiles;
        // this pair was issued one pair ago and nothing after it: all landed
        wait_vmcnt<0>();
        __syncthreads();
        int nv[2];
        bool fill = false;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            nv[t] = 0;
            if (t == 1 && !two) continue;
            const int j0 = kv_lo + (i + t) * kTileN;
            nv[t] = min(kTileN, kv_hi - j0);
            const bool page_ok = s_pages[(j0 - kv_lo) / kPage] >= 0;
            if (nv[t] < kTileN || !page_ok) {
                // rows past the sequence end (or of an invalid page) may hold
                // anything: zero them so 0 * V cannot produce a NaN
                CK_LDS char *kb = smem + ((i + t) % kStages) * kStageBytes;
                CK_LDS char *vb = kb + kTileBytes;
                const int z0 = page_ok ? nv[t] : 0;
                for (int idx = tid; idx < (kTileN - z0) * 16; idx += kThreads) {
                    const int tt = z0 + (idx >> 4), c = idx & 15;
                    *reinterpret_cast<CK_LDS u32x4 *>(kb + tt * 256 + c * 16) = u32x4{0, 0, 0, 0};
                    *reinterpret_cast<CK_LDS u32x4 *>(vb + tt * 256 + c * 16) = u32x4{0, 0, 0, 0};
                }
                fill = true;
            }
        }
        if (fill) __syncthreads();
        // the previous pair's slots are free: the pair after this one goes there
#pragma unroll
        for (int t = 0; t < 2; ++t)
            if (i + 2 + t < ntiles) issue_tile(i + 2 + t);

        const bool act0 = wave_active && th * 32 < nv[0];
        const bool act1 = wave_active && th * 32 < nv[1];  // tile i + 1 exists only after a full tile i
        if (act0) {
            f32x16 s0, s1;
            qk_tile(i % kStages, nv[0], s0);
            if (act1) qk_tile((i + 1) % kStages, nv[1], s1);
            // row max of the unscaled scores over both tiles; the scale is > 0,
            // so scaling the max gives the max of the scaled scores
            float smax = -INFINITY;
#pragma unroll
            for (int e = 0; e < 16; ++e) smax = fmaxf(smax, s0[e]);
            if (act1) {
#pragma unroll
                for (int e = 0; e < 16; ++e) smax = fmaxf(smax, s1[e]);
            }
            smax = max_xor32(smax) * a.scale_log2;  // the row's other tokens sit in lane l ^ 32
            const float m_new = fmaxf(m_run, smax);
            const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
            const float dm = exp2_fast(m_run - m_use);
            // p = exp2(s * scale * log2(e) - m): one FMA and one exp2 per score
            float ls = 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float p = exp2_fast(fmaf(s0[e], a.scale_log2, -m_use));
                s0[e] = p;
                ls += p;
            }
            if (act1) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float p = exp2_fast(fmaf(s1[e], a.scale_log2, -m_use));
                    s1[e] = p;
                    ls += p;
                }
            }
            // the two lane halves hold different tokens of the row: their sums
            // are kept apart and added once after the loop
            l_part = l_part * dm + ls;
            m_run = m_new;
            // rescale only when some row's max moved (wave-uniform branch)
            if (__builtin_amdgcn_ballot_w64(dm != 1.0f)) {
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int e = 0; e < 16; ++e) oacc[db][e] *= dm;
            }
            pv_tile(i % kStages, s0);
            if (act1) pv_tile((i + 1) % kStages, s1);
        }
    }

    // ---- merge the two token halves, then write whole rows --------------------------
    // The ring is free now. Wave (rb, 1) parks its O^T accumulators in the
    // 16 KB slab of row block rb; wave (rb, 0) folds them into its own, then
    // rewrites the slab as 32 normalised fp32 rows of 512 B (16-byte chunks
    // XOR-swizzled by row) and stores two whole rows per instruction, so every
    // global store is a full, contiguous 1 KB.
    const float l_run = l_part + __shfl_xor(l_part, 32);
    __syncthreads();
    CK_LDS float *slab = (CK_LDS float *)smem + rb * (32 * kD);  // [16 quads][64 lanes][4]
    CK_LDS float *xm = (CK_LDS float *)smem + 4 * 32 * kD;  // past the four slabs
    CK_LDS float *xl = xm + 4 * 64;
    if (th == 1) {
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4)
                *reinterpret_cast<CK_LDS f32x4 *>(slab + ((db * 4 + c4) * 64 + lane) * 4) =
                    f32x4{oacc[db][4 * c4], oacc[db][4 * c4 + 1], oacc[db][4 * c4 + 2], oacc[db][4 * c4 + 3]};
        xm[rb * 64 + lane] = m_run;
        xl[rb * 64 + lane] = l_run;
    }
    __syncthreads();
    if (th == 1 || !wave_active) return;  // wave-uniform
    const float m1 = xm[rb * 64 + lane], l1 = xl[rb * 64 + lane];
    const float mn = fmaxf(m_run, m1);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float f0 = exp2_fast(m_run - mu), f1 = exp2_fast(m1 - mu);
    const float lt = l_run * f0 + l1 * f1;
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    const float lse_v = lt > 0.f ? (mn + __log2f(lt)) * kLn2 : -INFINITY;
    f32x4 o1[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) o1[q] = *reinterpret_cast<const CK_LDS f32x4 *>(slab + (q * 64 + lane) * 4);
    // lane holds row lane%32, dims 32*db + 8*c4 + 4*hh .. +3 = 16-byte chunk 8*db + 2*c4 + hh
    const int my_row = lane & 31;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
            const int q = db * 4 + c4;
            const f32x4 o = f32x4{(oacc[db][4 * c4 + 0] * f0 + o1[q][0] * f1) * inv,
                                  (oacc[db][4 * c4 + 1] * f0 + o1[q][1] * f1) * inv,
                                  (oacc[db][4 * c4 + 2] * f0 + o1[q][2] * f1) * inv,
                                  (oacc[db][4 * c4 + 3] * f0 + o1[q][3] * f1) * inv};
            const int chunk = (8 * db + 2 * c4 + hh) ^ my_row;
            *reinterpret_cast<CK_LDS f32x4 *>(slab + my_row * kD + chunk * 4) = o;
        }
    if (row_valid) {
        if (a.num_splits == 1) {
            const float4 lv = make_float4(lse_v, lse_v, lse_v, lse_v);
            *reinterpret_cast<float4 *>(a.lse + qrow * 8 + 4 * hh) = lv;
        } else if (hh == 0) {
            a.part_lse[(int64_t)sp * a.num_rows + qrow] = lse_v;
        }
    }
    // the wave reads back only its own slab: no barrier, the LDS ops of one wave complete in order
    float *base = a.num_splits == 1 ? a.out : a.part_o + (int64_t)sp * a.num_rows * kD;
    const int chunk = lane & 31;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int rr = 2 * j + (lane >> 5);  // row within the block
        const int64_t qr = __shfl((int)qrow, rr);
        const f32x4 o = *reinterpret_cast<const CK_LDS f32x4 *>(slab + rr * kD + ((chunk ^ rr) * 4));
        if (wrow0 + rr < rows_b) *reinterpret_cast<f32x4 *>(base + qr * kD + chunk * 4) = o;
    }
}

// N-way LSE merge of split partials: 32 threads per row, 4 dims each. One
// pass with an online maximum; the partials of 8 splits are fetched with
// independent loads per round so the round trips overlap.
__global__ __launch_bounds__(256) void stage1_combine_kernel(const float *part_o, const float *part_lse,
                                                             int num_splits, int64_t rows,
                                                             float *out, float *lse) {
    constexpr int kBatch = 8;
    const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int d4 = threadIdx.x & 31;
    if (row >= rows) return;
    float m = -INFINITY, wsum = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < num_splits; s0 += kBatch) {
        float ls[kBatch];
        float4 o[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int s = s0 + j < num_splits ? s0 + j : num_splits - 1;
            ls[j] = s0 + j < num_splits ? part_lse[(int64_t)s * rows + row] : -INFINITY;
            o[j] = *reinterpret_cast<const float4 *>(part_o + ((int64_t)s * rows + row) * kD + 4 * d4);
        }
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
    static std::atomic<uint64_t> lds_set{0};
    rc = ensure_dynamic_lds(reinterpret_cast<const void *>(&stage1_kernel), kLdsBytes, lds_set);
    if (rc != CK_OK) return rc;
    hipLaunchKernelGGL(stage1_kernel, dim3((unsigned)grid), dim3(kThreads), kLdsBytes, s, a);
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
