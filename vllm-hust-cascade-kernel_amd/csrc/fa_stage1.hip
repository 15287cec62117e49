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
//   the row maximum the reference rounds on). Two kernels:
//   - stage1_tile_kernel (m-tile of 128 rows): 4 waves, one per SIMD with 512
//     registers. Iteration t runs the QK MFMAs of tile t + 1 and the PV MFMAs
//     of tile t in a fixed issue order, with one slice of tile t's softmax
//     and, every four MFMAs, one of the wave's DMAs between them. K and V
//     stream through separate 3-slot LDS rings (K one tile ahead of V).
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

// Software-pipelined whole-row kernel. 4 waves (one per SIMD, 512 registers
// each); wave w owns RB blocks of 32 query rows (rows 32 RB w .. + 32 RB of the
// workgroup's 128 RB) and every token of them, so each row has one
// online-softmax state and P is rounded on the row's own running maximum,
// which moves once per 64-token tile. Every K or V fragment read from LDS
// feeds RB MFMAs (RB = 2 halves the LDS bytes per MFMA).
// Iteration t runs the QK MFMAs of tile t + 1 and the PV MFMAs of tile t in a
// fixed order, with one slice of tile t's softmax and, every few MFMAs, one of
// the wave's 8 DMAs of the tile two ahead between them: the wave issues its
// VALU work and DMAs while the matrix pipe is busy. K and V stream through
// separate 3-slot LDS rings (K is read one iteration before V), so every DMA
// is issued two iterations before its first reader. Past the last tile the
// DMAs repeat into slots nobody reads again, so every iteration issues the
// same number and the vmcnt wait is exact.
constexpr int kTW = 4;                               // waves per workgroup
constexpr int kTSlots = 3;                           // ring depth of each of K and V
constexpr int kTBlk = kTBytes / 1024 / kTW;          // 1-KB DMAs of K (and of V) per wave per tile
constexpr int kTDma = 2 * kTBlk;                     // DMAs per wave per tile
constexpr int kTLds = 2 * kTSlots * kTBytes + kMaxSplitPages * 4;

template <int RB>
__global__ __launch_bounds__(kTW * 64) void stage1_tile_kernel(Stage1Args a) {
    constexpr int kRowsWg = kTW * 32 * RB;
    // the epilogue parks every row block's 16 KB of O in the (idle) rings; RB = 2
    // would also need more than a wave's 512 registers (it spills), so the
    // launcher instantiates RB = 1 only
    static_assert(kTW * RB * 32 * kD * 4 <= 2 * kTSlots * kTBytes, "epilogue slabs fit the rings");
    extern __shared__ __attribute__((aligned(16))) char smem_raw[];
    CK_LDS char *smem = (CK_LDS char *)smem_raw;
    CK_LDS char *kring = smem;
    CK_LDS char *vring = smem + kTSlots * kTBytes;
    CK_LDS int *s_pages = (CK_LDS int *)(smem + 2 * kTSlots * kTBytes);

    const int tid = threadIdx.x;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: DMA LDS addresses in SGPRs
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
    const int row0 = mt * kRowsWg;
    if (row0 >= rows_b) return;  // uniform over the workgroup

    const int wrow0 = row0 + wid * 32 * RB;
    const bool wave_active = wrow0 < rows_b;
    int64_t qrow[RB];
    bool row_valid[RB];
    bf16x8 qf[RB][8];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int r = wrow0 + rb * 32 + (lane & 31);
        row_valid[rb] = r < rows_b;
        const int t_local = r / a.group;
        const int h = g * a.group + (r - t_local * a.group);
        qrow[rb] = (int64_t)(qs + t_local) * a.num_heads + h;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            if (row_valid[rb]) {
                qf[rb][kk] = *reinterpret_cast<const bf16x8 *>(a.q + qrow[rb] * kD + 16 * kk + 8 * hh);
            } else {
                qf[rb][kk] = __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
            }
        }
    }
    const int kv_lo = sp * a.split_len;  // a multiple of the page size
    {
        const int pg0 = kv_lo / kPage;
        const int64_t avail = a.bt_cols - pg0;
        const int pg_n = (int)min((int64_t)(a.split_len / kPage), avail > 0 ? avail : (int64_t)0);
        for (int pi = tid; pi < pg_n; pi += kTW * 64) {
            const int page = a.bt[(int64_t)b * a.bt_cols + pg0 + pi];
            s_pages[pi] = (page >= 0 && (int64_t)page < a.num_blocks) ? page : -1;
        }
    }
    int64_t kvl = a.kv_seqlens[b];
    const int64_t kv_lim = a.bt_cols * kPage;
    if (kvl > kv_lim) kvl = kv_lim;
    if (kvl > a.kv_cap) kvl = a.kv_cap;
    if (kvl < 0 || a.num_blocks <= 0) kvl = 0;
    int kv_hi = kv_lo + a.split_len;
    if (kv_hi > (int)kvl) kv_hi = (int)kvl;
    const int ntok = kv_hi > kv_lo ? kv_hi - kv_lo : 0;
    const int ntiles = (ntok + kTTok - 1) / kTTok;

    wait_vmcnt<0>();
    __syncthreads();  // s_pages visible

    // DMA geometry: one wave instruction moves 4 token rows (1 KB); lane ->
    // token 4 blk + lane / 16 and LDS chunk lane % 16, which holds global chunk
    // (lane % 16) ^ tile_swz(token). Per-lane element offsets inside a tile.
    const int64_t head_stride = (int64_t)a.kv_heads * kD;
    uint32_t dma_off[kTBlk];
#pragma unroll
    for (int j = 0; j < kTBlk; ++j) {
        const int tt = (wid * kTBlk + j) * 4 + (lane >> 4);
        dma_off[j] = (uint32_t)(tt * head_stride + g * kD + (((lane & 15) ^ tile_swz(tt)) << 3));
    }
    // DMA j (0 .. kTDma-1: K blocks, then V blocks) of the wave's share of tile
    // t (K) or tile t - 1 (V) -- the two the iteration before t prefetches. A
    // tile past the end repeats the last tile into its own (dead) slot.
    auto tile_src = [&](int t) {  // called only when ntiles > 0
        const int tc = t < ntiles ? t : ntiles - 1;
        const int raw = __builtin_amdgcn_readfirstlane(s_pages[tc >> 1]);
        const int64_t tok0 = (int64_t)(raw < 0 ? 0 : raw) * kPage + (tc & 1) * kTTok;
        return tok0 * head_stride;
    };
    // a tile's 64 token rows of K or V as a buffer resource (scalar base): the
    // DMAs add only the fixed lane offsets
    const uint32_t tile_bytes = (uint32_t)(kTTok * head_stride * 2);
    auto dma_k = [&](int t, int j) {
        dma16_buf(buf_rsrc(a.k + tile_src(t), tile_bytes), (int)(dma_off[j] * 2), 0,
                  kring + (t % kTSlots) * kTBytes + (wid * kTBlk + j) * 1024);
    };
    auto dma_v = [&](int t, int j) {
        dma16_buf(buf_rsrc(a.v + tile_src(t), tile_bytes), (int)(dma_off[j] * 2), 0,
                  vring + (t % kTSlots) * kTBytes + (wid * kTBlk + j) * 1024);
    };
    // the iteration-t DMA group: K of tile t + 3 and V of tile t + 2; the two
    // tile bases are looked up once per iteration
    struct DmaGroup {
        ck_rsrc_t k, v;
        CK_LDS char *kd, *vd;
    };
    auto dma_group = [&](int t) {
        DmaGroup d;
        d.k = buf_rsrc(a.k + tile_src(t + 3), tile_bytes);
        d.v = buf_rsrc(a.v + tile_src(t + 2), tile_bytes);
        d.kd = kring + ((t + 3) % kTSlots) * kTBytes + wid * kTBlk * 1024;
        d.vd = vring + ((t + 2) % kTSlots) * kTBytes + wid * kTBlk * 1024;
        return d;
    };
    auto dma_step = [&](const DmaGroup &d, int j) {
        if (j < kTBlk) dma16_buf(d.k, (int)(dma_off[j] * 2), 0, d.kd + j * 1024);
        else dma16_buf(d.v, (int)(dma_off[j - kTBlk] * 2), 0, d.vd + (j - kTBlk) * 1024);
    };
    auto zero_rows = [&](CK_LDS char *slot, int z0) {
        for (int idx = tid; idx < (kTTok - z0) * 16; idx += kTW * 64) {
            const int tt = z0 + (idx >> 4), c = idx & 15;
            *reinterpret_cast<CK_LDS u32x4 *>(slot + tt * 256 + c * 16) = u32x4{0, 0, 0, 0};
        }
    };
    auto page_ok = [&](int t) { return s_pages[t >> 1] >= 0; };

    f32x16 oacc[RB][4];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) oacc[rb][db][i] = 0.f;
    float m_run[RB], l_part[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        m_run[rb] = -INFINITY;
        l_part[rb] = 0.f;
    }

    const int trG = (lane >> 4) & 3;
    const int tr_row = (lane & 15) >> 2;
    const int tr_e4 = lane & 3;
    const int ktok = lane & 31;
    auto vt_off = [&](int s16, int db, int second) {
        const int t1 = 16 * s16 + 4 * (trG >> 1) + tr_row + 8 * second;
        const int d = 32 * db + 16 * (trG & 1) + 4 * tr_e4;
        return tile_off(t1, d >> 3) + (d & 7) * 2;
    };
    // K fragment f of a tile (f = 2 kk + q2: 16-dim step kk of token block q2)
    auto kfrag = [&](const CK_LDS char *kb, int f) {
        return *reinterpret_cast<const CK_LDS bf16x8 *>(kb + tile_off(32 * (f & 1) + ktok, 2 * (f >> 1) + hh));
    };
    // S^T of the tile in `kb` without interleaving (prologue)
    auto qk_tile = [&](const CK_LDS char *kb, f32x16 (*sb)[2]) {
        const f32x16 zero16 = {};
#pragma unroll
        for (int f = 0; f < 16; ++f) {
            const bf16x8 kf = kfrag(kb, f);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
                sb[rb][f & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[rb][f >> 1],
                                                                        f < 2 ? zero16 : sb[rb][f & 1], 0, 0, 0);
        }
    };

    // ---- per-tile softmax pieces (p replaces s in place; P packed per 16 tokens) ----
    // group s16 of row block rb: elements 8 (s16 & 1) .. + 8 of token block s16 / 2
    float smax[RB], m_use[RB], dmv[RB], lsum[RB];
    bool rescale = false;
    auto soft_begin = [&]() {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            smax[rb] = -INFINITY;
            lsum[rb] = 0.f;
        }
    };
    auto max_chunk = [&](f32x16 (*sc)[2], int c) {  // c < 4 RB: 8 scores
        const int rb = c >> 2, q2 = (c >> 1) & 1, e0 = 8 * (c & 1);
#pragma unroll
        for (int e = e0; e < e0 + 8; ++e) smax[rb] = fmaxf(smax[rb], sc[rb][q2][e]);
    };
    auto max_finish = [&]() {
        bool any = false;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const float mx = max_xor32(smax[rb]) * a.scale_log2;
            const float m_new = fmaxf(m_run[rb], mx);
            m_use[rb] = (m_new == -INFINITY) ? 0.f : m_new;
            dmv[rb] = exp2_fast(m_run[rb] - m_use[rb]);
            m_run[rb] = m_new;
            any |= dmv[rb] != 1.0f;
        }
        // O moves only when some row's max moved (wave-uniform)
        rescale = __builtin_amdgcn_ballot_w64(any) != 0;
    };
    auto rescale_chunk = [&](int c) {  // c < 4 RB: 16 accumulators
        if (rescale) {
            const int rb = c >> 2, db = c & 3;
#pragma unroll
            for (int e = 0; e < 16; ++e) oacc[rb][db][e] *= dmv[rb];
        }
    };
    bf16x8 pbv[4][RB];
    auto exp_chunk = [&](f32x16 (*sc)[2], int s16, int rb, int hf) {  // 4 scores; hf 1 packs the group
        const int q2 = s16 >> 1, e0 = 8 * (s16 & 1) + 4 * hf;
#pragma unroll
        for (int e = e0; e < e0 + 4; ++e) {
            const float pv = exp2_fast(fmaf(sc[rb][q2][e], a.scale_log2, -m_use[rb]));
            sc[rb][q2][e] = pv;
            lsum[rb] += pv;
        }
        if (hf == 1) pbv[s16][rb] = pack_p(sc[rb][q2], 8 * (s16 & 1));
    };
    auto soft_end = [&]() {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) l_part[rb] = l_part[rb] * dmv[rb] + lsum[rb];
    };

    // One full tile of the main loop (t + 1 < ntiles): a fixed issue order, one
    // step per MFMA, fenced so the compiler keeps it.
    //   QK of tile t + 1 (16 RB MFMAs, K fragments read four ahead) with tile t's
    //   row max, step factors, O rescale and the exp of its 16-token groups 0-1;
    //   PV of tile t (16 RB MFMAs, V^T fragments read two 4-fragment groups
    //   ahead) with the exp of groups 2-3; a DMA every 4 RB MFMAs.
    constexpr int kNQ = 16 * RB;
    auto tile_body = [&](int t, f32x16 (*sc)[2], f32x16 (*sn)[2]) {
        const CK_LDS char *kb = kring + ((t + 1) % kTSlots) * kTBytes;
        const CK_LDS char *vb = vring + (t % kTSlots) * kTBytes;
        const f32x16 zero16 = {};
        const DmaGroup dg = dma_group(t);
        soft_begin();
        bf16x8 kfr[4];
#pragma unroll
        for (int f = 0; f < 4; ++f) kfr[f] = kfrag(kb, f);
#pragma unroll
        for (int i = 0; i < kNQ; ++i) {
            const int f = i / RB, rb = i % RB;
            sn[rb][f & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kfr[f & 3], qf[rb][f >> 1],
                                                                    f < 2 ? zero16 : sn[rb][f & 1], 0, 0, 0);
            if (rb == RB - 1 && f + 4 < 16) kfr[f & 3] = kfrag(kb, f + 4);
            // softmax slice: 4 RB max chunks, 4 RB rescale chunks, then the 4 RB exp
            // chunks of groups 0-1 (2 RB per group: row block, half)
            const int c = i;
            if (c < 4 * RB) {
                max_chunk(sc, c);
                if (c == 4 * RB - 1) max_finish();
            } else if (c < 8 * RB) {
                rescale_chunk(c - 4 * RB);
            } else if (c < 12 * RB) {
                const int x = c - 8 * RB;
                exp_chunk(sc, x / (2 * RB), (x / 2) % RB, x & 1);
            }
            if (i % (kNQ / (kTDma / 2)) == kNQ / (kTDma / 2) - 1) dma_step(dg, i / (kNQ / (kTDma / 2)));
            __builtin_amdgcn_sched_barrier(0);
        }
        uint2 vlo[3][4], vhi[3][4];
#pragma unroll
        for (int s0 = 0; s0 < 2; ++s0)
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                vlo[s0][db] = lds_read_tr16(vb + vt_off(s0, db, 0));
                vhi[s0][db] = lds_read_tr16(vb + vt_off(s0, db, 1));
            }
#pragma unroll
        for (int i = 0; i < kNQ; ++i) {
            const int fv = i / RB, rb = i % RB, s16 = fv >> 2, db = fv & 3, bsel = s16 % 3;
            const bf16x8 vf = __builtin_bit_cast(
                bf16x8, make_uint4(vlo[bsel][db].x, vlo[bsel][db].y, vhi[bsel][db].x, vhi[bsel][db].y));
            oacc[rb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pbv[s16][rb], oacc[rb][db], 0, 0, 0);
            if (rb == RB - 1 && s16 + 2 < 4) {
                vlo[(s16 + 2) % 3][db] = lds_read_tr16(vb + vt_off(s16 + 2, db, 0));
                vhi[(s16 + 2) % 3][db] = lds_read_tr16(vb + vt_off(s16 + 2, db, 1));
            }
            // exp of groups 2-3 (2 RB chunks each) over the first PV steps, each
            // group finished before its first MFMA (group 2 at step 8 RB)
            if (i < 4 * RB) exp_chunk(sc, 2 + i / (2 * RB), (i / 2) % RB, i & 1);
            if (i % (kNQ / (kTDma / 2)) == kNQ / (kTDma / 2) - 1)
                dma_step(dg, kTDma / 2 + i / (kNQ / (kTDma / 2)));
            __builtin_amdgcn_sched_barrier(0);
        }
        soft_end();
    };

    f32x16 s_a[RB][2], s_b[RB][2];
    // prologue: K of tiles 0-2 and V of tiles 0-1 in flight (repeats past the
    // end). A split with no tokens (a request shorter than the split's start)
    // issues nothing: every DMA source is a tile index clamped to ntiles - 1.
    if (ntiles > 0) {
#pragma unroll
        for (int j = 0; j < kTBlk; ++j) {
            dma_k(0, j);
            dma_k(1, j);
            dma_k(2, j);
            dma_v(0, j);
            dma_v(1, j);
        }
    }
    wait_vmcnt<0>();
    __syncthreads();
    if (ntiles > 0 && !page_ok(0)) {
        zero_rows(kring, 0);
        __syncthreads();
    }
    if (ntiles > 0 && wave_active) qk_tile(kring, s_a);

    // every tile but the last is full (64 tokens)
    auto tile_top = [&](int t) {
        // this iteration reads K of tile t + 1 and V of tile t (issued two
        // iterations ago); the previous iteration's group may stay in flight
        wait_vmcnt<kTDma>();
        __syncthreads();  // ... for every wave; and every wave is done with tile t - 1
        const bool v_fill = !page_ok(t);
        const bool k_fill = !page_ok(t + 1);
        if (v_fill) zero_rows(vring + (t % kTSlots) * kTBytes, 0);
        if (k_fill) zero_rows(kring + ((t + 1) % kTSlots) * kTBytes, 0);
        if (v_fill || k_fill) __syncthreads();
    };
    auto idle_dmas = [&](int t) {
        const DmaGroup dg = dma_group(t);
#pragma unroll
        for (int j = 0; j < kTDma; ++j) dma_step(dg, j);
    };
    int t = 0;
    for (; t + 2 < ntiles; t += 2) {
        tile_top(t);
        if (wave_active) tile_body(t, s_a, s_b);
        else idle_dmas(t);
        tile_top(t + 1);
        if (wave_active) tile_body(t + 1, s_b, s_a);
        else idle_dmas(t + 1);
    }
    if (t + 1 < ntiles) {
        tile_top(t);
        if (wave_active) {
            tile_body(t, s_a, s_b);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                s_a[rb][0] = s_b[rb][0];
                s_a[rb][1] = s_b[rb][1];
            }
        } else {
            idle_dmas(t);
        }
        ++t;
    }
    // the last tile: tokens past the split's end are masked (p = 0) and their V
    // rows zeroed, so 0 * V cannot produce a NaN from rows nobody wrote
    if (ntiles > 0) {
        wait_vmcnt<0>();
        __syncthreads();
        const int nv = ntok - t * kTTok;
        if (nv < kTTok || !page_ok(t)) {
            zero_rows(vring + (t % kTSlots) * kTBytes, page_ok(t) ? nv : 0);
            __syncthreads();
        }
        if (wave_active) {
            if (nv < kTTok) {
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int q2 = 0; q2 < 2; ++q2)
#pragma unroll
                        for (int e = 0; e < 16; ++e) {
                            const int tok = 32 * q2 + (e & 3) + 8 * (e >> 2) + 4 * hh;
                            if (tok >= nv) s_a[rb][q2][e] = -INFINITY;
                        }
            }
            const CK_LDS char *vb = vring + (t % kTSlots) * kTBytes;
            soft_begin();
            for (int c = 0; c < 4 * RB; ++c) max_chunk(s_a, c);
            max_finish();
            for (int c = 0; c < 4 * RB; ++c) rescale_chunk(c);
#pragma unroll
            for (int s16 = 0; s16 < 4; ++s16)
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
                    exp_chunk(s_a, s16, rb, 0);
                    exp_chunk(s_a, s16, rb, 1);
                }
            soft_end();
#pragma unroll
            for (int s16 = 0; s16 < 4; ++s16)
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const uint2 lo = lds_read_tr16(vb + vt_off(s16, db, 0));
                    const uint2 hi = lds_read_tr16(vb + vt_off(s16, db, 1));
                    const bf16x8 vf = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb)
                        oacc[rb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pbv[s16][rb], oacc[rb][db], 0, 0, 0);
                }
        }
    }

    // ---- normalise and write whole rows --------------------------------------------
    // Each wave writes its 32 RB rows through its own slab of the (now idle) rings
    // (32 rows x 512 B = 16 KB per row block), re-laid out as whole 512-byte rows
    // so each store instruction writes two contiguous rows.
    float l_run[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) l_run[rb] = l_part[rb] + __shfl_xor(l_part[rb], 32);
    __syncthreads();  // every wave is past its last ring read
    if (!wave_active) return;  // wave-uniform
    float *base = a.num_splits == 1 ? a.out : a.part_o + (int64_t)sp * a.num_rows * kD;
    const int my_row = lane & 31;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const float inv = l_run[rb] > 0.f ? 1.0f / l_run[rb] : 0.f;
        const float lse_v = l_run[rb] > 0.f ? (m_run[rb] + __log2f(l_run[rb])) * kLn2 : -INFINITY;
        CK_LDS float *slab = (CK_LDS float *)smem + (wid * RB + rb) * (32 * kD);
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4) {
                const f32x4 o = f32x4{oacc[rb][db][4 * c4 + 0] * inv, oacc[rb][db][4 * c4 + 1] * inv,
                                      oacc[rb][db][4 * c4 + 2] * inv, oacc[rb][db][4 * c4 + 3] * inv};
                const int chunk = (8 * db + 2 * c4 + hh) ^ my_row;
                *reinterpret_cast<CK_LDS f32x4 *>(slab + my_row * kD + chunk * 4) = o;
            }
        if (row_valid[rb]) {
            if (a.num_splits == 1) {
                const float4 lv = make_float4(lse_v, lse_v, lse_v, lse_v);
                *reinterpret_cast<float4 *>(a.lse + qrow[rb] * 8 + 4 * hh) = lv;
            } else if (hh == 0) {
                a.part_lse[(int64_t)sp * a.num_rows + qrow[rb]] = lse_v;
            }
        }
        // the wave reads back only its own slab: the LDS ops of one wave complete in order
        const int chunk = lane & 31;
        const int rbase = wrow0 + rb * 32;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int rr = 2 * j + (lane >> 5);
            const int64_t qr = __shfl((int)qrow[rb], rr);
            const f32x4 o = *reinterpret_cast<const CK_LDS f32x4 *>(slab + rr * kD + ((chunk ^ rr) * 4));
            if (rbase + rr < rows_b) *reinterpret_cast<f32x4 *>(base + qr * kD + chunk * 4) = o;
        }
    }
}

__global__ __launch_bounds__(kWW * 64) void stage1_wide_kernel(Stage1Args a) {
    extern __shared__ __attribute__((aligned(16))) char smem_raw[];
    stage1_wide_body<kWW, kWSlots>(a, (CK_LDS char *)smem_raw, blockIdx.x, gridDim.x, threadIdx.x, WgBarrier{});
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
        rc = ensure_dynamic_lds(reinterpret_cast<const void *>(&stage1_tile_kernel<1>), kTLds, lds_set1);
        if (rc != CK_OK) return rc;
        hipLaunchKernelGGL(stage1_tile_kernel<1>, dim3((unsigned)grid), dim3(kTW * 64), kTLds, s, a);
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
