// stage1_wide.h - the stage-1 arguments, tile helpers and the 256-row (wide)
// kernel body, shared by the stand-alone stage-1 kernels (fa_stage1.hip) and the
// fused cascade kernel (suffix_decode.hip), which runs the body on 4 of its waves.
#pragma once

#include "ck_common.h"

namespace ck {
namespace s1 {

constexpr int kD = 128;          // head dim (op contract)
constexpr int kPage = 128;       // paged block size (op contract)
constexpr int kMaxSplitPages = 256;   // page ids held in LDS per split

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

constexpr int kTTok = 64;                            // tokens per tile
constexpr int kTBytes = kTTok * kD * 2;              // 16 KB of K (or V) per tile

// 256-row variant for requests whose rows of one kv head fill more than 128:
// 8 waves (two per SIMD), wave w owns query rows 32 w .. + 32 and every token
// of them. Each 64-token K/V tile in LDS feeds 256 rows (twice the MFMA work
// per DMA byte and per barrier of the 128-row kernel), and while one wave of a
// SIMD waits on a fragment read, a DMA issue or its softmax, the other issues
// MFMAs. Per tile: QK (16 MFMAs, K fragments read four ahead), softmax with
// the running max moved once per tile, PV (16 MFMAs, V^T fragments read one
// 16-token group ahead). A 4-slot ring of K+V tiles, three tiles of DMA lead.
// The body is shared with the fused cascade kernel, where 4 waves run it (128
// rows, a 3-slot ring) beside 4 waves of suffix streaming: NW waves, SLOTS ring
// slots, its own barrier, workgroup lb of nlb, thread tid of the NW * 64.
constexpr int kWW = 8;
constexpr int kWSlots = 4;
constexpr int kWStage = 2 * kTBytes;  // K + V of one tile (32 KB)
template <int SLOTS>
constexpr int wide_lds_bytes() { return SLOTS * kWStage + kMaxSplitPages * 4; }
constexpr int kWLds = wide_lds_bytes<kWSlots>();

template <int NW, int SLOTS, class Bar>
__device__ __forceinline__ void stage1_wide_body(const Stage1Args &a, CK_LDS char *smem, int lb, int nlb, int tid,
                                                 const Bar &bar) {
    constexpr int kWRows = NW * 32;
    constexpr int kWBlk = kTBytes / 1024 / NW;  // 1-KB DMAs of K (and of V) per wave per tile
    static_assert(SLOTS >= 2 && SLOTS <= 4, "ring depth");
    static_assert(NW * 32 * kD * 4 <= SLOTS * kWStage, "epilogue slabs fit the ring");
    CK_LDS int *s_pages = (CK_LDS int *)(smem + SLOTS * kWStage);

    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: DMA LDS addresses in SGPRs
    const int lane = tid & 63;
    const int hh = lane >> 5;

    uint32_t w = xcd_remap(lb, nlb);
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
    const int row0 = mt * kWRows;
    if (row0 >= rows_b) return;  // uniform over the workgroup

    const int wrow0 = row0 + wid * 32;
    const bool wave_active = wrow0 < rows_b;
    const int r = wrow0 + (lane & 31);
    const bool row_valid = r < rows_b;
    const int t_local = r / a.group;
    const int h = g * a.group + (r - t_local * a.group);
    const int64_t qrow = (int64_t)(qs + t_local) * a.num_heads + h;
    bf16x8 qf[8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
        if (row_valid) {
            qf[kk] = *reinterpret_cast<const bf16x8 *>(a.q + qrow * kD + 16 * kk + 8 * hh);
        } else {
            qf[kk] = __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
        }
    }
    const int kv_lo = sp * a.split_len;
    {
        const int pg0 = kv_lo / kPage;
        const int64_t avail = a.bt_cols - pg0;
        const int pg_n = (int)min((int64_t)(a.split_len / kPage), avail > 0 ? avail : (int64_t)0);
        for (int pi = tid; pi < pg_n; pi += NW * 64) {
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
    bar.sync();  // s_pages visible

    const int64_t head_stride = (int64_t)a.kv_heads * kD;
    uint32_t dma_off[kWBlk];
#pragma unroll
    for (int j = 0; j < kWBlk; ++j) {
        const int tt = (wid * kWBlk + j) * 4 + (lane >> 4);
        dma_off[j] = (uint32_t)(tt * head_stride + g * kD + (((lane & 15) ^ tile_swz(tt)) << 3));
    }
    // DMAs of tile t (t < ntiles, page id raw) into ring slot `slot` (t % SLOTS):
    // the tile's 64 token rows of K and of V as buffer resources (scalar base),
    // the lane offsets fixed. Byte offsets from 32-bit factors (a page is at most
    // 2^31 bytes: 128 tokens x 2^16 heads x 256 B), the page id read a barrier
    // ahead and the slot counted, so the DMA issue is a few scalar instructions.
    const uint32_t tile_bytes = (uint32_t)(kTTok * head_stride * 2);
    const uint32_t page_bytes = 2 * tile_bytes;
    auto issue = [&](int t, int raw, int slot) {
        raw = __builtin_amdgcn_readfirstlane(raw);
        const uint64_t base = (uint64_t)(uint32_t)max(raw, 0) * page_bytes + ((t & 1) ? tile_bytes : 0u);
        const ck_rsrc_t rk = buf_rsrc(reinterpret_cast<const char *>(a.k) + base, tile_bytes);
        const ck_rsrc_t rv = buf_rsrc(reinterpret_cast<const char *>(a.v) + base, tile_bytes);
        CK_LDS char *kd = smem + slot * kWStage + wid * kWBlk * 1024;
#pragma unroll
        for (int j = 0; j < kWBlk; ++j) {
            dma16_buf(rk, (int)(dma_off[j] * 2), 0, kd + j * 1024);
            dma16_buf(rv, (int)(dma_off[j] * 2), 0, kd + kTBytes + j * 1024);
        }
    };

    f32x16 oacc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[db][i] = 0.f;
    float m_run = -INFINITY;
    float l_part = 0.f;

    const int trG = (lane >> 4) & 3;
    const int tr_row = (lane & 15) >> 2;
    const int tr_e4 = lane & 3;
    const int ktok = lane & 31;
    auto vt_off = [&](int s16, int db, int second) {
        const int t1 = 16 * s16 + 4 * (trG >> 1) + tr_row + 8 * second;
        const int d = 32 * db + 16 * (trG & 1) + 4 * tr_e4;
        return tile_off(t1, d >> 3) + (d & 7) * 2;
    };

    for (int t = 0; t < SLOTS - 1 && t < ntiles; ++t) issue(t, s_pages[t >> 1], t);
    int slot = 0;  // t % SLOTS
    for (int t = 0; t < ntiles; ++t) {
        // page ids of tile t and of the tile issued below, read before the waits
        const int pg_t = s_pages[t >> 1];
        const int pg_i = t + SLOTS - 1 < ntiles ? s_pages[(t + SLOTS - 1) >> 1] : 0;
        // tile t has landed once at most the DMAs of the tiles after it remain
        const int after = min(SLOTS - 2, ntiles - 1 - t);
        if (after >= 2) wait_vmcnt<4 * kWBlk>();
        else if (after == 1) wait_vmcnt<2 * kWBlk>();
        else wait_vmcnt<0>();
        bar.sync();  // ... in every wave; every wave is done with tile t - 1
        const int nv = min(kTTok, ntok - t * kTTok);
        const bool ok = pg_t >= 0;
        CK_LDS char *kb = smem + slot * kWStage;
        CK_LDS char *vb = kb + kTBytes;
        if (nv < kTTok || !ok) {
            // rows past the split's end or of an invalid page: zero them so 0 * V
            // cannot produce a NaN (an invalid page reads as zero rows)
            const int z0 = ok ? nv : 0;
            for (int idx = tid; idx < (kTTok - z0) * 16; idx += NW * 64) {
                const int tt = z0 + (idx >> 4), c = idx & 15;
                *reinterpret_cast<CK_LDS u32x4 *>(kb + tt * 256 + c * 16) = u32x4{0, 0, 0, 0};
                *reinterpret_cast<CK_LDS u32x4 *>(vb + tt * 256 + c * 16) = u32x4{0, 0, 0, 0};
            }
            bar.sync();
        }
        if (t + SLOTS - 1 < ntiles) issue(t + SLOTS - 1, pg_i, slot == 0 ? SLOTS - 1 : slot - 1);  // tile t - 1's slot
        slot = slot == SLOTS - 1 ? 0 : slot + 1;
        if (!wave_active) continue;

        // S^T of the two 32-token blocks, K fragments read four ahead
        f32x16 sb[2];
        {
            const f32x16 zero16 = {};
            auto kfrag = [&](int f) {
                return *reinterpret_cast<const CK_LDS bf16x8 *>(kb + tile_off(32 * (f & 1) + ktok, 2 * (f >> 1) + hh));
            };
            bf16x8 kfr[4];
#pragma unroll
            for (int f = 0; f < 4; ++f) kfr[f] = kfrag(f);
#pragma unroll
            for (int f = 0; f < 16; ++f) {
                sb[f & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kfr[f & 3], qf[f >> 1], f < 2 ? zero16 : sb[f & 1],
                                                                    0, 0, 0);
                if (f + 4 < 16) kfr[f & 3] = kfrag(f + 4);
            }
        }
        if (nv < kTTok) {
#pragma unroll
            for (int q2 = 0; q2 < 2; ++q2)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int tok = 32 * q2 + (e & 3) + 8 * (e >> 2) + 4 * hh;
                    if (tok >= nv) sb[q2][e] = -INFINITY;
                }
        }
        float smax = -INFINITY;
#pragma unroll
        for (int q2 = 0; q2 < 2; ++q2)
#pragma unroll
            for (int e = 0; e < 16; ++e) smax = fmaxf(smax, sb[q2][e]);
        smax = max_xor32(smax) * a.scale_log2;
        const float m_new = fmaxf(m_run, smax);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        const float dm = exp2_fast(m_run - m_use);
        m_run = m_new;
        float ls = 0.f;
        bf16x8 pb[4];
#pragma unroll
        for (int q2 = 0; q2 < 2; ++q2) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float pv = exp2_fast(fmaf(sb[q2][e], a.scale_log2, -m_use));
                sb[q2][e] = pv;
                ls += pv;
            }
            pb[2 * q2] = pack_p(sb[q2], 0);
            pb[2 * q2 + 1] = pack_p(sb[q2], 8);
        }
        l_part = l_part * dm + ls;
        if (__builtin_amdgcn_ballot_w64(dm != 1.0f)) {
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int e = 0; e < 16; ++e) oacc[db][e] *= dm;
        }
        // O^T += V^T P^T, V^T fragments read one 16-token group ahead
        {
            uint2 vlo[2][4], vhi[2][4];
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                vlo[0][db] = lds_read_tr16(vb + vt_off(0, db, 0));
                vhi[0][db] = lds_read_tr16(vb + vt_off(0, db, 1));
            }
#pragma unroll
            for (int s16 = 0; s16 < 4; ++s16) {
                if (s16 + 1 < 4) {
#pragma unroll
                    for (int db = 0; db < 4; ++db) {
                        vlo[(s16 + 1) & 1][db] = lds_read_tr16(vb + vt_off(s16 + 1, db, 0));
                        vhi[(s16 + 1) & 1][db] = lds_read_tr16(vb + vt_off(s16 + 1, db, 1));
                    }
                }
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const uint2 lo = vlo[s16 & 1][db], hi = vhi[s16 & 1][db];
                    const bf16x8 vf = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
                    oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb[s16], oacc[db], 0, 0, 0);
                }
            }
        }
    }

    // ---- normalise and write whole rows through the idle ring ------------------------
    const float l_run = l_part + __shfl_xor(l_part, 32);
    bar.sync();  // every wave is past its last ring read
    if (!wave_active) return;  // wave-uniform
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
    const float lse_v = l_run > 0.f ? (m_run + __log2f(l_run)) * kLn2 : -INFINITY;
    CK_LDS float *slab = (CK_LDS float *)smem + wid * (32 * kD);
    const int my_row = lane & 31;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
            const f32x4 o = f32x4{oacc[db][4 * c4 + 0] * inv, oacc[db][4 * c4 + 1] * inv,
                                  oacc[db][4 * c4 + 2] * inv, oacc[db][4 * c4 + 3] * inv};
            const int chunk = (8 * db + 2 * c4 + hh) ^ my_row;
            *reinterpret_cast<CK_LDS f32x4 *>(slab + my_row * kD + chunk * 4) = o;
        }
    if (row_valid) {
        if (a.num_splits == 1) {
            const float4 lv = make_float4(lse_v, lse_v, lse_v, lse_v);
            *reinterpret_cast<float4 *>(a.lse + qrow * 8 + 4 * hh) = lv;
        } else if (hh == 0) {
            __builtin_nontemporal_store(lse_v, a.part_lse + (int64_t)sp * a.num_rows + qrow);
        }
    }
    float *base = a.num_splits == 1 ? a.out : a.part_o + (int64_t)sp * a.num_rows * kD;
    const int chunk = lane & 31;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int rr = 2 * j + (lane >> 5);
        const int64_t qr = __shfl((int)qrow, rr);
        const f32x4 o = *reinterpret_cast<const CK_LDS f32x4 *>(slab + rr * kD + ((chunk ^ rr) * 4));
        // non-temporal: read once, by another kernel (combine, cascade epilogue)
        if (wrow0 + rr < rows_b) __builtin_nontemporal_store(o, reinterpret_cast<f32x4 *>(base + qr * kD + chunk * 4));
    }
}

}  // namespace s1
}  // namespace ck
