// gateup_swiglu.hip - gate_up GEMM with the f3 epilogue ladder on gfx950 MFMA.
//
// Semantics (reference: ascend-kernel/csrc/ops/f3_floor, kernel
// op_kernel/kernel_f3_floor.cpp:137-349, host op_host/f3_floor.cpp:59-124):
//   a [M, K] bf16 activations, b [2I, K] bf16 nn.Linear weight (gate rows
//   0..I-1, up rows I..2I-1). C = a b^T accumulated in fp32.
//   mode 1 (SwiGLU, a hook only in the reference, design.md:107-109):
//     d = bf16_RNE(silu(g) * u), g/u the fp32 accumulators, silu(x) = x/(1+e^-x);
//     the C workspace is not written (the point of the fusion).
//   modes 0/2/4/5/7/8: the workspace receives C = bf16_RNE(a b^T); d is the gate
//   window (0, 5), the up window (4), nothing (2, 7) or zeros (8).
//   mode 3: d = workspace[:, :I] (no GEMM).
//
// MI355X design:
// * D^T = W X^T on v_mfma_f32_32x32x16_bf16: A operand = weight rows, B operand
//   = activation rows, both K-contiguous in memory, so fragments are 16-byte
//   LDS reads and each accumulator lane ends up holding 4 consecutive output
//   columns (8-byte bf16 stores in the epilogue). The gate and up accumulators
//   of one output element sit in the same lane and register index: SwiGLU is
//   computed in registers in fp32 and stored once as bf16 -- the gate/up
//   product never reaches memory.
// * Main kernel (K a multiple of 32): workgroup tile 256 activation rows x
//   (128 gate + the matching 128 up weight rows), 4 waves (one per SIMD)
//   arranged 2 (activation) x 2 (weight); each wave owns 128 activation rows x
//   (64 gate + 64 up) weight rows, 16 accumulator tiles of 32x32 in the
//   accumulation registers, so per 16-deep k-substep 8 fragment reads feed 16
//   MFMAs (half an LDS read per MFMA). Operand tiles stream global -> LDS by
//   DMA (buffer_load_dwordx4 ... lds on per-block buffer resources: no staging
//   registers, no LDS write instructions, no vector address arithmetic). With K
//   a multiple of 64 a stage is 64 deep, so each staged
//   row is one whole 128-byte line and a DMA instruction fetches 8 whole lines
//   (with 32-deep stages it fetched 16 half lines: the address unit's cost per
//   byte doubles, and it bounded the kernel). Two such 64-KB stages would fill
//   the ring, so the ring is five 32-KB parts, one operand of one stage each:
//   the weights run two tiles ahead, the activations one. Rows are
//   XOR-swizzled at 16-byte granularity (the DMA lane fetches the chunk that
//   belongs at its LDS slot) so the 32-row fragment reads are bank-conflict
//   free. The fragments of substep s + 1 are read while the MFMAs of substep s
//   run, interleaved by scheduling barriers. A half-width instance (64 gate +
//   64 up rows, three 48-KB stages) runs when the full-width grid would leave
//   CUs idle (a few m-tiles, e.g. M = 256 at I = 14336: 224 workgroups instead
//   of 112). K = 32 mod 64 runs the same kernel on 32-deep stages (4-stage ring).
// * Decode-sized kernel (M <= 32, K % 256 == 0): the weight stream bounds the
//   op, so a workgroup takes 32 gate + 32 up rows (I / 32 workgroups, two per
//   CU) and its 4 waves each stream a quarter of K from global memory straight
//   into MFMA operand registers, several 64-deep steps ahead; the partial sums
//   meet in LDS once. It runs on 16x16x32 MFMA, whose operand layout (four lanes
//   per row) needs half the address lines per weight byte of the 32x32 one.
// * General kernel (any K % 16 == 0): 8 waves of 128 x (32 + 32), operands
//   staged global -> registers -> LDS.
// * Tiles are ordered M-fastest and XCD-aware so the workgroups sharing a
//   weight slice run on the same XCD and hit its L2.
#include "ck_common.h"

namespace ck {
namespace {

constexpr int kBM = 256;        // activation rows per workgroup
constexpr int kBNh = 128;       // gate columns per workgroup (and as many up columns)
constexpr int kBW = 2 * kBNh;   // weight rows staged per workgroup
constexpr int kBK = 64;
constexpr int kThreads = 512;
constexpr int kRowBytes = kBK * 2;                // 128 B per staged row
constexpr int kTileBytes = (kBM + kBW) * kRowBytes;  // 64 KB per stage
constexpr int kChunksPerThread = (kBM + kBW) * (kBK / 8) / kThreads;  // 8

struct GemmArgs {
    const uint16_t *a;
    const uint16_t *b;
    uint16_t *c;
    uint16_t *d;
    int64_t m;
    int64_t n_half;
    int64_t k;
    int64_t d_stride;
    int mtiles;
    int ntiles;
};

__device__ __forceinline__ int sw_off(int row, int c) { return row * kRowBytes + ((c ^ (row & 7)) << 4); }

__device__ __forceinline__ float silu_mul(float g, float u) {
    const float e = exp2_fast(-g * kLog2e);
    return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

template <int MODE>
__global__ __launch_bounds__(kThreads) void gateup_general_kernel(GemmArgs p) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int tid = threadIdx.x;
    const int wid = tid >> 6;
    const int lane = tid & 63;
    const int hh = lane >> 5;
    const int l32 = lane & 31;
    const int wa = wid >> 2;  // activation half: rows wa*128 .. +128
    const int ww = wid & 3;   // weight quarter: gate rows ww*32 .. +32 (and up)

    const uint32_t w = xcd_remap(blockIdx.x, gridDim.x);
    const int mi = w % p.mtiles;
    const int ni = w / p.mtiles;
    const int64_t m0 = (int64_t)mi * kBM;
    const int64_t n0 = (int64_t)ni * kBNh;
    const int ktiles = (int)((p.k + kBK - 1) / kBK);

    // staging assignment: chunk ci = tid + 512u -> staged row ci/8, 16-byte chunk ci%8
    const uint16_t *src[kChunksPerThread];
    bool rvalid[kChunksPerThread];
#pragma unroll
    for (int u = 0; u < kChunksPerThread; ++u) {
        const int ci = tid + kThreads * u;
        const int row = ci >> 3, c = ci & 7;
        if (row < kBM) {
            const int64_t gm = m0 + row;
            rvalid[u] = gm < p.m;
            src[u] = p.a + (rvalid[u] ? gm : 0) * p.k + c * 8;
        } else {
            const int wr = row - kBM;
            const int64_t gn = wr < kBNh ? n0 + wr : p.n_half + n0 + (wr - kBNh);
            rvalid[u] = true;
            src[u] = p.b + gn * p.k + c * 8;
        }
    }
    uint4 stage[kChunksPerThread];
    auto load_tile = [&](int kt) {
        const int64_t k0 = (int64_t)kt * kBK;
#pragma unroll
        for (int u = 0; u < kChunksPerThread; ++u) {
            const int c = (tid + kThreads * u) & 7;
            const bool ok = rvalid[u] && (k0 + c * 8) < p.k;
            stage[u] = ok ? *reinterpret_cast<const uint4 *>(src[u] + k0) : make_uint4(0, 0, 0, 0);
        }
    };
    auto store_tile = [&](int buf) {
        char *base = smem + buf * kTileBytes;
#pragma unroll
        for (int u = 0; u < kChunksPerThread; ++u) {
            const int ci = tid + kThreads * u;
            *reinterpret_cast<uint4 *>(base + sw_off(ci >> 3, ci & 7)) = stage[u];
        }
    };

    f32x16 acc[4][2];
#pragma unroll
    for (int ab = 0; ab < 4; ++ab)
#pragma unroll
        for (int gu = 0; gu < 2; ++gu)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[ab][gu][e] = 0.f;

    load_tile(0);
    store_tile(0);
    __syncthreads();
    if (ktiles > 1) load_tile(1);

    for (int kt = 0; kt < ktiles; ++kt) {
        const char *xa = smem + (kt & 1) * kTileBytes;
        const char *wb = xa + kBM * kRowBytes;
#pragma unroll
        for (int s = 0; s < kBK / 16; ++s) {
            const int ch = 2 * s + hh;
            bf16x8 wf[2], xf[4];
            wf[0] = *reinterpret_cast<const bf16x8 *>(wb + sw_off(ww * 32 + l32, ch));
            wf[1] = *reinterpret_cast<const bf16x8 *>(wb + sw_off(kBNh + ww * 32 + l32, ch));
#pragma unroll
            for (int ab = 0; ab < 4; ++ab)
                xf[ab] = *reinterpret_cast<const bf16x8 *>(xa + sw_off(wa * 128 + ab * 32 + l32, ch));
#pragma unroll
            for (int ab = 0; ab < 4; ++ab)
#pragma unroll
                for (int gu = 0; gu < 2; ++gu)
                    acc[ab][gu] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[gu], xf[ab], acc[ab][gu], 0, 0, 0);
        }
        if (kt + 1 < ktiles) store_tile((kt + 1) & 1);
        __syncthreads();
        if (kt + 2 < ktiles) load_tile(kt + 2);
    }

    // ---- epilogue: lane = activation row l32 of block ab; regs 4c..4c+3 =
    // output columns n0 + ww*32 + 8c + 4hh + 0..3 --------------------------------
#pragma unroll
    for (int ab = 0; ab < 4; ++ab) {
        const int64_t gm = m0 + wa * 128 + ab * 32 + l32;
        if (gm >= p.m) continue;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int64_t col = n0 + ww * 32 + 8 * c + 4 * hh;
            const float g0 = acc[ab][0][4 * c + 0], g1 = acc[ab][0][4 * c + 1];
            const float g2 = acc[ab][0][4 * c + 2], g3 = acc[ab][0][4 * c + 3];
            const float u0 = acc[ab][1][4 * c + 0], u1 = acc[ab][1][4 * c + 1];
            const float u2 = acc[ab][1][4 * c + 2], u3 = acc[ab][1][4 * c + 3];
            if (MODE == 1) {
                const uint2 dv = make_uint2(pack_bf16x2(silu_mul(g0, u0), silu_mul(g1, u1)),
                                            pack_bf16x2(silu_mul(g2, u2), silu_mul(g3, u3)));
                *reinterpret_cast<uint2 *>(p.d + gm * p.d_stride + col) = dv;
            } else {
                const uint2 gv = make_uint2(pack_bf16x2(g0, g1), pack_bf16x2(g2, g3));
                const uint2 uv = make_uint2(pack_bf16x2(u0, u1), pack_bf16x2(u2, u3));
                uint16_t *crow = p.c + gm * (2 * p.n_half);
                *reinterpret_cast<uint2 *>(crow + col) = gv;
                *reinterpret_cast<uint2 *>(crow + p.n_half + col) = uv;
                if (MODE == 0 || MODE == 5)
                    *reinterpret_cast<uint2 *>(p.d + gm * p.d_stride + col) = gv;
                else if (MODE == 4)
                    *reinterpret_cast<uint2 *>(p.d + gm * p.d_stride + col) = uv;
                else if (MODE == 8)
                    *reinterpret_cast<uint2 *>(p.d + gm * p.d_stride + col) = make_uint2(0, 0);
            }
        }
    }
}

// ---- main kernel: 4 waves x (128 x 64 WB), DMA-fed LDS ring ---------------------------
constexpr int kDThreads = 256;
constexpr int64_t kMaxDmaK = (int64_t)1 << 21;  // a 256-row operand block stays under 2^31 bytes
constexpr int kGroupM = 4;   // tile block one XCD runs at once: 4 m-tiles x 8 n-tiles
constexpr int kGroupN = 8;

// Workgroup tile of the DMA kernel: 256 activation rows x WB * 64 gate rows (and as
// many up rows); each wave holds WB 32-row blocks of gate and of up. WB = 2 is the
// 256 x (128 + 128) tile; WB = 1 halves the weight rows so that a small M (one
// m-tile) still spreads over twice the workgroups. BK = K per ring stage: 64 (rows
// of 128 bytes, one whole cache line per row and DMA lane group) when K allows,
// else 32 (64-byte rows). The ring holds as many stages as fit in 160 KB, at most 4.
template <int WB, int BK>
struct DmaTile {
    static constexpr int kNh = 64 * WB;                               // gate rows per workgroup
    static constexpr int kRowBytes = BK * 2;                          // 128 / 64 B per staged row
    static constexpr int kRows = kBM + 2 * kNh;                       // staged rows per stage
    static constexpr int kStageBytes = kRows * kRowBytes;             // 64 / 48 KB (BK 64), 32 / 24 KB (BK 32)
    static constexpr int kStages = BK == 64 ? (WB == 2 ? 2 : 3) : 4;
    static constexpr int kDmaPerWave = kStageBytes / 1024 / 4;        // 16 / 12 (BK 64), 8 / 6 (BK 32)
    static constexpr int kRowsPerDma = 1024 / kRowBytes;              // 8 / 16 rows per 1-KB DMA
    // 256 x (128 + 128) at BK 64: two 64-KB stages would be all the ring holds, so
    // the operands get rings of their own within five 32-KB parts instead (below)
    static constexpr bool kSplit = BK == 64 && WB == 2;
    static constexpr int kPart = kBM * kRowBytes;                     // 32 KB: one operand of one stage
    static constexpr int kLdsBytes = kSplit ? 5 * kPart : kStages * kStageBytes;  // 160 / 144 KB, 128 / 96 KB
    static constexpr int kSub = BK / 16;                              // 16-deep MFMA substeps per stage
    static constexpr int kMfmaSub = 8 * WB;                           // MFMAs per wave per substep
    static constexpr int kReads = 2 * WB + 4;                         // fragment reads per substep
    // DMAs of a stage issued right after the barrier that frees its slot (in the
    // stage's last substep); the rest go out in the first substep of the next stage
    static constexpr int kEarlyDma = BK == 64 && WB == 2 ? kDmaPerWave : kDmaPerWave / 2;
    static_assert(kLdsBytes <= 160 * 1024, "ring fits the LDS");
};

// Byte offset of 16-byte chunk ch of staged row `row`: chunk slot ch ^ f(row). A
// fragment read has 32 lanes on consecutive rows at one chunk, 16 lanes per LDS
// cycle over 256-byte bank windows: with 128-byte rows (two per window) f(row) =
// (row >> 1) & 7 puts the 16 rows of a cycle on 16 distinct 16-byte slots; with
// 64-byte rows (four per window) f(row) = ((row >> 1) ^ (row >> 2)) & 3 does (a
// plain ((row >> 1) & 3) collides rows r and r + 8).
template <int BK>
__device__ __forceinline__ int dsw_swz(int row) {
    if constexpr (BK == 64) return (row >> 1) & 7;
    else return ((row >> 1) ^ (row >> 2)) & 3;
}
template <int BK>
__device__ __forceinline__ int dsw_off(int row, int ch) { return row * (BK * 2) + ((ch ^ dsw_swz<BK>(row)) << 4); }

template <int MODE, int WB, int BK>
__global__ __launch_bounds__(kDThreads, 1) void gateup_dma_kernel(GemmArgs p) {
    using T = DmaTile<WB, BK>;
    constexpr int kBNhW = T::kNh;
    constexpr int kS = T::kStages;
    constexpr int kNS = T::kSub;
    constexpr int kD = T::kDmaPerWave;
    constexpr int kRB = T::kRowBytes;
    extern __shared__ __attribute__((aligned(16))) char smem_raw[];
    CK_LDS char *smem = (CK_LDS char *)smem_raw;
    const int tid = threadIdx.x;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: LDS addresses in SGPRs
    const int lane = tid & 63;
    const int hh = lane >> 5;
    const int l32 = lane & 31;
    const int wa = wid >> 1;  // activation half: rows wa*128 .. +128
    const int ww = wid & 1;   // weight half: gate rows ww*32WB .. +32WB (and up)

    const uint32_t w = xcd_remap(blockIdx.x, gridDim.x);
    // the 32 workgroups an XCD runs at once (consecutive w after the remap) form
    // a 4 (m) x 8 (n) block of tiles: 12 operand slices shared through its L2
    // per K step instead of 18 for a 16 x 2 column
    int mi, ni;
    if (p.mtiles % kGroupM == 0 && p.ntiles % kGroupN == 0) {
        const int grp = w / (kGroupM * kGroupN), in = w % (kGroupM * kGroupN);
        const int mgroups = p.mtiles / kGroupM;
        mi = (grp % mgroups) * kGroupM + in % kGroupM;
        ni = (grp / mgroups) * kGroupN + in / kGroupM;
    } else {
        mi = w % p.mtiles;
        ni = w / p.mtiles;
    }
    const int64_t m0 = (int64_t)mi * kBM;
    const int64_t n0 = (int64_t)ni * kBNhW;
    const int ktiles = (int)(p.k / BK);

    // DMA geometry: a DMA instruction fills kRowsPerDma consecutive staged rows;
    // lane l -> row + l / (kRB / 16), LDS slot l % (kRB / 16), which holds global
    // chunk slot ^ f(row): every lane group reads one whole row segment. DMA j of
    // wave w: j < kNA -> activation rows from kRowsPerDma (kNA w + j); then kNG
    // gate-row DMAs and kNG up-row DMAs, each wave a quarter of each block.
    //   The three operand blocks -- the m-tile's activation rows, the tile's gate
    // rows, its up rows -- are buffer resources (base and size in SGPRs), and the
    // block of DMA j is fixed by j alone. A DMA address is a per-lane 32-bit
    // offset into its block, fixed for the whole loop, plus the K tile's byte
    // offset in an SGPR: no vector arithmetic per DMA. Every offset stays inside its
    // block: the lane offset within the block's rows, the K tile offset within a row.
    constexpr int kLpr = kRB / 16;  // lanes per staged row
    constexpr int kRpd = T::kRowsPerDma;
    constexpr int kNA = kBM / (kRpd * 4);    // activation DMAs per wave per stage
    constexpr int kNG = kBNhW / (kRpd * 4);  // gate (and up) DMAs per wave per stage
    static_assert(kNA + 2 * kNG == kD, "every staged row has one DMA lane group");
    const int rowb = (int)p.k * 2;  // bytes per operand row (k <= kMaxDmaK)
    const int a_rows = p.m - m0 < kBM ? (int)(p.m - m0) : kBM;
    const ck_rsrc_t rsa = buf_rsrc(p.a + m0 * p.k, (uint32_t)(a_rows * rowb));
    const ck_rsrc_t rsg = buf_rsrc(p.b + n0 * p.k, (uint32_t)(kBNhW * rowb));
    const ck_rsrc_t rsu = buf_rsrc(p.b + (p.n_half + n0) * p.k, (uint32_t)(kBNhW * rowb));
    // staged row of DMA j's first row: within the stage, or (split ring) within
    // its operand's part; and its first row within its operand block
    auto srow0 = [&](int j) __attribute__((always_inline)) {
        if (j < kNA) return kRpd * (kNA * wid + j);
        const int wbase = T::kSplit ? 0 : kBM;
        if (j < kNA + kNG) return wbase + kRpd * (kNG * wid + j - kNA);
        return wbase + kBNhW + kRpd * (kNG * wid + j - kNA - kNG);
    };
    auto brow0 = [&](int j) __attribute__((always_inline)) {
        if (j < kNA) return kRpd * (kNA * wid + j);
        if (j < kNA + kNG) return kRpd * (kNG * wid + j - kNA);
        return kRpd * (kNG * wid + j - kNA - kNG);
    };
    int voff[kD];  // per-lane byte offset of DMA j in its block
#pragma unroll
    for (int j = 0; j < kD; ++j) {
        const int R = srow0(j) + lane / kLpr;  // staged row: its swizzle
        const int coff = ((lane % kLpr) ^ dsw_swz<BK>(R)) * 16;
        int row = brow0(j) + lane / kLpr;
        if (j < kNA && row >= a_rows) row = a_rows - 1;  // rows past m only feed output rows that are not stored
        voff[j] = row * rowb + coff;
    }
    // DMA j of K tile `src` into the stage (or part) at `base`
    auto dma_src = [&](int j, int src, CK_LDS char *base) __attribute__((always_inline)) {
        dma16_buf(j < kNA ? rsa : j < kNA + kNG ? rsg : rsu, voff[j], src * (BK * 2), base + srow0(j) * kRB);
    };
    f32x16 acc[4][WB][2];
#pragma unroll
    for (int ab = 0; ab < 4; ++ab)
#pragma unroll
        for (int gb = 0; gb < WB; ++gb)
#pragma unroll
            for (int gu = 0; gu < 2; ++gu)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[ab][gb][gu][e] = 0.f;

    // DMA j of this wave: K tile `src` into the ring slot of tile `slot`
    auto dma_one = [&](int slot, int src, int j) {
        dma_src(j, src, smem + (slot % kS) * T::kStageBytes);
    };
    // Split ring: part q holds the weights of tile q / 2 (q even) or its
    // activations (q odd) in slot q % 5, so the weight rows of tile t sit in
    // slot 2t % 5 and its activation rows in (2t + 1) % 5.
    // (the part offsets pass through readfirstlane: they stay one SGPR each instead of
    // the compiler distributing the modulo over every per-lane read address)
    auto wslot = [&](int t) { return smem + __builtin_amdgcn_readfirstlane(((2 * t) % 5) * T::kPart); };
    auto aslot = [&](int t) { return smem + __builtin_amdgcn_readfirstlane(((2 * t + 1) % 5) * T::kPart); };
    auto dma_w = [&](int t, int src, int jj) {  // weight DMA jj of tile t
        dma_src(kNA + jj, src, wslot(t));
    };
    auto dma_a = [&](int t, int src, int jj) {  // activation DMA jj of tile t
        dma_src(jj, src, aslot(t));
    };
    constexpr int kLate = kD - T::kEarlyDma;
    constexpr int kSpE = T::kMfmaSub / T::kEarlyDma > 1 ? T::kMfmaSub / T::kEarlyDma : 1;  // MFMAs per early DMA
    constexpr int kSpL = T::kMfmaSub / (kLate > 0 ? kLate : 1) > 1 ? T::kMfmaSub / (kLate > 0 ? kLate : 1) : 1;
    static_assert(kLate <= T::kMfmaSub && T::kEarlyDma <= T::kMfmaSub && T::kEarlyDma > 0,
                  "at most one DMA per MFMA");
    // fragment read r of substep s of the tile in ring slot `slot`: r < 2 WB -> weight
    // block (gb, gu) = (r >> 1, r & 1), r >= 2 WB -> activation block r - 2 WB. Every
    // block starts on a multiple of 32 rows, where the row swizzle repeats, so a
    // read is the slot's (scalar) base + the wave's block offset + an immediate for
    // the block + lsw[s], the lane's offset of (row l32, chunk 2s + hh) in a block.
    int lsw[kNS];
#pragma unroll
    for (int s = 0; s < kNS; ++s) lsw[s] = dsw_off<BK>(l32, 2 * s + hh);
    const int woff = ww * 32 * WB * kRB;  // wave-uniform
    const int aoff = wa * 128 * kRB;
#define CK_GEMM_READ(slot, s, r, WF, XF)                                                                      \
    do {                                                                                                      \
        const CK_LDS char *xa_ = T::kSplit ? aslot(slot)                                                      \
                                           : smem + __builtin_amdgcn_readfirstlane(((slot) % kS) * T::kStageBytes); \
        const CK_LDS char *xw_ = T::kSplit ? wslot(slot) : xa_ + kBM * kRB;                                   \
        if ((r) < 2 * WB)                                                                                     \
            WF[(r) >> 1][(r) & 1] = *reinterpret_cast<const CK_LDS bf16x8 *>(                                  \
                xw_ + woff + (((r) & 1) * kBNhW + ((r) >> 1) * 32) * kRB + lsw[s]);                            \
        else                                                                                                  \
            XF[(r) - 2 * WB] = *reinterpret_cast<const CK_LDS bf16x8 *>(                                      \
                xa_ + aoff + ((r) - 2 * WB) * 32 * kRB + lsw[s]);                                             \
    } while (0)
    // Reads in the order the next substep's MFMAs consume them: MFMA 0 needs weight
    // block 0 and activation block 0, then the other weight blocks one per MFMA,
    // then one activation block every 2 WB MFMAs, so every wait is partial.
    constexpr int kReadOrder[8] = {0, 2 * WB, 1, WB == 2 ? 2 : 3, WB == 2 ? 3 : 4, WB == 2 ? 5 : 5, 6, 7};
    // MFMA i of a substep: (ab, gb, gu) = (i / 2WB, (i / 2) % WB, i % 2)
#define CK_GEMM_MFMA(i, WF, XF)                                                                               \
    acc[(i) / (2 * WB)][((i) >> 1) % WB][(i) & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(                  \
        WF[((i) >> 1) % WB][(i) & 1], XF[(i) / (2 * WB)], acc[(i) / (2 * WB)][((i) >> 1) % WB][(i) & 1], 0, 0, 0)

    // DMA schedule: tile t + kS goes into tile t's slot, freed by the barrier in
    // tile t's last substep; kEarlyDma of its DMAs go out right after that barrier,
    // the rest in the first substep of tile t + 1. A tile index past the end repeats
    // the last tile into a slot nothing reads again, so every tile issues the same
    // DMAs and the vmcnt waits are exact.
    //   Split ring: weights run two tiles ahead, activations one. The weights of
    // tile t + 2 go out in tile t's first substep, into the part tile t - 1's
    // activations left at the barrier of tile t - 1; the activations of tile t + 2
    // in its last substep, into the part of tile t's weights, freed by the barrier
    // just before. At the barrier of tile t only the weights of tile t + 2 may
    // still be in flight.
    // prologue: tiles 0 .. kS-2 and the early DMAs of tile kS - 1 in flight (split:
    // tiles 0 and 1), tile 0 landed
    if constexpr (T::kSplit) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int src = min(t, ktiles - 1);
#pragma unroll
            for (int jj = 0; jj < kD / 2; ++jj) dma_w(t, src, jj);
#pragma unroll
            for (int jj = 0; jj < kD / 2; ++jj) dma_a(t, src, jj);
        }
        wait_vmcnt<kD>();
    } else {
        for (int t = 0; t < kS; ++t)
#pragma unroll
            for (int j = 0; j < kD; ++j)
                if (t < kS - 1 || j < T::kEarlyDma) dma_one(t, min(t, ktiles - 1), j);
        wait_vmcnt<(kS - 2) * kD + T::kEarlyDma>();
    }
    __syncthreads();
    bf16x8 wf[2][WB][2], xf[2][4];
#pragma unroll
    for (int r = 0; r < T::kReads; ++r) CK_GEMM_READ(0, 0, kReadOrder[r], wf[0], xf[0]);
    // Substep s of tile kt: its MFMAs with the next substep's fragment reads (tile
    // kt + 1's first substep after the last) and the DMAs between them, in a fixed
    // order (sched_barrier fences), so the wave issues its reads, address arithmetic
    // and DMAs while the matrix pipe is busy. Before the last substep: tile kt + 1
    // has landed and every read of tile kt is done (vmcnt wait + barrier).
    for (int kt = 0; kt < ktiles; ++kt) {
        const int ta = min(kt + kS - 1, ktiles - 1);  // late DMAs: tile kt + kS - 1
        const int tb = min(kt + kS, ktiles - 1);      // early DMAs: tile kt + kS
        const int t2 = min(kt + 2, ktiles - 1);       // split ring: tile kt + 2
#pragma unroll
        for (int s = 0; s < kNS; ++s) {
            if (s == kNS - 1) {
                // tile kt + 1 has landed once only the DMAs of tiles kt + 2 .. kt + kS - 1
                // (real or repeated; split: the weights of tile kt + 2) remain in flight
                if constexpr (T::kSplit) wait_vmcnt<kD / 2>();
                else wait_vmcnt<(kS - 2) * kD>();
                __syncthreads();
            }
            const int cur = s & 1, nxt = cur ^ 1;
            const int rslot = s == kNS - 1 ? kt + 1 : kt;
            const int rs = s == kNS - 1 ? 0 : s + 1;
#pragma unroll
            for (int i = 0; i < T::kMfmaSub; ++i) {
                CK_GEMM_MFMA(i, wf[cur], xf[cur]);
                if (WB == 2) {
                    if (i % 2 == 0) CK_GEMM_READ(rslot, rs, kReadOrder[i / 2], wf[nxt], xf[nxt]);
                } else {
                    if (i < T::kReads) CK_GEMM_READ(rslot, rs, kReadOrder[i], wf[nxt], xf[nxt]);
                }
                if constexpr (T::kSplit) {
                    // every second MFMA: weights of tile kt + 2 in substep 0,
                    // activations of tile kt + 2 in the last substep
                    if (s == 0 && i % 2 == 1) dma_w(kt + 2, t2, i / 2);
                    if (s == kNS - 1 && i % 2 == 1) dma_a(kt + 2, t2, i / 2);
                } else {
                    // late DMAs spread over substep 0, early ones over the last substep
                    if (s == 0 && i % kSpL == (kSpL > 1 ? 1 : 0) && i / kSpL < kLate)
                        dma_one(kt + kS - 1, ta, T::kEarlyDma + i / kSpL);
                    if (s == kNS - 1 && i % kSpE == (kSpE > 1 ? 1 : 0) && i / kSpE < T::kEarlyDma)
                        dma_one(kt + kS, tb, i / kSpE);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
#undef CK_GEMM_READ
#undef CK_GEMM_MFMA
    // repeated tiles may still be landing in the ring: drain before the
    // workgroup's LDS can be handed to another
    wait_vmcnt<0>();

    // ---- epilogue: lane = activation row l32 of block ab; regs 4c..4c+3 of weight
    // block gb = output columns n0 + ww*64 + gb*32 + 8c + 4hh + 0..3 -------------------
#pragma unroll
    for (int ab = 0; ab < 4; ++ab) {
        const int64_t gm = m0 + wa * 128 + ab * 32 + l32;
        if (gm >= p.m) continue;
#pragma unroll
        for (int gb = 0; gb < WB; ++gb) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int64_t col = n0 + ww * 32 * WB + gb * 32 + 8 * c + 4 * hh;
                const f32x16 &G = acc[ab][gb][0];
                const f32x16 &U = acc[ab][gb][1];
                const float g0 = G[4 * c + 0], g1 = G[4 * c + 1], g2 = G[4 * c + 2], g3 = G[4 * c + 3];
                const float u0 = U[4 * c + 0], u1 = U[4 * c + 1], u2 = U[4 * c + 2], u3 = U[4 * c + 3];
                if (MODE == 1) {
                    const uint2 dv = make_uint2(pack_bf16x2(silu_mul(g0, u0), silu_mul(g1, u1)),
                                                pack_bf16x2(silu_mul(g2, u2), silu_mul(g3, u3)));
                    *reinterpret_cast<uint2 *>(p.d + gm * p.d_stride + col) = dv;
                } else {
                    const uint2 gv = make_uint2(pack_bf16x2(g0, g1), pack_bf16x2(g2, g3));
                    const uint2 uv = make_uint2(pack_bf16x2(u0, u1), pack_bf16x2(u2, u3));
                    uint16_t *crow = p.c + gm * (2 * p.n_half);
                    *reinterpret_cast<uint2 *>(crow + col) = gv;
                    *reinterpret_cast<uint2 *>(crow + p.n_half + col) = uv;
                    if (MODE == 0 || MODE == 5)
                        *reinterpret_cast<uint2 *>(p.d + gm * p.d_stride + col) = gv;
                    else if (MODE == 4)
                        *reinterpret_cast<uint2 *>(p.d + gm * p.d_stride + col) = uv;
                    else if (MODE == 8)
                        *reinterpret_cast<uint2 *>(p.d + gm * p.d_stride + col) = make_uint2(0, 0);
                }
            }
        }
    }
}

// ---- decode-sized activations (M <= 32) --------------------------------------
// With few activation rows the op is bound by the weight stream (2I x K bf16),
// not by MFMA: the 256-row tile above would run I / 128 workgroups (112 at
// I = 14336) with half their DMAs fetching padding, and the bytes they keep in
// flight cap the stream near 2.8 TB/s. Here a workgroup takes 32 gate + 32 up
// weight rows against all activation rows (I / 32 workgroups, two per CU), and
// each of its 4 waves streams a quarter of K straight from global memory into
// MFMA operand registers, several steps ahead; the four partial accumulators
// meet in LDS once at the end.
//   On v_mfma_f32_16x16x32_bf16 four lanes share a row (K groups of 8), so a
//   16-byte-per-lane load covers 16 rows x 64 B: 16 address lines per
//   instruction, half what the 32x32 layout (two lanes per row) needs per weight
//   byte. Per 64-deep K step, lane (row r, group q) loads 32 contiguous bytes of
//   its row, K [64 s + 16 q, +16); MFMA j (of 2) takes the j-th 16 bytes of both
//   operands, i.e. K {64 s + 16 q + 8 j + t}, the same permutation on both sides,
//   hence the exact product. Each wave holds 4 weight tiles (gate/up x 2 blocks of
//   16 rows) per 16-row activation block (NB = 1 up to M = 16, 2 up to M = 32).
//   Activation rows past M load row M - 1: they feed only output rows that are
//   not stored.
constexpr int kSThreads = 256;  // 4 waves, wave w reduces K quarter w
constexpr int kSN = 32;         // gate rows (and as many up rows) per workgroup
constexpr int kSStep = 64;      // K per pipeline step
constexpr int kSDepth = 4;      // steps whose loads are in flight per wave (NB = 1)
constexpr int kSMaxM = 32;

template <int MODE, int NB>  // NB = 16-row activation blocks (M <= 16 NB)
__global__ __launch_bounds__(kSThreads) void gateup_skinny16_kernel(GemmArgs p) {
    typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
    // [wave][weight tile: gate b0, gate b1, up b0, up b1][activation block][register][lane]
    __shared__ float red[4][4][NB][4][64];
    const int tid = threadIdx.x;
    const int wid = tid >> 6;
    const int lane = tid & 63;
    const int r16 = lane & 15;
    const int q4 = lane >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * kSN;
    const int64_t kq = p.k / 4;
    const int steps = (int)(kq / kSStep);
    const int64_t koff = wid * kq + 16 * q4;
    const uint4 *wp[4];  // gate rows n0 + 16 b + r16, up rows n_half + n0 + 16 b + r16
#pragma unroll
    for (int t = 0; t < 4; ++t)
        wp[t] = reinterpret_cast<const uint4 *>(p.b + ((t < 2 ? 0 : p.n_half) + n0 + 16 * (t & 1) + r16) * p.k + koff);
    const uint4 *xp[NB];
#pragma unroll
    for (int ab = 0; ab < NB; ++ab) {
        const int64_t arow = 16 * ab + r16 < p.m ? 16 * ab + r16 : p.m - 1;
        xp[ab] = reinterpret_cast<const uint4 *>(p.a + arow * p.k + koff);
    }
    constexpr int kStepVec = kSStep * 2 / 16;  // uint4 per row per step (8)
    constexpr int kDepth = NB == 1 ? kSDepth : 3;  // registers: 48 per step at NB = 2

    uint4 W[kDepth][4][2], X[kDepth][NB][2];
    f32x4_t acc[4][NB];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int ab = 0; ab < NB; ++ab)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[t][ab][e] = 0.f;
#define CK_SKINNY16_LOAD(slot, st)                                          \
    do {                                                                    \
        const int64_t o_ = (int64_t)(st) * kStepVec;                        \
        _Pragma("unroll") for (int j_ = 0; j_ < 2; ++j_) {                  \
            _Pragma("unroll") for (int t_ = 0; t_ < 4; ++t_) W[slot][t_][j_] = wp[t_][o_ + j_]; \
            _Pragma("unroll") for (int b_ = 0; b_ < NB; ++b_) X[slot][b_][j_] = xp[b_][o_ + j_]; \
        }                                                                   \
    } while (0)
#pragma unroll
    for (int d = 0; d < kDepth; ++d)
        if (d < steps) CK_SKINNY16_LOAD(d, d);
    for (int s = 0; s < steps; s += kDepth) {
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            if (s + d < steps) {
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int ab = 0; ab < NB; ++ab) {
                        const bf16x8 xf = __builtin_bit_cast(bf16x8, X[d][ab][j]);
#pragma unroll
                        for (int t = 0; t < 4; ++t)
                            acc[t][ab] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                __builtin_bit_cast(bf16x8, W[d][t][j]), xf, acc[t][ab], 0, 0, 0);
                    }
                if (s + d + kDepth < steps) CK_SKINNY16_LOAD(d, s + d + kDepth);
            }
        }
    }
#undef CK_SKINNY16_LOAD

#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int ab = 0; ab < NB; ++ab)
#pragma unroll
            for (int e = 0; e < 4; ++e) red[wid][t][ab][e][lane] = acc[t][ab][e];
    __syncthreads();
    // thread -> (weight tile pair b: gate b and up b, activation block ab, accumulator
    // lane l): output row 16 ab + l % 16, columns n0 + 16 b + 4 (l / 16) + 0..3
    if (tid >= 2 * NB * 64) return;
    const int b = tid / (NB * 64);
    const int ab = (tid / 64) % NB;
    const int l = tid & 63;
    const int64_t gm = 16 * ab + (l & 15);
    if (gm >= p.m) return;
    float g[4], u[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        g[i] = red[0][b][ab][i][l] + red[1][b][ab][i][l] + red[2][b][ab][i][l] + red[3][b][ab][i][l];
        u[i] = red[0][2 + b][ab][i][l] + red[1][2 + b][ab][i][l] + red[2][2 + b][ab][i][l] + red[3][2 + b][ab][i][l];
    }
    const int64_t col = n0 + 16 * b + 4 * (l >> 4);
    if (MODE == 1) {
        *reinterpret_cast<uint2 *>(p.d + gm * p.d_stride + col) =
            make_uint2(pack_bf16x2(silu_mul(g[0], u[0]), silu_mul(g[1], u[1])),
                       pack_bf16x2(silu_mul(g[2], u[2]), silu_mul(g[3], u[3])));
    } else {
        const uint2 gv = make_uint2(pack_bf16x2(g[0], g[1]), pack_bf16x2(g[2], g[3]));
        const uint2 uv = make_uint2(pack_bf16x2(u[0], u[1]), pack_bf16x2(u[2], u[3]));
        uint16_t *crow = p.c + gm * (2 * p.n_half);
        *reinterpret_cast<uint2 *>(crow + col) = gv;
        *reinterpret_cast<uint2 *>(crow + p.n_half + col) = uv;
        if (MODE == 0 || MODE == 5)
            *reinterpret_cast<uint2 *>(p.d + gm * p.d_stride + col) = gv;
        else if (MODE == 4)
            *reinterpret_cast<uint2 *>(p.d + gm * p.d_stride + col) = uv;
        else if (MODE == 8)
            *reinterpret_cast<uint2 *>(p.d + gm * p.d_stride + col) = make_uint2(0, 0);
    }
}

// mode 3: d = workspace[:, :I] (epilogue-only rung), 8 columns per thread. The
// workspace and d are 8-byte aligned (the ABI contract) and d_stride % 4 == 0,
// so both sides move as two 8-byte words.
__global__ __launch_bounds__(256) void gate_window_copy_kernel(const uint16_t *c, uint16_t *d, int64_t m,
                                                               int64_t n_half, int64_t d_stride) {
    const int64_t per_row = n_half / 8;
    const int64_t total = m * per_row;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / per_row, q = i - r * per_row;
        const uint2 *src = reinterpret_cast<const uint2 *>(c + r * 2 * n_half + q * 8);
        const uint2 v0 = src[0], v1 = src[1];
        uint2 *dst = reinterpret_cast<uint2 *>(d + r * d_stride + q * 8);
        dst[0] = v0;
        dst[1] = v1;
    }
}

constexpr int64_t kNumCus = 256;  // MI355X

template <int MODE, int WB, int BK>
int launch_dma(GemmArgs p, hipStream_t s) {
    using T = DmaTile<WB, BK>;
    p.ntiles = (int)(p.n_half / T::kNh);
    const int64_t grid = (int64_t)p.mtiles * p.ntiles;
    static std::atomic<uint64_t> lds_set{0};
    int rc = ensure_dynamic_lds(reinterpret_cast<const void *>(&gateup_dma_kernel<MODE, WB, BK>), T::kLdsBytes,
                                lds_set);
    if (rc != CK_OK) return rc;
    hipLaunchKernelGGL((gateup_dma_kernel<MODE, WB, BK>), dim3((unsigned)grid), dim3(kDThreads), T::kLdsBytes, s,
                       p);
    CK_RETURN_LAUNCH();
}

template <int MODE>
int launch_gemm(const GemmArgs &p, hipStream_t s) {
    if (p.m <= kSMaxM && p.k % (4 * kSStep) == 0) {
        if (p.m <= 16)
            hipLaunchKernelGGL((gateup_skinny16_kernel<MODE, 1>), dim3((unsigned)(p.n_half / kSN)), dim3(kSThreads),
                               0, s, p);
        else
            hipLaunchKernelGGL((gateup_skinny16_kernel<MODE, 2>), dim3((unsigned)(p.n_half / kSN)), dim3(kSThreads),
                               0, s, p);
        CK_RETURN_LAUNCH();
    }
    const int64_t grid = (int64_t)p.mtiles * p.ntiles;
    if (p.k % 32 == 0 && p.k <= kMaxDmaK) {
        // The half-width tile (WB = 1) does about 3/4 of the full tile's work per
        // workgroup (its DMA bytes; half the MFMAs) with twice the workgroups: it
        // wins when it needs fewer than 4/3 as many rounds of resident workgroups
        // (one per CU), i.e. when the full-width grid leaves CUs idle.
        const int64_t rounds2 = (grid + kNumCus - 1) / kNumCus;
        const int64_t rounds1 = (2 * grid + kNumCus - 1) / kNumCus;
        const bool half = 3 * rounds1 < 4 * rounds2;
        // 128-byte staged rows (whole cache lines per DMA lane group) when K allows
        if (p.k % 64 == 0) return half ? launch_dma<MODE, 1, 64>(p, s) : launch_dma<MODE, 2, 64>(p, s);
        return half ? launch_dma<MODE, 1, 32>(p, s) : launch_dma<MODE, 2, 32>(p, s);
    }
    static std::atomic<uint64_t> lds_set_g{0};
    int rc = ensure_dynamic_lds(reinterpret_cast<const void *>(&gateup_general_kernel<MODE>), 2 * kTileBytes,
                                lds_set_g);
    if (rc != CK_OK) return rc;
    hipLaunchKernelGGL((gateup_general_kernel<MODE>), dim3((unsigned)grid), dim3(kThreads), 2 * kTileBytes, s, p);
    CK_RETURN_LAUNCH();
}

}  // namespace
}  // namespace ck

using namespace ck;

extern "C" int ck_f3_gateup_epilogue(const void *a, const void *b, void *workspace, void *d, int64_t m,
                                     int64_t n_half, int64_t k, int64_t mode, int64_t d_stride, void *stream) {
    if (m < 1 || k < 64 || k % 16 != 0 || n_half < kBNh || n_half % kBNh != 0) return CK_E_INVALID_ARG;
    if (!(mode >= 0 && mode <= 5) && mode != 7 && mode != 8) return CK_E_INVALID_ARG;
    if (d_stride < n_half || d_stride % 4 != 0) return CK_E_INVALID_ARG;
    if (!a || !b || !d) return CK_E_NULL_PTR;
    if (mode != 1 && !workspace) return CK_E_NULL_PTR;
    // operand rows are fetched 16 bytes at a time, results stored 8 bytes at a time
    if (reinterpret_cast<uintptr_t>(a) % 16 != 0 || reinterpret_cast<uintptr_t>(b) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(d) % 8 != 0 || reinterpret_cast<uintptr_t>(workspace) % 8 != 0)
        return CK_E_INVALID_ARG;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (mode == 3) {
        int64_t blocks = (m * (n_half / 8) + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(gate_window_copy_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                           static_cast<const uint16_t *>(workspace), static_cast<uint16_t *>(d), m, n_half,
                           d_stride);
        CK_RETURN_LAUNCH();
    }
    GemmArgs p;
    p.a = static_cast<const uint16_t *>(a);
    p.b = static_cast<const uint16_t *>(b);
    p.c = static_cast<uint16_t *>(workspace);
    p.d = static_cast<uint16_t *>(d);
    p.m = m;
    p.n_half = n_half;
    p.k = k;
    p.d_stride = d_stride;
    p.mtiles = (int)((m + kBM - 1) / kBM);
    p.ntiles = (int)(n_half / kBNh);
    if ((int64_t)p.mtiles * p.ntiles > 0x7FFFFFFF) return CK_E_INVALID_ARG;
    switch (mode) {
        case 0: return launch_gemm<0>(p, s);
        case 1: return launch_gemm<1>(p, s);
        case 2: return launch_gemm<2>(p, s);
        case 4: return launch_gemm<4>(p, s);
        case 5: return launch_gemm<5>(p, s);
        case 7: return launch_gemm<7>(p, s);
        default: return launch_gemm<8>(p, s);
    }
}
