// suffix_decode.hip - per-sequence paged decode attention over each sequence's
// own suffix pages (cascade stage 2) on gfx950: the stand-alone op and the
// fused cascade's streaming waves compute their windows on the matrix cores
// (the fused kernel above 4 query heads per group on the vector ALU).
//
// Role: replaces the closed CANN op npu_fused_infer_attention_score_v2 the
// reference calls for stage 2 (ascend-kernel/README.md:186-197): one query
// token per sequence, GQA, paged K/V, bf16 O plus a compact fp32 LSE that
// lse_merge folds into the stage-1 result. An empty suffix (kv length 0)
// yields O = 0, LSE = -inf, which the merge treats as weight 0.
//
// Arithmetic: S = q k^T * scale in fp32, online softmax in the log2 domain,
// P at fp32 precision (the matrix-core body feeds P as two bf16 terms whose
// sum is P within 2^-16) and fp32 accumulation, O = acc / l, LSE = ln(l) + max.
//
// MI355X design: HBM-bound streaming with a persistent, balanced grid and few
// instructions per byte (at 8 TB/s a CU receives about 15 bytes per cycle; a
// vector-ALU body of ~190 instructions per 32-token window was bound by its
// own issue, the matrix-core body takes ~90).
// * Suffix lengths vary widely (geometric in the benchmark), so the work is cut
//   into windows of 8 tokens per streaming wave (32 tokens on 4 waves) of one
//   sequence (the last window of a sequence may be short), and workgroup (kv
//   head group g, chunk c) takes the c-th 1/P of the list of all windows,
//   crossing sequence boundaries: every workgroup streams the same number of
//   windows and starts once.
// * Start-up: lengths -> window prefix sums (block scan in LDS), then a table
//   of the workgroup's windows (page id, valid tokens, sequence, segment
//   start/end) built in parallel in one round trip that also copies the first
//   q rows into LDS. The streaming loop reads the table from LDS; no load in
//   the loop depends on another load.
// * Two paged K/V layouts: NHD [blocks, 128, kv_heads, 128] (the stage-1 pool)
//   and BNSD [blocks, kv_heads, 128, 128] (the layout the reference's stage-2
//   op reads, ascend-kernel/README.md:182-183), so a BNSD pool needs no
//   transposing copy. A page, a token and a kv head are three strides.
// * K and V go straight from HBM into registers by buffer loads, no barrier in
//   the streaming loop. Each window gets a buffer descriptor (its first row as
//   base, its valid rows as range) built with scalar instructions, so a lane's
//   address is a fixed offset; rows past the sequence's end fall outside the
//   range (zeros, no bytes moved), and an invalid page id gets an empty range:
//   its rows read as zeros, the semantics of the pool's unmapped pages.
// * Token-major body (the stand-alone kernel, the fused kernel up to 4 heads):
//   scores S^T = K q^T and values O^T += V^T P^T on 16x16 bf16 MFMAs, V^T
//   through a per-wave LDS slot read back transposed (suffix_stream_body gives
//   the lane layouts). Dims-major body (the fused kernel above 4 heads): 8
//   packed bf16 dot products and a DPP sum per score, p through a per-wave LDS
//   row, 4 value FMAs per token and head. Either way the running max moves only
//   when a score exceeds it by more than 2^kTau (a wave-uniform branch), so
//   rescaling is rare; any reference point gives the same O and LSE.
// * Closing a sequence never stops the stream: each wave writes its partial
//   (O, m, l) into the segment's slot of an LDS exchange ring and counts itself
//   in with an LDS atomic. Token-major: once all partials are in, each wave
//   merges its share into an LDS stash (one wave doing the whole merge fell
//   behind the others by it at every close), written out after the phase's
//   loop. Dims-major: the last wave in merges and writes the result while the
//   others go on. A wave waits for a ring slot only if it runs a whole ring
//   ahead of the slowest wave, which itself never waits, so every wait ends.
// * Cascade (stage 1 + suffix + merge): one fused kernel, one workgroup per CU.
//   Waves 0-3 run the stage-1 body (MFMA, LDS tiles: matrix cores and LDS),
//   waves 4-7 stream suffix windows; each role synchronises only its own four
//   waves through an LDS counter barrier, so the two run side by side instead
//   of one kernel after the other, and a small epilogue kernel merges the two
//   results.
// * The range is processed in phases of at most 512 windows and 8 segments.
//   A phase starts with one round trip that fills the window table and copies
//   the q rows of its segments into LDS; the phase's loop has no barrier.
// * A segment that is a whole sequence writes bf16 O and the LSE directly; a
//   sequence cut by a chunk boundary leaves fp32 partials that a small fix-up
//   kernel folds (it also writes O = 0, LSE = -inf for empty suffixes).
#include <type_traits>

#include "ck_common.h"
#include "ck_internal.h"

// Bounded waits of this file's kernels that ran out (a broken invariant, never
// expected): counted here, read and reset by ck_wait_giveups.
static __device__ unsigned int g_wait_giveups;

namespace ck {
namespace {

// Calls f(std::integral_constant<int, I>{}) for I = 0 .. N - 1 (unrolled, I usable
// as a compile-time index).
template <int I, int N, class F>
__device__ __forceinline__ void static_for_from(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for_from<I + 1, N>(f);
    }
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
    static_for_from<0, N>(f);
}

constexpr int kD = 128;
constexpr int kPage = 128;
constexpr int kMaxGroup = 8;
constexpr int kMaxBatch = 1024;     // sequences per launch (prefix sums in LDS)
constexpr int kQSlots = 8;          // segments per phase (their q rows in LDS)
constexpr int kTable = 512;         // windows per table phase
constexpr float kTau = 8.0f;        // log2 headroom before the running max moves
constexpr uint32_t kOob = 0x80000000u;  // a buffer offset past every window's range
constexpr int kRsrcFlags = 0x00020000;  // buffer descriptor word 3 for gfx9 raw loads

// windows of loads in flight per streaming wave: token-major, 2 (24 registers
// per window and lane; 3 and 4 measured slower in the fused kernel), 1 in the
// stand-alone kernel above 4 heads (one workgroup per CU there: 1 measured
// faster than 2 and 3); dims-major (the fused kernel above 4 heads), 4.
constexpr int kTokDepth = 2;
constexpr int kFusedDepth = 4;
// Share of each fused workgroup's suffix windows that its streaming waves take
// (in 1/256); the stage-1 waves take the rest after their stage-1 unit.
constexpr int kFusedSplit = 208;
static_assert(kFusedSplit >= 128 && kFusedSplit < 256, "ChunkMap::none_empty assumes a share in [1/2, 1)");

// LDS layout (bytes) of the stream body for G query heads per group and NW waves;
// TOK (the token-major body) adds the merged results of a phase's segments,
// held until the phase's window loop is done, and each wave's V transpose slot:
// 8 token rows of 256 bytes at a 288-byte pitch (the pitch puts the 4 rows of a
// transpose read in distinct bank groups).
constexpr int kVtPitch = 288;
template <int G, int NW, bool TOK = false>
struct SfxLds {
    static constexpr int kCw = 0;                                        // int cw[kMaxBatch + 1]
    static constexpr int kLen = ((kMaxBatch + 1) * 4 + 15) / 16 * 16;   // int len[kMaxBatch]
    static constexpr int kWtot = kLen + kMaxBatch * 4;                   // int wtot[NW]
    static constexpr int kTab = kWtot + 64;               // int pair tab[kTable + 8] (8 padding entries)
    static constexpr int kPw = kTab + (kTable + 8) * 8;  // float pw[NW][8][8] p rows (dims-major)
    static constexpr int kQs = kPw + NW * 8 * 8 * 4;                     // bf16 q[kQSlots][G][kD]
    static constexpr int kX = TOK || G <= 4 ? 2 : 1;                     // exchange ring slots
    static constexpr int kXo = kQs + kQSlots * G * kD * 2;               // float xo[kX][NW][G][kD]
    static constexpr int kXml = kXo + kX * NW * G * kD * 4;              // float xml[kX][NW][G][2]
    static constexpr int kXsync = kXml + kX * NW * G * 2 * 4;            // int cnt[kX], gen[kX]
    static constexpr int kBar = kXsync + 2 * kX * 4;                     // int bar[2] (group barrier)
    static constexpr int kSo = (kBar + 8 + 15) / 16 * 16;                // float so[kQSlots][G][kD] (TOK)
    static constexpr int kSl = kSo + (TOK ? kQSlots * G * kD * 4 : 0);   // float sl[kQSlots][G]
    static constexpr int kSb = kSl + (TOK ? kQSlots * G * 4 : 0);        // int sb[kQSlots]
    static constexpr int kVt = (kSb + (TOK ? kQSlots * 4 : 0) + 15) / 16 * 16;  // char vt[NW][8][kVtPitch] (TOK)
    static constexpr int kBytes = kVt + (TOK ? NW * 8 * kVtPitch : 0);
    static_assert(kTab % 16 == 0 && kPw % 16 == 0 && kQs % 16 == 0 && kXo % 16 == 0 && kXml % 8 == 0 &&
                      kSo % 16 == 0,
                  "aligned LDS rows");
};

// window table entry: [0] = page id (-1: not a valid page), [1] = packed fields
__device__ __forceinline__ int tab_tv(int y) { return y & 127; }  // valid tokens 1 .. 64
__device__ __forceinline__ bool tab_first(int y) { return (y >> 7) & 1; }
__device__ __forceinline__ bool tab_last(int y) { return (y >> 8) & 1; }
__device__ __forceinline__ int tab_sub(int y) { return (y >> 9) & 3; }  // the window's quarter/half of its page
__device__ __forceinline__ int tab_b(int y) { return y >> 11; }


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
    int chunks;  // chunks of the window list per kv head group
    int split;   // 0: equal chunks; else chunk pairs, the first taking split/256 (ChunkMap)
    float scale_log2;
};

// Window ranges of the chunks of one kv head group (W windows): chunk c covers
// [lo(c), lo(c + 1)). split == 0: P equal chunks, lo(c) = c W / P. split > 0 (P
// even): chunks 2j and 2j + 1 share the j-th of P / 2 equal ranges, the first
// taking split / 256 of it (the fused cascade kernel's two roles on one CU).
// floor(x / d) for 0 <= x < 2^52, 1 <= d < 2^31 (here x <= W P with W < 2^31
// windows and P <= 2^20 chunks) from one IEEE double division: with
// n = floor(x / d), a quotient that is not the integer n is at most
// n + 1 - 1 / d, and rounding moves it up by at most (n + 1) 2^-53 < 1 / d
// (as (n + 1) d <= x + d < 2^53), so it truncates to n; an integer quotient is
// exact. A 64-bit integer division would expand to a few hundred scalar
// instructions per use, inline between the hot blocks of the kernels that map
// windows to chunks (the epilogue was 85% such code and missed the
// instruction cache on 6% of its fetches).
__device__ __forceinline__ int64_t div_nonneg(int64_t x, int64_t d) {
    return (int64_t)((double)x / (double)d);
}

struct ChunkMap {
    int64_t W;
    int P;
    int split;
    __device__ __forceinline__ int64_t lo(int c) const {
        if (split == 0) return div_nonneg((int64_t)c * W, P);
        const int h = P >> 1, j = c >> 1;
        const int64_t a = div_nonneg((int64_t)j * W, h);
        if ((c & 1) == 0) return a;
        return a + (((div_nonneg((int64_t)(j + 1) * W, h) - a) * split) >> 8);
    }
    // the chunk that owns window p < W
    __device__ __forceinline__ int owner(int64_t p) const {
        if (split == 0) return (int)div_nonneg((p + 1) * P - 1, W);
        const int j = (int)div_nonneg((p + 1) * (P >> 1) - 1, W);
        return 2 * j + (p >= lo(2 * j + 1) ? 1 : 0);
    }
    __device__ __forceinline__ bool empty(int c) const { return lo(c) == lo(c + 1); }
    // No chunk is empty once there are at least as many windows as chunks: equal
    // chunks then hold >= 1 window each, and each pair's range holds >= 2, of which
    // a share split / 256 in [1/2, 1) leaves >= 1 to either chunk. (Saves the
    // divisions of empty(), which dominated the fix-up's and epilogue's time.)
    __device__ __forceinline__ bool none_empty() const { return W >= P; }
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// Every control used below (quad_perm, row_half_mirror, row_ror) reads a lane of
// the same 16-lane row, so bound_ctrl never applies; setting it lets the
// compiler fold the move into the consuming add (v_add_f32_dpp).
#define CK_DPP(x, ctrl) __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), ctrl, 0xF, 0xF, true))

// x[l] op x[l ^ 16] and x[l] op x[l ^ 32] through v_permlane16_swap /
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
// Sum / max over the 8 lanes l, l^8, l^16, ..., l^56 (the token slots of a wave).
__device__ __forceinline__ float sum_slots(float x) {
    x += CK_DPP(x, 0x128);  // row_ror:8: the other 8 of the 16-lane row
    return sum_xor32(sum_xor16(x));
}
__device__ __forceinline__ float max_slots(float x) {
    x = fmaxf(x, CK_DPP(x, 0x128));
    return max_xor32(max_xor16(x));
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                           false);
}
// 16-dim bf16 dot product: one chain of 8 (the callers interleave one chain per
// query head, which covers the chain's latency; two chains per head cost a
// second zero-initialised accumulator and an add)
__device__ __forceinline__ float dot16(const u32x4 &k0, const u32x4 &k1, const u32x4 &q0, const u32x4 &q1) {
    // the chain's first product takes its zero as an inline constant (the
    // compiler materialises the zero in a register for the tied-accumulator form)
    float d;
    asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(d) : "v"(k0[0]), "v"(q0[0]));
#pragma unroll
    for (int i = 1; i < 4; ++i) d = dot2(k0[i], q0[i], d);
#pragma unroll
    for (int i = 0; i < 4; ++i) d = dot2(k1[i], q1[i], d);
    return d;
}

__device__ __forceinline__ int64_t clamp_len(const SuffixArgs &a, int64_t kvl) {
    const int64_t lim = a.bt_cols * kPage;
    if (kvl > lim) kvl = lim;
    if (kvl > a.kv_cap) kvl = a.kv_cap;
    if (a.num_blocks <= 0) kvl = 0;
    return kvl < 0 ? 0 : kvl;
}

// The stream body on NW waves (thread tid of the group's NW * 64) as workgroup lb
// of a grid of a.kv_heads * a.chunks, with the group's LDS at smem and its own
// barrier. Windows hold 8 NW tokens.
//
// Two bodies:
// * TOK = false (dims-major, vector ALU; the fused kernel above 4 heads): lane
//   (t, c) holds token t and dims 8c .. 8c+7 and 64+8c .. 64+8c+7 of K; lane
//   (hf, dd) holds dims 4dd .. 4dd+3 of 4 tokens of V, p reaches it through a
//   per-wave LDS row and q is read from LDS per window. 4 accumulators per head.
// * TOK = true (token-major on the matrix cores, 4 waves): a wave owns 8
//   tokens of every window, and lane (g, n) = (lane / 16, lane % 16):
// * S^T = K q^T on v_mfma_f32_16x16x32_bf16: A = K, row n = token n of the wave's
//   8 (rows 8-15 read nothing: zeros), dims 32 s + 8 g .. + 7 at step s, straight
//   from global memory; B = q of head n, the same dims. The result puts token
//   4 g + r, head n in register r of lane (g, n); lanes of rows 8-15 (g >= 2) and
//   of heads n >= G get score -inf through the scale's addend, hence p = 0.
// * O^T += V^T P^T on v_mfma_f32_16x16x16_bf16, one 16-dim tile of O per MFMA: B =
//   P^T is the score layout itself (lane (g, n): tokens 4 g .. 4 g + 3 of head n),
//   and A = V^T comes from the V rows through the wave's LDS slot by
//   ds_read_b64_tr_b16 (lane (g, n): dim n of the tile, tokens 4 g .. 4 g + 3).
//   P enters as two bf16 terms, hi = p truncated and lo = p - hi rounded (|p - hi|
//   < 2^-7 p, so p = hi + lo within 2^-16 p): fp32 P for the arithmetic's purposes.
// * The softmax state of head n sits in lane (g, n), the same for every g: the
//   running max is reduced over the 4 groups when it moves, the row sum when the
//   segment closes, and O^T needs no reduction (the MFMA summed the tokens).
// * The merged result of a segment waits in an LDS stash, and the waves write a
//   phase's results out together after its window loop: a store in the loop
//   would count in the same vmcnt as the window loads, so every later wait of
//   the merging wave would also wait for its acknowledgement (or for loads
//   issued after it), a stall of about a round trip per merge.
//
// Two bodies on one CU may share one scan: the body given scan_src (the other
// body's LDS) skips its own, waits until scan_flag is set and reads the other's
// lengths and window prefix sums; the body given only scan_flag sets it once its
// scan is complete.
template <int G, int NW, int D, bool TOK, class Bar>
__device__ __forceinline__ void suffix_stream_body(const SuffixArgs &a, CK_LDS char *smem, int lb, int tid,
                                                   const Bar &bar, CK_LDS int *scan_flag = nullptr,
                                                   const CK_LDS char *scan_src = nullptr) {
    static_assert(!TOK || NW == 4, "token-major body: 4 waves");
    static_assert(D + 1 <= 8, "table padding: D + 1 entries past a phase");
    constexpr int NB = D + 1;  // register ring slots: D windows in flight + the one in use
    constexpr int kThr = NW * 64;
    constexpr int kWin = 8 * NW;         // tokens per window
    constexpr int kWpp = kPage / kWin;   // windows per page
    using L = SfxLds<G, NW, TOK>;
    CK_LDS int *cw = (CK_LDS int *)((scan_src ? scan_src : smem) + L::kCw);
    CK_LDS int *len = (CK_LDS int *)((scan_src ? scan_src : smem) + L::kLen);
    CK_LDS int *wtot = (CK_LDS int *)(smem + L::kWtot);
    CK_LDS i32x2 *tab = (CK_LDS i32x2 *)(smem + L::kTab);
    CK_LDS char *qs = smem + L::kQs;
    constexpr int R = L::kX;
    CK_LDS float *xo = (CK_LDS float *)(smem + L::kXo);
    CK_LDS float *xml = (CK_LDS float *)(smem + L::kXml);
    CK_LDS int *xcnt = (CK_LDS int *)(smem + L::kXsync);  // waves counted into each slot
    CK_LDS int *xgen = xcnt + R;                             // merges completed in each slot
    CK_LDS float *so = (CK_LDS float *)(smem + L::kSo);      // TOK: merged O of the phase's segments
    CK_LDS float *sl = (CK_LDS float *)(smem + L::kSl);      // TOK: their LSE
    CK_LDS int *sb = (CK_LDS int *)(smem + L::kSb);          // TOK: their sequence

    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int t = lane >> 3;  // K: token slot, token 8 wid + t of each window
    const int c = lane & 7;   // K: dims 8c .. 8c+7 and 64+8c .. 64+8c+7
    const int hf = lane >> 5; // V: tokens hf, 2 + hf, 4 + hf, 6 + hf of the wave's 8
    const int dd = lane & 31; // V: dims 4 dd .. 4 dd + 3
    const int g = lb % a.kv_heads;  // kv head group: query heads g * G .. + G
    const int chunk = lb / a.kv_heads;
    const int gk = g / a.kv_sub;            // the physical kv head they read

    if (tid < R) {
        xcnt[tid] = 0;
        xgen[tid] = 0;
    }

    // ---- lengths and window prefix sums (kPer sequences per thread, block scan) ----
    if (scan_src == nullptr) {
        constexpr int kPer = kMaxBatch / kThr;
        // every load goes out before any is used (one round trip, not kPer): the
        // index is clamped into the batch, and entries past it are dropped below
        int64_t raw[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) raw[j] = a.kv_seqlens[min(kPer * tid + j, a.batch - 1)];
        int lv[kPer];
        int local = 0;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = kPer * tid + j;
            const int ln = i < a.batch ? (int)clamp_len(a, raw[j]) : 0;
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
        bar.sync();
        int wave_off = 0;
        for (int ww = 0; ww < wid; ++ww) wave_off += wtot[ww];
        int run = wave_off + x - local;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = kPer * tid + j;
            run += lv[j];
            if (i < a.batch) cw[i + 1] = run;
        }
        if (tid == 0) cw[0] = 0;
        bar.sync();
        if (lb == 0)
            for (int i = tid; i <= a.batch; i += kThr) a.cw_out[i] = cw[i];
        if (scan_flag != nullptr && tid == 0) *(volatile CK_LDS int *)scan_flag = 1;  // after the barrier above
    } else {
        // the other body's scan (bounded: it always completes, long before this
        // bound; a wait that runs out is counted)
        int spin = 0;
        for (; *(volatile CK_LDS int *)scan_flag == 0 && spin < (1 << 22); ++spin) __builtin_amdgcn_s_sleep(1);
        if (spin == (1 << 22)) count_giveup(&g_wait_giveups);
    }

    const int W = cw[a.batch];
    const ChunkMap cm{W, a.chunks, a.split};
    const int w0 = (int)cm.lo(chunk);
    const int w1 = (int)cm.lo(chunk + 1);
    if (w0 >= w1) return;  // uniform over the workgroup

    // ---- q rows: the s-th segment of a phase in slot s ------------------------------
    // The q rows of one sequence are G * 256 contiguous bytes: one or two wave DMAs.
    auto dma_q = [&](int bq, int slot) {
#pragma unroll
        for (int u0 = 0; u0 < G * 16; u0 += 64) {
            if (u0 + lane < G * 16)
                dma16(a.q + ((int64_t)bq * a.num_heads + g * G) * kD + (u0 + lane) * 8,
                      qs + slot * G * (kD * 2) + u0 * 16);
        }
    };
    // Largest b in [0, batch] with cw[b] <= x: two ballots over the wave's lanes
    // (a stride-S sample of cw, then the S entries after the last sample <= x)
    // instead of a binary search of ~10 dependent LDS reads.
    auto find_seq = [&](int x) {
        const int S = (a.batch + 64) / 64;  // 64 S > batch
        const uint64_t m1 = __builtin_amdgcn_ballot_w64(cw[min(lane * S, a.batch)] <= x);
        const int base = (__builtin_popcountll(m1) - 1) * S;  // cw is nondecreasing, cw[0] = 0 <= x
        const uint64_t m2 = __builtin_amdgcn_ballot_w64(lane < S && cw[min(base + lane, a.batch)] <= x);
        return base + __builtin_popcountll(m2) - 1;
    };

    // ---- per-lane constants ------------------------------------------------------------
    const int64_t tokb = a.tok_stride * 2;                      // bytes between token rows
    const uint32_t koff = (uint32_t)((8 * wid + t) * tokb + c * 16);   // K byte offset in a window
    const uint32_t voff = (uint32_t)((8 * wid + hf) * tokb + dd * 8);  // dims-major V byte offset
    const uint32_t win_bytes = (uint32_t)(kWin * tokb);          // a window's buffer range
    const char *kbase = reinterpret_cast<const char *>(a.k) + (int64_t)gk * a.head_off * 2;
    const char *vbase = reinterpret_cast<const char *>(a.v) + (int64_t)gk * a.head_off * 2;
    const int64_t pgb = a.page_stride * 2;
    const uint32_t pg32 = (uint32_t)pgb, win32 = win_bytes, tok32 = (uint32_t)tokb;  // token-major addressing
    // token-major body: lane (mg, mn); its K rows (token 8 wid + mn, 16 bytes at
    // 64 s + 16 mg for step s; rows 8-15 read nothing), its V bytes (lane (t, c):
    // token t, bytes 16 c and 128 + 16 c, at koff) in the wave's LDS slot, read
    // back transposed (tile T at + 32 T), and the addend of its scores (-inf: a
    // padding row or head)
    const int mn = lane & 15, mg = lane >> 4;
    const uint32_t kfoff = mn < 8 ? (uint32_t)((8 * wid + mn) * tokb + 16 * mg) : kOob;
    CK_LDS char *vt = smem + L::kVt + wid * 8 * kVtPitch;
    const int vwo = t * kVtPitch + 16 * c;
    const int vro = (4 * (mg & 1) + (mn >> 2)) * kVtPitch + 8 * (mn & 3);
    const float sbias = (mg < 2 && mn < G) ? 0.f : -INFINITY;

    float m[G], l[G], acc[G][4];  // dims-major: per head, 4 value accumulators
    // token-major: the O^T tiles (dims 16 T + 4 mg + r of head mn), head mn's
    // softmax state (m; m + kTau, the rescale trigger; the exponent offset, m or
    // 0 while m = -inf; this lane's share of the row sum), q fragments, and the
    // P^T operand (hi, lo) of the pending window
    f32x4 oacc[8];
    float m1, mt1, mz1, l1;
    u32x4 qf[4];
    uint32_t ph[2], pl[2];
    int nclose = 0;  // segments closed so far (exchange ring position)
    int qslot = 0;   // segment of the current phase
    u32x4 kbuf[NB][TOK ? 4 : 2];
    using VSlot = std::conditional_t<TOK, u32x4[2], u32x2[4]>;
    VSlot vbuf[NB];
    int eyr[NB];               // packed table fields of the window in each ring slot
    constexpr int kPwRow = (G + 3) / 4 * 4;  // floats per token in this wave's p rows
    static_assert(kPwRow <= 8, "p row");
    CK_LDS float *pw = (CK_LDS float *)(smem + L::kPw) + wid * 64;

    // A window's loads: the buffer descriptor of its rows (K or V) starts at the
    // window and spans its valid tokens, so the range check returns 0 for the rows
    // of tokens past the sequence's end (or of an invalid page: range 0) and the
    // lane offsets are constants. The offset from 32-bit factors: a page is at most
    // 2^31 bytes (128 tokens x 2^16 heads x 256 B), a window's offset in its page
    // below that. A step spends few instructions on addresses: the stream wave's
    // instruction count per window is its critical path.
    struct TokWin {
        int64_t off;
        int range;
    };
    auto tok_win = [&](i32x2 e) __attribute__((always_inline)) {
        const int page = __builtin_amdgcn_readfirstlane(e[0]);
        const int ey = __builtin_amdgcn_readfirstlane(e[1]);
        const uint64_t off = (uint64_t)(uint32_t)max(page, 0) * pg32 + (uint32_t)tab_sub(ey) * win32;
        return TokWin{(int64_t)off, page < 0 ? 0 : (int)(tab_tv(ey) * tok32)};
    };

    // K/V loads of the window with table entry e (e[0] < 0: invalid page; a padding
    // entry past the phase end reads nothing) into one ring slot
    auto issue = [&](i32x2 e, u32x4 &k0, u32x4 &k1, VSlot &vv) __attribute__((always_inline)) {
        const TokWin w = tok_win(e);
        const __amdgpu_buffer_rsrc_t rk =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(kbase + w.off), (short)0, w.range, kRsrcFlags);
        const __amdgpu_buffer_rsrc_t rv =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(vbase + w.off), (short)0, w.range, kRsrcFlags);
        k0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, (int)koff, 0, 0));
        k1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, (int)(koff + 128), 0, 0));
        if constexpr (!TOK) {  // the dims-major body's loads
#pragma unroll
            for (int j = 0; j < 4; ++j)
                vv[j] = __builtin_bit_cast(
                    u32x2, __builtin_amdgcn_raw_buffer_load_b64(rv, (int)(voff + (uint32_t)(2 * j * tokb)), 0, 0));
        }
    };

    // token-major: a window's K rows as the 4 A fragments of its score MFMAs
    auto issue_kfrag = [&](const TokWin &w, u32x4 *kf) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t r =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(kbase + w.off), (short)0, w.range, kRsrcFlags);
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
            kf[s4] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(kfoff + 64 * s4), 0, 0));
    };

    // token-major: a window's V rows (lane (t, c): token t, bytes 16 c and 128 + 16 c),
    // issued after the values of the window whose ring slot they reuse
    auto issue_v = [&](const TokWin &w, u32x4 &x0, u32x4 &x1) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t r =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(vbase + w.off), (short)0, w.range, kRsrcFlags);
        x0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)koff, 0, 0));
        x1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(koff + 128), 0, 0));
    };

    // The merged result of sequence b's segment for query head h, dims 4 d4 .. 4 d4
    // + 3 (O normalised): bf16 O and the LSE when the segment is the whole
    // sequence, else an fp32 partial in the chunk's head or tail slot.
    auto write_result = [&](int b, int h, int d4, f32x4 on, float lse_v) __attribute__((always_inline)) {
        const bool head_part = cw[b] < w0;
        const bool tail_part = cw[b + 1] > w1;
        if (!head_part && !tail_part) {
            const int64_t row = (int64_t)b * a.num_heads + g * G + h;
            *reinterpret_cast<uint2 *>(a.out + row * kD + 4 * d4) =
                make_uint2(pack_bf16x2(on[0], on[1]), pack_bf16x2(on[2], on[3]));
            if (d4 == 0) a.lse[row] = lse_v;
        } else {
            const int64_t pidx = (((int64_t)g * a.chunks + chunk) * 2 + (head_part ? 0 : 1)) * G + h;
            // non-temporal: read once, by the fix-up or cascade epilogue kernel
            __builtin_nontemporal_store(on, reinterpret_cast<f32x4 *>(a.part_o + pidx * kD + 4 * d4));
            if (d4 == 0) a.part_lse[pidx] = lse_v;
        }
    };

    // Merges query-head / dim pair u (h = u / 32, dims 4 (u % 32) .. + 3) of the NW
    // partials in exchange slot r: TOK into stash entry e, else straight out for
    // sequence b.
    auto merge_pair = [&](int u, int r, int b, int e) __attribute__((always_inline)) {
        const CK_LDS float *xo_r = xo + r * NW * G * kD;
        const CK_LDS float *xml_r = xml + r * NW * G * 2;
        const int h = u >> 5, d4 = u & 31;
        float mx = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) mx = fmaxf(mx, xml_r[(ww * G + h) * 2]);
        const float mz = mx == -INFINITY ? 0.f : mx;
        float lt = 0.f;
        f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) {
            const float f = exp2_fast(xml_r[(ww * G + h) * 2] - mz);
            lt = fmaf(xml_r[(ww * G + h) * 2 + 1], f, lt);
            const f32x4 xa = *reinterpret_cast<const CK_LDS f32x4 *>(xo_r + (ww * G + h) * kD + 4 * d4);
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = fmaf(xa[i], f, o[i]);
        }
        const float inv = lt > 0.f ? 1.0f / lt : 0.f;
        const float lse_v = lt > 0.f ? (mx + __log2f(lt)) * kLn2 : -INFINITY;
        const f32x4 on = f32x4{o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv};
        if constexpr (TOK) {
            *reinterpret_cast<CK_LDS f32x4 *>(so + (e * G + h) * kD + 4 * d4) = on;
            if (d4 == 0) sl[e * G + h] = lse_v;
        } else {
            write_result(b, h, d4, on, lse_v);
        }
    };

    // TOK: this wave's share of the merge of close k (exchange slot k % R, sequence
    // b, stash entry e) once all NW partials are in (bounded wait: every wave
    // closes the same segments), so no single wave carries the whole merge. The
    // slot's arrival count only grows, NW per use, so use k / R is complete at
    // NW (k / R + 1) and nothing is reset or published: a wave at close k has
    // passed close k - 1's wait, for which every wave arrived after its reads of
    // close k - 2, the slot's previous use. Each step of a close costs an LDS round
    // trip, slow while the stage-1 waves keep the LDS busy, so the close has few.
    auto merge_share = [&](int k, int b, int e) __attribute__((always_inline)) {
        static_assert(!TOK || R == 2, "the slot reuse argument above takes two slots");
        const int r = k % R;
        const int target = NW * (k / R + 1);
        {
            int spin = 0;
            for (; *(volatile CK_LDS int *)(xcnt + r) < target && spin < (1 << 22); ++spin)
                __builtin_amdgcn_s_sleep(1);
            if (spin == (1 << 22)) count_giveup(&g_wait_giveups);
        }
        asm volatile("" ::: "memory");
        constexpr int kPer = 32 * G / NW;  // pairs per wave
        static_assert(!TOK || (kPer * NW == 32 * G && kPer <= 64), "pairs split evenly over the waves");
        if (lane < kPer) merge_pair(wid * kPer + lane, r, b, e);
        if (wid == 0 && lane == 0) sb[e] = b;
    };

    // Token-major: the state of a new segment, set at the start and by every close
    // (a segment opens at the chunk's first window or right after the previous
    // segment's close).
    auto reset_seg = [&]() __attribute__((always_inline)) {
        m1 = -INFINITY;
        mt1 = -INFINITY;
        mz1 = 0.f;
        l1 = 0.f;
#pragma unroll
        for (int T = 0; T < 8; ++T) oacc[T] = f32x4{0.f, 0.f, 0.f, 0.f};
    };

    // Closes segment b (sequence b's windows in this range): folds the lanes' partial
    // sums, hands the wave's (O, m, l) to the exchange ring, and the last wave in
    // merges the NW partials and writes the result (TOK: into the phase's stash).
    auto close_seg = [&](int b) __attribute__((always_inline)) {
        // token-major: head mn's row sum over the 4 groups; O^T needs no reduction
        // (the MFMAs summed over the tokens). Dims-major: each head's row sum over
        // the 8 token slots, its accumulators over the two half-waves.
        float lt1 = 0.f;
        if constexpr (TOK) {
            lt1 = sum_xor32(sum_xor16(l1));
        } else {
#pragma unroll
            for (int h = 0; h < G; ++h) l[h] = sum_slots(l[h]);
#pragma unroll
            for (int h = 0; h < G; ++h) {
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[h][e] = sum_xor32(acc[h][e]);
            }
        }
        const int r = nclose % R;
        const int want = nclose / R;  // merges the slot has seen before this segment
        // dims-major: the slot's previous segment must be merged (bounded: a wait
        // that never ended would mean a broken invariant, and results then are
        // wrong, not hung; such a wait is counted). Token-major: see merge_share.
        if constexpr (!TOK) {
            int spin = 0;
            for (; *(volatile CK_LDS int *)(xgen + r) != want && spin < (1 << 22); ++spin)
                __builtin_amdgcn_s_sleep(1);
            if (spin == (1 << 22)) count_giveup(&g_wait_giveups);
        }
        CK_LDS float *xo_r = xo + r * NW * G * kD;
        CK_LDS float *xml_r = xml + r * NW * G * 2;
        if constexpr (TOK) {
            if (mn < G) {
#pragma unroll
                for (int T = 0; T < 8; ++T)
                    *reinterpret_cast<CK_LDS f32x4 *>(xo_r + (wid * G + mn) * kD + 16 * T + 4 * mg) = oacc[T];
                if (mg == 0) {
                    xml_r[(wid * G + mn) * 2] = m1;
                    xml_r[(wid * G + mn) * 2 + 1] = lt1;
                }
            }
        } else if (hf == 0) {
#pragma unroll
            for (int h = 0; h < G; ++h)
                *reinterpret_cast<CK_LDS f32x4 *>(xo_r + (wid * G + h) * kD + 4 * dd) =
                    f32x4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
        }
        if (!TOK && lane == 0) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                xml_r[(wid * G + h) * 2] = m[h];
                xml_r[(wid * G + h) * 2 + 1] = l[h];
            }
        }
        // a wave's LDS operations are performed in the order it issues them: its rows
        // are in before its arrival counts (token-major: no wait for that; the
        // dims-major path waits, as before)
        if constexpr (TOK) asm volatile("" ::: "memory");
        else asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if constexpr (TOK) {
            if (lane == 0) __hip_atomic_fetch_add(xcnt + r, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            merge_share(nclose, b, qslot);
        } else {
            int old = 0;
            if (lane == 0) old = __hip_atomic_fetch_add(xcnt + r, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            old = __builtin_amdgcn_readfirstlane(old);
            if (old == NW - 1) {
                // the last wave in: merge the NW partials of every query head
                asm volatile("" ::: "memory");
#pragma unroll 1
                for (int u0 = 0; u0 < 32 * G; u0 += 64) {
                    if (u0 + lane < 32 * G) merge_pair(u0 + lane, r, b, 0);
                }
                // free the slot: reset its count, then publish the merge
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                if (lane == 0) xcnt[r] = 0;
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                if (lane == 0) xgen[r] = want + 1;
            }
        }
        ++nclose;
        ++qslot;
        if constexpr (TOK) reset_seg();
    };

    i32x2 enext = i32x2{-1, 0};  // the table entry of the next window to issue
    // One window of a phase: issue window n + D into the slot freed last step,
    // compute window n from slot J = n % NB, close its segment if it ends here.
    auto step = [&](auto jc, int n, int np) __attribute__((always_inline)) {
      if constexpr (!TOK) {
        constexpr int J = decltype(jc)::value;
        constexpr int JI = (J + D) % NB;  // slot of window n + D (freed by window n - 1)
        const i32x2 ei = enext;           // tab[n + D], read a step ahead
        issue(ei, kbuf[JI][0], kbuf[JI][1], vbuf[JI]);
        eyr[JI] = __builtin_amdgcn_readfirstlane(ei[1]);
        const int ey = eyr[J];
        enext = tab[n + D + 1];  // at most np + D: a padding entry past the phase
        const int b = tab_b(ey);
        const int t1 = min(max(tab_tv(ey) - 8 * wid, 0), 8);
        const CK_LDS char *qrow = qs + qslot * G * (kD * 2) + c * 16;
        if (tab_first(ey)) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                m[h] = -INFINITY;
                l[h] = 0.f;
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[h][e] = 0.f;
            }
        }
        if (t1 > 0) {
            const u32x4 k0 = kbuf[J][0], k1 = kbuf[J][1];
            float s[G];  // scores, then p in place
            bool trig = false;
#pragma unroll
            for (int h = 0; h < G; ++h) {  // q from LDS per window
                const u32x4 q0 = *reinterpret_cast<const CK_LDS u32x4 *>(qrow + h * (kD * 2));
                const u32x4 q1 = *reinterpret_cast<const CK_LDS u32x4 *>(qrow + h * (kD * 2) + 128);
                s[h] = sum8(dot16(k0, k1, q0, q1)) * a.scale_log2;
            }
            if (t1 < 8) {
#pragma unroll
                for (int h = 0; h < G; ++h) s[h] = t < t1 ? s[h] : -INFINITY;
            }
#pragma unroll
            for (int h = 0; h < G; ++h) trig |= s[h] > m[h] + kTau;  // m = -inf: always
            if (__builtin_amdgcn_ballot_w64(trig)) {
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    const float m_new = fmaxf(m[h], max_slots(s[h]));
                    if (m_new > m[h]) {
                        const float f = exp2_fast(m[h] - m_new);  // 0 from -inf
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[h][e] *= f;
                        l[h] *= f;
                        m[h] = m_new;
                    }
                }
            }
#pragma unroll
            for (int h = 0; h < G; ++h) {
                s[h] = exp2_fast(s[h] - (m[h] == -INFINITY ? 0.f : m[h]));  // 0 for masked tokens
                l[h] += s[h];
            }
            // p of token t -> this wave's row t (lanes c = 0), read back per V token
            if (c == 0) {
#pragma unroll
                for (int h4 = 0; h4 < kPwRow; h4 += 4)
                    *reinterpret_cast<CK_LDS f32x4 *>(pw + t * 8 + h4) =
                        f32x4{s[h4], h4 + 1 < G ? s[h4 + 1] : 0.f, h4 + 2 < G ? s[h4 + 2] : 0.f,
                              h4 + 3 < G ? s[h4 + 3] : 0.f};
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x2 vv = vbuf[J][j];
                const float v0 = bf16_lo(vv[0]), v1 = bf16_hi(vv[0]), v2 = bf16_lo(vv[1]), v3 = bf16_hi(vv[1]);
#pragma unroll
                for (int h4 = 0; h4 < kPwRow; h4 += 4) {
                    const f32x4 pv = *reinterpret_cast<const CK_LDS f32x4 *>(pw + (2 * j + hf) * 8 + h4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (h4 + e < G) {
                            acc[h4 + e][0] = fmaf(pv[e], v0, acc[h4 + e][0]);
                            acc[h4 + e][1] = fmaf(pv[e], v1, acc[h4 + e][1]);
                            acc[h4 + e][2] = fmaf(pv[e], v2, acc[h4 + e][2]);
                            acc[h4 + e][3] = fmaf(pv[e], v3, acc[h4 + e][3]);
                        }
                    }
                }
            }
        }

        if (tab_last(ey)) close_seg(b);
      }
    };

    int eypend = 0;  // packed table fields of window n - 1 (token-major)
    // Token-major values of the pending window: its V rows (lane (t, c) holds 32
    // bytes of token t) into the wave's LDS slot, back as the V^T fragments of the 8
    // dim tiles, then O^T += V^T P^T for the hi and the lo term of P. The slot is
    // written and read by this wave only, whose LDS operations run in issue order.
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    auto pv_tok = [&](const VSlot &vv) __attribute__((always_inline)) {
      if constexpr (TOK) {
        *reinterpret_cast<CK_LDS u32x4 *>(vt + vwo) = vv[0];
        *reinterpret_cast<CK_LDS u32x4 *>(vt + vwo + 128) = vv[1];
        uint2 vtf[8];
#pragma unroll
        for (int T = 0; T < 8; ++T) vtf[T] = lds_read_tr16(vt + vro + 32 * T);
        const s16x4 bh = __builtin_bit_cast(s16x4, uint2{ph[0], ph[1]});
        const s16x4 bl = __builtin_bit_cast(s16x4, uint2{pl[0], pl[1]});
#pragma unroll
        for (int T = 0; T < 8; ++T) {
            const s16x4 av = __builtin_bit_cast(s16x4, vtf[T]);
            oacc[T] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, bh, oacc[T], 0, 0, 0);
            oacc[T] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, bl, oacc[T], 0, 0, 0);
        }
      }
    };
    // Token-major window step, pipelined by one window: step n issues the K rows of
    // window n + D, computes the scores of window n and the values of window n - 1
    // (its P kept from the step before, its V rows still in their ring slot) -- two
    // independent chains in one basic block, so each fills the other's latencies --
    // then issues window n + D's V rows into the slot window n - 1's values just
    // left, closes window n - 1's segment if it ends there and finishes window n's
    // softmax. The table entry of the window to issue was read one step ahead and
    // the packed fields of each window travel in the ring with its data.
    auto step_tok = [&](auto jc, int n, int np) __attribute__((always_inline)) {
      if constexpr (TOK) {
        constexpr int J = decltype(jc)::value;
        constexpr int JI = (J + D) % NB;  // window n + D, into the slot of window n - 1
        const i32x2 ei = enext;
        const TokWin wi = tok_win(ei);
        issue_kfrag(wi, kbuf[JI]);
        const int ey = eyr[J];
        const int eyp = eypend;
        eyr[JI] = __builtin_amdgcn_readfirstlane(ei[1]);
        if (tab_first(ey)) {
            // window n opens a segment: q of head mn (heads past G: any finite row,
            // their scores are -inf), in the slot after the segment window n - 1
            // may still close
            const CK_LDS char *qrow =
                qs + ((qslot + (tab_last(eyp) ? 1 : 0)) * G + (mn < G ? mn : 0)) * (kD * 2) + 16 * mg;
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) qf[s4] = *reinterpret_cast<const CK_LDS u32x4 *>(qrow + 64 * s4);
        }
        enext = tab[n + D + 1];  // at most np + D: a padding entry past the phase
        f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
            sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kbuf[J][s4]),
                                                         __builtin_bit_cast(bf16x8, qf[s4]), sc, 0, 0, 0);
        pv_tok(vbuf[JI]);
        issue_v(wi, vbuf[JI][0], vbuf[JI][1]);
        if (tab_last(eyp)) close_seg(tab_b(eyp));
        eypend = ey;
        float s[4];  // scores of tokens 4 mg + r, head mn; then p
#pragma unroll
        for (int r = 0; r < 4; ++r) s[r] = fmaf(sc[r], a.scale_log2, sbias);
        {
            const int t1 = min(max(tab_tv(ey) - 8 * wid, 0), 8);
            if (t1 < 8) {
                asm volatile("");  // a branch (a sequence's last window)
#pragma unroll
                for (int r = 0; r < 4; ++r) s[r] = 4 * mg + r < t1 ? s[r] : -INFINITY;
            }
        }
        bool trig = false;
#pragma unroll
        for (int r = 0; r < 4; ++r) trig |= s[r] > mt1;  // m = -inf: any real score
        if (__builtin_amdgcn_ballot_w64(trig)) {
            // head mn's max over its 8 tokens (the 4 groups), the same in its 4 lanes
            const float x = max_xor32(max_xor16(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]))));
            if (x > m1) {
                const float f = exp2_fast(m1 - x);  // 0 from -inf
#pragma unroll
                for (int T = 0; T < 8; ++T) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) oacc[T][r] *= f;
                }
                l1 *= f;
                m1 = x;
                mt1 = x + kTau;
                mz1 = x;
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s[r] = exp2_fast(s[r] - mz1);  // 0 for masked tokens and padding lanes
            l1 += s[r];
        }
        // P^T of window n for the next step: hi = p truncated to bf16 (exact in fp32),
        // lo = p - hi (exact) rounded to bf16
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t u0 = __float_as_uint(s[2 * i]), u1 = __float_as_uint(s[2 * i + 1]);
            ph[i] = __builtin_amdgcn_perm(u1, u0, 0x07060302u);
            pl[i] = pack_bf16x2(s[2 * i] - __uint_as_float(u0 & 0xFFFF0000u),
                                s[2 * i + 1] - __uint_as_float(u1 & 0xFFFF0000u));
        }
      }
    };
    // after a phase's last window (np - 1, in slot (np - 1) % NB): its values and
    // its segment's close
    auto drain_tok = [&](int np) __attribute__((always_inline)) {
      if constexpr (TOK) {
        const int js = (np - 1) % NB;  // wave-uniform
        static_for<NB>([&](auto jc) __attribute__((always_inline)) {
            if (js == decltype(jc)::value) pv_tok(vbuf[decltype(jc)::value]);
        });
        if (tab_last(eypend)) close_seg(tab_b(eypend));
      }
    };

    // ---- phases of up to kTable windows and kQSlots segments: table and q rows,
    //      prologue loads, streaming loop --------------------------------------------
    const int nwin = w1 - w0;
    if constexpr (TOK) reset_seg();  // the chunk's first window opens a segment
    for (int p0 = 0; p0 < nwin;) {
        if (p0 > 0) {
            wait_vmcnt<0>();
            bar.sync();  // every wave is done with the previous phase's table and q rows
        }
        // The phase's segments: the first kQSlots non-empty sequences from the one
        // holding window w0 + p0 that start inside the chunk, read from one ballot
        // over 64 candidate sequences (every wave finds the same list on its own).
        const int bq0 = find_seq(w0 + p0);  // non-empty: cw[bq0 + 1] > w0 + p0
        const int bc = min(bq0 + lane, a.batch - 1);
        const int c_lo = cw[bc], c_hi = cw[bc + 1], c_len = len[bc];
        uint64_t segm = __builtin_amdgcn_ballot_w64(bq0 + lane < a.batch && c_hi > c_lo && c_lo < w1);
        int segb[kQSlots], seg_lo[kQSlots], seg_hi[kQSlots], seg_len[kQSlots];
#pragma unroll
        for (int sg = 0; sg < kQSlots; ++sg) {
            seg_lo[sg] = 0x7FFFFFFF;  // never selected below
            segb[sg] = seg_hi[sg] = seg_len[sg] = 0;
            if (segm != 0) {
                const int l = __builtin_ctzll(segm);
                segm &= segm - 1;
                segb[sg] = bq0 + l;
                seg_lo[sg] = __builtin_amdgcn_readlane(c_lo, l);
                seg_hi[sg] = __builtin_amdgcn_readlane(c_hi, l);
                seg_len[sg] = __builtin_amdgcn_readlane(c_len, l);
                if (sg % NW == wid) dma_q(segb[sg], sg);
            }
        }
        int p1 = min(p0 + kTable, nwin);
        if (segm != 0) {
            p1 = min(p1, __builtin_amdgcn_readlane(c_lo, __builtin_ctzll(segm)) - w0);  // the next segment opens the next phase
        } else if (bq0 + 64 < a.batch) {
            p1 = min(p1, cw[bq0 + 64] - w0);  // candidates beyond the 64 examined: the next phase
        }
        const int np = p1 - p0;
        // D + 1 padding entries past the phase (no loads, no tokens) for the
        // one-step-ahead table reads of its last windows
        for (int i = tid; i < np + D + 1; i += kThr) {
            if (i >= np) {
                tab[i] = i32x2{-1, 0};
                continue;
            }
            const int wg = w0 + p0 + i;
            int b = segb[0], lo_b = seg_lo[0], hi_b = seg_hi[0], len_b = seg_len[0];
#pragma unroll
            for (int sg = 1; sg < kQSlots; ++sg) {
                if (seg_lo[sg] <= wg) {  // the last segment starting at or before window wg
                    b = segb[sg];
                    lo_b = seg_lo[sg];
                    hi_b = seg_hi[sg];
                    len_b = seg_len[sg];
                }
            }
            const int k = wg - lo_b;
            const int tv = min(len_b - k * kWin, kWin);
            const int first = wg == max(lo_b, w0);
            const int last = wg == min(hi_b, w1) - 1;
            const int page = a.bt[(int64_t)b * a.bt_cols + k / kWpp];
            const bool ok = page >= 0 && (int64_t)page < a.num_blocks;
            const int ey = tv | (first << 7) | (last << 8) | ((k % kWpp) << 9) | (b << 11);
            tab[i] = i32x2{ok ? page : -1, ey};
        }
        wait_vmcnt<0>();  // q rows and page ids in
        bar.sync();
        qslot = 0;
#pragma unroll
        for (int j = 0; j < D; ++j) {
            if constexpr (TOK) {
                const i32x2 e = tab[j];  // j < D: a padding entry when j >= np
                const TokWin w = tok_win(e);
                issue_kfrag(w, kbuf[j]);
                issue_v(w, vbuf[j][0], vbuf[j][1]);
                eyr[j] = __builtin_amdgcn_readfirstlane(e[1]);
            } else {
                const i32x2 e = tab[j];  // j < D: a padding entry when j >= np
                issue(e, kbuf[j][0], kbuf[j][1], vbuf[j]);
                eyr[j] = __builtin_amdgcn_readfirstlane(e[1]);
            }
        }
        if constexpr (!TOK) enext = tab[D];
        if constexpr (TOK) {
            enext = tab[D];
            // "window -1" of the pipelined step (slot NB - 1): no values, no close;
            // its V slot is zeroed so that p = 0 times it stays 0
            ph[0] = ph[1] = pl[0] = pl[1] = 0u;
            vbuf[NB - 1][0] = u32x4{0u, 0u, 0u, 0u};
            vbuf[NB - 1][1] = u32x4{0u, 0u, 0u, 0u};
            eypend = 0;
        }
        // full rounds of NB steps, then the rest: the ring slot of every step is a
        // compile-time constant and no step leaves the loop early, so the
        // compiler's vmcnt bookkeeping sees one path around the back edge
        int n = 0;
        for (int it = np / NB; it > 0; --it) {
            static_for<NB>([&](auto jc) __attribute__((always_inline)) {
                if constexpr (TOK) step_tok(jc, n + decltype(jc)::value, np);
                else step(jc, n + decltype(jc)::value, np);
            });
            n += NB;
        }
        const int rem = np - n;
        static_for<NB>([&](auto jc) __attribute__((always_inline)) {
            if (decltype(jc)::value < rem) {
                if constexpr (TOK) step_tok(jc, n + decltype(jc)::value, np);
                else step(jc, n + decltype(jc)::value, np);
            }
        });
        drain_tok(np);
        if constexpr (TOK) {
            // the phase's merged results out, by every wave of the role: each merge
            // is done once every wave is past its last close
            bar.sync();
            const int nseg = qslot;  // segments closed in this phase (the same in every wave)
            for (int i = tid; i < nseg * G * 32; i += kThr) {
                const int e = i / (G * 32), u = i % (G * 32);
                const int h = u >> 5, d4 = u & 31;
                write_result(sb[e], h, d4, *reinterpret_cast<const CK_LDS f32x4 *>(so + (e * G + h) * kD + 4 * d4),
                             sl[e * G + h]);
            }
        }
        p0 = p1;
    }
}

// The stand-alone stream kernel: the token-major body on the matrix cores (the
// fused kernel's streaming body) on 4 waves and at most 256 registers; two
// workgroups per CU up to 4 query heads per group (64 KB of LDS each), one above
// (103 KB at 8 heads: the grid's second half runs as the first half's
// workgroups finish; a 4-segment layout that fits two per CU measured no faster).
template <int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void suffix_stream_kernel(SuffixArgs a) {
    extern __shared__ __attribute__((aligned(16))) char smem_raw[];
    suffix_stream_body<G, 4, (G > 4 ? 1 : kTokDepth), true>(a, (CK_LDS char *)smem_raw, blockIdx.x, threadIdx.x,
                                                           WgBarrier{});
}
static_assert(SfxLds<4, 4, true>::kBytes <= 80 * 1024, "two stand-alone workgroups per CU up to 4 heads");
static_assert(SfxLds<kMaxGroup, 4, true>::kBytes <= 160 * 1024, "one above");

// Folds the partials of one query head of a sequence cut by chunk boundaries
// (chunks ca < cb): the tail slot (1) of chunk ca and the head slot (0) of every
// later chunk that holds windows, weighted by exp(lse - max). Online over batches
// of kB chunks whose loads all go out before any is used: one memory round trip
// per batch, not one per chunk (a long sequence spans many chunks, and the
// slowest sequence sets the kernel's time).
template <int G>
__device__ __forceinline__ void fold_cut(const float *part_o, const float *part_lse, int g, const ChunkMap &cm,
                                         int hq, int d4, int ca, int cb, float4 &o_out, float &lse_out) {
    constexpr int kB = 8;
    auto pidx = [&](int ch, int sl) { return (((int64_t)g * cm.P + ch) * 2 + sl) * G + hq; };
    float m = -INFINITY, wsum = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int c0 = ca; c0 <= cb; c0 += kB) {
        float pl[kB];
        float4 po[kB];
        bool ok[kB];
        // a chunk with no windows wrote nothing (chunk ca holds the sequence's
        // start); empty chunks exist only below one window per chunk, and their
        // test runs as a rolled loop off the common path
        uint32_t okm = cb - c0 + 1 >= kB ? (1u << kB) - 1 : (1u << (cb - c0 + 1)) - 1;
        if (!cm.none_empty()) {
#pragma unroll 1
            for (int j = 0; j < kB; ++j)
                if (c0 + j <= cb && c0 + j != ca && cm.empty(c0 + j)) okm &= ~(1u << j);
        }
#pragma unroll
        for (int j = 0; j < kB; ++j) {
            const int ch = min(c0 + j, cb);  // clamped: every load is in bounds
            ok[j] = (okm >> j) & 1;
            const int64_t p = pidx(ch, c0 + j == ca ? 1 : 0);
            pl[j] = part_lse[p];
            po[j] = *reinterpret_cast<const float4 *>(part_o + p * kD + 4 * d4);
        }
        float mb = m;
#pragma unroll
        for (int j = 0; j < kB; ++j)
            if (ok[j]) mb = fmaxf(mb, pl[j]);
        const float mu = mb == -INFINITY ? 0.f : mb;
        const float r = exp2_fast((m - mu) * kLog2e);  // 0 from m = -inf
        acc.x *= r;
        acc.y *= r;
        acc.z *= r;
        acc.w *= r;
        wsum *= r;
#pragma unroll
        for (int j = 0; j < kB; ++j) {
            if (!ok[j]) continue;
            const float wgt = exp2_fast((pl[j] - mu) * kLog2e);
            acc.x = fmaf(wgt, po[j].x, acc.x);
            acc.y = fmaf(wgt, po[j].y, acc.y);
            acc.z = fmaf(wgt, po[j].z, acc.z);
            acc.w = fmaf(wgt, po[j].w, acc.w);
            wsum += wgt;
        }
        m = mb;
    }
    const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
    o_out = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
    lse_out = wsum > 0.f ? m + __logf(wsum) : -INFINITY;
}

// One workgroup of 32 G threads per (sequence, kv head): empty suffixes get
// O = 0, LSE = -inf; a sequence cut by chunk boundaries gets its partials
// folded; others return. The window prefix sums and the grid arithmetic come as
// leading scalar parameters (preloaded into SGPRs at wave launch, as for the
// cascade epilogue), so the first load waits for no kernel-argument load.
template <int G>
__global__ __launch_bounds__(kMaxGroup * 32) void suffix_fixup_kernel(const int32_t *cw, int kv_heads, int batch,
                                                                      SuffixArgs a) {
    const int b = blockIdx.x / kv_heads;
    const int g = blockIdx.x % kv_heads;
    const int hq = threadIdx.x >> 5;
    const int d4 = threadIdx.x & 31;
    const int64_t beg = cw[b], end = cw[b + 1], W = cw[batch];
    const int64_t row = (int64_t)b * a.num_heads + g * G + hq;
    if (end == beg) {
        *reinterpret_cast<uint2 *>(a.out + row * kD + 4 * d4) = make_uint2(0, 0);
        if (d4 == 0) a.lse[row] = -INFINITY;
        return;
    }
    const ChunkMap cm{W, a.chunks, a.split};
    const int ca = cm.owner(beg);
    const int cb = cm.owner(end - 1);
    if (ca == cb) return;  // written by the stream kernel
    float4 o;
    float l;
    fold_cut<G>(a.part_o, a.part_lse, g, cm, hq, d4, ca, cb, o, l);
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
// What those first loads need (the prefix sums, the stage-1 result and the row
// arithmetic) comes as scalar kernel parameters ahead of the struct: the
// compiler preloads leading scalar parameters into SGPRs at wave launch, which
// takes the kernel-argument load off the first round trip.
// The host fills the whole struct; launch_epilogue passes s1, cw, b0, nb,
// num_heads and kv_heads again as the leading parameters the kernel reads.
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
    int split;
};

template <int G>
__global__ __launch_bounds__(kMaxGroup * 32) void cascade_epilogue_kernel(const int32_t *cw, const float *s1o, const float *s1lse,
                                                                         int64_t rows, int kv_heads, int nb, int num_heads,
                                                                         int b0, int splits, EpilogueArgs e) {
    constexpr int kBatch = 8;   // splits folded per rescale step
    constexpr int kPreS = 16;   // splits loaded up front
    const int bl = blockIdx.x / kv_heads;
    const int g = blockIdx.x % kv_heads;
    const int hq = threadIdx.x >> 5;
    const int d4 = threadIdx.x & 31;
    const int h = g * G + hq;
    const int64_t row = (int64_t)(b0 + bl) * num_heads + h;

    const int64_t beg = cw[bl], end = cw[bl + 1], W = cw[nb];

    // ---- stage-1 loads: the first kPreS splits of this query row ------------------
    float ls[kPreS];
    float4 os[kPreS];
    if (splits <= 1) {
        os[0] = *reinterpret_cast<const float4 *>(s1o + row * kD + 4 * d4);
        ls[0] = s1lse[row * 8];
    } else {
#pragma unroll
        for (int j = 0; j < kPreS; ++j) {
            const int s = j < splits ? j : splits - 1;
            ls[j] = s1lse[(int64_t)s * rows + row];
            os[j] = *reinterpret_cast<const float4 *>(s1o + ((int64_t)s * rows + row) * kD + 4 * d4);
        }
    }

    // ---- suffix: empty, whole (bf16 result) or cut by chunk boundaries ------------
    float l2 = -INFINITY;
    float4 o2 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (end > beg) {
        const ChunkMap cm{W, e.chunks, e.split};
        const int ca = cm.owner(beg);
        const int cb = cm.owner(end - 1);
        if (ca == cb) {
            const int64_t r2 = (int64_t)bl * num_heads + h;
            const uint2 w = *reinterpret_cast<const uint2 *>(e.o2 + r2 * kD + 4 * d4);
            o2 = make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
            l2 = e.lse2[r2];
        } else {
            fold_cut<G>(e.part_o, e.part_lse, g, cm, hq, d4, ca, cb, o2, l2);
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
                lb[j] = s1lse[(int64_t)s * rows + row];
                ob[j] = *reinterpret_cast<const float4 *>(s1o + ((int64_t)s * rows + row) * kD + 4 * d4);
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

// Fused cascade kernel: workgroup i runs stage-1 unit i on waves 0-3 (the
// 128-row body with a 3-slot ring) and suffix chunk 2j on waves 4-7 (the stream
// body on 4 waves, 32-token windows) side by side on one CU: each SIMD holds one
// MFMA wave and one streaming wave, which fill each other's stalls, and the
// prefix pages and the suffix pages stream at the same time. When its stage-1
// unit is done, waves 0-3 stream suffix chunk 2j + 1, the last (256 - split) /
// 256 of the workgroup's windows, in the LDS the stage-1 tiles used: the two
// roles end together instead of the stage-1 waves idling while the suffix
// waves finish. Each role has its own LDS region and barrier; neither waits
// for the other.
constexpr int kFusedS1Lds = s1::wide_lds_bytes<3>();
template <int G>
using FusedSfx = SfxLds<G, 4, (G <= 4)>;  // the stream body's layout on 4 waves (token-major up to 4 heads)
template <int G>
constexpr int fused_lds_bytes() { return kFusedS1Lds + FusedSfx<G>::kBytes + 32; }
static_assert(fused_lds_bytes<4>() <= 160 * 1024 && fused_lds_bytes<kMaxGroup>() <= 160 * 1024,
              "one fused workgroup per CU");
static_assert(FusedSfx<4>::kBytes <= kFusedS1Lds && FusedSfx<kMaxGroup>::kBytes <= kFusedS1Lds,
              "the stage-1 waves' stream body fits the tile ring");

template <int G>
__global__ __launch_bounds__(512) void cascade_fused_kernel(s1::Stage1Args s1a, int n1, SuffixArgs sa, int n2) {
    extern __shared__ __attribute__((aligned(16))) char smem_raw[];
    CK_LDS char *smem = (CK_LDS char *)smem_raw;
    CK_LDS int *bars = (CK_LDS int *)(smem + kFusedS1Lds + FusedSfx<G>::kBytes);
    if (threadIdx.x < 5) bars[threadIdx.x] = 0;  // two role barriers, the scan flag
    __syncthreads();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int role = wave < 4 ? 1 : 0;  // 1: stage-1 waves (suffix chunk 2j + 1 afterwards)
    const GroupBarrier bar{bars + 2 * (1 - role), bars + 2 * (1 - role) + 1, 4, &g_wait_giveups};
    if (role == 1 && (int)blockIdx.x < n1) {
        s1::stage1_wide_body<4, 3>(s1a, smem, blockIdx.x, n1, threadIdx.x, bar);
        // The stream body's arguments stay in scalar registers across the stage-1
        // body (the compiler loads them with the kernel's other arguments at the
        // start): without a use here it reloads them from the kernel-argument
        // segment after the barrier below, a memory round trip on the stage-1
        // waves' way to their suffix windows (0.3-0.5 us per step).
        asm volatile("" ::"s"(sa.q), "s"(sa.head_off), "s"(sa.scale_log2), "s"(sa.cw_out));
        bar.sync();  // every stage-1 wave is done with the tile ring
    }
    if ((int)blockIdx.x < n2) {
        // The stream roles take kv head group blockIdx + 3 (mod kv_heads) while the
        // stage-1 unit order puts kv head x on XCD x (blockIdx % 8) at the usual
        // shapes: a workgroup's two roles then read different kv heads. Pages of
        // some kv heads are slower to fetch than others (by their address bits: up
        // to ~15% measured), and with both roles on one head their slowness stacked
        // on the same workgroups, which set the kernel's end (1.1-1.6 us per step).
        constexpr int kRoleRot = 3;
        const int g = ((int)blockIdx.x + kRoleRot) % sa.kv_heads, j = (int)blockIdx.x / sa.kv_heads;
        // the streaming waves scan the lengths; the stage-1 waves reuse that scan
        suffix_stream_body<G, 4, (G <= 4 ? kTokDepth : kFusedDepth), (G <= 4)>(
            sa, smem + (role ? 0 : kFusedS1Lds), (2 * j + role) * sa.kv_heads + g, threadIdx.x & 255, bar, bars + 4,
            role ? smem + kFusedS1Lds : nullptr);
    }
}

int64_t ceil_div(int64_t x, int64_t y) { return (x + y - 1) / y; }

// partial (O, LSE) slots: 2 per (query head, chunk) -- the same count for any
// split of the heads into kv head groups
int64_t group_parts(int64_t num_heads, int64_t chunks) { return num_heads * chunks * 2; }

template <int G>
void launch_epilogue(const EpilogueArgs &e, unsigned grid, hipStream_t st) {
    hipLaunchKernelGGL(cascade_epilogue_kernel<G>, dim3(grid), dim3(32 * G), 0, st, e.cw, e.s1.o, e.s1.lse, e.s1.rows,
                       e.kv_heads, e.nb, e.num_heads, (int)e.b0, e.s1.splits, e);
}

template <int G>
int launch_fused(const s1::Stage1Args &s1a, int64_t n1, const SuffixArgs &a, const EpilogueArgs &epi,
                 hipStream_t st) {
    static std::atomic<uint64_t> lds_set{0};
    constexpr int kLds = fused_lds_bytes<G>();
    int rc = ensure_dynamic_lds(reinterpret_cast<const void *>(&cascade_fused_kernel<G>), kLds, lds_set);
    if (rc != CK_OK) return rc;
    const int64_t n2 = (int64_t)a.kv_heads * (a.chunks / 2);  // chunk pairs (a.split > 0)
    const int64_t grid = n1 > n2 ? n1 : n2;
    hipLaunchKernelGGL(cascade_fused_kernel<G>, dim3((unsigned)grid), dim3(512), kLds, st, s1a, (int)n1, a, (int)n2);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return static_cast<int>(e);
    launch_epilogue<G>(epi, (unsigned)(a.batch * a.kv_heads), st);
    CK_RETURN_LAUNCH();
}

template <int G>
int launch_suffix(const SuffixArgs &a, bool fixup, const EpilogueArgs *epi, hipStream_t st) {
    static std::atomic<uint64_t> lds_set{0};
    constexpr int kLds = SfxLds<G, 4, true>::kBytes;
    int rc = ensure_dynamic_lds(reinterpret_cast<const void *>(&suffix_stream_kernel<G>), kLds, lds_set);
    if (rc != CK_OK) return rc;
    hipLaunchKernelGGL(suffix_stream_kernel<G>, dim3((unsigned)(a.kv_heads * a.chunks)), dim3(256), kLds, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return static_cast<int>(e);
    if (fixup)
        hipLaunchKernelGGL(suffix_fixup_kernel<G>, dim3((unsigned)(a.batch * a.kv_heads)), dim3(32 * G), 0, st,
                           (const int32_t *)a.cw_out, a.kv_heads, a.batch, a);
    if (epi) launch_epilogue<G>(*epi, (unsigned)(a.batch * a.kv_heads), st);
    CK_RETURN_LAUNCH();
}

int check_suffix_dims(int64_t batch, int64_t num_heads, int64_t kv_heads, int64_t head_dim, int64_t kv_cap) {
    if (batch < 0 || batch > 0x7FFFFFFF || kv_cap < 0) return CK_E_INVALID_ARG;  // sequence indices are 32-bit
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

// Workgroups per kv head group: two resident workgroups per CU (16 waves of at
// most 128 registers, under 80 KB of LDS each), so the grid holds 512
// workgroups over all kv head groups and starts at once.
int64_t suffix_default_chunks(int64_t num_heads, int64_t kv_heads) {
    const int64_t groups = kv_heads * suffix_sub_groups(num_heads, kv_heads);
    const int64_t p = 512 / groups;
    return p > 0 ? p : 1;
}

int64_t suffix_fused_chunks(int64_t num_heads, int64_t kv_heads) {
    const int64_t groups = kv_heads * suffix_sub_groups(num_heads, kv_heads);
    const int64_t p = 256 / groups;
    return 2 * (p > 0 ? p : 1);  // a pair of chunks per fused workgroup
}

int64_t suffix_group_ws_bytes(int64_t nb, int64_t num_heads, int64_t kv_heads, int64_t chunks) {
    const int64_t parts = group_parts(num_heads, chunks);
    return parts * (kD + 1) * (int64_t)sizeof(float) + (nb + 1) * (int64_t)sizeof(int32_t) + 256;
}

int suffix_launch_group(const void *q, const void *k, const void *v, const int32_t *block_table, int64_t bt_cols,
                        const int64_t *kv_seqlens, int64_t b0, int64_t nb, int64_t num_heads, int64_t kv_heads,
                        int64_t num_blocks, int64_t kv_layout, float scale, int64_t kv_cap, int64_t chunks,
                        void *out, float *lse, void *group_ws, const Stage1Result *cascade, void *final_out,
                        float *final_lse, hipStream_t stream, const s1::Stage1Args *fused, int64_t fused_units) {
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
    a.split = fused && cascade ? kFusedSplit : 0;
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
        e.split = a.split;
    }
    if (fused && cascade) {
        switch (G) {
            case 1: return launch_fused<1>(*fused, fused_units, a, e, stream);
            case 2: return launch_fused<2>(*fused, fused_units, a, e, stream);
            case 3: return launch_fused<3>(*fused, fused_units, a, e, stream);
            case 4: return launch_fused<4>(*fused, fused_units, a, e, stream);
            case 5: return launch_fused<5>(*fused, fused_units, a, e, stream);
            case 6: return launch_fused<6>(*fused, fused_units, a, e, stream);
            case 7: return launch_fused<7>(*fused, fused_units, a, e, stream);
            default: return launch_fused<8>(*fused, fused_units, a, e, stream);
        }
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
                                 lse + b0 * num_heads, workspace, nullptr, nullptr, nullptr, st, nullptr, 0);
        if (rc != CK_OK) return rc;
    }
    return CK_OK;
}

extern "C" int ck_wait_giveups(uint64_t *count, int reset) {
    if (!count) return CK_E_NULL_PTR;
    unsigned int v = 0;
    hipError_t e = hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_wait_giveups), sizeof(v), 0, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return static_cast<int>(e);
    *count = v;
    if (reset) {
        const unsigned int zero = 0;
        e = hipMemcpyToSymbol(HIP_SYMBOL(g_wait_giveups), &zero, sizeof(zero), 0, hipMemcpyHostToDevice);
        if (e != hipSuccess) return static_cast<int>(e);
    }
    return CK_OK;
}
