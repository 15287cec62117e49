// add_rms_norm.hip - residual add + RMSNorm statistics (+ apply) on gfx950.
//
// Semantics (reference: ascend-kernel/csrc/ops/add_rms_norm_stats, design.md:37-62 and
// the fp64 model test/add_rms_norm_stats_ref.py:139-156), per row of [M, K]:
//   mode 0: x_out = rd(x1 + x2);         rstd = 1 / sqrt(mean_k(x_out^2) + eps)
//   mode 1: xo = x1 (the rounded residual); rstd as above;
//           y = rd(rd(xo * rstd) * gamma + beta)
//   mode 2: rstd of rd(x1 + x2) only
// rd() rounds to the data dtype. The statistics are taken on the ROUNDED
// residual, as the reference's golden does.
//
// Rounding contract. The reference model evaluates in fp64 and casts with
// torch's double -> bf16/fp16 conversion, which goes through fp32 (round to
// nearest even twice). This kernel does the same: the sum of squares, the
// mean, sqrt, the reciprocal and the two apply products run in fp64 (each
// square of a 16-bit value is exact in fp32 and 5120 of them sum in fp64 with a
// relative error below 1e-12), and every rd() is fp64 -> fp32 -> dtype, both
// RNE. x1 + x2 of two 16-bit values is exact in fp32 up to a 16-binade gap
// and otherwise lands far from a dtype tie, so rd(x1 + x2) is computed from
// the fp32 sum. rstd is returned as fp32 (RNE of the fp64 value).
//
// MI355X design: HBM-bound (mode 0 moves 3 M K elements). One wave per row:
// a row of K <= 5120 16-bit values is at most 10 16-byte chunks per lane,
// loaded with one buffer load per chunk (a buffer resource spanning the row
// returns zeros past its end, so there is no branch and all of a wave's loads
// are in flight together) and kept in registers between the statistics pass
// and the write pass, so every input byte is read once.
// Four rows per 256-thread workgroup; the grid also covers the padding rows
// of rstd (ceil(M / 8) * 8 rows, the reference's 32-byte output groups,
// op_host/add_rms_norm_stats.cpp:111-113), which are written 0.
#include <cmath>

#include "ck_common.h"

namespace ck {
namespace {

constexpr int kMaxK = 5120;                       // op contract (one row per wave)
constexpr int kMaxChunks = kMaxK / 8 / kWave;     // 16-byte chunks per lane: 10
constexpr int kRowsPerBlock = 4;
constexpr int kRstdGroup = 8;

struct NormArgs {
    const uint16_t *x1;
    const uint16_t *x2;
    const uint16_t *gamma;
    const uint16_t *beta;  // null = no bias
    uint16_t *x_out;
    float *rstd;
    uint16_t *y;
    int64_t m_rows;
    int64_t m_pad;
    int chunks;         // k / 8
    double eps;
};

// 16-bit element <-> fp32 for the two data dtypes.
template <bool kBf16>
__device__ __forceinline__ float lo16(uint32_t w) {
    if constexpr (kBf16) return __uint_as_float(w << 16);
    else return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
}
template <bool kBf16>
__device__ __forceinline__ float hi16(uint32_t w) {
    if constexpr (kBf16) return __uint_as_float(w & 0xFFFF0000u);
    else return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}
// two fp32 values -> packed dtype pair, RNE
template <bool kBf16>
__device__ __forceinline__ uint32_t pack16(float lo, float hi) {
    if constexpr (kBf16) {
        return pack_bf16x2(lo, hi);
    } else {
        const uint32_t a = __builtin_bit_cast(uint16_t, (_Float16)lo);
        const uint32_t b = __builtin_bit_cast(uint16_t, (_Float16)hi);
        return a | (b << 16);
    }
}
// fp64 -> fp32 (RNE) kept opaque to the optimiser: LLVM folds the chain
// fp64 -> fp32 -> 16-bit into one correctly rounded fp64 -> 16-bit conversion,
// which differs from the two-step rounding at fp32 values that sit on a
// 16-bit tie (about 2^-16 of the elements).
__device__ __forceinline__ float to_f32_opaque(double x) {
    float f = (float)x;
    asm volatile("" : "+v"(f));
    return f;
}
// rd() of an fp64 value as the reference casts it: fp64 -> fp32 -> dtype
template <bool kBf16>
__device__ __forceinline__ float rd64(double x) {
    const float f = to_f32_opaque(x);
    if constexpr (kBf16) return bf16_lo(pack_bf16x2(f, 0.f));
    else return (float)(_Float16)f;
}

// Buffer resource over `bytes` bytes at p: loads past the end return 0 and
// stores past the end are dropped, so a row's ragged last chunk needs no branch
// and every wave issues all its loads back to back.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void *p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bload(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ void bstore(__amdgpu_buffer_rsrc_t r, int off, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((__vector_size__(16))) unsigned, v), r,
                                           off, 0, 0);
}

__device__ __forceinline__ double wave_sum(double x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

template <bool kBf16, int kMode, bool kBeta>
__global__ __launch_bounds__(kRowsPerBlock * kWave) void add_rms_norm_kernel(NormArgs a) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= a.m_pad) return;
    if (row >= a.m_rows) {  // rstd padding rows
        if (lane == 0) a.rstd[row] = 0.f;
        return;
    }
    const int row_bytes = a.chunks * 16;
    const int64_t base = row * (int64_t)a.chunks * 8;  // elements

    // ---- load the row (x_out for mode 1, rd(x1 + x2) otherwise) -------------------
    u32x4 xo[kMaxChunks];
    const auto r1 = row_rsrc(a.x1 + base, row_bytes);
#pragma unroll
    for (int i = 0; i < kMaxChunks; ++i) xo[i] = bload(r1, (lane + kWave * i) * 16);
    if constexpr (kMode != 1) {
        u32x4 xb[kMaxChunks];
        const auto r2 = row_rsrc(a.x2 + base, row_bytes);
#pragma unroll
        for (int i = 0; i < kMaxChunks; ++i) xb[i] = bload(r2, (lane + kWave * i) * 16);
#pragma unroll
        for (int i = 0; i < kMaxChunks; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                xo[i][e] = pack16<kBf16>(lo16<kBf16>(xo[i][e]) + lo16<kBf16>(xb[i][e]),
                                         hi16<kBf16>(xo[i][e]) + hi16<kBf16>(xb[i][e]));
    }
    if constexpr (kMode == 0) {
        const auto ro = row_rsrc(a.x_out + base, row_bytes);
#pragma unroll
        for (int i = 0; i < kMaxChunks; ++i) bstore(ro, (lane + kWave * i) * 16, xo[i]);
    }

    // ---- statistics in fp64 (chunks past K hold zeros) -----------------------------
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < kMaxChunks; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // the square of a 16-bit value is exact in fp32; converting the
            // product (not the element) also keeps the fp64 elements of the
            // apply pass from being held live across the reduction
            const float l = lo16<kBf16>(xo[i][e]), h = hi16<kBf16>(xo[i][e]);
            ss += (double)(l * l);
            ss += (double)(h * h);
        }
    ss = wave_sum(ss);
    const double rstd = 1.0 / sqrt(ss / (double)(a.chunks * 8) + a.eps);
    if (lane == 0) a.rstd[row] = (float)rstd;

    // ---- apply ------------------------------------------------------------------------
    if constexpr (kMode == 1) {
        const auto rg = row_rsrc(a.gamma, row_bytes);
        const auto rb = row_rsrc(a.beta, kBeta ? row_bytes : 0);
        const auto ry = row_rsrc(a.y + base, row_bytes);
        u32x4 gw[kMaxChunks];
#pragma unroll
        for (int i = 0; i < kMaxChunks; ++i) gw[i] = bload(rg, (lane + kWave * i) * 16);
        // one chunk at a time (the fences keep the fp64 temporaries of one chunk
        // live at once, so the kernel keeps 4 waves per SIMD)
#pragma unroll
        for (int i = 0; i < kMaxChunks; ++i) {
            const int off = (lane + kWave * i) * 16;
            const u32x4 bw = kBeta ? bload(rb, off) : u32x4{0, 0, 0, 0};
            u32x4 out;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const double m0 = rd64<kBf16>((double)lo16<kBf16>(xo[i][e]) * rstd);
                const double m1 = rd64<kBf16>((double)hi16<kBf16>(xo[i][e]) * rstd);
                const double y0 = m0 * (double)lo16<kBf16>(gw[i][e]) + (double)lo16<kBf16>(bw[e]);
                const double y1 = m1 * (double)hi16<kBf16>(gw[i][e]) + (double)hi16<kBf16>(bw[e]);
                out[e] = pack16<kBf16>(to_f32_opaque(y0), to_f32_opaque(y1));
            }
            bstore(ry, off, out);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

template <bool kBf16>
int launch_norm(const NormArgs &a, int64_t mode, hipStream_t s) {
    const int64_t blocks = (a.m_pad + kRowsPerBlock - 1) / kRowsPerBlock;
    if (blocks > 0x7FFFFFFF) return CK_E_INVALID_ARG;
    const dim3 grid((unsigned)blocks), block(kRowsPerBlock * kWave);
    if (mode == 0) hipLaunchKernelGGL((add_rms_norm_kernel<kBf16, 0, false>), grid, block, 0, s, a);
    else if (mode == 2) hipLaunchKernelGGL((add_rms_norm_kernel<kBf16, 2, false>), grid, block, 0, s, a);
    else if (a.beta) hipLaunchKernelGGL((add_rms_norm_kernel<kBf16, 1, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((add_rms_norm_kernel<kBf16, 1, false>), grid, block, 0, s, a);
    CK_RETURN_LAUNCH();
}

}  // namespace
}  // namespace ck

extern "C" int ck_add_rms_norm_stats(const void *x1, const void *x2, const void *gamma, const void *beta,
                                     void *x_out, float *rstd, void *y, int64_t m_rows, int64_t k_dim,
                                     int dtype, int64_t mode, double eps, void *stream) {
    using namespace ck;
    if (dtype != CK_DTYPE_BF16 && dtype != CK_DTYPE_F16) return CK_E_INVALID_ARG;
    if (mode < 0 || mode > 2) return CK_E_INVALID_ARG;
    if (m_rows < 0 || k_dim <= 0 || k_dim > kMaxK || k_dim % 16 != 0) return CK_E_INVALID_ARG;
    if (!(eps > 0.0) || !std::isfinite(eps)) return CK_E_INVALID_ARG;
    if (m_rows == 0) return CK_OK;
    if (!x1 || !rstd) return CK_E_NULL_PTR;
    if (mode != 1 && !x2) return CK_E_NULL_PTR;
    if (mode == 0 && !x_out) return CK_E_NULL_PTR;
    if (mode == 1 && (!gamma || !y)) return CK_E_NULL_PTR;
    // rows, gamma and beta move 16 bytes per lane
    if (!aligned_to(x1, 16) || !aligned_to(x2, 16) || !aligned_to(gamma, 16) || !aligned_to(beta, 16) ||
        !aligned_to(x_out, 16) || !aligned_to(y, 16) || !aligned_to(rstd, 4))
        return CK_E_INVALID_ARG;
    NormArgs a;
    a.x1 = static_cast<const uint16_t *>(x1);
    a.x2 = static_cast<const uint16_t *>(x2);
    a.gamma = static_cast<const uint16_t *>(gamma);
    a.beta = mode == 1 ? static_cast<const uint16_t *>(beta) : nullptr;
    a.x_out = static_cast<uint16_t *>(x_out);
    a.rstd = rstd;
    a.y = static_cast<uint16_t *>(y);
    a.m_rows = m_rows;
    a.m_pad = (m_rows + kRstdGroup - 1) / kRstdGroup * kRstdGroup;
    a.chunks = (int)(k_dim / 8);
    a.eps = eps;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    return dtype == CK_DTYPE_BF16 ? launch_norm<true>(a, mode, s) : launch_norm<false>(a, mode, s);
}
