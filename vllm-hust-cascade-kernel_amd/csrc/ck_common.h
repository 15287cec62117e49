// ck_common.h - shared device helpers for the gfx950 cascade-decode kernels.
//
// Everything here targets CDNA4 (gfx950) only: 64-lane wavefronts, MFMA
// bf16 tiles, 160 KB LDS per CU, 8 XCDs with private L2.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/cascade_kernels.h"

namespace ck {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

constexpr int kWave = 64;
constexpr int kNumXcd = 8;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---- bf16 <-> fp32 -----------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// float -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return ((u >> 16) | 0x40u) & 0xFFFFu;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// 2^x on the hardware exp unit.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- XCD-aware block order ----------------------------------------------------
// Workgroups are dispatched round-robin over the 8 XCDs (block b runs on XCD
// b % 8). Remap so that consecutive logical work ids land on the same XCD and
// share its L2: logical = xcd * per_xcd + b / 8 for the first floor(n/8)*8 blocks.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t b, uint32_t n) {
    uint32_t full = (n / kNumXcd) * kNumXcd;
    if (b >= full) return b;
    uint32_t per = n / kNumXcd;
    return (b % kNumXcd) * per + b / kNumXcd;
}

}  // namespace ck

// Host-side launch check: converts a launch error into the ABI's return code.
#define CK_RETURN_LAUNCH()                                     \
    do {                                                       \
        hipError_t _e = hipGetLastError();                     \
        return _e == hipSuccess ? CK_OK : static_cast<int>(_e); \
    } while (0)
