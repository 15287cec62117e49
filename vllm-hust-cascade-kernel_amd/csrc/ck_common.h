// ck_common.h - shared device helpers for the gfx950 cascade-decode kernels.
//
// Everything here targets CDNA4 (gfx950) only: 64-lane wavefronts, MFMA
// bf16 tiles, 160 KB LDS per CU, 8 XCDs with private L2.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/cascade_kernels.h"

namespace ck {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(unsigned)))) unsigned u32x4;

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
// Two floats -> packed bf16 pair, round to nearest even (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
    const bf16x2v v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

#define CK_LDS __attribute__((address_space(3)))

// 16-byte global -> LDS DMA (gfx950 global_load_lds_dwordx4): lane l's 16 bytes
// land at lds_base + 16 * l; lds_base must be wave-uniform. Issued as inline asm
// so the compiler does not guard every later LDS read with a vmcnt(0) wait (it
// cannot prove transpose reads do not alias the DMA); callers wait explicitly
// with wait_vmcnt<N>() and a workgroup barrier before reading the data.
__device__ __forceinline__ void dma16(const void *g, CK_LDS void *lds_base) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_base);
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(m0), "v"(g)
                 : "memory", "m0");
}

// A raw buffer resource (V#) for `bytes` bytes from `base`: the 4 dwords
// buffer_load takes in SGPRs (wave-uniform by construction). A lane whose
// per-lane offset is at or past `bytes` reads zeros (the scalar offset is not
// range-checked).
typedef int ck_rsrc_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ ck_rsrc_t buf_rsrc(const void *base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    ck_rsrc_t r;
    r[0] = (int)__builtin_amdgcn_readfirstlane((uint32_t)a);
    r[1] = (int)(__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) & 0xffffu);  // stride 0
    r[2] = (int)__builtin_amdgcn_readfirstlane(bytes);
    r[3] = 0x00020000;
    return r;
}

// 16-byte buffer -> LDS DMA (buffer_load_dwordx4 ... lds): lane l reads
// rsrc.base + voff(l) + soff and its 16 bytes land at lds_base + 16 * l; voff is
// a per-lane 32-bit offset, soff and lds_base wave-uniform. Inline asm like dma16.
__device__ __forceinline__ void dma16_buf(const ck_rsrc_t &rsrc, int voff, int soff, CK_LDS void *lds_base) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_base);
    const int so = __builtin_amdgcn_readfirstlane(soff);
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(m0), "v"(voff), "s"(rsrc), "s"(so)
                 : "memory", "m0");
}

// 4-byte global -> LDS DMA (global_load_lds_dword): lane l's word lands at
// lds_base + 4 * l.
__device__ __forceinline__ void dma4(const void *g, CK_LDS void *lds_base) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_base);
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off"
                 :
                 : "s"(m0), "v"(g)
                 : "memory", "m0");
}

// Wait until at most N vector-memory operations of this wave are outstanding
// (gfx9 s_waitcnt encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Same with a wave-uniform count known only at run time. A count above the
// largest case waits for fewer outstanding operations, which is stricter.
__device__ __forceinline__ void wait_vmcnt_dyn(int n) {
#define CK_WAIT_CASE(N) \
    case N:             \
        wait_vmcnt<N>(); \
        break;
    switch (n) {
        CK_WAIT_CASE(0) CK_WAIT_CASE(1) CK_WAIT_CASE(2) CK_WAIT_CASE(3) CK_WAIT_CASE(4) CK_WAIT_CASE(5)
        CK_WAIT_CASE(6) CK_WAIT_CASE(7) CK_WAIT_CASE(8) CK_WAIT_CASE(9) CK_WAIT_CASE(10) CK_WAIT_CASE(11)
        CK_WAIT_CASE(12) CK_WAIT_CASE(13) CK_WAIT_CASE(14) CK_WAIT_CASE(15) CK_WAIT_CASE(16)
        CK_WAIT_CASE(17) CK_WAIT_CASE(18) CK_WAIT_CASE(19) CK_WAIT_CASE(20)
        default:
            if (n < 0) wait_vmcnt<0>();
            else wait_vmcnt<20>();
            break;
    }
#undef CK_WAIT_CASE
}

// LDS transpose read (gfx950 ds_read_b64_tr_b16). Within each 16-lane group,
// result lane i receives element (i % 4) of the 8-byte rows addressed by source
// lanes i/4, i/4+4, i/4+8, i/4+12. A group that addresses a 4-token x 16-element
// block (lane s -> token s/4, elements 4(s%4)..+3) therefore gets element i of
// the 4 tokens in lane i.
__device__ __forceinline__ uint2 lds_read_tr16(const CK_LDS char *p) {
    typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s16x4;
    s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((CK_LDS s16x4 *)p);
    return __builtin_bit_cast(uint2, v);
}

// 2^x on the hardware exp unit.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// max(x[l], x[l ^ 32]) in every lane: v_permlane32_swap exchanges the upper
// half of its first operand with the lower half of its second, so swapping x
// with itself leaves x[l ^ 32] in one result and x[l] in the other (a VALU
// exchange, no LDS round trip).
__device__ __forceinline__ float max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// A bounded wait that ran out: counted in `counter` (a global word the host
// reads back) from lane 0 with a vector atomic, so a broken invariant -- a wave
// that went on past a barrier or into a slot still in use, whose results are
// then wrong -- never passes silently.
__device__ __forceinline__ void count_giveup(unsigned int *counter) {
    if (__lane_id() == 0) __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup barrier (the stand-alone kernels) and a barrier among the waves of
// one role of a workgroup that runs two roles side by side: sense-free counting
// on two LDS words (arrivals, generation). A wave reads the generation before it
// counts itself in, so the generation cannot move before it has. The wait is
// bounded (2^24 sleeps, far beyond any real wait); a wait that runs out is
// counted in *giveups.
struct WgBarrier {
    __device__ __forceinline__ void sync() const { __syncthreads(); }
};
struct GroupBarrier {
    CK_LDS int *cnt;
    CK_LDS int *gen;
    int n;  // waves of the group
    unsigned int *giveups;
    __device__ __forceinline__ void sync() const {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's LDS writes are done
        const int g0 = __builtin_amdgcn_readfirstlane(*(volatile CK_LDS int *)gen);
        int old = 0;
        if (__lane_id() == 0) old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        old = __builtin_amdgcn_readfirstlane(old);
        if (old == n - 1) {
            if (__lane_id() == 0) {
                *cnt = 0;
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                *(volatile CK_LDS int *)gen = g0 + 1;
            }
        } else {
            int spin = 0;
            for (; *(volatile CK_LDS int *)gen == g0 && spin < (1 << 24); ++spin) __builtin_amdgcn_s_sleep(1);
            if (spin == (1 << 24)) count_giveup(giveups);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
};

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

// Host-side argument check: p is a multiple of n bytes (null counts as aligned).
inline bool aligned_to(const void *p, uintptr_t n) { return reinterpret_cast<uintptr_t>(p) % n == 0; }

// Raises a kernel's dynamic-LDS limit to `bytes` on the current device, once
// per device (bit d of `done` records device d). Safe to call from several
// threads at once: the attribute call is idempotent and the bit is set
// atomically after it succeeds. Returns CK_OK or the hipError_t.
inline int ensure_dynamic_lds(const void *fn, int bytes, std::atomic<uint64_t> &done) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return static_cast<int>(e);
    const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t)1 << dev : 0;
    if (bit && (done.load(std::memory_order_acquire) & bit)) return CK_OK;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return static_cast<int>(e);
    done.fetch_or(bit, std::memory_order_release);
    return CK_OK;
}

}  // namespace ck

// Host-side launch check: converts a launch error into the ABI's return code.
#define CK_RETURN_LAUNCH()                                     \
    do {                                                       \
        hipError_t _e = hipGetLastError();                     \
        return _e == hipSuccess ? CK_OK : static_cast<int>(_e); \
    } while (0)
