// lse_merge.hip - LSE-space merge of two partial attention results (gfx950).
//
// Per row r (fp32 arithmetic, the operation order of the reference kernel
// ascend-kernel/csrc/ops/lse_merge/op_kernel/kernel_lse_merge.cpp:237-289):
//   m = max(l1, l2); w1 = exp(l1 - m); w2 = exp(l2 - m); s = w1 + w2
//   out = (o1 * w1 + o2 * w2) * (1 / s)            bf16 out: round to nearest even
//   lse_out = m + log(s)                            (optional)
// A -inf side has weight exactly 0 and contributes nothing (even non-finite O
// filler); two -inf sides give out = 0, lse_out = -inf (the reference has no
// guard there and produces NaN).
//
// Design: purely HBM-bound (about 10 B/element moved, 5 flops). Each thread
// owns 8 consecutive elements of one row (16 B of bf16 / 32 B of fp32 per
// operand, one vector load each); dim/8 threads share a row and recompute its
// two weights from the (L1-resident) lse values, which keeps the kernel a single
// streaming pass with no LDS and no synchronisation. A grid-stride loop covers
// any row count with a launch sized to the chip.
#include "ck_common.h"

namespace ck {
namespace {

template <int DT>
struct Vec8;  // 8 consecutive elements loaded as fp32

template <>
struct Vec8<CK_DTYPE_BF16> {
    static __device__ __forceinline__ void load(const void *base, int64_t idx, float (&x)[8]) {
        uint4 w = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(base) + idx);
        x[0] = bf16_lo(w.x); x[1] = bf16_hi(w.x);
        x[2] = bf16_lo(w.y); x[3] = bf16_hi(w.y);
        x[4] = bf16_lo(w.z); x[5] = bf16_hi(w.z);
        x[6] = bf16_lo(w.w); x[7] = bf16_hi(w.w);
    }
    static __device__ __forceinline__ void store(void *base, int64_t idx, const float (&x)[8]) {
        uint4 w;
        w.x = pack_bf16x2(x[0], x[1]);
        w.y = pack_bf16x2(x[2], x[3]);
        w.z = pack_bf16x2(x[4], x[5]);
        w.w = pack_bf16x2(x[6], x[7]);
        *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(base) + idx) = w;
    }
};

template <>
struct Vec8<CK_DTYPE_F32> {
    static __device__ __forceinline__ void load(const void *base, int64_t idx, float (&x)[8]) {
        const float4 *p = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(base) + idx);
        float4 a = p[0], b = p[1];
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    }
    static __device__ __forceinline__ void store(void *base, int64_t idx, const float (&x)[8]) {
        float4 *p = reinterpret_cast<float4 *>(reinterpret_cast<float *>(base) + idx);
        p[0] = make_float4(x[0], x[1], x[2], x[3]);
        p[1] = make_float4(x[4], x[5], x[6], x[7]);
    }
};

struct MergeArgs {
    const void *o1;
    const void *o2;
    const float *lse1;
    const float *lse2;
    void *out;
    float *lse_out;
    int64_t rows;
    int64_t dim;
    int64_t s1;
    int64_t s2;
};

template <int T1, int T2, int TO>
__global__ __launch_bounds__(256) void lse_merge_kernel(MergeArgs a) {
    const int64_t chunks_per_row = a.dim >> 3;
    const int64_t total = a.rows * chunks_per_row;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < total; c += stride) {
        const int64_t r = c / chunks_per_row;
        const int64_t e = c * 8;  // element offset (rows are contiguous, dim % 8 == 0)
        const float l1 = a.lse1[r * a.s1];
        const float l2 = a.lse2[r * a.s2];
        const float m = fmaxf(l1, l2);
        float x1[8], x2[8], y[8];
        Vec8<T1>::load(a.o1, e, x1);
        Vec8<T2>::load(a.o2, e, x2);
        if (m == -INFINITY) {
#pragma unroll
            for (int i = 0; i < 8; ++i) y[i] = 0.f;
            Vec8<TO>::store(a.out, e, y);
            if (a.lse_out != nullptr && c == r * chunks_per_row) a.lse_out[r] = -INFINITY;
            continue;
        }
        const float w1 = expf(l1 - m);
        const float w2 = expf(l2 - m);
        const float s = w1 + w2;
        const float sinv = 1.0f / s;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            // A zero weight contributes exactly nothing, even when that side's
            // O holds non-finite filler (an empty suffix).
            float t1 = (w1 == 0.f) ? 0.f : x1[i] * w1;
            float t2 = (w2 == 0.f) ? 0.f : x2[i] * w2;
            y[i] = (t1 + t2) * sinv;
        }
        Vec8<TO>::store(a.out, e, y);
        if (a.lse_out != nullptr && c == r * chunks_per_row) a.lse_out[r] = m + logf(s);
    }
}

template <int T1, int T2, int TO>
int launch_merge(const MergeArgs &a, hipStream_t stream) {
    const int64_t total = a.rows * (a.dim >> 3);
    int64_t blocks = (total + 255) / 256;
    // 256 CUs x 8 resident workgroups is enough to saturate HBM; the
    // grid-stride loop covers the rest.
    if (blocks > 2048) blocks = 2048;
    hipLaunchKernelGGL((lse_merge_kernel<T1, T2, TO>), dim3((unsigned)blocks), dim3(256), 0,
                       stream, a);
    CK_RETURN_LAUNCH();
}

}  // namespace
}  // namespace ck

using namespace ck;

extern "C" int ck_lse_merge(const void *o1, int o1_dtype, const void *o2, int o2_dtype,
                            const float *lse1, int64_t lse1_stride, const float *lse2,
                            int64_t lse2_stride, void *out, int out_dtype, float *lse_out,
                            int64_t rows, int64_t dim, void *stream) {
    if (rows < 0 || dim <= 0 || dim % 16 != 0) return CK_E_INVALID_ARG;
    if (lse1_stride < 1 || lse1_stride > 64 || lse2_stride < 1 || lse2_stride > 64)
        return CK_E_INVALID_ARG;
    auto okdt = [](int d) { return d == CK_DTYPE_BF16 || d == CK_DTYPE_F32; };
    if (!okdt(o1_dtype) || !okdt(o2_dtype) || !okdt(out_dtype)) return CK_E_INVALID_ARG;
    if (rows == 0) return CK_OK;
    if (!o1 || !o2 || !lse1 || !lse2 || !out) return CK_E_NULL_PTR;
    // 8 elements per lane per operand: 16 bytes of bf16, 32 of fp32
    if (!aligned_to(o1, 16) || !aligned_to(o2, 16) || !aligned_to(out, 16) || !aligned_to(lse1, 4) ||
        !aligned_to(lse2, 4) || !aligned_to(lse_out, 4))
        return CK_E_INVALID_ARG;
    MergeArgs a{o1, o2, lse1, lse2, out, lse_out, rows, dim, lse1_stride, lse2_stride};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int key = o1_dtype * 4 + o2_dtype * 2 + out_dtype;
    switch (key) {
        case 0: return launch_merge<0, 0, 0>(a, s);
        case 1: return launch_merge<0, 0, 1>(a, s);
        case 2: return launch_merge<0, 1, 0>(a, s);
        case 3: return launch_merge<0, 1, 1>(a, s);
        case 4: return launch_merge<1, 0, 0>(a, s);
        case 5: return launch_merge<1, 0, 1>(a, s);
        case 6: return launch_merge<1, 1, 0>(a, s);
        default: return launch_merge<1, 1, 1>(a, s);
    }
}
