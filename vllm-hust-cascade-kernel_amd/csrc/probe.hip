// probe.hip - measured ceilings for the roofline denominators (benchmark-only
// entry points; no production path calls them).
//
// Role: the reference keeps a benchmark-only bandwidth probe beside its
// production ops (ascend-kernel/csrc/ops/bw_probe/design.md:1-30: the same
// bytes with the compute taken out, to measure what an access pattern can
// reach). Here the two ceilings the cascade and GEMM numbers are judged
// against are measured on the GPU the bench runs on:
// * ck_bw_probe: a streaming read of `bytes` (variant 0; each lane XOR-folds
//   its 16-byte loads and writes one word to `sink`) or a copy of `bytes`
//   (variant 1), grid-stride with four loads per lane in flight and 8
//   workgroups of 4 waves per CU -- the occupancy at which a plain stream
//   reaches its highest rate on MI355X.
// * ck_mfma_probe: back-to-back v_mfma_f32_32x32x16_bf16 on register operands
//   with 8 independent accumulators per wave (no memory traffic in the loop),
//   2 waves per SIMD; FLOPs = 2 * 32 * 32 * 16 per MFMA.
#include "ck_common.h"

namespace ck {
namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeGrid = 2048;  // 8 workgroups of 4 waves per CU on 256 CUs
static_assert((int64_t)kProbeGrid * kProbeThreads * 4 == CK_PROBE_SINK_BYTES, "one sink word per thread");

__global__ __launch_bounds__(kProbeThreads) void bw_read_kernel(const uint4 *__restrict__ p, int64_t n,
                                                              unsigned *__restrict__ sink) {
    int64_t i = (int64_t)blockIdx.x * kProbeThreads + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * kProbeThreads;
    unsigned acc = 0;
#pragma unroll 4
    for (; i < n; i += stride) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    sink[(int64_t)blockIdx.x * kProbeThreads + threadIdx.x] = acc;
}

__global__ __launch_bounds__(kProbeThreads) void bw_copy_kernel(const uint4 *__restrict__ p,
                                                              uint4 *__restrict__ q, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * kProbeThreads + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * kProbeThreads;
#pragma unroll 4
    for (; i < n; i += stride) q[i] = p[i];
}

__global__ __launch_bounds__(kProbeThreads) void mfma_rate_kernel(int64_t iters, float *__restrict__ sink) {
    const int lane = threadIdx.x & 63;
    // operands that depend on the lane (the compiler cannot fold the products)
    const float fa = 1.0f + 1e-3f * lane, fb = 1.0f - 1e-3f * lane;
    bf16x8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = (__bf16)(fa + e * 1e-2f);
        b[e] = (__bf16)(fb - e * 1e-2f);
    }
    f32x16 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;
    for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) s += acc[j][e];
    sink[(int64_t)blockIdx.x * kProbeThreads + threadIdx.x] = s;
}

}  // namespace
}  // namespace ck

using namespace ck;

extern "C" int ck_bw_probe(const void *src, void *dst, int64_t bytes, int variant, void *sink, int64_t sink_bytes,
                           void *stream) {
    if (bytes < 16 || bytes % 16 != 0) return CK_E_INVALID_ARG;
    if (variant != 0 && variant != 1) return CK_E_INVALID_ARG;
    if (!src || (variant == 1 && !dst) || (variant == 0 && !sink)) return CK_E_NULL_PTR;
    if (!aligned_to(src, 16) || !aligned_to(dst, 16) || !aligned_to(sink, 4)) return CK_E_INVALID_ARG;
    if (variant == 0 && sink_bytes < CK_PROBE_SINK_BYTES) return CK_E_WORKSPACE;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int64_t n = bytes / 16;
    if (variant == 0)
        hipLaunchKernelGGL(bw_read_kernel, dim3(kProbeGrid), dim3(kProbeThreads), 0, st,
                           static_cast<const uint4 *>(src), n, static_cast<unsigned *>(sink));
    else
        hipLaunchKernelGGL(bw_copy_kernel, dim3(kProbeGrid), dim3(kProbeThreads), 0, st,
                           static_cast<const uint4 *>(src), static_cast<uint4 *>(dst), n);
    CK_RETURN_LAUNCH();
}

extern "C" int ck_mfma_probe(int64_t iterations, void *sink, int64_t sink_bytes, double *flops, void *stream) {
    if (iterations <= 0 || iterations > ((int64_t)1 << 24)) return CK_E_INVALID_ARG;
    if (!sink || !flops) return CK_E_NULL_PTR;
    if (!aligned_to(sink, 4)) return CK_E_INVALID_ARG;
    constexpr int kGrid = 512;  // 2 workgroups of 4 waves per CU: 2 waves per SIMD
    if (sink_bytes < CK_PROBE_SINK_BYTES) return CK_E_WORKSPACE;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(mfma_rate_kernel, dim3(kGrid), dim3(kProbeThreads), 0, st, iterations,
                       static_cast<float *>(sink));
    *flops = (double)kGrid * (kProbeThreads / 64) * (double)iterations * 16.0 * (2.0 * 32 * 32 * 16);
    CK_RETURN_LAUNCH();
}
