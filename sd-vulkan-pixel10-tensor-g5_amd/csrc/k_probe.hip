// Calibration kernels: the practical ceilings of the GPU the library runs on, measured
// with the same clock and power state as the engine's kernels (the role of the
// reference's micro-benchmarks, VulkanBench.kt:10-19, which time single shaders).
//
//  * mfma_probe_kernel: dense f16 MFMA (v_mfma_f32_32x32x16_f16) from registers only,
//    eight waves per block, four independent accumulators per wave; block 0 records
//    the shader-clock and real-time (100 MHz) counters around its loop, so the run also
//    gives the shader clock under sustained MFMA load.
//  * copy_probe_kernel: streaming 16-byte copy, four loads in flight per thread.
#include "sdu_internal.h"

#include <algorithm>

namespace sdu {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(512) void mfma_probe_kernel(float* sink, long long* clk, int iters) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // operands of ordinary magnitude (data-dependent switching is part of the power draw)
    half8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = (_Float16)(((lane * 7 + e * 13) % 31 - 15) * 0.0625f);
        b[e] = (_Float16)(((wave * 5 + lane * 3 + e * 11) % 29 - 14) * 0.0625f);
    }
    floatx16 acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = floatx16{};
    const long long t0 = __builtin_amdgcn_s_memtime();
    const long long r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[i], 0, 0, 0);
    }
    const long long t1 = __builtin_amdgcn_s_memtime();
    const long long r1 = __builtin_amdgcn_s_memrealtime();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) s += acc[i][lane & 15];
    if (s == 1234.5f) sink[threadIdx.x] = s;  // keeps the MFMAs live; never true in practice
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        clk[0] = t1 - t0;
        clk[1] = r1 - r0;
    }
}

__global__ __launch_bounds__(256) void copy_probe_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                         int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * 1024;
    for (int64_t i = (int64_t)blockIdx.x * 1024 + threadIdx.x; i < n; i += stride) {
        uint4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (i + k * 256 < n) v[k] = src[i + k * 256];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (i + k * 256 < n) dst[i + k * 256] = v[k];
    }
}

hipError_t mfma_probe_launch(float* sink, long long* clk, int blocks, int iters, hipStream_t s) {
    if (blocks < 1 || iters < 1) return hipErrorInvalidValue;
    SDU_LAUNCH(mfma_probe_kernel, dim3(blocks), dim3(512), 0, s, sink, clk, iters);
    return hipGetLastError();
}

hipError_t copy_probe_launch(const void* src, void* dst, size_t bytes, hipStream_t s) {
    if (bytes % 16) return hipErrorInvalidValue;
    const int64_t n = (int64_t)(bytes / 16);
    const int blocks = (int)std::min<int64_t>((n + 1023) / 1024, 256 * 16);
    SDU_LAUNCH(copy_probe_kernel, dim3(blocks), dim3(256), 0, s, (const uint4*)src, (uint4*)dst, n);
    return hipGetLastError();
}

}  // namespace sdu
