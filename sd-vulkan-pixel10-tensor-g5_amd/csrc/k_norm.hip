// GroupNorm(+SiLU) and LayerNorm for NHWC fp16 activations (memory-bound).
//
// GroupNorm replaces groupnorm_f32.comp / groupnorm_silu.comp (vk_engine.cpp:548-549):
// statistics per (image, group), eps inside the rsqrt, affine, optional SiLU.
// The reference reduces one group per 256-thread workgroup; here the image is
// split into pixel chunks so the whole chip streams the tensor:
//   pass 1 (stats): each block reads a chunk of pixels x all channels with 16-byte
//     loads, reduces per-group sum and sum of squares in fp32 and adds them to a
//     per-(image, group) fp64 accumulator with one atomic per group.  The
//     accumulator must be zero on entry (a fill kernel clears it once per forward).
//   pass 2 (apply): mean = S1/N, var = S2/N - mean^2 in fp64; then
//     y = x * a_c + b_c (a_c = rstd_g gamma_c, b_c = beta_c - mean_g a_c),
//     optional SiLU, 16-byte loads and stores.
// Both passes accept a second source concatenated along channels (the up-path
// skip concat, vk_engine.cpp:678-688), so the concat is never materialised.
//
// LayerNorm replaces layernorm_f32.comp (vk_engine.cpp:652): one wave per token,
// exact two-pass mean / variance in registers.
#include "sdu_internal.h"

namespace sdu {

static constexpr int GN_THREADS = 256;
static constexpr int GN_CHUNK_ELEMS = 8192;  // elements per stats / apply block
static constexpr int GN_MAXG = 32;
static constexpr int GN_MAXC = 2560;

struct GnGeom {
    int P, nchunk;  // P pixels per chunk
};

static GnGeom gn_geom(int HW, int C) {
    GnGeom g;
    g.P = (GN_CHUNK_ELEMS + C - 1) / C;
    if (g.P < 1) g.P = 1;
    g.nchunk = (HW + g.P - 1) / g.P;
    return g;
}

size_t groupnorm_acc_bytes(int B, int G) { return (size_t)B * G * 2 * sizeof(double); }

__device__ __forceinline__ uint4 load_src(const f16* x, const f16* x2, int C1, int C2, int64_t pix,
                                          int ch) {
    if (ch < C1) return *(const uint4*)(x + pix * C1 + ch);
    return *(const uint4*)(x2 + pix * C2 + (ch - C1));
}

__global__ __launch_bounds__(GN_THREADS) void gn_stats_kernel(const f16* x, const f16* x2, int C1,
                                                              int C2, int HW, int P, int G,
                                                              double* acc) {
    const int C = C1 + C2, V = C / 8, cpg = C / G;
    const int chunk = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const int p0 = chunk * P;
    const int pn = min(P, HW - p0);
    const int64_t pixb = (int64_t)b * HW + p0;
    // thread -> (vector column(s), pixel phase); R phases stride over the pixels
    const bool narrow = V <= GN_THREADS;
    const int R = narrow ? GN_THREADS / V : 1;
    const int ph = narrow ? tid / V : 0;
    __shared__ float s1[GN_MAXC], s2[GN_MAXC];  // [R][C] (narrow) or [C]
    for (int v0 = 0; v0 < (narrow ? 1 : V); v0 += GN_THREADS) {
        const int v = narrow ? tid % V : v0 + tid;
        const bool active = narrow ? tid < R * V : v < V;
        if (!active) continue;
        float a[8], q[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) { a[e] = 0.f; q[e] = 0.f; }
        for (int p = ph; p < pn; p += R) {
            const uint4 raw = load_src(x, x2, C1, C2, pixb + p, v * 8);
            const f16* hv = (const f16*)&raw;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float f = (float)hv[e];
                a[e] += f;
                q[e] += f * f;
            }
        }
        const int base = (narrow ? ph * C : 0) + v * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) { s1[base + e] = a[e]; s2[base + e] = q[e]; }
    }
    __syncthreads();
    // per-group reduction: 8 threads per group
    const int g = tid / 8, sub = tid % 8;
    float ga = 0.f, gq = 0.f;
    if (g < G) {
        const int n = R * cpg;
        for (int idx = sub; idx < n; idx += 8) {
            const int r = idx / cpg, ch = g * cpg + idx % cpg;
            ga += s1[r * C + ch];
            gq += s2[r * C + ch];
        }
    }
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) {
        ga += __shfl_xor(ga, off);
        gq += __shfl_xor(gq, off);
    }
    if (g < G && sub == 0) {
        atomicAdd(&acc[(b * G + g) * 2 + 0], (double)ga);
        atomicAdd(&acc[(b * G + g) * 2 + 1], (double)gq);
    }
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + __expf(-x)); }

__global__ __launch_bounds__(GN_THREADS) void gn_apply_kernel(const f16* x, const f16* x2, int C1,
                                                              int C2, const f16* gamma,
                                                              const f16* beta, f16* y, int HW,
                                                              int P, int G, float eps, int silu,
                                                              const double* acc) {
    const int C = C1 + C2, V = C / 8, cpg = C / G;
    const int chunk = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    __shared__ float tab[2 * GN_MAXC];
    __shared__ float s_mean[GN_MAXG], s_rstd[GN_MAXG];
    if (tid < G) {
        const double n = (double)HW * cpg;
        const double mean = acc[(b * G + tid) * 2 + 0] / n;
        const double var = fmax(acc[(b * G + tid) * 2 + 1] / n - mean * mean, 0.0);
        s_mean[tid] = (float)mean;
        s_rstd[tid] = (float)(1.0 / sqrt(var + (double)eps));
    }
    __syncthreads();
    for (int c = tid; c < C; c += GN_THREADS) {
        const int gg = c / cpg;
        const float sc = s_rstd[gg] * (float)gamma[c];
        tab[c] = sc;
        tab[C + c] = (float)beta[c] - s_mean[gg] * sc;
    }
    __syncthreads();
    const int p0 = chunk * P;
    const int pn = min(P, HW - p0);
    const int64_t pixb = (int64_t)b * HW + p0;
    for (int i = tid; i < pn * V; i += GN_THREADS) {
        const int p = i / V, v = i - p * V;
        const uint4 raw = load_src(x, x2, C1, C2, pixb + p, v * 8);
        const f16* hv = (const f16*)&raw;
        uint4 outv;
        f16* ov = (f16*)&outv;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int c = v * 8 + e;
            float z = (float)hv[e] * tab[c] + tab[C + c];
            if (silu) z = silu_f(z);
            ov[e] = (f16)z;
        }
        *(uint4*)(y + (pixb + p) * C + v * 8) = outv;
    }
}

__global__ void zero_kernel(uint4* p, int64_t n16) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n16) p[i] = make_uint4(0, 0, 0, 0);
}

hipError_t zero_launch(void* p, size_t bytes, hipStream_t s) {
    const int64_t n16 = (int64_t)((bytes + 15) / 16);
    if (n16 == 0) return hipSuccess;
    launch_timed("zero_kernel", 0.0, 16.0 * n16, [&] {
        hipLaunchKernelGGL(zero_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, s, (uint4*)p, n16);
    });
    return hipGetLastError();
}

hipError_t groupnorm_launch(const f16* x, const f16* x2, int C1, int C2, const f16* gamma,
                            const f16* beta, f16* y, int B, int HW, int G, float eps, int silu,
                            double* acc, hipStream_t s) {
    const int C = C1 + C2;
    if (G > GN_MAXG || C > GN_MAXC || C % G || C % 8 || C1 % 8 || (C2 && !x2)) return hipErrorInvalidValue;
    GnGeom g = gn_geom(HW, C);
    const double xbytes = 2.0 * B * HW * C;
    launch_timed("gn_stats_kernel", 0.0, xbytes, [&] {
        hipLaunchKernelGGL(gn_stats_kernel, dim3(g.nchunk, B), dim3(GN_THREADS), 0, s, x, x2, C1, C2, HW,
                           g.P, G, acc);
    });
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_timed("gn_apply_kernel", 0.0, 2.0 * xbytes, [&] {
        hipLaunchKernelGGL(gn_apply_kernel, dim3(g.nchunk, B), dim3(GN_THREADS), 0, s, x, x2, C1, C2, gamma,
                           beta, y, HW, g.P, G, eps, silu, (const double*)acc);
    });
    return hipGetLastError();
}

// ----------------------------------------------------------------- LayerNorm

template <int NV>  // vectors of 8 per lane (C <= NV * 512)
__global__ __launch_bounds__(256) void ln_kernel(const f16* x, const f16* gamma, const f16* beta,
                                                 f16* y, int T, int C, float eps) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    const int V = C / 8;
    float v[NV][8];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int vi = lane + i * 64;
        if (vi < V) {
            uint4 raw = *(const uint4*)(x + (int64_t)t * C + vi * 8);
            const f16* hv = (const f16*)&raw;
#pragma unroll
            for (int e = 0; e < 8; ++e) { v[i][e] = (float)hv[e]; s += v[i][e]; }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[i][e] = 0.f;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    const float mean = s / (float)C;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
        if (lane + i * 64 < V)
#pragma unroll
            for (int e = 0; e < 8; ++e) { const float d = v[i][e] - mean; q += d * d; }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) q += __shfl_xor(q, off);
    const float rstd = rsqrtf(q / (float)C + eps);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int vi = lane + i * 64;
        if (vi < V) {
            uint4 gr = *(const uint4*)(gamma + vi * 8), br = *(const uint4*)(beta + vi * 8);
            const f16* gh = (const f16*)&gr;
            const f16* bh = (const f16*)&br;
            uint4 outv;
            f16* ov = (f16*)&outv;
#pragma unroll
            for (int e = 0; e < 8; ++e) ov[e] = (f16)((v[i][e] - mean) * rstd * (float)gh[e] + (float)bh[e]);
            *(uint4*)(y + (int64_t)t * C + vi * 8) = outv;
        }
    }
}

hipError_t layernorm_launch(const f16* x, const f16* gamma, const f16* beta, f16* y, int T, int C,
                            float eps, hipStream_t s) {
    if (C % 8 || C > 4 * 512) return hipErrorInvalidValue;
    dim3 grid((T + 3) / 4), block(256);
    static const char* kNames[4] = {"ln_kernel<1>", "ln_kernel<2>", "ln_kernel<3>", "ln_kernel<4>"};
    const int v = C <= 512 ? 0 : C <= 1024 ? 1 : C <= 1536 ? 2 : 3;
    launch_timed(kNames[v], 0.0, 4.0 * T * C, [&] {
        if (v == 0) hipLaunchKernelGGL(ln_kernel<1>, grid, block, 0, s, x, gamma, beta, y, T, C, eps);
        else if (v == 1) hipLaunchKernelGGL(ln_kernel<2>, grid, block, 0, s, x, gamma, beta, y, T, C, eps);
        else if (v == 2) hipLaunchKernelGGL(ln_kernel<3>, grid, block, 0, s, x, gamma, beta, y, T, C, eps);
        else hipLaunchKernelGGL(ln_kernel<4>, grid, block, 0, s, x, gamma, beta, y, T, C, eps);
    });
    return hipGetLastError();
}

}  // namespace sdu
