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
// When one (image, group) slab is small (HW * C/G <= 32K elements: the 32x32 and
// smaller levels of the 64x64 UNet) and fits the registers of a 512-thread block,
// a single kernel does it all: the slab is loaded once into registers, the sums and
// sums of squares of x minus the group's first value are reduced in one pass (the
// shift keeps the one-pass variance free of cancellation when the mean dwarfs the
// spread), and the normalised values are stored -- one launch, one read and one
// write of the tensor.
//
// LayerNorm replaces layernorm_f32.comp (vk_engine.cpp:652): one wave per token,
// exact two-pass mean / variance in registers.
#include "sdu_internal.h"

#include <cstdio>

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

// Apply y = act((x - mean_g) * rstd_g * gamma + beta) to one image per blockIdx.y.
// The image is cut into chunks of GNA_VEC vectors of 8 channels (vector i: pixel
// i / V, channels 8 * (i % V) ..); block x handles chunks x, x + gridDim.x, ... and
// loads the next chunk while it writes the current one.  The first chunk's loads are
// issued before the group statistics are formed, so their latencies overlap.
// CST = false: acc holds the per-group sums [B][G][2] of gn_stats_kernel.
// CST = true: acc and st2 hold per-channel sums [B][C1][2] and [B][C2][2] written by
// the GEMM epilogues that produced x and x2; 8 threads add up each group's channels.
// 2 vectors per thread and chunk: the apply passes of B=2 took 127 against 136 us per 64x64
// forward and 309 against 318 us per 96x96 forward with 4 (B=16 434 against 431 us)
static constexpr int GNA_VPT = 2;
static constexpr int GNA_VEC = GN_THREADS * GNA_VPT;

// Branch-free loads of one chunk (index clamped to the last vector of the image).
__device__ __forceinline__ void gna_load(const f16* x, const f16* x2, int C1, int C2, int V, int nvec,
                                         int64_t pix0, int chunk, uint4 (&raw)[GNA_VPT]) {
#pragma unroll
    for (int k = 0; k < GNA_VPT; ++k) {
        const int i = min(chunk * GNA_VEC + k * GN_THREADS + (int)threadIdx.x, nvec - 1);
        const int p = i / V;
        const int ch = (i - p * V) * 8;
        const f16* src = ch < C1 ? x + (pix0 + p) * C1 + ch : x2 + (pix0 + p) * C2 + (ch - C1);
        raw[k] = *(const uint4*)src;
    }
}

template <bool CST>
__global__ __launch_bounds__(GN_THREADS) void gn_apply_kernel(const f16* x, const f16* x2, int C1,
                                                              int C2, const f16* gamma,
                                                              const f16* beta, f16* y, int HW, int G,
                                                              float eps, int silu, const double* acc,
                                                              const double* st2) {
    const int C = C1 + C2, V = C / 8, cpg = C / G;
    const int b = blockIdx.y, tid = threadIdx.x;
    const int nvec = HW * V;  // < 2^31 (checked by the launchers)
    const int nchunk = (nvec + GNA_VEC - 1) / GNA_VEC;
    const int64_t pix0 = (int64_t)b * HW;
    uint4 raw[GNA_VPT];
    gna_load(x, x2, C1, C2, V, nvec, pix0, blockIdx.x, raw);
    // gamma / beta of the channel octets this thread turns into table entries
    uint4 gv[2], bv[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int o = min(tid + j * GN_THREADS, V - 1);
        gv[j] = *(const uint4*)(gamma + o * 8);
        bv[j] = *(const uint4*)(beta + o * 8);
    }
    __shared__ float s_mean[GN_MAXG], s_rstd[GN_MAXG];
    __shared__ float4 tab[GN_MAXC / 2];  // per channel octet: 2 x (scale[4]), 2 x (shift[4])
    const double n = (double)HW * cpg;
    if (CST) {
        const int g = tid / 8, sub = tid % 8;
        double ga = 0.0, gq = 0.0;
        if (g < G) {
            // 4 channels per round, loads issued together (clamped, weighted 0 / 1)
            for (int i0 = sub; i0 < cpg; i0 += 32) {
                double2 qv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int c = g * cpg + min(i0 + 8 * u, cpg - 1);
                    const double* q = c < C1 ? acc + ((int64_t)b * C1 + c) * 2 : st2 + ((int64_t)b * C2 + (c - C1)) * 2;
                    qv[u] = *(const double2*)q;
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const bool use = i0 + 8 * u < cpg;
                    ga += use ? qv[u].x : 0.0;
                    gq += use ? qv[u].y : 0.0;
                }
            }
        }
#pragma unroll
        for (int off = 1; off < 8; off <<= 1) {
            ga += __shfl_xor(ga, off);
            gq += __shfl_xor(gq, off);
        }
        if (g < G && sub == 0) {
            const double mean = ga / n;
            const double var = fmax(gq / n - mean * mean, 0.0);
            s_mean[g] = (float)mean;
            s_rstd[g] = (float)(1.0 / sqrt(var + (double)eps));
        }
    } else if (tid < G) {
        const double mean = acc[(b * G + tid) * 2 + 0] / n;
        const double var = fmax(acc[(b * G + tid) * 2 + 1] / n - mean * mean, 0.0);
        s_mean[tid] = (float)mean;
        s_rstd[tid] = (float)(1.0 / sqrt(var + (double)eps));
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int o = tid + j * GN_THREADS;
        if (o >= V) break;
        const f16* hg = (const f16*)&gv[j];
        const f16* hb = (const f16*)&bv[j];
        float sc[8], sh[8];
        int g = o * 8 / cpg, nb = (g + 1) * cpg;  // group of channel o*8, its end
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if (o * 8 + e >= nb) { ++g; nb += cpg; }  // channels step by one: one group at a time
            sc[e] = s_rstd[g] * (float)hg[e];
            sh[e] = (float)hb[e] - s_mean[g] * sc[e];
        }
        tab[o * 4 + 0] = make_float4(sc[0], sc[1], sc[2], sc[3]);
        tab[o * 4 + 1] = make_float4(sc[4], sc[5], sc[6], sc[7]);
        tab[o * 4 + 2] = make_float4(sh[0], sh[1], sh[2], sh[3]);
        tab[o * 4 + 3] = make_float4(sh[4], sh[5], sh[6], sh[7]);
    }
    __syncthreads();
    for (int chunk = blockIdx.x; chunk < nchunk; chunk += gridDim.x) {
        uint4 nxt[GNA_VPT];
        const int cn = chunk + gridDim.x;
        if (cn < nchunk) gna_load(x, x2, C1, C2, V, nvec, pix0, cn, nxt);
#pragma unroll
        for (int k = 0; k < GNA_VPT; ++k) {
            const int i = chunk * GNA_VEC + k * GN_THREADS + tid;
            if (i >= nvec) continue;
            const int p = i / V, o = i - p * V;
            const float4 s0 = tab[o * 4 + 0], s1 = tab[o * 4 + 1], h0 = tab[o * 4 + 2], h1 = tab[o * 4 + 3];
            const float sc[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
            const float sh[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
            const f16* hv = (const f16*)&raw[k];
            uint4 outv;
            f16* ov = (f16*)&outv;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float z = (float)hv[e] * sc[e] + sh[e];
                if (silu) z = silu_f(z);
                ov[e] = (f16)z;
            }
            *(uint4*)(y + (pix0 + p) * C + o * 8) = outv;
        }
#pragma unroll
        for (int k = 0; k < GNA_VPT; ++k) raw[k] = nxt[k];
    }
}

// Blocks per image for gn_apply_kernel: about 2048 blocks in all, each taking the
// same number of chunks (+-1).
static int gna_blocks(int HW, int C, int B) {
    const int nchunk = (int)(((int64_t)HW * (C / 8) + GNA_VEC - 1) / GNA_VEC);
    const int per = (nchunk * B + 2047) / 2048;  // chunks per block
    return (nchunk + per - 1) / per;
}

__global__ void zero_kernel(uint4* p, int64_t n16) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n16) p[i] = make_uint4(0, 0, 0, 0);
}

// ----------------------------------------------------------------- single-pass GroupNorm

// 512 threads: the 8x8 - 32x32 slabs (2.5K - 20K elements) leave most of a 1024-thread
// block idle through its block reductions; per forward the GroupNorms took 418 against
// 434 us at B=2 64x64 and 898 against 976 us at B=16 (256 threads: 467 / 921 us).
static constexpr int GNF_THREADS = 512;

// Sums over the block of two floats per thread, in fp64 across waves; every thread
// gets the results.
__device__ __forceinline__ double2 gnf_block_sum2(float v, float u, double2* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        v += __shfl_xor(v, off);
        u += __shfl_xor(u, off);
    }
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (lane == 0) red[wave] = make_double2((double)v, (double)u);
    __syncthreads();
    double2 t = make_double2(0.0, 0.0);
#pragma unroll
    for (int w = 0; w < GNF_THREADS / 64; ++w) {
        t.x += red[w].x;
        t.y += red[w].y;
    }
    return t;
}

// One block per (group, image), grid G * B.  Thread t owns VW consecutive channels (vector
// t % (cpg/VW) of the group) and pixels t / (cpg/VW) + k*P (P = pixels per sweep of the
// block), k < EP: each load / store is one VW*2-byte vector at a fixed stride, and
// vectors never straddle the concat split (C1 and C/G are multiples of VW).
template <int VW>
struct GnfVec;
template <>
struct GnfVec<2> {
    typedef uint32_t T;
    static __device__ T load(__amdgpu_buffer_rsrc_t rs, int off) { return __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0); }
};
template <>
struct GnfVec<4> {
    typedef uint2 T;
    static __device__ T load(__amdgpu_buffer_rsrc_t rs, int off) {
        return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0));
    }
};
template <>
struct GnfVec<8> {
    typedef uint4 T;
    static __device__ T load(__amdgpu_buffer_rsrc_t rs, int off) {
        return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }
};

template <int EP, int VW>
__global__ __launch_bounds__(GNF_THREADS) void gn_fused_kernel(const f16* x, const f16* x2, int C1, int C2,
                                                               const f16* gamma, const f16* beta, f16* y,
                                                               int B, int HW, int G, float eps, int silu) {
    typedef typename GnfVec<VW>::T V;
    __shared__ double2 red[GNF_THREADS / 64];
    const int C = C1 + C2, cpg = C / G, vpg = cpg / VW;
    // Workgroups are dealt round-robin over the 8 XCDs, each with its own L2.  The
    // groups of one image share the 128-byte lines of every pixel row, so each XCD is
    // given whole images (consecutive groups): a line then crosses the fabric once.
    const int nblk = gridDim.x;
    const int q = (nblk & 7) ? (int)blockIdx.x : (int)(blockIdx.x & 7) * (nblk >> 3) + (int)(blockIdx.x >> 3);
    const int g = q % G, b = q / G, tid = threadIdx.x;
    const int P = GNF_THREADS / vpg;
    const int cv = tid % vpg, pp0 = tid / vpg;
    const bool act = pp0 < P;
    const int pp = act ? pp0 : P - 1;
    const int c = g * cpg + VW * cv;
    // All loads are issued before any is used, with 32-bit byte offsets into the
    // source; pixels past HW reload pixel HW-1 and are not accumulated.
    V raw[EP];
    {
        const bool first = c < C1;
        const int Cs = first ? C1 : C2;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(first ? x : x2), (short)0, B * HW * Cs * 2, 0x00020000);
        const int vo = ((int)b * HW * Cs + (first ? c : c - C1)) * 2;
#pragma unroll
        for (int k = 0; k < EP; ++k) raw[k] = GnfVec<VW>::load(rs, vo + min(pp + k * P, HW - 1) * Cs * 2);
    }
    // One pass over the values shifted by the group's first value (the same element
    // for every thread): the sum and sum of squares of x - shift do not cancel for a
    // group whose mean is large against its spread.  (x - shift is exact in fp32.)
    const int c0 = g * cpg;
    const float shift = (float)(c0 < C1 ? x[(int64_t)b * HW * C1 + c0] : x2[(int64_t)b * HW * C2 + (c0 - C1)]);
    float s = 0.f, ss = 0.f;
#pragma unroll
    for (int k = 0; k < EP; ++k) {
        if (act && pp + k * P < HW) {
            const f16* h = (const f16*)&raw[k];
#pragma unroll
            for (int e = 0; e < VW; ++e) {
                const float dv = (float)h[e] - shift;
                s += dv;
                ss += dv * dv;
            }
        }
    }
    const double n = (double)HW * cpg;
    const double2 t = gnf_block_sum2(s, ss, red);
    const double m1 = t.x / n;
    const double mean = shift + m1;
    const double var = fmax(t.y / n - m1 * m1, 0.0);
    const float mf = (float)mean;
    const float rstd = (float)(1.0 / sqrt(var + (double)eps));
    float sc[VW], sh[VW];
#pragma unroll
    for (int e = 0; e < VW; ++e) {
        sc[e] = rstd * (float)gamma[c + e];
        sh[e] = (float)beta[c + e] - mf * sc[e];
    }
    f16* dst = y + c;
#pragma unroll
    for (int k = 0; k < EP; ++k) {
        const int p = pp + k * P;
        if (!act || p >= HW) continue;
        const f16* h = (const f16*)&raw[k];
        V o;
        f16* oh = (f16*)&o;
#pragma unroll
        for (int e = 0; e < VW; ++e) {
            float z = (float)h[e] * sc[e] + sh[e];
            if (silu) z = silu_f(z);
            oh[e] = (f16)z;
        }
        *(V*)(dst + ((int64_t)b * HW + p) * C) = o;
    }
}

hipError_t zero_launch(void* p, size_t bytes, hipStream_t s) {
    const int64_t n16 = (int64_t)((bytes + 15) / 16);
    if (n16 == 0) return hipSuccess;
    launch_timed("zero_kernel", 0.0, 16.0 * n16, [&] {
        SDU_LAUNCH(zero_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, s, (uint4*)p, n16);
    });
    return hipGetLastError();
}

hipError_t groupnorm_launch(const f16* x, const f16* x2, int C1, int C2, const f16* gamma,
                            const f16* beta, f16* y, int B, int HW, int G, float eps, int silu,
                            double* acc, hipStream_t s) {
    const int C = C1 + C2;
    if (G > GN_MAXG || C > GN_MAXC || C % G || C % 8 || C1 % 8 || (C2 && !x2) || (int64_t)HW * C >= 0x7fffffff)
        return hipErrorInvalidValue;
    const double xbytes = 2.0 * B * HW * C;
    const int cpg = C / G;
    // channels per thread: the widest vector that divides the group and the concat split
    const int vw = (cpg % 8 == 0 && C1 % 8 == 0) ? 8 : (cpg % 4 == 0 && C1 % 4 == 0) ? 4 : 2;
    const int sweep = cpg % 2 == 0 ? GNF_THREADS / (cpg / vw) : 0;  // pixels per block sweep
    const int nsweep = sweep ? (HW + sweep - 1) / sweep : 1 << 30;
    // one block per (image, group) wins while the slab is small (up to 64K elements: the
    // 32x32 concat GroupNorms of B=2, 1920 channels 17.8 against 20.7 us for statistics +
    // apply, 1280 channels 13.9 against 17.8); larger slabs stream faster through the
    // chunked two-kernel path, which spreads them over the chip
    if (cpg % 2 == 0 && C1 % 2 == 0 && cpg / vw <= GNF_THREADS && nsweep <= 32 &&
        (int64_t)HW * cpg <= 65536 && 2 * (int64_t)B * HW * C < 0x7fffffff) {
        const int ep = nsweep <= 4 ? 4 : nsweep <= 8 ? 8 : nsweep <= 16 ? 16 : 32;
        char name[40];
        snprintf(name, sizeof name, "gn_fused_kernel<%d,%d>", ep, vw);
        const dim3 grid(G * B);
        launch_timed(name, 0.0, 2.0 * xbytes, [&] {
#define GNF_LAUNCH(EPV, VWV)                                                                                 \
    SDU_LAUNCH((gn_fused_kernel<EPV, VWV>), grid, dim3(GNF_THREADS), 0, s, x, x2, C1, C2, gamma, beta, y, \
                       B, HW, G, eps, silu)
#define GNF_VW(EPV)                      \
    if (vw == 8) GNF_LAUNCH(EPV, 8);     \
    else if (vw == 4) GNF_LAUNCH(EPV, 4); \
    else GNF_LAUNCH(EPV, 2)
            if (ep == 4) { GNF_VW(4); }
            else if (ep == 8) { GNF_VW(8); }
            else if (ep == 16) { GNF_VW(16); }
            else { GNF_VW(32); }
#undef GNF_VW
#undef GNF_LAUNCH
        });
        return hipGetLastError();
    }
    GnGeom g = gn_geom(HW, C);
    launch_timed("gn_stats_kernel", 0.0, xbytes, [&] {
        SDU_LAUNCH(gn_stats_kernel, dim3(g.nchunk, B), dim3(GN_THREADS), 0, s, x, x2, C1, C2, HW,
                           g.P, G, acc);
    });
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 agrid(gna_blocks(HW, C, B), B);
    launch_timed("gn_apply_kernel<0>", 0.0, 2.0 * xbytes, [&] {
        SDU_LAUNCH(gn_apply_kernel<false>, agrid, dim3(GN_THREADS), 0, s, x, x2, C1, C2, gamma, beta, y,
                           HW, G, eps, silu, (const double*)acc, (const double*)nullptr);
    });
    return hipGetLastError();
}

hipError_t groupnorm_apply_stats_launch(const f16* x, const f16* x2, int C1, int C2, const double* st1,
                                        const double* st2, const f16* gamma, const f16* beta, f16* y,
                                        int B, int HW, int G, float eps, int silu, hipStream_t s) {
    const int C = C1 + C2;
    if (G > GN_MAXG || C > GN_MAXC || C % G || C % 8 || C1 % 8 || (C2 && (!x2 || !st2)) || !st1 ||
        (int64_t)HW * C >= 0x7fffffff)
        return hipErrorInvalidValue;
    const double xbytes = 2.0 * B * HW * C;
    const dim3 agrid(gna_blocks(HW, C, B), B);
    launch_timed("gn_apply_kernel<1>", 0.0, 2.0 * xbytes, [&] {
        SDU_LAUNCH(gn_apply_kernel<true>, agrid, dim3(GN_THREADS), 0, s, x, x2, C1, C2, gamma, beta, y, HW,
                           G, eps, silu, st1, st2);
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
        if (v == 0) SDU_LAUNCH(ln_kernel<1>, grid, block, 0, s, x, gamma, beta, y, T, C, eps);
        else if (v == 1) SDU_LAUNCH(ln_kernel<2>, grid, block, 0, s, x, gamma, beta, y, T, C, eps);
        else if (v == 2) SDU_LAUNCH(ln_kernel<3>, grid, block, 0, s, x, gamma, beta, y, T, C, eps);
        else SDU_LAUNCH(ln_kernel<4>, grid, block, 0, s, x, gamma, beta, y, T, C, eps);
    });
    return hipGetLastError();
}

}  // namespace sdu
