// Layout conversion, elementwise ops, the fused CFG + LCM step, and the seeded
// weight generator.
//
//  * nchw_to_nhwc: the C-ABI edge.  The reference's boundary tensors are fp32
//    [C, B*HW] / NCHW (vk_engine.cpp:874-913); inside, activations are NHWC fp16.
//  * silu / add / add_bias / geglu: SILU, ADD, AB2, GEGLU shaders
//    (silu_f32.comp, add_f32.comp, addbias2_f32.comp, geglu_f32.comp) as
//    standalone ops of the C ABI.  Inside the UNet graph they are fused into GEMM
//    epilogues.
//  * lcm_step: CFG combine (VulkanUnetPipeline.kt:86) + LcmScheduler.step
//    (LcmScheduler.kt:56-82) in one pass, also writing the next UNet input.
//  * gen: device side of the seeded generator specified in oracle/gen.c.
#include "sdu_internal.h"

namespace sdu {

__global__ void nchw_to_nhwc_kernel(const float* src, f16* dst, int B, int Bsrc, int C, int Cpad,
                                    int HW, int tanh_clamp) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)B * HW * Cpad;
    if (i >= total) return;
    const int c = (int)(i % Cpad);
    const int64_t pix = i / Cpad;
    const int b = (int)(pix / HW), p = (int)(pix % HW);
    float v = 0.f;
    if (c < C) v = src[((int64_t)(b % Bsrc) * C + c) * HW + p];
    if (tanh_clamp) v = 3.0f * tanhf(v * (1.0f / 3.0f));
    dst[i] = (f16)v;
}

hipError_t nchw_to_nhwc_launch(const float* src, f16* dst, int B, int Bsrc, int C, int Cpad, int HW,
                               hipStream_t s, int tanh_clamp) {
    const int64_t total = (int64_t)B * HW * Cpad;
    launch_timed("nchw_to_nhwc_kernel", 0.0, 4.0 * Bsrc * C * HW + 2.0 * total, [&] {
        SDU_LAUNCH(nchw_to_nhwc_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                           src, dst, B, Bsrc, C, Cpad, HW, tanh_clamp);
    });
    return hipGetLastError();
}

// The VAE decoder's input: the UNet latent z (NCHW fp32 [B,4,H,W]) divided by the
// scaling factor and through post_quant_conv (1x1, 4 -> 4, fp32 arithmetic), as NHWC
// fp16 [B,H,W,8] with channels 4..7 zero.  One thread per pixel, one 16-byte store.
__global__ void vae_stage_kernel(const float* z, const f16* w, const f16* bias, f16* y, int B, int HW,
                                 float inv_scale) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)B * HW) return;
    const int b = (int)(i / HW), p = (int)(i % HW);
    float zi[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) zi[c] = z[((int64_t)b * 4 + c) * HW + p] * inv_scale;
    uint4 o = make_uint4(0, 0, 0, 0);
    f16* oh = (f16*)&o;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        float acc = (float)bias[c];
#pragma unroll
        for (int k = 0; k < 4; ++k) acc += (float)w[c * 4 + k] * zi[k];
        oh[c] = (f16)acc;
    }
    *(uint4*)(y + i * 8) = o;
}

hipError_t vae_stage_launch(const float* z, const f16* w, const f16* bias, f16* y, int B, int HW, float inv_scale,
                            hipStream_t s) {
    if (B < 1 || HW < 1) return hipErrorInvalidValue;
    const int64_t n = (int64_t)B * HW;
    launch_timed("vae_stage_kernel", 32.0 * n, 16.0 * n + 16.0 * n, [&] {
        SDU_LAUNCH(vae_stage_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, z, w, bias, y, B, HW,
                   inv_scale);
    });
    return hipGetLastError();
}

// Softmax of the rows of an fp32 score matrix [rows][n] (row stride n) times `scale`,
// stored fp16 [rows][n]: one 256-thread block per row; max, then the sum of
// 2^((s - max) * scale * log2 e), then the normalised values.
__device__ __forceinline__ float block_reduce(float v, bool is_max, float* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(v, off);
        v = is_max ? fmaxf(v, o) : v + o;
    }
    const int w = threadIdx.x >> 6;
    __syncthreads();  // red reused across calls
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    v = red[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) v = is_max ? fmaxf(v, red[i]) : v + red[i];
    return v;
}

__global__ __launch_bounds__(256) void softmax_rows_kernel(const float* s, f16* p, int n, float c) {
    __shared__ float red[4];
    const float* sr = s + (int64_t)blockIdx.x * n;
    f16* pr = p + (int64_t)blockIdx.x * n;
    float m = -INFINITY;
    for (int j = threadIdx.x; j < n; j += 256) m = fmaxf(m, sr[j]);
    m = block_reduce(m, true, red);
    float sum = 0.f;
    for (int j = threadIdx.x; j < n; j += 256) sum += __builtin_amdgcn_exp2f((sr[j] - m) * c);
    sum = block_reduce(sum, false, red);
    const float inv = 1.0f / sum;
    for (int j = threadIdx.x; j < n; j += 256) pr[j] = (f16)(__builtin_amdgcn_exp2f((sr[j] - m) * c) * inv);
}

hipError_t softmax_rows_launch(const float* s, f16* p, int rows, int n, float scale, hipStream_t st) {
    if (rows < 1 || n < 1) return hipErrorInvalidValue;
    const float c = scale * 1.4426950408889634f;
    launch_timed("softmax_rows_kernel", 0.0, (double)rows * n * 6.0, [&] {
        SDU_LAUNCH(softmax_rows_kernel, dim3((unsigned)rows), dim3(256), 0, st, s, p, n, c);
    });
    return hipGetLastError();
}

// The UNet forward's inputs in one launch, outside its graph: the latent NCHW fp32
// [B,C,H,W] -> NHWC fp16 [B,H,W,Cpad] (channels >= C zero), the context fp32 -> fp16,
// and ntemb floats of the time projection copied.  Threads [0, nlat) take the latent,
// the next nctx the context, the next ntemb the time projection, the next nzero16 clear
// 16-byte words at zero_dst; thread 0 also stores out_ptr to *out_slot (when set).
__global__ void stage_in_kernel(const float* lat, const float* ctx, const float* temb, f16* lat16, f16* ctx16,
                                float* temb_dst, int B, int C, int Cpad, int HW, int64_t nctx, int ntemb,
                                uint4* zero_dst, int64_t nzero16, void** out_slot, void* out_ptr) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i == 0 && out_slot) *out_slot = out_ptr;
    const int64_t nlat = (int64_t)B * HW * Cpad;
    if (i < nlat) {
        const int c = (int)(i % Cpad);
        const int64_t pix = i / Cpad;
        const int b = (int)(pix / HW), p = (int)(pix % HW);
        lat16[i] = (f16)(c < C ? lat[((int64_t)b * C + c) * HW + p] : 0.f);
        return;
    }
    i -= nlat;
    if (i < nctx) {
        ctx16[i] = (f16)ctx[i];
        return;
    }
    i -= nctx;
    if (i < ntemb) {
        temb_dst[i] = temb[i];
        return;
    }
    i -= ntemb;
    if (i < nzero16) zero_dst[i] = make_uint4(0, 0, 0, 0);
}

hipError_t stage_in_launch(const float* lat, const float* ctx, const float* temb, f16* lat16, f16* ctx16,
                           float* temb_dst, int B, int C, int Cpad, int HW, int64_t nctx, int ntemb,
                           hipStream_t s, void* zero_dst, size_t zero_bytes, void** out_slot, void* out_ptr) {
    const int64_t nlat = (int64_t)B * HW * Cpad, nz = (int64_t)((zero_bytes + 15) / 16);
    const int64_t total = nlat + nctx + ntemb + nz;
    launch_timed("stage_in_kernel", 0.0, 4.0 * B * C * HW + 2.0 * nlat + 6.0 * nctx + 8.0 * ntemb + 16.0 * nz, [&] {
        SDU_LAUNCH(stage_in_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, lat, ctx, temb, lat16,
                   ctx16, temb_dst, B, C, Cpad, HW, nctx, ntemb, (uint4*)zero_dst, nz, out_slot, out_ptr);
    });
    return hipGetLastError();
}

// One thread per 8 channels of one token.
__global__ void embed_kernel(const int32_t* ids, const f16* tok, const f16* pos, f16* out, int B, int S, int C,
                             int vocab) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int cpr = C / 8;
    if (i >= (int64_t)B * S * cpr) return;
    const int64_t row = i / cpr;
    const int c8 = (int)(i - row * cpr) * 8;
    const int t = (int)(row % S);
    const int id = min(max(ids[row], 0), vocab - 1);
    const uint4 a = *(const uint4*)(tok + (int64_t)id * C + c8);
    const uint4 p = *(const uint4*)(pos + (int64_t)t * C + c8);
    const f16* ah = (const f16*)&a;
    const f16* ph = (const f16*)&p;
    uint4 o;
    f16* oh = (f16*)&o;
#pragma unroll
    for (int e = 0; e < 8; ++e) oh[e] = (f16)((float)ah[e] + (float)ph[e]);
    *(uint4*)(out + row * C + c8) = o;
}

hipError_t embed_launch(const int32_t* ids, const f16* tok, const f16* pos, f16* out, int B, int S, int C,
                        int vocab, hipStream_t s) {
    if (B < 1 || S < 1 || C % 8 || vocab < 1) return hipErrorInvalidValue;
    const int64_t total = (int64_t)B * S * (C / 8);
    launch_timed("embed_kernel", 0.0, 4.0 * B * S * C + 4.0 * B * S, [&] {
        SDU_LAUNCH(embed_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, ids, tok, pos, out, B, S, C,
                   vocab);
    });
    return hipGetLastError();
}

__global__ void f32_to_f16_kernel(const float* src, f16* dst, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = (f16)src[i];
}
__global__ void f16_to_f32_kernel(const f16* src, float* dst, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = (float)src[i];
}
hipError_t f32_to_f16_launch(const float* src, f16* dst, int64_t n, hipStream_t s) {
    launch_timed("f32_to_f16_kernel", 0.0, 6.0 * n, [&] {
        SDU_LAUNCH(f32_to_f16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, dst, n);
    });
    return hipGetLastError();
}
hipError_t f16_to_f32_launch(const f16* src, float* dst, int64_t n, hipStream_t s) {
    launch_timed("f16_to_f32_kernel", 0.0, 6.0 * n, [&] {
        SDU_LAUNCH(f16_to_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, dst, n);
    });
    return hipGetLastError();
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + __expf(-x)); }

// float -> fp16 (round to nearest even) of a value that must first be rounded to
// float: the empty asm pins the float intermediate, otherwise the compiler folds
// (f16)(float)double into one double -> half rounding, which differs from the
// two-step rounding the generator and the scheduler specify.
__device__ __forceinline__ f16 f16_via_f32(float f) {
    asm volatile("" : "+v"(f));
    return (f16)f;
}

// Elementwise ops over n fp16 values: 8 per thread with 16-byte loads and stores when
// every pointer is 16-byte aligned, one per thread otherwise.
template <bool V8>
__global__ void silu_kernel(const f16* x, f16* y, int64_t n) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (V8) {
        const int64_t i = t * 8;
        if (i + 8 <= n) {
            const uint4 v = *(const uint4*)(x + i);
            const f16* h = (const f16*)&v;
            uint4 o;
            f16* oh = (f16*)&o;
#pragma unroll
            for (int e = 0; e < 8; ++e) oh[e] = (f16)silu_f((float)h[e]);
            *(uint4*)(y + i) = o;
        } else {
            for (int64_t j = i; j < n; ++j) y[j] = (f16)silu_f((float)x[j]);
        }
    } else if (t < n) {
        y[t] = (f16)silu_f((float)x[t]);
    }
}
template <bool V8>
__global__ void add_kernel(const f16* a, const f16* b, f16* y, int64_t n) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (V8) {
        const int64_t i = t * 8;
        if (i + 8 <= n) {
            const uint4 u = *(const uint4*)(a + i), v = *(const uint4*)(b + i);
            const f16* ha = (const f16*)&u;
            const f16* hb = (const f16*)&v;
            uint4 o;
            f16* oh = (f16*)&o;
#pragma unroll
            for (int e = 0; e < 8; ++e) oh[e] = (f16)((float)ha[e] + (float)hb[e]);
            *(uint4*)(y + i) = o;
        } else {
            for (int64_t j = i; j < n; ++j) y[j] = (f16)((float)a[j] + (float)b[j]);
        }
    } else if (t < n) {
        y[t] = (f16)((float)a[t] + (float)b[t]);
    }
}
__global__ void add_bias_kernel(f16* y, const f16* bias, int64_t n, int C) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = (f16)((float)y[i] + (float)bias[i % C]);
}
__global__ void geglu_kernel(const f16* g, f16* y, int T, int C2) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)T * C2) return;
    const int64_t t = i / C2;
    const int c = (int)(i - t * C2);
    const float a = (float)g[t * 2 * C2 + c], bb = (float)g[t * 2 * C2 + C2 + c];
    y[i] = (f16)(a * gelu_erf(bb));
}

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

hipError_t silu_launch(const f16* x, f16* y, int64_t n, hipStream_t s) {
    const bool v8 = al16(x) && al16(y);
    const int64_t th = v8 ? (n + 7) / 8 : n;
    launch_timed(v8 ? "silu_kernel<1>" : "silu_kernel<0>", 0.0, 4.0 * n, [&] {
        if (v8) SDU_LAUNCH(silu_kernel<true>, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s, x, y, n);
        else SDU_LAUNCH(silu_kernel<false>, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s, x, y, n);
    });
    return hipGetLastError();
}
hipError_t add_launch(const f16* a, const f16* b, f16* y, int64_t n, hipStream_t s) {
    const bool v8 = al16(a) && al16(b) && al16(y);
    const int64_t th = v8 ? (n + 7) / 8 : n;
    launch_timed(v8 ? "add_kernel<1>" : "add_kernel<0>", 0.0, 6.0 * n, [&] {
        if (v8) SDU_LAUNCH(add_kernel<true>, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s, a, b, y, n);
        else SDU_LAUNCH(add_kernel<false>, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s, a, b, y, n);
    });
    return hipGetLastError();
}
hipError_t add_bias_launch(f16* y, const f16* bias, int64_t n, int C, hipStream_t s) {
    SDU_LAUNCH(add_bias_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, y, bias, n, C);
    return hipGetLastError();
}
hipError_t geglu_launch(const f16* g, f16* y, int T, int C2, hipStream_t s) {
    const int64_t n = (int64_t)T * C2;
    SDU_LAUNCH(geglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g, y, T, C2);
    return hipGetLastError();
}

// ----------------------------------------------------------------- CFG + LCM step

__global__ void lcm_step_kernel(float* x, const float* eps2, const float* noise, int64_t n,
                                LcmCoeffs c, f16* unet_in, int C, int HW, int Cpad) {
    // Every operation rounds separately, in the order of the host formulas, so the device
    // loop reproduces a host loop bit for bit: contraction into FMAs is off for the
    // expressions below (a fused u + s (c - u) differs whenever s (c - u) is inexact).
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    // eps = u + s (c - u) in float32 (VulkanUnetPipeline.kt:86)
    const float ec = eps2[i];
    const float g = c.guidance_dev ? *c.guidance_dev : c.guidance;
    float eps = ec;
    if (!c.cond_only) {
        const float eu = eps2[n + i];
        const float d = ec - eu;
        const float sd = g * d;
        eps = eu + sd;
    }
    // LcmScheduler.kt:70-79 in float64
    const double xv = (double)x[i];
    const double be = c.sqrt_beta * (double)eps;
    const double x0 = (xv - be) / c.sqrt_alpha;
    const double t0 = c.c_out * x0, t1 = c.c_skip * xv;
    const double den = t0 + t1;
    float out;
    if (c.last) {
        out = (float)den;
    } else {
        const double u0 = c.sqrt_alpha_prev * den, u1 = c.sqrt_beta_prev * (double)noise[i];
        out = (float)(u0 + u1);
    }
    x[i] = out;
    if (unet_in) {
        // i indexes the NCHW latent [C, HW]; write NHWC [2, HW, Cpad] for both slots
        const int ch = (int)(i / HW), p = (int)(i % HW);
        const f16 h = f16_via_f32(out);
        unet_in[(int64_t)p * Cpad + ch] = h;
        unet_in[((int64_t)HW + p) * Cpad + ch] = h;
    }
}

hipError_t lcm_step_launch(float* x, const float* eps2, const float* noise, int64_t n, LcmCoeffs c,
                           f16* unet_in, int C, int HW, int Cpad, hipStream_t s) {
    launch_timed("lcm_step_kernel", 0.0, 16.0 * n, [&] {
        SDU_LAUNCH(lcm_step_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, eps2,
                           noise, n, c, unet_in, C, HW, Cpad);
    });
    return hipGetLastError();
}

__global__ void fill_f32_kernel(float* p, float v, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

hipError_t fill_f32_launch(float* p, float v, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    launch_timed("fill_f32_kernel", 0.0, 4.0 * n, [&] {
        SDU_LAUNCH(fill_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, v, n);
    });
    return hipGetLastError();
}

// ----------------------------------------------------------------- generator

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ULL;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

uint64_t splitmix64(uint64_t x) { return mix64(x); }

uint64_t fnv1a64(const char* s) {
    uint64_t h = 0xCBF29CE484222325ULL;
    for (; *s; ++s) { h ^= (uint8_t)*s; h *= 0x100000001B3ULL; }
    return h;
}

__global__ void gen_kernel(f16* dst, GenDesc g) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= g.n) return;
    if (g.constant) { dst[i] = f16_via_f32((float)g.mean); return; }
    int64_t ci;  // canonical index
    if (g.layout == GL_CONV_OHWI) {
        // device [co, kh, kw, ci_pad] -> canonical [co, ci, kh, kw]
        const int c = (int)(i % g.ci_pad);
        int64_t r = i / g.ci_pad;
        const int kx = (int)(r % g.kw); r /= g.kw;
        const int ky = (int)(r % g.kh);
        const int o = (int)(r / g.kh);
        if (c >= g.ci) { dst[i] = (f16)0.f; return; }
        ci = (((int64_t)o * g.ci + c) * g.kh + ky) * g.kw + kx;
    } else if (g.layout == GL_GEGLU_PERM) {
        // device row r: 64-row blocks [32 rows of the first half | 32 of the second]
        const int64_t r = i / g.cols;
        const int col = (int)(i % g.cols);
        const int64_t blk = r / 64, w = r % 64;
        const int64_t cr = (w < 32) ? blk * 32 + w : (int64_t)g.half_rows + blk * 32 + (w - 32);
        ci = cr * g.cols + col;
    } else {
        ci = i;
    }
    const uint64_t h1 = mix64(g.key + 2ULL * (uint64_t)ci);
    const uint64_t h2 = mix64(g.key + 2ULL * (uint64_t)ci + 1ULL);
    const double u1 = (double)((h1 >> 11) + 1ULL) * 0x1.0p-53;
    const double u2 = (double)(h2 >> 11) * 0x1.0p-53;
    const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    dst[i] = f16_via_f32((float)__dadd_rn(g.mean, __dmul_rn(g.stdv, z)));
}

// fp32 N(0, 1) draws of the same generator (TpuUnetPipeline.kt:100 draws the per-step
// noise as FloatArray(latSize) { gaussian(rnd) }): value = float(z).
__global__ void gen_normal_f32_kernel(float* dst, int64_t n, uint64_t key) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t h1 = mix64(key + 2ULL * (uint64_t)i);
    const uint64_t h2 = mix64(key + 2ULL * (uint64_t)i + 1ULL);
    const double u1 = (double)((h1 >> 11) + 1ULL) * 0x1.0p-53;
    const double u2 = (double)(h2 >> 11) * 0x1.0p-53;
    dst[i] = (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}

hipError_t gen_normal_f32_launch(float* dst, int64_t n, uint64_t key, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    launch_timed("gen_normal_f32_kernel", 0.0, 4.0 * n, [&] {
        SDU_LAUNCH(gen_normal_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, dst, n, key);
    });
    return hipGetLastError();
}

hipError_t gen_launch(f16* dst, const GenDesc& g, hipStream_t s) {
    SDU_LAUNCH(gen_kernel, dim3((unsigned)((g.n + 255) / 256)), dim3(256), 0, s, dst, g);
    return hipGetLastError();
}


// ----------------------------------------------------------------- weight folding
//
// A transformer's feed-forward output and its proj_out are consecutive linear maps
// with a residual between them:
//   t' = t + Wf.g + bf,   out = Wp.t' + bp + x
// so out = [Wp.Wf | Wp] . [g | t] + (Wp.bf + bp) + x: one GEMM over the two-source
// A = [g | t] with K = 5C instead of two GEMMs (same FLOPs, one launch and one
// intermediate fewer).  wcat [C, 5C] row-major: columns [0, 4C) = Wp.Wf (fp32 sums
// of fp16 products, rounded once), [4C, 5C) = Wp.  bcat [C] = Wp.bf + bp.

namespace {
constexpr int FT = 64;   // output tile (rows o x columns k)
constexpr int FJ = 16;   // reduction chunk
}

// Block: 256 threads, a 64 x 64 tile of wcat, each thread 4 x 4 outputs.
__global__ __launch_bounds__(256) void fold_ffout_kernel(const f16* Wp, const f16* Wf, f16* wcat, int C) {
    __shared__ float sp[FT][FJ + 1];  // Wp[o0 + r][j0 + c]
    __shared__ float sf[FJ][FT + 1];  // Wf[j0 + r][k0 + c]
    const int K4 = 4 * C, K5 = 5 * C;
    const int k0 = blockIdx.x * FT, o0 = blockIdx.y * FT;
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    if (k0 >= K4) {  // the Wp copy columns
        for (int i = threadIdx.x; i < FT * FT; i += 256) {
            const int o = o0 + i / FT, k = k0 + i % FT;
            if (o < C && k < K5) wcat[(int64_t)o * K5 + k] = Wp[(int64_t)o * C + (k - K4)];
        }
        return;
    }
    float acc[4][4] = {};
    for (int j0 = 0; j0 < C; j0 += FJ) {
        for (int i = threadIdx.x; i < FT * FJ; i += 256) {
            const int r = i / FJ, c = i % FJ;
            const int o = o0 + r, j = j0 + c;
            sp[r][c] = (o < C && j < C) ? (float)Wp[(int64_t)o * C + j] : 0.f;
            const int r2 = i / FT, c2 = i % FT;
            const int j2 = j0 + r2, k = k0 + c2;
            sf[r2][c2] = (j2 < C && k < K4) ? (float)Wf[(int64_t)j2 * K4 + k] : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < FJ; ++j) {
            float a[4], b[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) { a[u] = sp[ty * 4 + u][j]; b[u] = sf[j][tx * 4 + u]; }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[u][v] = fmaf(a[u], b[v], acc[u][v]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int o = o0 + ty * 4 + u, k = k0 + tx * 4 + v;
            if (o < C && k < K4) wcat[(int64_t)o * K5 + k] = (f16)acc[u][v];
        }
}

__global__ void fold_ffout_bias_kernel(const f16* Wp, const f16* bf, const f16* bp, f16* bcat, int C) {
    const int o = blockIdx.x * blockDim.x + threadIdx.x;
    if (o >= C) return;
    float s = 0.f;
    for (int j = 0; j < C; ++j) s = fmaf((float)Wp[(int64_t)o * C + j], (float)bf[j], s);
    bcat[o] = (f16)(s + (float)bp[o]);
}

hipError_t fold_ffout_launch(const f16* Wp, const f16* bp, const f16* Wf, const f16* bf, f16* wcat, f16* bcat,
                             int C, hipStream_t s) {
    if (C <= 0 || C % 16) return hipErrorInvalidValue;  // 4C: whole 64-column tiles
    SDU_LAUNCH(fold_ffout_kernel, dim3((5 * C + FT - 1) / FT, (C + FT - 1) / FT), dim3(256), 0, s, Wp, Wf,
                       wcat, C);
    SDU_LAUNCH(fold_ffout_bias_kernel, dim3((C + 255) / 256), dim3(256), 0, s, Wp, bf, bp, bcat, C);
    return hipGetLastError();
}

// A resnet's 1x1 shortcut summed into its conv2: wcat [Co, 9 Ci2 + Cs] rows =
// [conv2 row (OHWI, 9 Ci2) | shortcut row (Cs)], bcat = b2 + bs.
__global__ void fold_shortcut_kernel(const f16* w2, const f16* b2, const f16* ws, const f16* bs, f16* wcat,
                                     f16* bcat, int Co, int K2, int Cs) {
    const int o = blockIdx.y;
    const int K = K2 + Cs;
    for (int k = blockIdx.x * blockDim.x + threadIdx.x; k < K; k += gridDim.x * blockDim.x)
        wcat[(int64_t)o * K + k] = k < K2 ? w2[(int64_t)o * K2 + k] : ws[(int64_t)o * Cs + (k - K2)];
    if (blockIdx.x == 0 && threadIdx.x == 0) bcat[o] = (f16)((float)b2[o] + (float)bs[o]);
}

hipError_t fold_shortcut_launch(const f16* w2, const f16* b2, const f16* ws, const f16* bs, f16* wcat, f16* bcat,
                                int Co, int Ci2, int Cs, hipStream_t s) {
    if (Co <= 0 || Ci2 <= 0 || Cs <= 0) return hipErrorInvalidValue;
    SDU_LAUNCH(fold_shortcut_kernel, dim3(8, Co), dim3(256), 0, s, w2, b2, ws, bs, wcat, bcat, Co, 9 * Ci2, Cs);
    return hipGetLastError();
}

// Sub-pixel weights (GemmArgs::subpix): block (o, phase), thread c over the input
// channels; each of the 4 taps (ty, tx) sums the 1, 2 or 4 source taps (ky, kx) with
// ty = (py + ky + 1) / 2 - py, tx = (px + kx + 1) / 2 - px in fp32.
__global__ void fold_subpix_kernel(const f16* w3, f16* w4, int Co, int Ci) {
    const int o = blockIdx.x, ph = blockIdx.y, py = ph >> 1, px = ph & 1;
    for (int c = threadIdx.x; c < Ci; c += blockDim.x) {
        float t[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ky = 0; ky < 3; ++ky)
#pragma unroll
            for (int kx = 0; kx < 3; ++kx) {
                const int ty = (py + ky + 1) / 2 - py, tx = (px + kx + 1) / 2 - px;
                t[ty * 2 + tx] += (float)w3[((int64_t)o * 9 + ky * 3 + kx) * Ci + c];
            }
#pragma unroll
        for (int q = 0; q < 4; ++q) w4[(((int64_t)ph * Co + o) * 4 + q) * Ci + c] = (f16)t[q];
    }
}

hipError_t fold_subpix_launch(const f16* w3, f16* w4, int Co, int Ci, hipStream_t s) {
    if (Co <= 0 || Ci <= 0) return hipErrorInvalidValue;
    SDU_LAUNCH(fold_subpix_kernel, dim3(Co, 4), dim3(256), 0, s, w3, w4, Co, Ci);
    return hipGetLastError();
}

// LayerNorm affine folded into the Linear after it, one block per output row n:
// Wf[n, k] = fp16(gamma[k] W[n, k]), sf[n] = sum_k Wf[n, k] (of the rounded values the
// GEMM multiplies), bf[n] = b[n] + sum_k beta[k] W[n, k].
__global__ __launch_bounds__(256) void fold_ln_kernel(const f16* W, const f16* b, const f16* gamma,
                                                      const f16* beta, f16* Wf, float* bf, float* sf, int K,
                                                      float oscale, int nscale) {
    const int n = blockIdx.x;
    const float cn = n < nscale ? oscale : 1.f;
    float ss = 0.f, sb = 0.f;
    for (int k = threadIdx.x; k < K; k += 256) {
        const float w = (float)W[(int64_t)n * K + k];
        const f16 wq = (f16)(w * (float)gamma[k] * cn);
        Wf[(int64_t)n * K + k] = wq;
        ss += (float)wq;
        sb += (float)beta[k] * w;
    }
    for (int off = 32; off > 0; off >>= 1) {
        ss += __shfl_xor(ss, off);
        sb += __shfl_xor(sb, off);
    }
    __shared__ float part[2][4];
    if ((threadIdx.x & 63) == 0) { part[0][threadIdx.x >> 6] = ss; part[1][threadIdx.x >> 6] = sb; }
    __syncthreads();
    if (threadIdx.x == 0) {
        sf[n] = part[0][0] + part[0][1] + part[0][2] + part[0][3];
        bf[n] = cn * ((b ? (float)b[n] : 0.f) + part[1][0] + part[1][1] + part[1][2] + part[1][3]);
    }
}

hipError_t fold_ln_launch(const f16* W, const f16* b, const f16* gamma, const f16* beta, f16* Wf, float* bf,
                          float* sf, int N, int K, hipStream_t s, float oscale, int nscale) {
    if (N <= 0 || K <= 0) return hipErrorInvalidValue;
    SDU_LAUNCH(fold_ln_kernel, dim3(N), dim3(256), 0, s, W, b, gamma, beta, Wf, bf, sf, K, oscale, nscale);
    return hipGetLastError();
}

}  // namespace sdu
