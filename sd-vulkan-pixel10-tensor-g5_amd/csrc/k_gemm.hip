// MFMA GEMM / implicit-GEMM convolution for gfx950 (CDNA4).
//
// C[M,N] = A[M,K] . W[N,K]^T, fp16 operands, fp32 accumulation on
// v_mfma_f32_32x32x16_f16.  Replaces the reference's matmul_f32.comp (MM) and
// every conv route of vk_engine.cpp:578-608 (1x1 GEMM, Winograd, im2col + GEMM):
//   * A_DENSE: A is row-major [M, lda]; columns [K1, K) may come from a second
//     source (the 1x1 shortcut over the up-path concat, vk_engine.cpp:634, :754).
//   * A_CONV3: A is the implicit im2col of an NHWC image for a 3x3 conv, pad 1,
//     stride 1/2 (downsample, :689-692), optional nearest-2x upsample folded into
//     the index math (upsample, :693-697).  K index = tap*Cin + ci.
// Epilogue (fused; the reference runs these as separate AB/AB2/ADD/GEGLU passes):
// + bias[n] + bias2[n] (fp32 time projection), GEGLU over interleaved a/b column
// blocks, + residual, store fp16 / fp32 / fp32-NCHW.
// Split-K writes fp32 partial tiles; a reduce kernel applies the epilogue.
#include "sdu_internal.h"

#include <algorithm>

namespace sdu {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

static constexpr int BK = 64;            // K tile (halves)
static constexpr int LDS_STRIDE = BK + 8; // padded row stride (halves) against bank conflicts

__device__ __forceinline__ float gelu_erf(float x) {
    return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
}

// Final value for output element (m, output column nout) given the fp32 GEMM
// results for column n (and its GEGLU gate partner).
__device__ __forceinline__ void epi_store(const GemmArgs& a, int m, int n, float v, float gate,
                                          int nout) {
    if (a.bias) v += (float)a.bias[n];
    if (a.bias2) v += a.bias2[n];
    if (a.geglu) {
        int ng = n + 32;
        if (a.bias) gate += (float)a.bias[ng];
        if (a.bias2) gate += a.bias2[ng];
        v = v * gelu_erf(gate);
    }
    if (a.res) v += (float)a.res[(int64_t)m * a.ldr + nout];
    if (a.out_mode == OUT_F16) {
        ((f16*)a.C)[(int64_t)m * a.ldc + nout] = (f16)v;
    } else if (a.out_mode == OUT_F32) {
        ((float*)a.C)[(int64_t)m * a.ldc + nout] = v;
    } else {
        int b = m / a.hw_out, p = m - b * a.hw_out;
        ((float*)a.C)[((int64_t)b * a.ldc + nout) * a.hw_out + p] = v;
    }
}

template <int MT, int NT, int WM, int WN>
__global__ __launch_bounds__(WM* WN * 64) void gemm_kernel(GemmArgs a) {
    constexpr int NTH = WM * WN * 64;
    constexpr int TMW = MT / WM, TNW = NT / WN;  // wave tile
    constexpr int FM = TMW / 32, FN = TNW / 32;   // 32x32 MFMA tiles per wave
    constexpr int A_CH = MT * (BK / 8) / NTH;     // 16-byte chunks per thread
    constexpr int B_CH = NT * (BK / 8) / NTH;
    static_assert(A_CH * NTH == MT * (BK / 8), "A tile split");
    static_assert(B_CH * NTH == NT * (BK / 8), "B tile split");

    __shared__ __attribute__((aligned(16))) f16 As[2][MT * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) f16 Bs[2][NT * LDS_STRIDE];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave % WM, wn = wave / WM;

    // XCD-aware block order: consecutive hardware block ids go round-robin over the
    // 8 XCDs; give each XCD a contiguous range of logical tiles so neighbouring
    // tiles (same A rows) share that XCD's L2.
    const int tiles_n = (a.N + NT - 1) / NT;
    const int tiles_m = (a.M + MT - 1) / MT;
    const int nblk = tiles_m * tiles_n;
    int bid = blockIdx.x;
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    const int tm = bid / tiles_n, tn = bid - tm * tiles_n;
    const int m0 = tm * MT, n0 = tn * NT;

    const int kbeg = blockIdx.z * a.k_per_split;
    const int kend = min(a.K, kbeg + a.k_per_split);
    const int nk = (kend - kbeg + BK - 1) / BK;

    // Per-thread A-row geometry (conv mode): image base pointer and output coords.
    int a_row[A_CH], a_kc[A_CH];
    int a_b[A_CH], a_oy[A_CH], a_ox[A_CH];
    bool a_ok[A_CH];
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
        int c = tid + i * NTH;
        a_row[i] = c / (BK / 8);
        a_kc[i] = c % (BK / 8);
        int m = m0 + a_row[i];
        a_ok[i] = m < a.M;
        if (a.amode == A_CONV3) {
            int hw = a.Ho * a.Wo;
            int mm = a_ok[i] ? m : 0;
            a_b[i] = mm / hw;
            int p = mm - a_b[i] * hw;
            a_oy[i] = p / a.Wo;
            a_ox[i] = p - a_oy[i] * a.Wo;
        } else {
            a_b[i] = a_oy[i] = a_ox[i] = 0;
        }
    }
    int b_row[B_CH], b_kc[B_CH];
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
        int c = tid + i * NTH;
        b_row[i] = c / (BK / 8);
        b_kc[i] = c % (BK / 8);
    }

    uint4 ra[A_CH], rb[B_CH];
    const uint4 zero4 = make_uint4(0, 0, 0, 0);
    const bool tap_uniform = (a.amode == A_CONV3) && (a.Cin % BK == 0);

    auto load_tiles = [&](int kt) {
        const int k0 = kbeg + kt * BK;
        int tap_u = 0, c_u = 0;
        if (tap_uniform) { tap_u = k0 / a.Cin; c_u = k0 - tap_u * a.Cin; }
#pragma unroll
        for (int i = 0; i < A_CH; ++i) {
            const int k = k0 + a_kc[i] * 8;
            uint4 v = zero4;
            if (a_ok[i] && k < kend) {
                const int m = m0 + a_row[i];
                if (a.amode == A_DENSE) {
                    const f16* p = (k < a.K1) ? a.A + (int64_t)m * a.lda + k
                                              : a.A2 + (int64_t)m * a.lda2 + (k - a.K1);
                    v = *(const uint4*)p;
                } else {
                    int tap, c;
                    if (tap_uniform) { tap = tap_u; c = c_u + a_kc[i] * 8; }
                    else { tap = k / a.Cin; c = k - tap * a.Cin; }
                    const int ky = tap / 3, kx = tap - ky * 3;
                    int iy, ix;
                    bool ok;
                    if (a.upsample) {
                        int uy = a_oy[i] + ky - 1, ux = a_ox[i] + kx - 1;
                        ok = (uy >= 0) & (uy < 2 * a.Hin) & (ux >= 0) & (ux < 2 * a.Win);
                        iy = uy >> 1; ix = ux >> 1;
                    } else {
                        iy = a_oy[i] * a.stride + ky - 1;
                        ix = a_ox[i] * a.stride + kx - 1;
                        ok = (iy >= 0) & (iy < a.Hin) & (ix >= 0) & (ix < a.Win);
                    }
                    if (ok)
                        v = *(const uint4*)(a.A + (((int64_t)a_b[i] * a.Hin + iy) * a.Win + ix) * a.Cin + c);
                }
            }
            ra[i] = v;
        }
#pragma unroll
        for (int i = 0; i < B_CH; ++i) {
            const int k = k0 + b_kc[i] * 8;
            const int n = n0 + b_row[i];
            uint4 v = zero4;
            if (n < a.N && k < kend) v = *(const uint4*)(a.Wt + (int64_t)n * a.K + k);
            rb[i] = v;
        }
    };
    auto store_tiles = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_CH; ++i)
            *(uint4*)&As[buf][a_row[i] * LDS_STRIDE + a_kc[i] * 8] = ra[i];
#pragma unroll
        for (int i = 0; i < B_CH; ++i)
            *(uint4*)&Bs[buf][b_row[i] * LDS_STRIDE + b_kc[i] * 8] = rb[i];
    };

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = floatx16{};

    if (nk > 0) {
        load_tiles(0);
        store_tiles(0);
    }
    __syncthreads();

    const int lrow = lane & 31, lk = (lane >> 5) * 8;
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load_tiles(kt + 1);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            half8 af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *(const half8*)&As[buf][(wm * TMW + i * 32 + lrow) * LDS_STRIDE + ks * 16 + lk];
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bf[j] = *(const half8*)&Bs[buf][(wn * TNW + j * 32 + lrow) * LDS_STRIDE + ks * 16 + lk];
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store_tiles(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue
    const int col_l = lane & 31, rq = (lane >> 5) * 4;
    if (a.partial) {
        float* P = a.partial + (int64_t)blockIdx.z * a.M * a.N;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int n = n0 + wn * TNW + j * 32 + col_l;
                if (n >= a.N) continue;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int m = m0 + wm * TMW + i * 32 + (e >> 2) * 8 + rq + (e & 3);
                    if (m < a.M) P[(int64_t)m * a.N + n] = acc[i][j][e];
                }
            }
        return;
    }
    if (a.geglu) {
        // column tiles (2t, 2t+1) of the wave hold the a and b halves of one
        // 64-row weight block; output column = 32 * block + lane%32.
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; j += 2) {
                const int n = n0 + wn * TNW + j * 32 + col_l;
                if (n >= a.N) continue;
                const int nout = (n >> 6) * 32 + col_l;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int m = m0 + wm * TMW + i * 32 + (e >> 2) * 8 + rq + (e & 3);
                    if (m < a.M) epi_store(a, m, n, acc[i][j][e], acc[i][j + 1][e], nout);
                }
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int n = n0 + wn * TNW + j * 32 + col_l;
            if (n >= a.N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm * TMW + i * 32 + (e >> 2) * 8 + rq + (e & 3);
                if (m < a.M) epi_store(a, m, n, acc[i][j][e], 0.f, n);
            }
        }
}

// Sum split-K partials and apply the epilogue; one thread per output element.
__global__ void splitk_reduce_kernel(GemmArgs a) {
    const int nout_cols = a.geglu ? a.N / 2 : a.N;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)a.M * nout_cols) return;
    const int m = (int)(idx / nout_cols);
    const int nout = (int)(idx - (int64_t)m * nout_cols);
    const int n = a.geglu ? (nout >> 5) * 64 + (nout & 31) : nout;
    const int64_t mn = (int64_t)a.M * a.N;
    float v = 0.f, g = 0.f;
    for (int z = 0; z < a.splits; ++z) {
        v += a.partial[z * mn + (int64_t)m * a.N + n];
        if (a.geglu) g += a.partial[z * mn + (int64_t)m * a.N + n + 32];
    }
    epi_store(a, m, n, v, g, nout);
}

// ----------------------------------------------------------------- dispatch

namespace {
struct Tile { int mt, nt; };

int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Tile + split choice: aim for >= ~2 blocks per CU on 256 CUs.
void plan(const GemmArgs& a, Tile& t, int& splits, int& kps) {
    t = (a.N <= 64) ? Tile{128, 64} : Tile{128, 128};
    if (a.geglu) t = Tile{128, 128};
    const int blocks = ceil_div(a.M, t.mt) * ceil_div(a.N, t.nt);
    const int nkt = ceil_div(a.K, BK);
    splits = 1;
    const int target = 512;
    if (blocks < target && nkt >= 8) {
        splits = std::min(std::min(ceil_div(target, blocks), nkt / 4), 32);
        if (splits < 1) splits = 1;
    }
    kps = ceil_div(nkt, splits) * BK;
    splits = ceil_div(a.K, kps);
}
}  // namespace

size_t gemm_workspace_bytes(const GemmArgs& a) {
    Tile t; int splits, kps;
    plan(a, t, splits, kps);
    return splits > 1 ? (size_t)splits * a.M * a.N * sizeof(float) : 0;
}

hipError_t gemm_launch(GemmArgs a, float* ws, hipStream_t s) {
    Tile t; int splits, kps;
    plan(a, t, splits, kps);
    if (a.A2 == nullptr) a.K1 = a.K;
    a.splits = splits;
    a.k_per_split = kps;
    a.partial = splits > 1 ? ws : nullptr;
    if (splits > 1 && ws == nullptr) return hipErrorInvalidValue;
    dim3 grid(ceil_div(a.M, t.mt) * ceil_div(a.N, t.nt), 1, splits);
    if (t.mt == 128 && t.nt == 128)
        hipLaunchKernelGGL((gemm_kernel<128, 128, 2, 2>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((gemm_kernel<128, 64, 2, 2>), grid, dim3(256), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    const int nout = a.geglu ? a.N / 2 : a.N;
    const int64_t total = (int64_t)a.M * nout;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ----------------------------------------------------------------- GEMV (time MLP)

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + __expf(-x)); }

// One wave per output row; fp32 input vector, fp16 weights [N, K], K % 8 == 0.
__global__ __launch_bounds__(256) void gemv_kernel(const float* x, const f16* W, const f16* bias,
                                                   float* y, int N, int K, int act_in, int act_out) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;
    float s = 0.f;
    for (int k = lane * 8; k < K; k += 64 * 8) {
        uint4 wv = *(const uint4*)(W + (int64_t)n * K + k);
        const f16* wh = (const f16*)&wv;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float xv = x[k + i];
            if (act_in) xv = silu_f(xv);
            s += xv * (float)wh[i];
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (lane == 0) {
        if (bias) s += (float)bias[n];
        if (act_out) s = silu_f(s);
        y[n] = s;
    }
}

hipError_t gemv_launch(const float* x, const f16* W, const f16* bias, float* y, int N, int K,
                       int act_in, int act_out, hipStream_t s) {
    hipLaunchKernelGGL(gemv_kernel, dim3((N + 3) / 4), dim3(256), 0, s, x, W, bias, y, N, K, act_in,
                       act_out);
    return hipGetLastError();
}

}  // namespace sdu
