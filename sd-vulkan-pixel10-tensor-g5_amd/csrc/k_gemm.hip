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

static constexpr int BK = 64;  // K tile (halves)

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

// All-zero 16-byte source for DMA lanes outside the operands (conv padding, K tail).
__device__ __attribute__((aligned(64))) uint4 g_zero_page[4];

// s_waitcnt vmcnt(N) lgkmcnt(0): at most N vector-memory ops (the DMA of later
// tiles) outstanding, and every LDS read of this wave complete, so that after the
// following barrier no wave still reads the ring stage the next DMA overwrites.
template <int N>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
}

// Main loop: 3-stage LDS ring fed by global_load_lds_dwordx4 (direct to LDS, no
// register staging), so two K tiles are in flight while the third is consumed;
// one s_barrier per K tile.  LDS rows are 128 bytes (64 halves) with the 16-byte
// chunk index XOR-swizzled by ((row >> 1) & 7): the DMA writes stay linear per
// wave and the 32x32x16 fragment reads (32 rows x 16 B per half-wave) are free of
// bank conflicts.
template <int MT, int NT, int WM, int WN>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs a) {
    constexpr int NTH = 256, NS = 3;
    static_assert(WM * WN == 4, "four waves");
    constexpr int TMW = MT / WM, TNW = NT / WN;  // wave tile
    constexpr int FM = TMW / 32, FN = TNW / 32;   // 32x32 MFMA tiles per wave
    constexpr int STAGE = (MT + NT) * BK;         // halves per ring stage
    constexpr int AI = MT / 32, BI = NT / 32;     // DMA instructions per thread per K tile
    constexpr int LPT = AI + BI;
    static_assert(MT % 32 == 0 && NT % 32 == 0 && LPT < 64, "tile shape");

    __shared__ __attribute__((aligned(1024))) f16 smem[NS * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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

    // DMA lane assignment: instruction i of wave w fills tile rows
    // [i*32 + w*8, +8); lane l lands in row +(l>>3), physical chunk l&7, which holds
    // logical chunk (l&7) ^ ((row>>1)&7).
    const int lrow8 = lane >> 3, pchunk = lane & 7;
    int a_m[AI], a_c[AI], a_b[AI], a_oy[AI], a_ox[AI];
#pragma unroll
    for (int i = 0; i < AI; ++i) {
        const int row = i * 32 + wave * 8 + lrow8;
        a_c[i] = pchunk ^ ((row >> 1) & 7);
        const int m = min(m0 + row, a.M - 1);  // rows past M compute garbage that is never stored
        a_m[i] = m;
        if (a.amode == A_CONV3) {
            const int hw = a.Ho * a.Wo;
            a_b[i] = m / hw;
            const int p = m - a_b[i] * hw;
            a_oy[i] = p / a.Wo;
            a_ox[i] = p - a_oy[i] * a.Wo;
        } else {
            a_b[i] = a_oy[i] = a_ox[i] = 0;
        }
    }
    int b_n[BI], b_c[BI];
#pragma unroll
    for (int i = 0; i < BI; ++i) {
        const int row = i * 32 + wave * 8 + lrow8;
        b_c[i] = pchunk ^ ((row >> 1) & 7);
        b_n[i] = min(n0 + row, a.N - 1);
    }
    const bool tap_uniform = (a.amode == A_CONV3) && (a.Cin % BK == 0);
    const void* zero = (const void*)g_zero_page;

    // Source address of each lane's 16-byte chunk, chosen with selects (no
    // divergent branches around the DMA: exactly AI + BI DMA instructions per
    // thread and K tile, which the vmcnt waits below count on).
    auto issue = [&](int kt, int stage) __attribute__((always_inline)) {
        const int k0 = kbeg + kt * BK;
        f16* sA = smem + stage * STAGE;
        f16* sB = sA + MT * BK;
        if (a.amode == A_DENSE) {
#pragma unroll
            for (int i = 0; i < AI; ++i) {
                const int k = k0 + a_c[i] * 8;
                const bool second = k >= a.K1;
                const f16* base = second ? a.A2 : a.A;
                const int64_t off = second ? (int64_t)a_m[i] * a.lda2 + (k - a.K1) : (int64_t)a_m[i] * a.lda + k;
                const void* src = (k < kend) ? (const void*)(base + off) : zero;
                __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(sA + (i * 32 + wave * 8) * BK),
                                                 16, 0, 0);
            }
        } else {
            int tap_u = 0, c_u = 0;
            if (tap_uniform) { tap_u = k0 / a.Cin; c_u = k0 - tap_u * a.Cin; }
#pragma unroll
            for (int i = 0; i < AI; ++i) {
                const int k = k0 + a_c[i] * 8;
                const int tap = tap_uniform ? tap_u : k / a.Cin;
                const int c = tap_uniform ? c_u + a_c[i] * 8 : k - tap * a.Cin;
                const int ky = tap / 3, kx = tap - ky * 3;
                const int uy = a_oy[i] * a.stride + ky - 1, ux = a_ox[i] * a.stride + kx - 1;
                const int hlim = a.upsample ? 2 * a.Hin : a.Hin, wlim = a.upsample ? 2 * a.Win : a.Win;
                const bool ok = (k < kend) & (uy >= 0) & (uy < hlim) & (ux >= 0) & (ux < wlim);
                const int iy = a.upsample ? (uy >> 1) : uy, ix = a.upsample ? (ux >> 1) : ux;
                const int64_t off = (((int64_t)a_b[i] * a.Hin + iy) * a.Win + ix) * a.Cin + c;
                const void* src = ok ? (const void*)(a.A + off) : zero;
                __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(sA + (i * 32 + wave * 8) * BK),
                                                 16, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < BI; ++i) {
            const int k = k0 + b_c[i] * 8;
            const void* src = (k < kend) ? (const void*)(a.Wt + (int64_t)b_n[i] * a.K + k) : zero;
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(sB + (i * 32 + wave * 8) * BK),
                                             16, 0, 0);
        }
    };

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = floatx16{};

    // fragment addressing: row (base + lrow), logical chunk 2*ks + (lane>>5)
    const int lrow = lane & 31, hl = lane >> 5, sw = (lrow >> 1) & 7;
    if (nk > 0) issue(0, 0);
    if (nk > 1) issue(1, 1);
    for (int kt = 0; kt < nk; ++kt) {
        if (kt + 1 < nk) wait_vmcnt_lgkm0<LPT>();
        else wait_vmcnt_lgkm0<0>();
        __builtin_amdgcn_s_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (kt + 2 < nk) issue(kt + 2, (kt + 2) % NS);
        const f16* sA = smem + (kt % NS) * STAGE;
        const f16* sB = sA + MT * BK;
        // fragments double-buffered in registers: reads of k-step ks+1 are in
        // flight while the MFMAs of k-step ks run
        half8 af[2][FM], bf[2][FN];
        auto load_frags = [&](int ks, int slot) __attribute__((always_inline)) {
            const int pc = ((ks * 2 + hl) ^ sw) * 8;
#pragma unroll
            for (int i = 0; i < FM; ++i) af[slot][i] = *(const half8*)(sA + (wm * TMW + i * 32 + lrow) * BK + pc);
#pragma unroll
            for (int j = 0; j < FN; ++j) bf[slot][j] = *(const half8*)(sB + (wn * TNW + j * 32 + lrow) * BK + pc);
        };
        load_frags(0, 0);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            if (ks + 1 < BK / 16) load_frags(ks + 1, (ks + 1) & 1);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[ks & 1][i], bf[ks & 1][j], acc[i][j], 0, 0, 0);
        }
        // Schedule of the unrolled K tile: reads(0), reads(1), mfma(0), reads(2),
        // mfma(1), reads(3), mfma(2), mfma(3) -- the fragments of k-step ks+1 are
        // in flight (in their own registers) during the MFMAs of k-step ks.
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * (FM + FN), 0);  // DS reads
#pragma unroll
        for (int ks = 0; ks < BK / 16 - 2; ++ks) {
            __builtin_amdgcn_sched_group_barrier(0x008, FM * FN, 0);  // MFMAs
            __builtin_amdgcn_sched_group_barrier(0x100, FM + FN, 0);  // DS reads
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * FM * FN, 0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
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
    // Stage the fp32 tile through LDS (reusing the operand ring).  The vector path
    // then gives each thread one fixed 8-column slice of several rows: epilogue
    // operands are all loaded before any store (the residual may alias the
    // output), and stores are 16-byte.
    constexpr int CST = NT + 4;  // padded fp32 row stride
    static_assert(MT * CST * 4 <= NS * STAGE * 2, "C tile fits the operand LDS");
    float* Cs = (float*)smem;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int r = wm * TMW + i * 32 + (e >> 2) * 8 + rq + (e & 3);
                Cs[r * CST + wn * TNW + j * 32 + col_l] = acc[i][j][e];
            }
    __syncthreads();
    if (a.out_mode == OUT_F32_NCHW || (a.N & 7)) {
        // narrow outputs (conv_out, N = 4): one element per thread iteration
        const int nto = a.geglu ? NT / 2 : NT;
        for (int idx = tid; idx < MT * nto; idx += NTH) {
            const int r = idx / nto, oc = idx - r * nto;
            const int tc = a.geglu ? (oc >> 5) * 64 + (oc & 31) : oc;
            const int m = m0 + r, n = n0 + tc;
            if (m >= a.M || n >= a.N) continue;
            const int nout = a.geglu ? (n0 >> 1) + oc : n;
            epi_store(a, m, n, Cs[r * CST + tc], a.geglu ? Cs[r * CST + tc + 32] : 0.f, nout);
        }
        return;
    }
    const int NTO = NT / (a.geglu ? 2 : 1);  // output columns of this tile
    const int cpr = NTO / 8;                  // 8-column chunks per row
    const int oc = (tid % cpr) * 8;           // fixed output column slice of this thread
    const int r0 = tid / cpr, rstep = NTH / cpr;
    // tile column of the (first) source value for output column oc
    const int tc = a.geglu ? (oc >> 5) * 64 + (oc & 31) : oc;
    const int n = n0 + tc;
    const int nout = a.geglu ? (n0 >> 1) + oc : n;
    if (n >= a.N) return;
    float badd[8], gadd[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) { badd[e] = 0.f; gadd[e] = 0.f; }
    if (a.bias) {
        const uint4 bv = *(const uint4*)(a.bias + n);
        const f16* bh = (const f16*)&bv;
#pragma unroll
        for (int e = 0; e < 8; ++e) badd[e] = (float)bh[e];
        if (a.geglu) {
            const uint4 gv = *(const uint4*)(a.bias + n + 32);
            const f16* gh = (const f16*)&gv;
#pragma unroll
            for (int e = 0; e < 8; ++e) gadd[e] = (float)gh[e];
        }
    }
    if (a.bias2) {
#pragma unroll
        for (int e = 0; e < 8; ++e) badd[e] += a.bias2[n + e];
        if (a.geglu) {
#pragma unroll
            for (int e = 0; e < 8; ++e) gadd[e] += a.bias2[n + 32 + e];
        }
    }
    constexpr int MAXR = MT * NT / 8 / NTH;  // rows per thread (non-GEGLU; GEGLU uses half)
    uint4 rres[MAXR];
    if (a.res) {
#pragma unroll
        for (int k = 0; k < MAXR; ++k) {
            const int r = r0 + k * rstep;
            const int m = m0 + r;
            rres[k] = make_uint4(0, 0, 0, 0);
            if (r < MT && m < a.M) rres[k] = *(const uint4*)(a.res + (int64_t)m * a.ldr + nout);
        }
    }
#pragma unroll
    for (int k = 0; k < MAXR; ++k) {
        const int r = r0 + k * rstep;
        const int m = m0 + r;
        if (r >= MT || m >= a.M) continue;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            v[e] = Cs[r * CST + tc + e] + badd[e];
            if (a.geglu) v[e] *= gelu_erf(Cs[r * CST + tc + 32 + e] + gadd[e]);
        }
        if (a.res) {
            const f16* rh = (const f16*)&rres[k];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] += (float)rh[e];
        }
        if (a.out_mode == OUT_F16) {
            uint4 o;
            f16* oh = (f16*)&o;
#pragma unroll
            for (int e = 0; e < 8; ++e) oh[e] = (f16)v[e];
            *(uint4*)((f16*)a.C + (int64_t)m * a.ldc + nout) = o;
        } else {
            float* cp = (float*)a.C + (int64_t)m * a.ldc + nout;
            *(float4*)cp = make_float4(v[0], v[1], v[2], v[3]);
            *(float4*)(cp + 4) = make_float4(v[4], v[5], v[6], v[7]);
        }
    }
}

// Sum split-K partials and apply the epilogue.  Vector path: one thread per 8
// output columns (N % 8 == 0 and not NCHW); otherwise one thread per element.
__global__ void splitk_reduce_kernel(GemmArgs a) {
    const int nout_cols = a.geglu ? a.N / 2 : a.N;
    const int64_t mn = (int64_t)a.M * a.N;
    const bool vec = a.out_mode != OUT_F32_NCHW && (a.N & 7) == 0;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (!vec) {
        if (idx >= (int64_t)a.M * nout_cols) return;
        const int m = (int)(idx / nout_cols);
        const int nout = (int)(idx - (int64_t)m * nout_cols);
        const int n = a.geglu ? (nout >> 5) * 64 + (nout & 31) : nout;
        float v = 0.f, g = 0.f;
        for (int z = 0; z < a.splits; ++z) {
            v += a.partial[z * mn + (int64_t)m * a.N + n];
            if (a.geglu) g += a.partial[z * mn + (int64_t)m * a.N + n + 32];
        }
        epi_store(a, m, n, v, g, nout);
        return;
    }
    const int cpr = nout_cols / 8;
    if (idx >= (int64_t)a.M * cpr) return;
    const int m = (int)(idx / cpr);
    const int nout = (int)(idx - (int64_t)m * cpr) * 8;
    const int n = a.geglu ? (nout >> 5) * 64 + (nout & 31) : nout;
    float v[8], g[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) { v[e] = 0.f; g[e] = 0.f; }
    for (int z = 0; z < a.splits; ++z) {
        const float* p = a.partial + z * mn + (int64_t)m * a.N + n;
        const float4 p0 = *(const float4*)p, p1 = *(const float4*)(p + 4);
        v[0] += p0.x; v[1] += p0.y; v[2] += p0.z; v[3] += p0.w;
        v[4] += p1.x; v[5] += p1.y; v[6] += p1.z; v[7] += p1.w;
        if (a.geglu) {
            const float4 q0 = *(const float4*)(p + 32), q1 = *(const float4*)(p + 36);
            g[0] += q0.x; g[1] += q0.y; g[2] += q0.z; g[3] += q0.w;
            g[4] += q1.x; g[5] += q1.y; g[6] += q1.z; g[7] += q1.w;
        }
    }
    uint4 rr = make_uint4(0, 0, 0, 0);
    if (a.res) rr = *(const uint4*)(a.res + (int64_t)m * a.ldr + nout);
    const f16* rh = (const f16*)&rr;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        float x = v[e], gt = g[e];
        if (a.bias) { x += (float)a.bias[n + e]; if (a.geglu) gt += (float)a.bias[n + 32 + e]; }
        if (a.bias2) { x += a.bias2[n + e]; if (a.geglu) gt += a.bias2[n + 32 + e]; }
        if (a.geglu) x *= gelu_erf(gt);
        if (a.res) x += (float)rh[e];
        o[e] = x;
    }
    if (a.out_mode == OUT_F16) {
        uint4 ov;
        f16* oh = (f16*)&ov;
#pragma unroll
        for (int e = 0; e < 8; ++e) oh[e] = (f16)o[e];
        *(uint4*)((f16*)a.C + (int64_t)m * a.ldc + nout) = ov;
    } else {
        float* cp = (float*)a.C + (int64_t)m * a.ldc + nout;
        *(float4*)cp = make_float4(o[0], o[1], o[2], o[3]);
        *(float4*)(cp + 4) = make_float4(o[4], o[5], o[6], o[7]);
    }
}

// ----------------------------------------------------------------- dispatch

namespace {
struct Cfg {
    int mt, nt, per_cu;  // tile, resident blocks per CU (LDS-limited)
    double eff;          // relative per-FLOP throughput of the tile shape
    const char* name;
};
// 256x128: waves 128x64; 128x128: waves 64x64; 128x64: waves 64x32.
const Cfg kCfgs[3] = {{256, 128, 1, 1.0, "gemm_256x128"},
                      {128, 128, 1, 0.8, "gemm_128x128"},
                      {128, 64, 2, 0.6, "gemm_128x64"}};

int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Pick the tile shape and split-K factor with the lowest modelled time:
// block waves over 256 CUs x per-block MFMA time, plus the fp32 partial round
// trip and the reduce launch when K is split.
void plan(const GemmArgs& a, int& ci, int& splits, int& kps) {
    const double cu_flops = 2.5e15 / 256.0;
    const int nkt = ceil_div(a.K, BK);
    double best = 1e30;
    ci = 0; splits = 1; kps = nkt * BK;
    for (int c = 0; c < 3; ++c) {
        const Cfg& g = kCfgs[c];
        if (a.geglu && g.nt < 128) continue;  // GEGLU pairs 32-column blocks within a 64-wide wave tile
        const int tiles = ceil_div(a.M, g.mt) * ceil_div(a.N, g.nt);
        static const int cand[] = {1, 2, 3, 4, 6, 8, 12, 16, 24, 32};
        for (int s : cand) {
            if (s > 1 && nkt / s < 4) break;
            const int kt_per = ceil_div(nkt, s);
            const int se = ceil_div(nkt, kt_per);
            const long blocks = (long)tiles * se;
            const long slots = 256L * g.per_cu;
            const long waves = (blocks + slots - 1) / slots;
            const double blk_t = 2.0 * g.mt * g.nt * kt_per * BK * g.per_cu / (g.eff * cu_flops);
            double t = waves * blk_t + 1.5e-6;
            if (se > 1) t += (double)se * a.M * a.N * 8.0 / 4.0e12 + 2.5e-6;
            if (t < best * 0.97) { best = t; ci = c; splits = se; kps = kt_per * BK; }
        }
    }
}
}  // namespace

const char* gemm_kernel_name(const GemmArgs& a) {
    int ci, splits, kps;
    plan(a, ci, splits, kps);
    return kCfgs[ci].name;
}

size_t gemm_workspace_bytes(const GemmArgs& a) {
    int ci, splits, kps;
    plan(a, ci, splits, kps);
    return splits > 1 ? (size_t)splits * a.M * a.N * sizeof(float) : 0;
}

hipError_t gemm_launch(GemmArgs a, float* ws, hipStream_t s) {
    int ci, splits, kps;
    plan(a, ci, splits, kps);
    if (a.A2 == nullptr) a.K1 = a.K;
    a.splits = splits;
    a.k_per_split = kps;
    a.partial = splits > 1 ? ws : nullptr;
    if (splits > 1 && ws == nullptr) return hipErrorInvalidValue;
    const Cfg& g = kCfgs[ci];
    dim3 grid(ceil_div(a.M, g.mt) * ceil_div(a.N, g.nt), 1, splits);
    if (ci == 0) hipLaunchKernelGGL((gemm_kernel<256, 128, 2, 2>), grid, dim3(256), 0, s, a);
    else if (ci == 1) hipLaunchKernelGGL((gemm_kernel<128, 128, 2, 2>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((gemm_kernel<128, 64, 2, 2>), grid, dim3(256), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    const int nout = a.geglu ? a.N / 2 : a.N;
    const bool vec = a.out_mode != OUT_F32_NCHW && (a.N & 7) == 0;
    const int64_t total = (int64_t)a.M * (vec ? nout / 8 : nout);
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
