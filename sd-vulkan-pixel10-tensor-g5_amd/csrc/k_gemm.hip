// MFMA GEMM / implicit-GEMM convolution for gfx950 (CDNA4).
//
// C[M,N] = A[M,K] . W[N,K]^T, fp16 operands, fp32 accumulation on
// v_mfma_f32_32x32x16_f16.  Replaces the reference's matmul_f32.comp (MM) and
// every conv route of vk_engine.cpp:578-608 (1x1 GEMM, Winograd, im2col + GEMM):
//   * A_DENSE: A is row-major [M, lda]; columns [K1, K) may come from a second
//     source (the 1x1 shortcut over the up-path concat, vk_engine.cpp:634, :754).
//   * A_CONV3: A is the implicit im2col of an NHWC image for a 3x3 conv, pad 1,
//     stride 1/2 (downsample, :689-692), optional nearest-2x upsample folded into
//     the index math (upsample, :693-697).  K index = tap*Cin + ci.  Columns past
//     9*Cin may come from one or two dense sources of the same pixels: a resnet's
//     1x1 shortcut (:634) summed into its conv2.
// Epilogue (fused; the reference runs these as separate AB/AB2/ADD/GEGLU passes):
// + bias[n] + bias2[n] (fp32 time projection), GEGLU over interleaved a/b column
// blocks, + residual, activation (ReLU / quick-GELU), store fp16 / fp32 / fp32-NCHW.  A LayerNorm (layernorm_f32.comp,
// vk_engine.cpp:652, :658, :666) between two GEMMs runs inside them: the producer adds
// each output row's sum and sum of squares into a row-statistics buffer, and the
// consumer, reading the un-normalised rows as A, applies rstd * (acc - mean * colsum(W))
// with the LayerNorm's affine folded into its W and bias.
// Split-K, two ways: the last block of a tile to arrive sums the tile's fp32 partials
// and runs the epilogue (few splits), or a reduce kernel does (many splits).
#include "sdu_internal.h"

#include <cstdio>

#include <algorithm>

namespace sdu {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));


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
    v = apply_act(a.act, v);
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

// The same with the tiles issued after the one about to be read still in flight: at
// most `ahead` (<= A) tiles of LPT DMA instructions each.
template <int LPT, int A>
__device__ __forceinline__ void wait_tiles(int ahead) {
    if constexpr (A == 0) wait_vmcnt_lgkm0<0>();
    else if (ahead >= A) wait_vmcnt_lgkm0<A * LPT>();
    else wait_tiles<LPT, A - 1>(ahead);
}

// Sum the per-thread column statistics of a block over the threads that own the same
// 8 columns (thread t owns chunk t % CPR; chunk c covers columns col0 + 8c ..) through
// LDS and add them to the per-(image, channel) fp64 statistics, one atomic per value,
// the sums spread over all threads (each one's NTH / CPR LDS reads issued together).
// red must hold NTH * 32 floats and be free (the caller's last LDS use is complete
// after the first barrier here).  Value v of thread t sits at v * NTH + (t ^ v): the
// stores (one v, consecutive t) and the loads (consecutive v, one t) both fall on
// distinct banks (a thread-major layout, 32 floats per thread, put every lane of a
// store on one bank).
template <int NTH, int CPR>
__device__ __forceinline__ void stats_flush(const GemmArgs& a, const float (&st)[2][2][8], int b0,
                                            int m_last, int col0, float* red) {
    static_assert(NTH % 32 == 0, "swizzle stays within a row");
    const int tid = threadIdx.x;
    __syncthreads();
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int v = sl * 16 + q * 8 + e;
                red[v * NTH + (tid ^ v)] = st[sl][q][e];
            }
    __syncthreads();
    const int nslot = m_last / a.stats_hw != b0 ? 2 : 1;
    // value v of chunk c: slot v / 16, sum (0) or sum of squares (1) = (v / 8) % 2, column v % 8
    // (thread t owns chunk t % CPR; threads past the last whole group of CPR kept zeros)
#pragma unroll
    for (int q = tid; q < CPR * 32; q += NTH) {
        const int c = q >> 5, v = q & 31;
        const int col = col0 + c * 8 + (v & 7);
        if ((v >> 4) >= nslot || col >= a.N) continue;
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < NTH / CPR; ++j) t += red[v * NTH + ((c + j * CPR) ^ v)];
        atomicAdd(&a.stats[((int64_t)(b0 + (v >> 4)) * a.N + col) * 2 + ((v >> 3) & 1)], (double)t);
    }
}

// Sum split-K partials and apply the epilogue.  Vector path: 8 output columns
// (N % 8 == 0 and not NCHW); scalar path: one element.
__device__ __forceinline__ void reduce_scalar(const GemmArgs& a, int m, int nout) {
    const int64_t mn = (int64_t)a.M * a.N;
    const int n = a.geglu ? (nout >> 5) * 64 + (nout & 31) : nout;
    float v = 0.f, g = 0.f;
    for (int z = 0; z < a.splits; ++z) {
        v += a.partial[z * mn + (int64_t)m * a.N + n];
        if (a.geglu) g += a.partial[z * mn + (int64_t)m * a.N + n + 32];
    }
    epi_store(a, m, n, v, g, nout);
}

// Sum the split-K partials of 8 output columns (nout ..) for R rows m[r] and apply the
// epilogue; rows whose bit in `valid` is clear are read (m clamped by the caller) but
// not stored.  Every load of a round of U splits over all R rows is issued before any
// is added (the last round re-reads split splits-1 and weights the repeats 0), and
// the bias / residual loads come first.  GG = false: no GEGLU.  ov[r] = the stored
// fp16 values (OUT_F16).
template <int R, bool GG>
__device__ __forceinline__ void reduce_rows(const GemmArgs& a, const int (&m)[R], unsigned valid, int nout,
                                            uint4 (&ov)[R]) {
    // All loads are unconditional (absent operands read the zero page) and every
    // loaded value is used, so the compiler keeps them in flight together.
    const int64_t mn = (int64_t)a.M * a.N;
    const bool geglu = GG && a.geglu;
    const int n = geglu ? (nout >> 5) * 64 + (nout & 31) : nout;
    const f16* zh = (const f16*)g_zero_page;
    const float* zf = (const float*)g_zero_page;
    const uint4 bv = *(const uint4*)(a.bias ? a.bias + n : zh);
    const uint4 gbv = *(const uint4*)(a.bias && geglu ? a.bias + n + 32 : zh);
    const float4 c0 = *(const float4*)(a.bias2 ? a.bias2 + n : zf);
    const float4 c1 = *(const float4*)(a.bias2 ? a.bias2 + n + 4 : zf);
    const float4 d0 = *(const float4*)(a.bias2 && geglu ? a.bias2 + n + 32 : zf);
    const float4 d1 = *(const float4*)(a.bias2 && geglu ? a.bias2 + n + 36 : zf);
    uint4 rr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rr[r] = *(const uint4*)(a.res ? a.res + (int64_t)m[r] * a.ldr + nout : zh);
    float v[R][8], g[R][8];
    {
        const f16* bh = (const f16*)&bv;
        const f16* gh = (const f16*)&gbv;
        const float cb[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
        const float db[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                v[r][e] = (float)bh[e] + cb[e];
                g[r][e] = (float)gh[e] + db[e];
            }
    }
    // splits per round: 8 for one plain row (16 float4 in flight), else 4
    constexpr int U = (R == 1 && !GG) ? 8 : 4;
    for (int z0 = 0; z0 < a.splits; z0 += U) {
        float4 p0[R][U], p1[R][U], q0[GG ? R : 1][U], q1[GG ? R : 1][U];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float* p = a.partial + min(z0 + u, a.splits - 1) * mn + (int64_t)m[r] * a.N + n;
                p0[r][u] = *(const float4*)p;
                p1[r][u] = *(const float4*)(p + 4);
                if (GG) {
                    q0[GG ? r : 0][u] = *(const float4*)(geglu ? p + 32 : zf);
                    q1[GG ? r : 0][u] = *(const float4*)(geglu ? p + 36 : zf);
                }
            }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool use = z0 + u < a.splits;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float x[8] = {p0[r][u].x, p0[r][u].y, p0[r][u].z, p0[r][u].w,
                                    p1[r][u].x, p1[r][u].y, p1[r][u].z, p1[r][u].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) v[r][e] += use ? x[e] : 0.f;
                if (GG) {
                    const float4 x0 = q0[GG ? r : 0][u], x1 = q1[GG ? r : 0][u];
                    const float y[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) g[r][e] += use ? y[e] : 0.f;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const f16* rh = (const f16*)&rr[r];
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float x = v[r][e];
            if (geglu) x *= gelu_erf(g[r][e]);
            if (a.res) x += (float)rh[e];
            o[e] = apply_act(a.act, x);
        }
        ov[r] = make_uint4(0, 0, 0, 0);
        if (!(valid >> r & 1)) continue;
        if (a.out_mode == OUT_F16) {
            f16* oh = (f16*)&ov[r];
#pragma unroll
            for (int e = 0; e < 8; ++e) oh[e] = (f16)o[e];
            *(uint4*)((f16*)a.C + (int64_t)m[r] * a.ldc + nout) = ov[r];
        } else {
            float* cp = (float*)a.C + (int64_t)m[r] * a.ldc + nout;
            *(float4*)cp = make_float4(o[0], o[1], o[2], o[3]);
            *(float4*)(cp + 4) = make_float4(o[4], o[5], o[6], o[7]);
        }
    }
}

__global__ void splitk_reduce_kernel(GemmArgs a) {
    const int nout_cols = a.geglu ? a.N / 2 : a.N;
    const bool vec = a.out_mode != OUT_F32_NCHW && (a.N & 7) == 0;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (!vec) {
        if (idx >= (int64_t)a.M * nout_cols) return;
        const int m = (int)(idx / nout_cols);
        reduce_scalar(a, m, (int)(idx - (int64_t)m * nout_cols));
        return;
    }
    const int cpr = nout_cols / 8;
    if (idx >= (int64_t)a.M * cpr) return;
    const int m[1] = {(int)(idx / cpr)};
    uint4 o[1];
    const int nout = (int)(idx - (int64_t)m[0] * cpr) * 8;
    if (a.geglu) reduce_rows<1, true>(a, m, 1u, nout, o);
    else reduce_rows<1, false>(a, m, 1u, nout, o);
}

// 8 consecutive fp32 values from 16-byte-aligned LDS
__device__ __forceinline__ void ld8(const float* p, float (&v)[8]) {
    const float4 x = *(const float4*)p, y = *(const float4*)(p + 4);
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w; v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
}

// Main loop: NS-stage LDS ring fed by global_load_lds_dwordx4 (direct to LDS, no
// register staging), NS-1 K tiles in flight while one is consumed, one s_barrier
// per K tile.  LDS rows are BK halves (64 or 128 bytes) with the 16-byte chunk
// index XOR-swizzled per row, so the DMA writes stay linear per wave and the
// 32x32x16 fragment reads (32 rows x 16 B per half-wave) are free of bank
// conflicts.  Fragments are double-buffered in registers: the LDS reads of
// k-step ks+1 are in flight during the MFMAs of k-step ks.
template <int BKT>
__device__ __forceinline__ int lds_swizzle(int row) {
    return BKT == 64 ? ((row >> 1) & 7) : ((row >> 2) & 3);
}

// Two blocks per CU (4 waves per SIMD) where the ring leaves LDS for two: the
// register budget is then 128 VGPRs.
//
// MF: the MFMA, v_mfma_f32_32x32x16_f16 (32) or v_mfma_f32_16x16x32_f16 (16).  The 16x16
// form lets a wave tile be an odd number of 16-column blocks: the 64x160 tile (4 waves of
// 32x80) covers N = 320 in two tiles with no padded column and gives M = 8192 exactly 256
// tiles, one per CU.  Its lane layout: A / B operand lane l, row / column l % 16, K
// elements 8 (l / 16) .. + 8 of a 32-deep k-step; accumulator element e of lane l: row
// 4 (l / 16) + e, column l % 16.  With MF 16 the wave tile is 32 rows (one epilogue pass).
template <int MT, int NT, int WM, int WN, int BKT, int NS, int AM, int MF = 32>
__global__ __launch_bounds__(WM* WN * 64) __attribute__((amdgpu_waves_per_eu(MT == 256 || MF == 16 ? 2 : 4)))
void gemm_kernel(GemmArgs a) {
    constexpr int NW = WM * WN, NTH = NW * 64;
    constexpr int TMW = MT / WM, TNW = NT / WN;  // wave tile
    static_assert(MF == 32 || (MF == 16 && TMW == 32 && TNW % 16 == 0), "16x16 MFMA wave tile");
    constexpr int FM = MF == 32 ? TMW / 32 : 1;   // 32-row epilogue passes per wave
    constexpr int FN = MF == 32 ? TNW / 32 : 1;   // 32x32 MFMA tiles per wave row (MF 32)
    constexpr int FM16 = TMW / 16, FN16 = TNW / 16;  // 16x16 MFMA tiles per wave (MF 16)
    constexpr int CPR = BKT / 8;                  // 16-byte chunks per LDS row
    constexpr int RPI = 1024 / (BKT * 2);         // rows one wave DMA instruction fills
    constexpr int AI = MT / RPI / NW, BI = NT / RPI / NW;  // DMA instructions per thread per tile
    constexpr int LPT = AI + BI;
    constexpr int STAGE = (MT + NT) * BKT;        // halves per ring stage
    constexpr int KS = BKT / 16;                  // MFMA k-steps per tile
    constexpr bool DENSE = AM == A_DENSE;
    static_assert(AI * RPI * NW == MT && BI * RPI * NW == NT, "DMA split");
    static_assert(NS >= 2 && (NS - 2) * LPT < 64, "ring depth");

    __shared__ __attribute__((aligned(1024))) f16 smem[NS * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM, wn = wave / WM;

    // XCD-aware block order: consecutive hardware block ids go round-robin over the
    // 8 XCDs; give each XCD a contiguous range of logical tiles (XCD x: the nblk / 8
    // tiles, one more for the first nblk % 8 XCDs, after those of XCDs < x), so that
    // neighbouring tiles share that XCD's L2.  Neighbours share A rows (M-major order)
    // or, when the weights are the larger operand, W columns (N-major order).
    const int tiles_n = (a.N + NT - 1) / NT;
    const int tiles_m = (a.M + MT - 1) / MT;
    const int nblk = tiles_m * tiles_n;
    const int xcd = blockIdx.x & 7, per = nblk >> 3, extra = nblk & 7;
    const int bid = xcd * per + min(xcd, extra) + (blockIdx.x >> 3);
    int tm, tn;
    if (a.n_major) {
        tn = bid / tiles_m;
        tm = bid - tn * tiles_m;
    } else {
        tm = bid / tiles_n;
        tn = bid - tm * tiles_n;
    }
    const int m0 = tm * MT, n0 = tn * NT;
    // sub-pixel conv (GemmArgs::subpix): the tile's phase (a tile never straddles two)
    // and the first GEMM row of that phase
    const bool subpix = AM == A_CONV3 && a.subpix;
    const int sp_rows = a.M >> 2;
    const int sp_ph = subpix ? m0 / sp_rows : 0, sp_base = sp_ph * sp_rows;

    const int kbeg = blockIdx.z * a.k_per_split;
    const int kend = min(a.K, kbeg + a.k_per_split);
    const int nk = (kend - kbeg + BKT - 1) / BKT;

    // DMA lane assignment: instruction i of wave w fills tile rows
    // [(i*NW + w)*RPI, +RPI); lane l lands in row +(l / CPR), physical chunk l % CPR,
    // which holds logical chunk (l % CPR) ^ swizzle(row).
    //
    // Steady-state K tiles load through buffer_load ... lds: the operand base is a
    // wave-uniform buffer resource, each lane's byte offset is precomputed once (row
    // offset + chunk), and the K position is the scalar soffset, so a dense or weight
    // DMA costs no VALU.  Implicit-conv rows add a scalar tap offset and select
    // 0x80000000 for taps outside the image: an offset past the resource's range reads
    // zeros.  Rows past M / N repeat the last row (results never stored).  K tails,
    // tiles straddling the dense two-source split, and the conv cases whose tap
    // changes within a tile (Cin % BK != 0, upsampled input) take a per-lane pointer
    // path with global_load_lds and a zero page.  Every path issues exactly AI + BI
    // DMA instructions per thread and K tile, which the vmcnt waits below count on.
    const int lr = lane / CPR, pchunk = lane % CPR;
    const f16* zero = (const f16*)g_zero_page;
    constexpr uint32_t kOOB = 0x80000000u;
    const __amdgpu_buffer_rsrc_t rsB =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.Wt, (short)0, (subpix ? 4 : 1) * a.N * a.K * 2, 0x00020000);
    uint32_t voB[BI];
    int b_c[BI];
#pragma unroll
    for (int i = 0; i < BI; ++i) {
        const int row = (i * NW + wave) * RPI + lr;
        b_c[i] = (pchunk ^ lds_swizzle<BKT>(row)) * 8;
        voB[i] = (uint32_t)(((sp_ph * a.N + min(n0 + row, a.N - 1)) * a.K + b_c[i]) * 2);
    }
    int a_c[AI];          // element offset of the lane's chunk within the K tile
    int a_m[AI];          // dense: row (clamped)
    uint32_t voA[AI];     // dense: byte offset of (row, chunk) in A
    uint32_t voA2[AI];    // byte offset of (row, chunk) in A2 (dense second source, conv tail)
    uint32_t voA3[AI];    // conv: byte offset of (row, chunk) in A3
    int a_off[AI];        // conv: element offset of tap (0,0) of the lane's output pixel (+chunk)
    int a_vm[AI];         // conv: bit ky*3+kx set when that tap is inside the image
    int a_b[AI], a_oy[AI], a_ox[AI];  // conv geometry for the per-lane path
#pragma unroll
    for (int i = 0; i < AI; ++i) {
        const int row = (i * NW + wave) * RPI + lr;
        a_c[i] = (pchunk ^ lds_swizzle<BKT>(row)) * 8;
        const int m = min(m0 + row, a.M - 1);
        a_m[i] = m;
        if (DENSE) {
            voA[i] = (uint32_t)((m * a.lda + a_c[i]) * 2);
            voA2[i] = a.A2 ? (uint32_t)((m * a.lda2 + a_c[i]) * 2) : 0u;
        } else {
            voA2[i] = a.A2 ? (uint32_t)((m * a.lda2 + a_c[i]) * 2) : 0u;
            voA3[i] = a.A3 ? (uint32_t)((m * a.lda3 + a_c[i]) * 2) : 0u;
            if (subpix) {
                // input pixel (iy, ix) of phase (py, px): 2x2 taps at rows iy + py - 1 + ty,
                // columns ix + px - 1 + tx
                const int hwi = a.Hin * a.Win, q = m - sp_base;
                const int bb = q / hwi, r = q - bb * hwi, iy = r / a.Win, ix = r - iy * a.Win;
                const int y0 = iy + (sp_ph >> 1) - 1, x0 = ix + (sp_ph & 1) - 1;
                a_b[i] = bb; a_oy[i] = iy; a_ox[i] = ix;
                a_off[i] = ((bb * a.Hin + y0) * a.Win + x0) * a.Cin + a_c[i];
                int vm = 0;
#pragma unroll
                for (int ty = 0; ty < 2; ++ty)
#pragma unroll
                    for (int tx = 0; tx < 2; ++tx)
                        if (y0 + ty >= 0 && y0 + ty < a.Hin && x0 + tx >= 0 && x0 + tx < a.Win) vm |= 1 << (ty * 2 + tx);
                a_vm[i] = vm;
                continue;
            }
            const int hw = a.Ho * a.Wo;
            const int bb = m / hw, p = m - bb * hw;
            const int oy = p / a.Wo, ox = p - oy * a.Wo;
            a_b[i] = bb; a_oy[i] = oy; a_ox[i] = ox;
            const int y0 = oy * a.stride - 1, x0 = ox * a.stride - 1;
            a_off[i] = ((bb * a.Hin + y0) * a.Win + x0) * a.Cin + a_c[i];
            int vm = 0;
#pragma unroll
            for (int ky = 0; ky < 3; ++ky)
#pragma unroll
                for (int kx = 0; kx < 3; ++kx) {
                    const int uy = (a.upsample ? oy - 1 : y0) + ky, ux = (a.upsample ? ox - 1 : x0) + kx;
                    const int hl = a.upsample ? 2 * a.Hin : a.Hin, wl = a.upsample ? 2 * a.Win : a.Win;
                    if (uy >= 0 && uy < hl && ux >= 0 && ux < wl) vm |= 1 << (ky * 3 + kx);
                }
            a_vm[i] = vm;
        }
    }
    const __amdgpu_buffer_rsrc_t rsA = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.A, (short)0,
        DENSE ? a.M * a.lda * 2 : a.Bn * a.Hin * a.Win * a.Cin * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsA2 = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.A2 ? a.A2 : a.A), (short)0, a.A2 ? a.M * a.lda2 * 2 : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsA3 = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.A3 ? a.A3 : a.A), (short)0, a.A3 ? a.M * a.lda3 * 2 : 0, 0x00020000);
    // conv fast path: each K tile lies inside one tap (Cin % BKT == 0) and the input
    // is not upsampled, so the tap offset is one scalar per tile.  The K tiles of the
    // conv part go channel-chunk-major: the 9 taps of one BKT-channel chunk back to back
    // (virtual tile v = chunk * 9 + tap, real K offset tap * Cin + chunk * BKT), so the
    // block's input pixels (its rows and their halo) are re-read for the next tap while
    // that chunk is still in L2, rather than after a sweep over all Cin channels.  A
    // split-K block takes a contiguous range of virtual tiles.
    const bool conv_fast = AM == A_CONV3 && a.Cin % BKT == 0 && !a.upsample;
    const int ntap = subpix ? 4 : 9;  // 3x3 taps, or the sub-pixel form's 2x2
    int tap_next = 0, c_next = 0;  // tap / channel of the next tile issued (fast path)
    if (conv_fast) {
        const int v0 = kbeg / BKT, chunk = v0 / ntap;
        tap_next = v0 - chunk * ntap;
        c_next = chunk * BKT;
    }

    auto dma = [&](const f16* src, f16* dst) __attribute__((always_inline)) {
        __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
    };
    auto bdma = [&](__amdgpu_buffer_rsrc_t rs, uint32_t vo, int so, f16* dst) __attribute__((always_inline)) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)dst, 16, vo, so, 0, 0);
    };
    auto issue = [&](int kt, int stage) __attribute__((always_inline)) {
        const int k0 = kbeg + kt * BKT;
        const bool tail = k0 + BKT > kend;  // partial K tile
        int kw = k0;                        // the tile's real K offset (weights)
        f16* sA = smem + stage * STAGE;
        f16* sB = sA + MT * BKT;
        if (DENSE) {
            const bool in1 = !a.A2 || k0 + BKT <= a.K1, in2 = a.A2 && k0 >= a.K1;
            if (!tail && in1) {
#pragma unroll
                for (int i = 0; i < AI; ++i) bdma(rsA, voA[i], k0 * 2, sA + (i * NW + wave) * RPI * BKT);
            } else if (!tail && in2) {
#pragma unroll
                for (int i = 0; i < AI; ++i)
                    bdma(rsA2, voA2[i], (k0 - a.K1) * 2, sA + (i * NW + wave) * RPI * BKT);
            } else {
#pragma unroll
                for (int i = 0; i < AI; ++i) {
                    const int k = k0 + a_c[i];
                    const f16* src = (a.A2 && k >= a.K1) ? a.A2 + (int64_t)a_m[i] * a.lda2 + (k - a.K1)
                                                         : a.A + (int64_t)a_m[i] * a.lda + k;
                    dma(k < kend ? src : zero, sA + (i * NW + wave) * RPI * BKT);
                }
            }
        } else if (a.A2 && k0 >= a.K1) {
            // conv dense tail: whole tiles (K1, K2, K multiples of the K tile), after
            // every conv tile, so the fast path's tap counters are not advanced
            if (!a.A3 || k0 < a.K2) {
#pragma unroll
                for (int i = 0; i < AI; ++i) bdma(rsA2, voA2[i], (k0 - a.K1) * 2, sA + (i * NW + wave) * RPI * BKT);
            } else {
#pragma unroll
                for (int i = 0; i < AI; ++i) bdma(rsA3, voA3[i], (k0 - a.K2) * 2, sA + (i * NW + wave) * RPI * BKT);
            }
        } else if (conv_fast) {
            const int tap = tap_next, ky = subpix ? tap >> 1 : tap / 3, kx = tap - ky * (subpix ? 2 : 3);
            const int toff = (ky * a.Win + kx) * a.Cin + c_next;
            kw = tap * a.Cin + c_next;
            if (++tap_next == ntap) { tap_next = 0; c_next += BKT; }
#pragma unroll
            for (int i = 0; i < AI; ++i) {
                const bool ok = ((a_vm[i] >> tap) & 1) && !(tail && k0 + a_c[i] >= kend);
                bdma(rsA, ok ? (uint32_t)((a_off[i] + toff) * 2) : kOOB, 0, sA + (i * NW + wave) * RPI * BKT);
            }
        } else {
#pragma unroll
            for (int i = 0; i < AI; ++i) {
                const int k = k0 + a_c[i];
                const int tap = k / a.Cin, c = k - tap * a.Cin;
                const int ky = tap / 3, kx = tap - ky * 3;
                const int uy = a_oy[i] * a.stride + ky - 1, ux = a_ox[i] * a.stride + kx - 1;
                const bool ok = (k < kend) && ((a_vm[i] >> tap) & 1);
                const int iy = a.upsample ? (uy >> 1) : uy, ix = a.upsample ? (ux >> 1) : ux;
                const int64_t off = (((int64_t)a_b[i] * a.Hin + iy) * a.Win + ix) * a.Cin + c;
                dma(ok ? a.A + off : zero, sA + (i * NW + wave) * RPI * BKT);
            }
        }
        if (!tail) {
#pragma unroll
            for (int i = 0; i < BI; ++i) bdma(rsB, voB[i], kw * 2, sB + (i * NW + wave) * RPI * BKT);
        } else {
#pragma unroll
            for (int i = 0; i < BI; ++i)
                bdma(rsB, k0 + b_c[i] < kend ? voB[i] + k0 * 2 : kOOB, 0, sB + (i * NW + wave) * RPI * BKT);
        }
    };

    // Epilogue thread mapping (vector path: one fixed 8-column slice per thread, rows
    // r0 + k * rstep of each staged pass), and the residual rows of that slice.  Where
    // they cost few registers (PRE) they are loaded here, so that their latency hides
    // under the K loop; otherwise per pass in the epilogue.  Only a block that runs
    // the epilogue loads them; no block writes output rows another block reads here.
    constexpr int PR = WM * 32;                // staged rows per pass
    // staged rows per thread per pass (non-GEGLU): the threads of one staged row are the
    // NT / 8 chunk owners, NTH / (NT / 8) rows go per step
    constexpr int MAXR = (PR + NTH / (NT / 8) - 1) / (NTH / (NT / 8));
    const bool narrow = a.out_mode == OUT_F32_NCHW || (a.N & 7);
    const int NTO = NT / (a.geglu ? 2 : 1);  // output columns of this tile
    const int cpr = NTO / 8;                  // 8-column chunks per row
    const int oc = (tid % cpr) * 8;           // fixed output column slice of this thread
    const int r0 = tid / cpr, rstep = NTH / cpr;
    const int tc = a.geglu ? (oc >> 5) * 64 + (oc & 31) : oc;  // tile column of oc's source
    const int n = n0 + tc;
    const int nout = a.geglu ? (n0 >> 1) + oc : n;
    constexpr bool PRE = FM * MAXR <= 2;
    // (with a tile width whose 8-column chunks do not divide the thread count, the
    // threads past the last whole row group stay out of the vector epilogue)
    const bool ep_on = tid < rstep * cpr;
    const bool use_res = a.res && !narrow && n < a.N && (!a.partial || a.fixup);
    uint4 rres[FM][MAXR];
    auto load_res = [&](int ip) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < MAXR; ++k) {
            const int sr = r0 + k * rstep;
            const int m = min(m0 + (sr >> 5) * TMW + ip * 32 + (sr & 31), a.M - 1);
            rres[ip][k] = make_uint4(0, 0, 0, 0);
            if (use_res && sr < PR) rres[ip][k] = *(const uint4*)(a.res + (int64_t)m * a.ldr + nout);
        }
    };
    if (PRE) {
#pragma unroll
        for (int ip = 0; ip < FM; ++ip) load_res(ip);
    }

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = floatx16{};
    floatx4 acc16[MF == 16 ? FM16 : 1][MF == 16 ? FN16 : 1];
#pragma unroll
    for (int i = 0; i < (MF == 16 ? FM16 : 1); ++i)
#pragma unroll
        for (int j = 0; j < (MF == 16 ? FN16 : 1); ++j) acc16[i][j] = floatx4{};
    // LayerNorm consumer: the PPT consecutive lanes of tile row t / PPT load its 64-column
    // partials j = t % PPT, + PPT, ... (issued before the first K tiles, added after),
    // and thread t < NT the column sum of tile column t
    constexpr int PPT = NTH / MT, MAXP = 20 / PPT;  // lanes per row, partials per lane (K <= 1280)
    const bool lnc = DENSE && a.ln_part != nullptr;
    float2 ln_v[MAXP];
    float ln_cs_t = 0.f;
    if (lnc) {
        const int mm = min(m0 + tid / PPT, a.M - 1), T = a.K >> 6;
#pragma unroll
        for (int i = 0; i < MAXP; ++i) {
            const int j = tid % PPT + i * PPT;
            ln_v[i] = j < T ? *(const float2*)(a.ln_part + ((int64_t)j * a.M + mm) * 2) : make_float2(0.f, 0.f);
        }
        if (tid < NT && n0 + tid < a.N) ln_cs_t = a.ln_colsum[n0 + tid];
    }

    // fragment addressing: row (base + lrow), logical chunk 2*ks + (lane>>5);
    // every fragment base row is a multiple of 32, so the swizzle depends on lrow only
    const int lrow = lane & 31, hl = lane >> 5, sw = lds_swizzle<BKT>(lrow);
#pragma unroll
    for (int p = 0; p < NS - 1; ++p)
        if (p < nk) issue(p, p);
    float ln_s1 = 0.f, ln_s2 = 0.f;
    if (lnc) {
#pragma unroll
        for (int i = 0; i < MAXP; ++i) { ln_s1 += ln_v[i].x; ln_s2 += ln_v[i].y; }
    }
    for (int kt = 0; kt < nk; ++kt) {
        // tile kt must have landed; the tiles issued after it may still be in flight
        wait_tiles<LPT, NS - 2>(min(NS - 2, nk - 1 - kt));
        __builtin_amdgcn_s_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        // wave priority: highest while issuing the next tile's DMA, raised through this
        // tile's fragment reads and MFMAs, normal at the wait (B=2 -0.3%, B=16 -0.8%)
        __builtin_amdgcn_s_setprio(2);
        if (kt + NS - 1 < nk) issue(kt + NS - 1, (kt + NS - 1) % NS);
        __builtin_amdgcn_s_setprio(1);
        const f16* sA = smem + (kt % NS) * STAGE;
        const f16* sB = sA + MT * BKT;
        if constexpr (MF == 32) {
        half8 af[2][FM], bf[2][FN];
        auto load_frags = [&](int ks, int slot) __attribute__((always_inline)) {
            const int pc = ((ks * 2 + hl) ^ sw) * 8;
#pragma unroll
            for (int i = 0; i < FM; ++i) af[slot][i] = *(const half8*)(sA + (wm * TMW + i * 32 + lrow) * BKT + pc);
#pragma unroll
            for (int j = 0; j < FN; ++j) bf[slot][j] = *(const half8*)(sB + (wn * TNW + j * 32 + lrow) * BKT + pc);
        };
        load_frags(0, 0);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if (ks + 1 < KS) load_frags(ks + 1, (ks + 1) & 1);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[ks & 1][i], bf[ks & 1][j], acc[i][j], 0, 0, 0);
        }
        // Schedule of the unrolled K tile: reads(0), reads(1), mfma(0), reads(2),
        // mfma(1), ... -- the fragments of k-step ks+1 are in flight during the
        // MFMAs of k-step ks.
        if (KS >= 2) {
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * (FM + FN), 0);  // DS reads
#pragma unroll
            for (int ks = 0; ks < KS - 2; ++ks) {
                __builtin_amdgcn_sched_group_barrier(0x008, FM * FN, 0);  // MFMAs
                __builtin_amdgcn_sched_group_barrier(0x100, FM + FN, 0);  // DS reads
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 2 * FM * FN, 0);
        }
        } else {
        // 16x16x32: row / column lane & 15, logical chunk 4 * ks + (lane >> 4); the
        // fragment base rows are multiples of 16, so the swizzle depends on lane & 15 only
        constexpr int KS16 = BKT / 32;
        const int sw16 = lds_swizzle<BKT>(lane & 15);
        half8 af[2][FM16], bf[2][FN16];
        auto load_frags = [&](int ks, int slot) __attribute__((always_inline)) {
            const int pc = ((ks * 4 + (lane >> 4)) ^ sw16) * 8;
#pragma unroll
            for (int i = 0; i < FM16; ++i)
                af[slot][i] = *(const half8*)(sA + (wm * TMW + i * 16 + (lane & 15)) * BKT + pc);
#pragma unroll
            for (int j = 0; j < FN16; ++j)
                bf[slot][j] = *(const half8*)(sB + (wn * TNW + j * 16 + (lane & 15)) * BKT + pc);
        };
        load_frags(0, 0);
#pragma unroll
        for (int ks = 0; ks < KS16; ++ks) {
            if (ks + 1 < KS16) load_frags(ks + 1, (ks + 1) & 1);
#pragma unroll
            for (int i = 0; i < FM16; ++i)
#pragma unroll
                for (int j = 0; j < FN16; ++j)
                    acc16[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[ks & 1][i], bf[ks & 1][j], acc16[i][j], 0, 0, 0);
        }
        if (KS16 >= 2) {
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * (FM16 + FN16), 0);  // DS reads
#pragma unroll
            for (int ks = 0; ks < KS16 - 2; ++ks) {
                __builtin_amdgcn_sched_group_barrier(0x008, FM16 * FN16, 0);  // MFMAs
                __builtin_amdgcn_sched_group_barrier(0x100, FM16 + FN16, 0);  // DS reads
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 2 * FM16 * FN16, 0);
        }
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_setprio(0);
    }

    // ---- epilogue
    const int col_l = lane & 31, rq = (lane >> 5) * 4;
    float2 ln_rs = make_float2(1.f, 0.f);  // (rstd, -mean * rstd) of row tid / PPT
    if (lnc) {
        // the row's PPT lanes add their partials
#pragma unroll
        for (int off = 1; off < PPT; off <<= 1) {
            ln_s1 += __shfl_xor(ln_s1, off);
            ln_s2 += __shfl_xor(ln_s2, off);
        }
        // one-pass statistics as the reference's layernorm_f32.comp (clamped at 0)
        const float inv_k = 1.0f / (float)a.K;
        const float mean = ln_s1 * inv_k;
        const float rstd = rsqrtf(fmaxf(ln_s2 * inv_k - mean * mean, 0.f) + a.ln_eps);
        ln_rs = make_float2(rstd, -mean * rstd);
    }
    if (a.partial && !a.fixup) {
        // split K, reduce kernel: fp32 partial [split][M][N]
        float* P = a.partial + (int64_t)blockIdx.z * a.M * a.N;
        if constexpr (MF == 32) {
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
        } else {
#pragma unroll
        for (int i = 0; i < FM16; ++i)
#pragma unroll
            for (int j = 0; j < FN16; ++j) {
                const int n = n0 + wn * TNW + j * 16 + (lane & 15);
                if (n >= a.N) continue;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int m = m0 + wm * TMW + i * 16 + 4 * (lane >> 4) + e;
                    if (m < a.M) P[(int64_t)m * a.N + n] = acc16[i][j][e];
                }
            }
        }
        return;
    }
    if (a.partial) {
        // Split K, in-kernel sum: store the accumulators as they sit in registers (float4 q of
        // fragment (i, j) of wave w at ((((w * FM + i) * FN + j) * 4 + q) * 64 + lane) * 16
        // bytes into the block's slot of the tile), then count the tile's arrivals.  The
        // last block to arrive sums the slots and goes on to the epilogue; the others
        // are done.  No block waits for another.
        //
        // Ordering.  The slots are written and read only with device-coherent (sc1)
        // buffer stores and loads, which bypass the per-XCD L2's non-coherent state: an
        // sc1 store is written through to the device-coherent level, and its vmcnt
        // decrement is that write's acknowledgement; an sc1 load fetches from that level.
        // Each wave waits for its slot stores (vmcnt 0) before the block barrier; thread 0
        // then increments the tile counter (a device-scope atomic, performed at that same
        // level) and the last arriver's slot loads are issued only after it has read the
        // final count (block barrier).  So every slot store is complete at the coherent
        // level before the count that releases the tile, and the loads read that level.
        // This is a hardware-level ordering of gfx950's cache policy bits, not a HIP
        // memory-model release / acquire: the model's agent-scope release and acquire
        // (buffer_wbl2 / buffer_inv of the whole L2 around the atomic) made the B=2 64x64
        // forward 11% slower (5.92 vs 5.34 ms), so they are not used.
        constexpr int SLOT = MT * NT;       // floats per slot
        constexpr int CPOL_SC1 = 1 << 4;    // buffer cache policy: device-coherent
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        const __amdgpu_buffer_rsrc_t rsP = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(a.partial + (int64_t)bid * a.splits * SLOT), (short)0, a.splits * SLOT * 4, 0x00020000);
        // the lane's accumulators as QPL float4 quads: quad (i * FN + j) * 4 + q is elements
        // 4q .. 4q+3 of the 32x32 fragment (i, j), or quad i * FN16 + j the 16x16 fragment
        constexpr int QPL = MF == 32 ? FM * FN * 4 : FM16 * FN16;
        auto get_quad = [&](int qi) __attribute__((always_inline)) -> f32x4 {
            if constexpr (MF == 32) {
                const int i = qi / (FN * 4), j = (qi / 4) % FN, q = qi % 4;
                return f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
            } else {
                const floatx4 v = acc16[qi / FN16][qi % FN16];
                return f32x4{v[0], v[1], v[2], v[3]};
            }
        };
        auto add_quad = [&](int qi, f32x4 v) __attribute__((always_inline)) {
            if constexpr (MF == 32) {
                const int i = qi / (FN * 4), j = (qi / 4) % FN, q = qi % 4;
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += v[e];
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) acc16[qi / FN16][qi % FN16][e] += v[e];
            }
        };
        const uint32_t vo_w = (uint32_t)((wave * QPL * 64 + lane) * 16);
#pragma unroll
        for (int qi = 0; qi < QPL; ++qi)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, get_quad(qi)), rsP, vo_w + qi * 1024,
                                                   blockIdx.z * SLOT * 4, CPOL_SC1);
        wait_vmcnt_lgkm0<0>();  // this wave's slot stores are complete
        __syncthreads();        // ... for every wave; no wave still reads the ring
        int* const flag = (int*)smem;
        if (tid == 0) {
            const unsigned prev = __hip_atomic_fetch_add(a.tile_cnt + bid, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const bool last = prev == (unsigned)a.splits - 1;
            // ready for the next launch on this workspace
            if (last) __hip_atomic_store(a.tile_cnt + bid, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *flag = last;
        }
        __syncthreads();
        if (!*flag) return;
        // The tile is the sum of all slots in slot order (the own slot re-read), so
        // the result does not depend on which block arrived last.  Slots go in rounds
        // of SPR, every load of a round issued before any is added (slot indices
        // clamped, repeats not added).
        constexpr int SPR = QPL >= 16 ? 1 : (QPL >= 8 ? 2 : 4);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = floatx16{};
#pragma unroll
        for (int i = 0; i < (MF == 16 ? FM16 : 1); ++i)
#pragma unroll
            for (int j = 0; j < (MF == 16 ? FN16 : 1); ++j) acc16[i][j] = floatx4{};
        for (int z0 = 0; z0 < a.splits; z0 += SPR) {
            f32x4 pv[SPR][QPL];
#pragma unroll
            for (int u = 0; u < SPR; ++u) {
                const int so = min(z0 + u, a.splits - 1) * SLOT * 4;
#pragma unroll
                for (int qi = 0; qi < QPL; ++qi)
                    pv[u][qi] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsP, vo_w + qi * 1024, so, CPOL_SC1));
            }
#pragma unroll
            for (int u = 0; u < SPR; ++u) {
                const bool use = z0 + u < a.splits;
#pragma unroll
                for (int qi = 0; qi < QPL; ++qi) add_quad(qi, use ? pv[u][qi] : f32x4{0.f, 0.f, 0.f, 0.f});
            }
        }
    }
    // The fp32 tile goes through LDS (reusing the ring) in FM passes of WM*32 rows
    // (rows wm*TMW + i*32 + [0,32) of pass i).  In the vector path each thread owns
    // one fixed 8-column slice; the residual was loaded before any store (it may
    // alias the output), and stores are 16-byte.
    constexpr int CST = NT + 4;  // padded fp32 row stride
    static_assert(PR * CST * 4 <= NS * STAGE * 2, "C pass fits the operand LDS");
    static_assert(NTH * 32 * 4 <= NS * STAGE * 2, "statistics flush fits the operand LDS");
    float* Cs = (float*)smem;
    // LayerNorm consumer tables after the C pass area: (rstd, -mean * rstd) per tile
    // row, column sums of the tile's columns (written after the first pass barrier)
    constexpr int TBL = PR * CST;
    static_assert((TBL + 2 * MT + NT) * 4 <= NS * STAGE * 2, "LayerNorm tables fit the operand LDS");
    float2* const ln_rt = (float2*)(Cs + TBL);
    float* const ln_cs = Cs + TBL + 2 * MT;
    float badd[8], gadd[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) { badd[e] = 0.f; gadd[e] = 0.f; }
    if (!narrow && n < a.N) {
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
    }
    // per-channel output statistics (GroupNorm of the consumer): this thread's 8
    // columns over its rows, for the tile's first image (slot 0) and the next (slot 1)
    const bool do_st = a.stats != nullptr && !narrow;
    // (sub-pixel conv: statistics rows counted within the phase, stats_hw = Hin * Win)
    const int st_b0 = do_st ? (m0 - sp_base) / a.stats_hw : 0;
    const int st_mb = sp_base + (st_b0 + 1) * a.stats_hw;  // first row of the next image
    float st[2][2][8];
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
        for (int e = 0; e < 8; ++e) { st[sl][0][e] = 0.f; st[sl][1][e] = 0.f; }
    // per-row output statistics (LayerNorm of the consumer): this thread's 8 columns
    // of each of its rows
    const bool do_rs = a.row_part != nullptr && !narrow;
    float rsum[FM][MAXR], rsq[FM][MAXR];
#pragma unroll
    for (int ip = 0; ip < FM; ++ip)
#pragma unroll
        for (int k = 0; k < MAXR; ++k) { rsum[ip][k] = 0.f; rsq[ip][k] = 0.f; }
#pragma unroll
    for (int ip = 0; ip < FM; ++ip) {
        __syncthreads();
        if (lnc && ip == 0) {
            if (tid % PPT == 0) ln_rt[tid / PPT] = ln_rs;
            if (tid < NT) ln_cs[tid] = ln_cs_t;
        }
        if constexpr (MF == 32) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int r = wm * 32 + (e >> 2) * 8 + rq + (e & 3);
                Cs[r * CST + wn * TNW + j * 32 + col_l] = acc[ip][j][e];
            }
        } else {
#pragma unroll
        for (int i = 0; i < FM16; ++i)
#pragma unroll
            for (int j = 0; j < FN16; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = wm * 32 + i * 16 + 4 * (lane >> 4) + e;
                    Cs[r * CST + wn * TNW + j * 16 + (lane & 15)] = acc16[i][j][e];
                }
        }
        __syncthreads();
        // staged row s <-> tile row (s / 32) * TMW + ip * 32 + s % 32
        if (narrow) {
            const int nto = a.geglu ? NT / 2 : NT;
            for (int idx = tid; idx < PR * nto; idx += NTH) {
                const int sr = idx / nto, o = idx - sr * nto;
                const int t = a.geglu ? (o >> 5) * 64 + (o & 31) : o;
                const int m = m0 + (sr >> 5) * TMW + ip * 32 + (sr & 31), nn = n0 + t;
                if (m >= a.M || nn >= a.N) continue;
                epi_store(a, m, nn, Cs[sr * CST + t], a.geglu ? Cs[sr * CST + t + 32] : 0.f,
                          a.geglu ? (n0 >> 1) + o : nn);
            }
            continue;
        }
        if (n >= a.N || !ep_on) continue;
        if (!PRE) load_res(ip);
#pragma unroll
        for (int k = 0; k < MAXR; ++k) {
            const int sr = r0 + k * rstep;
            const int m = m0 + (sr >> 5) * TMW + ip * 32 + (sr & 31);
            if (sr >= PR || m >= a.M) continue;
            // the row's 8 (GEGLU: 2 x 8) staged values as 16-byte LDS reads (rows are
            // CST = NT + 4 floats, tc a multiple of 8: 16-byte aligned)
            // (LayerNorm consumer: rstd * (acc - mean * colsum) + bias)
            const float* crow = Cs + sr * CST + tc;
            float2 lt = make_float2(1.f, 0.f);
            if (lnc) lt = ln_rt[(sr >> 5) * TMW + ip * 32 + (sr & 31)];
            float v[8];
            ld8(crow, v);
            if (lnc) {
                float sn[8];
                ld8(ln_cs + tc, sn);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = fmaf(lt.x, v[e], lt.y * sn[e]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] += badd[e];
            if (a.geglu) {
                float g[8];
                ld8(crow + 32, g);
                if (lnc) {
                    float sn[8];
                    ld8(ln_cs + tc + 32, sn);
#pragma unroll
                    for (int e = 0; e < 8; ++e) g[e] = fmaf(lt.x, g[e], lt.y * sn[e]);
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] *= gelu_erf(g[e] + gadd[e]);
            }
            if (a.res) {
                const f16* rh = (const f16*)&rres[ip][k];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] += (float)rh[e];
            }
            if (a.act) {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = apply_act(a.act, v[e]);
            }
            if (a.out_mode == OUT_F16) {
                uint4 o;
                f16* oh = (f16*)&o;
#pragma unroll
                for (int e = 0; e < 8; ++e) oh[e] = (f16)v[e];
                int mo = m;  // output row (sub-pixel conv: the phase's pixel in the upsampled image)
                if (subpix) {
                    const int hwi = a.Hin * a.Win, q = m - sp_base;
                    const int bb = q / hwi, r = q - bb * hwi, iy = r / a.Win, ix = r - iy * a.Win;
                    mo = (bb * a.Ho + 2 * iy + (sp_ph >> 1)) * a.Wo + 2 * ix + (sp_ph & 1);
                }
                *(uint4*)((f16*)a.C + (int64_t)mo * a.ldc + nout) = o;
                if (do_rs) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float f = (float)oh[e];
                        rsum[ip][k] += f;
                        rsq[ip][k] += f * f;
                    }
                }
                if (do_st) {
                    const bool s1 = m >= st_mb;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float f = (float)oh[e];
                        if (s1) { st[1][0][e] += f; st[1][1][e] += f * f; }
                        else { st[0][0][e] += f; st[0][1][e] += f * f; }
                    }
                }
            } else {
                float* cp = (float*)a.C + (int64_t)m * a.ldc + nout;
                *(float4*)cp = make_float4(v[0], v[1], v[2], v[3]);
                *(float4*)(cp + 4) = make_float4(v[4], v[5], v[6], v[7]);
            }
        }
    }
    if (do_st) stats_flush<NTH, NT / 8>(a, st, st_b0, min(a.M, m0 + MT) - 1 - sp_base, n0, (float*)smem);
    if (do_rs) {
        // the cpr threads of a row are consecutive lanes, each 8 of them one 64-column
        // group: add their partial sums; the first of the 8 stores the group's partial
#pragma unroll
        for (int ip = 0; ip < FM; ++ip)
#pragma unroll
            for (int k = 0; k < MAXR; ++k) {
                float s1 = rsum[ip][k], s2 = rsq[ip][k];
#pragma unroll
                for (int off = 1; off < 8; off <<= 1) {
                    s1 += __shfl_xor(s1, off);
                    s2 += __shfl_xor(s2, off);
                }
                const int sr = r0 + k * rstep;
                const int m = m0 + (sr >> 5) * TMW + ip * 32 + (sr & 31);
                if ((oc & 63) == 0 && sr < PR && m < a.M && n < a.N)
                    *(float2*)(a.row_part + ((int64_t)(n >> 6) * a.M + m) * 2) = make_float2(s1, s2);
            }
    }
}

// 3x3 conv (pad 1, stride 1, no upsample) with at most 8 output channels (the UNet's
// conv_out, 320 -> 4): an MFMA tile would be 64 columns wide for 4, and 64 such tiles
// cannot fill the chip.  One thread per (pixel, K slice), 16 pixels x 16 slices per
// block: slice s takes the 8-channel chunks j = s, s + 16, ... of the pixel's 9 Cin / 8
// (tap-major, as W's K index) with fp16 dot products into fp32, the weights staged
// in LDS (dynamic, CO * 9 * Cin * 2 bytes); the 16 slices of a pixel are consecutive
// lanes, added by shuffles, and the first runs the common epilogue.  Loads go in
// batches of 12 chunks (two batches at Cin = 320), all issued before any is used.  A
// block takes 16-pixel groups g, g + gridDim.x, ... (at most kNarrowBlocks blocks), so on
// large images (the VAE's 512x512 conv_out) the staged weights serve many groups.
constexpr int kNarrowPix = 16, kNarrowSlices = 16, kNarrowBatch = 12, kNarrowBlocks = 2048;
template <int CO>
__global__ __launch_bounds__(256) void conv3_narrow_kernel(GemmArgs a) {
    if (a.c_ind) a.C = *a.c_ind;
    typedef _Float16 half2v __attribute__((ext_vector_type(2)));
    extern __shared__ uint4 wsm[];  // [CO][nchunk]
    const int cpt = a.Cin / 8, nchunk = 9 * cpt;
    {
        // CO * nchunk <= 4096 chunks (narrow_conv): at most 16 per thread, loads first
        constexpr int SMAX = 4096 / (kNarrowPix * kNarrowSlices);
        uint4 wv[SMAX];
#pragma unroll
        for (int u = 0; u < SMAX; ++u) {
            const int i = threadIdx.x + u * kNarrowPix * kNarrowSlices, co = i / nchunk, j = i - co * nchunk;
            wv[u] = make_uint4(0, 0, 0, 0);
            if (i < CO * nchunk && co < a.N) wv[u] = *(const uint4*)(a.Wt + (int64_t)co * a.K + j * 8);
        }
#pragma unroll
        for (int u = 0; u < SMAX; ++u) {
            const int i = threadIdx.x + u * kNarrowPix * kNarrowSlices;
            if (i < CO * nchunk) wsm[i] = wv[u];
        }
    }
    __syncthreads();
    const int tid = threadIdx.x, sl = tid % kNarrowSlices;
    const int ngroups = (a.M + kNarrowPix - 1) / kNarrowPix;
    for (int grp = blockIdx.x; grp < ngroups; grp += gridDim.x) {
        const int p = grp * kNarrowPix + tid / kNarrowSlices;
        const int m = min(p, a.M - 1);
        const int hw = a.Ho * a.Wo, bb = m / hw, r = m - bb * hw, oy = r / a.Wo, ox = r - oy * a.Wo;
        float acc[CO];
#pragma unroll
        for (int co = 0; co < CO; ++co) acc[co] = 0.f;
        // chunks in batches: every load of a batch issued before any is used
        for (int j0 = sl; j0 < nchunk; j0 += kNarrowSlices * kNarrowBatch) {
            uint4 x[kNarrowBatch];
#pragma unroll
            for (int u = 0; u < kNarrowBatch; ++u) {
                const int j = j0 + u * kNarrowSlices;
                const int tap = j / cpt, c8 = j - tap * cpt;
                const int iy = oy + tap / 3 - 1, ix = ox + tap % 3 - 1;
                x[u] = make_uint4(0, 0, 0, 0);
                if (j < nchunk && iy >= 0 && iy < a.Hin && ix >= 0 && ix < a.Win)
                    x[u] = *(const uint4*)(a.A + (((int64_t)bb * a.Hin + iy) * a.Win + ix) * a.Cin + c8 * 8);
            }
#pragma unroll
            for (int u = 0; u < kNarrowBatch; ++u) {
                const int j = j0 + u * kNarrowSlices;
                if (j >= nchunk) break;
                const half2v* xh = (const half2v*)&x[u];
#pragma unroll
                for (int co = 0; co < CO; ++co) {
                    const uint4 w = wsm[co * nchunk + j];
                    const half2v* wh = (const half2v*)&w;
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[co] = __builtin_amdgcn_fdot2(xh[q], wh[q], acc[co], false);
                }
            }
        }
#pragma unroll
        for (int co = 0; co < CO; ++co)
#pragma unroll
            for (int off = 1; off < kNarrowSlices; off <<= 1) acc[co] += __shfl_xor(acc[co], off);
        if (sl == 0 && p < a.M) {
#pragma unroll
            for (int co = 0; co < CO; ++co)
                if (co < a.N) epi_store(a, p, co, acc[co], 0.f, co);
        }
    }
}

// The narrow conv takes a 3x3 conv when its weights (up to 8 outputs) fit 64 KB of LDS.
static bool narrow_conv(const GemmArgs& a) {
    return a.amode == A_CONV3 && a.N <= 8 && a.stride == 1 && !a.upsample && !a.A2 && !a.stats && !a.geglu &&
           !a.row_part && a.Cin % 8 == 0 && 8 * 9 * (a.Cin / 8) <= 4096 && a.M > 0;
}

namespace {
struct Cfg {
    int mt, nt, per_cu;   // tile, resident blocks per CU (LDS-limited)
    double rate1, rate2;  // measured MFMA FLOP/s of one CU running 1 / 2 such blocks
    double t_fix;         // per-block prologue + epilogue time
    int spr;              // split slots per modelled round of the summing block's tail
    double conv_f;        // rate factor with the implicit-conv A (the tap gather)
};
// 0: 256x128, 8 waves of 64x64, BK 64, 2-stage ring (96 KB: one block per CU)
// 1: 128x128, 8 waves of 64x32, BK 64, 2-stage ring (64 KB: two per CU, 4 waves per SIMD)
// 2: 128x64,  8 waves of 32x32, BK 64, 3-stage ring (72 KB: two per CU, 4 waves per SIMD)
// 3: 64x160,  4 waves of 32x80 (16x16x32 MFMAs), BK 64, 2-stage ring (56 KB: two per CU)
// Rates and fixed costs from dense GEMMs that give every CU one or two blocks, at
// K = 512 and 4096 (the difference gives the rate, the rest the fixed cost).  The
// 128x128 two-block rate is set above that fit (3.54): the 64x64 convs over the up
// path's concatenated inputs run two splits as co-resident pairs faster than it
// predicts (640 -> 320: 56.6 us with 2 splits against 62.4 with 4), and whole forwards
// compared in one call take 5.09 against 5.10 ms (B=2 64x64), 9.69 against 9.78 (96x96)
// and 21.45 against 21.45 (B=16).  The implicit-conv A (a tap gather per row) costs the
// 64-column tile about 20% of its rate.
// The 64x160 tile covers N = 320 with no padded column and M = 8192 with 256 tiles, so it
// fills the chip where 128-row tiles leave a quarter of the CUs idle, but its own rate is
// lower (4 waves, 46 FLOP per operand byte against 64): its parameters are fitted to 18
// UNet GEMMs timed with both tiles in one forward (B=2 and 16, 64x64 latents).  In whole
// forwards the planner then takes it for the 64x64 level's convs at B=2 (M = 8192,
// N = 320: 38.5 against 41.8 us at K = 2880, 83.4 against 93.0 at K = 8640), the 77-token
// cross K/V GEMM (21.2 against 24.6 us) and two B=16 feed-forward outputs, each faster
// than before; it loses at larger M (B=16 conv, M = 65536: 192.6 against 178.3 us).
constexpr int kNumCfg = 4;
// The tail model counts one slot per round for the 128-row tiles and two for the others
// (their kernels load 1, 2, 4 and 2 slots per round): moving the 128x128 tile to its
// kernel's 2 sends the 64x64 and 48x48 levels' concat convs from the reduce launch to the
// in-kernel sum and changed them by -10% to +15% each, no gain over a forward.
const Cfg kCfgs[kNumCfg] = {{256, 128, 1, 3.5e12, 3.5e12, 4.5e-6, 1, 1.0},
                            {128, 128, 2, 2.76e12, 3.9e12, 3.0e-6, 1, 1.0},
                            {128, 64, 2, 2.23e12, 3.03e12, 2.5e-6, 2, 0.8},
                            {64, 160, 2, 2.0e12, 3.4e12, 6.0e-6, 2, 0.9}};
// full kernel names, as the instantiations (tile configuration, A mode: 0 dense, 1 implicit conv,
// then the MFMA)
const char* const kNames[kNumCfg][2] = {{"gemm_kernel<256,128,4,2,64,2,0,32>", "gemm_kernel<256,128,4,2,64,2,1,32>"},
                                        {"gemm_kernel<128,128,2,4,64,2,0,32>", "gemm_kernel<128,128,2,4,64,2,1,32>"},
                                        {"gemm_kernel<128,64,4,2,64,3,0,32>", "gemm_kernel<128,64,4,2,64,3,1,32>"},
                                        {"gemm_kernel<64,160,2,2,64,2,0,16>", "gemm_kernel<64,160,2,2,64,2,1,16>"}};

int ceil_div(int a, int b) { return (a + b - 1) / b; }

// In-kernel split-K sum: tile counters at the head of the workspace (one per tile),
// the slots the summing block loads per round (as the kernel's SPR), and the
// modelled cost of its tail.
constexpr int kMaxSplitTiles = 16384;
constexpr size_t kCounterBytes = kMaxSplitTiles * sizeof(unsigned);
constexpr double kFixBase = 1.0e-6, kFixRound = 0.9e-6;

// The epilogue keeps output statistics for two images per tile: the MT rows of a tile
// (MT-aligned) must not reach a third image.
bool stats_tile_ok(int mt, int hw) { return hw >= mt || mt == 2 * hw; }

// Pick the tile shape and split-K factor with the lowest modelled time.  Blocks are
// spread evenly over the 256 CUs; the busiest CU runs its blocks two at a time where
// the tile allows two per CU (a lone block cannot keep a CU busy: rate1 < rate2),
// each round paying a fixed prologue / epilogue cost.  A split K adds the fp32
// partial round trip (mostly L2 / Infinity Cache resident) and the serial tail of
// the block that sums a tile's partials.
void plan(const GemmArgs& a, int& ci, int& splits, int& kps, bool& fix) {
    const int nkt = ceil_div(a.K, 64);
    double best = 1e30;
    ci = 1; splits = 1; kps = nkt * 64; fix = false;
    for (int c = 0; c < kNumCfg; ++c) {
        const Cfg& g = kCfgs[c];
        if (a.geglu && g.nt % 128) continue;  // GEGLU pairs 32-column blocks within a 64-wide wave tile
        // LayerNorm row partials: one per 64 columns, summed by 8 consecutive lanes
        if (a.row_part && g.nt % 64) continue;
        // the LayerNorm consumer's epilogue runs 5-8% slower in the 4-wave 64x160 tile than
        // the 128x128 tile at K = 1280 (M = 1152, N = 3840: 27.8 against 25.7 us), which
        // the model does not see
        if (a.ln_part && g.mt == 64) continue;
        // (sub-pixel conv: whole phases per tile; statistics images of Hin * Win rows)
        if (a.subpix && (a.M >> 2) % g.mt) continue;
        if (a.stats && !stats_tile_ok(g.mt, a.subpix ? a.Hin * a.Win : a.stats_hw)) continue;
        const int tiles = ceil_div(a.M, g.mt) * ceil_div(a.N, g.nt);
        static const int cand[] = {1, 2, 3, 4, 6, 8, 12, 16, 24, 32};
        for (int s : cand) {
            if (s > 1 && nkt / s < 4) break;
            const int kt_per = ceil_div(nkt, s);
            const int se = ceil_div(nkt, kt_per);
            const long blocks = (long)tiles * se;
            const long load = (blocks + 255) / 256;  // blocks on the busiest CU
            const double w = 2.0 * g.mt * g.nt * kt_per * 64.0;
            const long pairs = g.per_cu >= 2 ? load / 2 : 0, singles = load - 2 * pairs;
            const double cf = a.amode == A_CONV3 ? g.conv_f : 1.0;
            double t = pairs * (2.0 * w / (g.rate2 * cf) + g.t_fix) + singles * (w / (g.rate1 * cf) + g.t_fix);
            // a split adds the partial round trip, and either the reduce launch (about
            // 5.5 us, 2 us more with statistics) or the serial tail of each tile's last
            // block (the count, then its rounds of slot loads)
            bool fx = false;
            if (se > 1) {
                const double part = (double)se * a.M * a.N * 8.0 / 20.0e12;
                // (with output statistics only the in-kernel sum: the reduce keeps none)
                const double t_red = (a.stats || a.row_part || a.ln_part || a.subpix) ? 1e30 : part + 5.5e-6;
                const int rounds = ceil_div(se, g.spr);
                const double t_fix = tiles <= kMaxSplitTiles ? part + kFixBase + kFixRound * rounds : 1e30;
                fx = t_fix < t_red;
                t += fx ? t_fix : t_red;
            }
            if (t < best * 0.98) { best = t; ci = c; splits = se; kps = kt_per * 64; fix = fx; }
        }
    }
}
}  // namespace

bool gemm_stats_supported(int hw) { return stats_tile_ok(128, hw); }

const char* gemm_kernel_name(const GemmArgs& a) {
    if (narrow_conv(a)) return a.N <= 4 ? "conv3_narrow_kernel<4>" : "conv3_narrow_kernel<8>";
    int ci, splits, kps;
    bool fix;
    plan(a, ci, splits, kps, fix);
    return kNames[ci][a.amode == A_CONV3];
}

size_t gemm_counter_bytes() { return kCounterBytes; }

size_t gemm_workspace_bytes(const GemmArgs& a) {
    if (narrow_conv(a)) return 0;
    int ci, splits, kps;
    bool fix;
    plan(a, ci, splits, kps, fix);
    if (splits == 1) return 0;
    const Cfg& g = kCfgs[ci];
    const size_t tiles = (size_t)ceil_div(a.M, g.mt) * ceil_div(a.N, g.nt);
    return kCounterBytes + (fix ? tiles * g.mt * g.nt : (size_t)a.M * a.N) * splits * sizeof(float);
}

template <int AM>
static void launch_cfg(int ci, dim3 grid, const GemmArgs& a, hipStream_t s) {
    if (ci == 0) SDU_LAUNCH((gemm_kernel<256, 128, 4, 2, 64, 2, AM>), grid, dim3(512), 0, s, a);
    else if (ci == 1) SDU_LAUNCH((gemm_kernel<128, 128, 2, 4, 64, 2, AM>), grid, dim3(512), 0, s, a);
    else if (ci == 2) SDU_LAUNCH((gemm_kernel<128, 64, 4, 2, 64, 3, AM>), grid, dim3(512), 0, s, a);
    else SDU_LAUNCH((gemm_kernel<64, 160, 2, 2, 64, 2, AM, 16>), grid, dim3(256), 0, s, a);
}

hipError_t gemm_launch(GemmArgs a, float* ws, hipStream_t s) {
    if (narrow_conv(a)) {
        if (a.Ho != a.Hin || a.Wo != a.Win || a.M != a.Bn * a.Ho * a.Wo || a.K != 9 * a.Cin ||
            2 * (int64_t)a.Bn * a.Hin * a.Win * a.Cin > 0x7fffffff)
            return hipErrorInvalidValue;
        a.splits = 1;
        a.partial = nullptr;
        const int co = a.N <= 4 ? 4 : 8;
        const size_t lds = (size_t)co * 9 * a.Cin * 2;
        const dim3 grid(std::min((a.M + kNarrowPix - 1) / kNarrowPix, kNarrowBlocks));
        const double flops = 2.0 * a.M * a.N * a.K;
        const double bytes = 2.0 * a.Bn * a.Hin * a.Win * a.Cin + 2.0 * a.N * a.K +
                             (double)a.M * a.N * (a.out_mode == OUT_F16 ? 2.0 : 4.0) + (a.res ? 2.0 * a.M * a.N : 0.0);
        launch_timed(co == 4 ? "conv3_narrow_kernel<4>" : "conv3_narrow_kernel<8>", flops, bytes, [&] {
            if (co == 4) SDU_LAUNCH(conv3_narrow_kernel<4>, grid, dim3(kNarrowPix * kNarrowSlices), lds, s, a);
            else SDU_LAUNCH(conv3_narrow_kernel<8>, grid, dim3(kNarrowPix * kNarrowSlices), lds, s, a);
        });
        return hipGetLastError();
    }
    if (a.c_ind) return hipErrorInvalidValue;  // the narrow conv only
    int ci, splits, kps;
    bool fix;
    plan(a, ci, splits, kps, fix);
    if (a.A2 == nullptr) a.K1 = a.K;
    if (a.A3 == nullptr) a.K2 = a.K;
    if (a.A3 && (a.amode != A_CONV3 || !a.A2)) return hipErrorInvalidValue;
    // (a consumer thread sums up to 10 row partials; 2 or 4 threads per tile row)
    if (a.ln_part && (a.amode != A_DENSE || a.A2 || !a.ln_colsum || a.out_mode != OUT_F16 || (a.N & 7) ||
                      (a.K & 63) || a.K > 1280 || !(a.ln_eps > 0.f) || (splits > 1 && !fix)))
        return hipErrorInvalidValue;
    if (a.row_part && (a.out_mode != OUT_F16 || a.geglu || (a.N & 63) || (splits > 1 && !fix)))
        return hipErrorInvalidValue;
    if (a.subpix) {
        if (a.amode != A_CONV3 || a.upsample || a.stride != 1 || a.A2 || a.A3 || a.Cin % 64 || a.K != 4 * a.Cin ||
            a.Ho != 2 * a.Hin || a.Wo != 2 * a.Win || a.M != a.Bn * a.Ho * a.Wo || a.res || a.row_part ||
            a.ln_part || a.geglu || a.out_mode != OUT_F16 || (a.N & 7) || (a.M >> 2) % kCfgs[ci].mt ||
            (splits > 1 && !fix) || (a.stats && a.stats_hw != a.Ho * a.Wo))
            return hipErrorInvalidValue;
        if (a.stats) a.stats_hw = a.Hin * a.Win;  // the kernel counts rows within a phase
    }
    if (a.amode == A_CONV3 && a.A2 &&
        (a.K1 != 9 * a.Cin || a.K1 % 64 || a.K2 % 64 || a.K % 64 || a.K2 <= a.K1 || a.K <= a.K1 ||
         (a.A3 && a.K2 >= a.K) || a.stride != 1 || a.upsample || a.Ho != a.Hin || a.Wo != a.Win ||
         a.M != a.Bn * a.Ho * a.Wo || a.lda2 < a.K2 - a.K1 || (a.A3 && a.lda3 < a.K - a.K2)))
        return hipErrorInvalidValue;
    a.splits = splits;
    a.k_per_split = kps;
    a.fixup = fix;
    // tile order: N-major when the weights outweigh the A source (a conv's A is its input
    // image, whose 9 taps hit the same L2 lines)
    {
        const double w_b = 2.0 * a.N * a.K;
        const double a_b = a.amode == A_CONV3 ? 2.0 * a.Bn * a.Hin * a.Win * a.Cin + 2.0 * a.M * (a.K - a.K1)
                                              : 2.0 * a.M * a.K;
        a.n_major = w_b > a_b;
    }
    a.tile_cnt = splits > 1 ? (unsigned*)ws : nullptr;
    a.partial = splits > 1 ? (float*)((char*)ws + kCounterBytes) : nullptr;
    if (splits > 1 && ws == nullptr) return hipErrorInvalidValue;
    // operands are addressed with 32-bit byte offsets (buffer resources)
    const int64_t lim = 0x7fffffff;
    if ((a.subpix ? 8 : 2) * (int64_t)a.N * a.K > lim) return hipErrorInvalidValue;
    if (a.amode == A_DENSE && (2 * (int64_t)a.M * a.lda > lim || (a.A2 && 2 * (int64_t)a.M * a.lda2 > lim)))
        return hipErrorInvalidValue;
    if (a.amode == A_CONV3 && (2 * (int64_t)a.Bn * a.Hin * a.Win * a.Cin > lim ||
                               (a.A2 && 2 * (int64_t)a.M * a.lda2 > lim) || (a.A3 && 2 * (int64_t)a.M * a.lda3 > lim)))
        return hipErrorInvalidValue;
    const Cfg& g = kCfgs[ci];
    if (a.stats && (a.out_mode != OUT_F16 || a.geglu || (a.N & 7) || a.stats_hw < 64 ||
                    !stats_tile_ok(g.mt, a.stats_hw)))
        return hipErrorInvalidValue;
    dim3 grid(ceil_div(a.M, g.mt) * ceil_div(a.N, g.nt), 1, splits);
    // algorithmic traffic: A once (the conv source image, not its im2col), W once, output
    // (+ residual) once.  A split's fp32 partials are overhead, not algorithmic traffic:
    // they are counted nowhere, and the reduce launch reports no algorithmic bytes
    const int nout = a.geglu ? a.N / 2 : a.N;
    const double a_bytes = a.amode == A_CONV3 ? 2.0 * a.Bn * a.Hin * a.Win * a.Cin + 2.0 * a.M * (a.K - a.K1)
                                              : 2.0 * a.M * a.K;
    const double out_bytes = (double)a.M * nout * (a.out_mode == OUT_F16 ? 2.0 : 4.0) +
                             (a.res ? 2.0 * a.M * nout : 0.0);
    // (the sub-pixel conv is counted as the 3x3 conv it computes: 9 taps of Cin, the 3x3
    // weights; it issues 4 / 9 of those FLOPs)
    const double kop = a.subpix ? 9.0 * a.Cin : (double)a.K;
    const double flops = 2.0 * a.M * a.N * kop;
    const double k_bytes = a_bytes + 2.0 * a.N * kop + out_bytes;
    launch_timed(kNames[ci][a.amode == A_CONV3], flops, k_bytes, [&] {
        if (a.amode == A_DENSE) launch_cfg<A_DENSE>(ci, grid, a, s);
        else launch_cfg<A_CONV3>(ci, grid, a, s);
    });
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1 || fix) return e;
    return splitk_reduce_launch(a, 0.0, s);
}

hipError_t splitk_reduce_launch(const GemmArgs& a, double bytes, hipStream_t s) {
    const int nout = a.geglu ? a.N / 2 : a.N;
    const bool vec = a.out_mode != OUT_F32_NCHW && (a.N & 7) == 0;
    const int64_t total = (int64_t)a.M * (vec ? nout / 8 : nout);
    // 128-thread blocks: the reduces of the 8x8 and 16x16 convs (20-80K threads) spread over
    // more CUs; per B=2 64x64 forward 226 against 238 us with 256 (512: 272 us)
    launch_timed("splitk_reduce_kernel", 0.0, bytes, [&] {
        SDU_LAUNCH(splitk_reduce_kernel, dim3((unsigned)((total + 127) / 128)), dim3(128), 0, s, a);
    });
    return hipGetLastError();
}

// ----------------------------------------------------------------- GEMV (time MLP)

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + __expf(-x)); }

// y[n] = act_out(sum_k act_in(x[k]) W[n][k] + bias[n]).  act_in(x) is formed once per
// block in LDS; each wave then takes GV_ROWS rows, lane l the 8-column chunks l, l+64,
// ..., with all of a chunk's row loads issued together.  K % 8 == 0, K <= GV_MAXK.
static constexpr int GV_ROWS = 4;
static constexpr int GV_MAXK = 2048;
// NV vectors at once (x [NV][K], y [NV][N]): each weight row is read once for all of
// them; every vector's sums run in the same order as with NV = 1.
template <int NV>
__global__ __launch_bounds__(256) void gemv_kernel(const float* x, const f16* W, const f16* bias,
                                                   float* y, int N, int K, int act_in, int act_out) {
    __shared__ __attribute__((aligned(16))) float xs[NV][GV_MAXK];
    for (int k = threadIdx.x; k < K; k += 256)
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const float t = x[(int64_t)v * K + k];
            xs[v][k] = act_in ? silu_f(t) : t;
        }
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * GV_ROWS;
    float s[GV_ROWS][NV];
#pragma unroll
    for (int r = 0; r < GV_ROWS; ++r)
#pragma unroll
        for (int v = 0; v < NV; ++v) s[r][v] = 0.f;
#pragma unroll
    for (int j = 0; j < GV_MAXK / 512; ++j) {
        const int k = (lane + 64 * j) * 8;
        if (k >= K) break;
        uint4 wv[GV_ROWS];
#pragma unroll
        for (int r = 0; r < GV_ROWS; ++r) wv[r] = *(const uint4*)(W + (int64_t)min(row0 + r, N - 1) * K + k);
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const float4 x0 = *(const float4*)&xs[v][k], x1 = *(const float4*)&xs[v][k + 4];
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int r = 0; r < GV_ROWS; ++r) {
                const f16* wh = (const f16*)&wv[r];
#pragma unroll
                for (int i = 0; i < 8; ++i) s[r][v] += xv[i] * (float)wh[i];
            }
        }
    }
#pragma unroll
    for (int r = 0; r < GV_ROWS; ++r)
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            float t = s[r][v];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) t += __shfl_xor(t, off);
            const int n = row0 + r;
            if (lane == 0 && n < N) {
                if (bias) t += (float)bias[n];
                if (act_out) t = silu_f(t);
                y[(int64_t)v * N + n] = t;
            }
        }
}

hipError_t gemv_launch(const float* x, const f16* W, const f16* bias, float* y, int N, int K,
                       int act_in, int act_out, hipStream_t s, int nvec) {
    if (N <= 0 || K <= 0 || K % 8 || K > GV_MAXK || nvec < 1) return hipErrorInvalidValue;
    const dim3 grid((N + 4 * GV_ROWS - 1) / (4 * GV_ROWS));
    for (int v0 = 0; v0 < nvec;) {
        const int nv = nvec - v0 >= 4 ? 4 : nvec - v0 >= 2 ? 2 : 1;
        const float* xv = x + (int64_t)v0 * K;
        float* yv = y + (int64_t)v0 * N;
        char name[24];
        snprintf(name, sizeof name, "gemv_kernel<%d>", nv);
        launch_timed(name, 2.0 * nv * N * K, 2.0 * N * K + 4.0 * nv * (N + K), [&] {
            if (nv == 4) SDU_LAUNCH(gemv_kernel<4>, grid, dim3(256), 0, s, xv, W, bias, yv, N, K, act_in, act_out);
            else if (nv == 2) SDU_LAUNCH(gemv_kernel<2>, grid, dim3(256), 0, s, xv, W, bias, yv, N, K, act_in, act_out);
            else SDU_LAUNCH(gemv_kernel<1>, grid, dim3(256), 0, s, xv, W, bias, yv, N, K, act_in, act_out);
        });
        v0 += nv;
    }
    return hipGetLastError();
}

}  // namespace sdu
