// Internal interfaces between the host runtime (runtime.cpp, unet.cpp, capi.cpp)
// and the gfx950 kernels (k_*.hip).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstddef>

namespace sdu {

typedef _Float16 f16;

// GELU with the erf of Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7): the branch-free
// form the reference's geglu_f32.comp evaluates, gelu(x) = 0.5 x (1 + erf(x / sqrt 2)).
__device__ __forceinline__ float erf_as(float x) {
    const float ax = fabsf(x);
    const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * ax);
    const float p = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t +
                     0.254829592f) * t;
    return copysignf(1.0f - p * __expf(-ax * ax), x);
}
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erf_as(x * 0.70710678118654752f)); }

// ----------------------------------------------------------------- kernel timing
// Eager profiling hook.  While a KernelTimer is installed on the calling thread
// (only inside sdu_profile, never during graph capture), every kernel launch of
// the k_*.hip launchers goes through it with its algorithmic FLOPs and HBM bytes,
// so that each kernel is timed on its own.
struct KernelTimer {
    virtual ~KernelTimer() = default;
    virtual void run(const char* kernel, double flops, double bytes, void (*fn)(const void*),
                     const void* arg) = 0;
};
extern thread_local KernelTimer* g_kernel_timer;

// Start / stop events of the launch the eager profiler is timing (null otherwise).
// Every kernel is launched through SDU_LAUNCH: while these are set it goes through
// hipExtLaunchKernelGGL, whose events record the start and end of that kernel's own
// execution on the stream (no marker packets around it); otherwise it is a plain launch.
extern thread_local hipEvent_t g_launch_ev0, g_launch_ev1;
#define SDU_LAUNCH(kern, grid, block, shm, stream, ...)                                               \
    do {                                                                                              \
        if (::sdu::g_launch_ev0)                                                                     \
            hipExtLaunchKernelGGL(kern, grid, block, shm, stream, ::sdu::g_launch_ev0, ::sdu::g_launch_ev1, 0, \
                                  __VA_ARGS__);                                                       \
        else                                                                                          \
            hipLaunchKernelGGL(kern, grid, block, shm, stream, __VA_ARGS__);                          \
    } while (0)

template <class F>
inline void launch_timed(const char* kernel, double flops, double bytes, const F& f) {
    if (g_kernel_timer)
        g_kernel_timer->run(kernel, flops, bytes, [](const void* p) { (*(const F*)p)(); }, &f);
    else
        f();
}

// ----------------------------------------------------------------- GEMM
// C[M,N] = A[M,K] . W[N,K]^T with a fused epilogue.  A is either a dense
// row-major matrix (optionally split over two sources along K) or the implicit
// im2col of an NHWC image for a 3x3 conv (pad 1, stride 1/2, optional 2x
// nearest upsample of the input), optionally followed along K by up to two dense
// sources (a 1x1 conv over another tensor of the same pixels, summed into the
// same outputs).
enum AMode { A_DENSE = 0, A_CONV3 = 1 };
// Output activation of a GEMM / conv: none, ReLU (the TAESD decoder's convs and block
// fuse) or quick-GELU x * sigmoid(1.702 x) (the CLIP text encoder's fc1).
enum ActFn { ACT_NONE = 0, ACT_RELU = 1, ACT_QUICK_GELU = 2 };
__device__ __forceinline__ float apply_act(int act, float v) {
    if (act == ACT_RELU) return fmaxf(v, 0.f);
    if (act == ACT_QUICK_GELU) return v / (1.0f + __expf(-1.702f * v));
    return v;
}
enum OutMode { OUT_F16 = 0, OUT_F32 = 1, OUT_F32_NCHW = 2 };

struct GemmArgs {
    int M, N, K;
    // A operand
    int amode;
    const f16* A;     // dense: [M, lda]; conv: NHWC input [B, Hin, Win, Cin]
    int lda;
    const f16* A2;    // dense: columns [K1, K) come from A2 [M, lda2]; conv: columns
    int lda2;         //   [K1 = 9 Cin, K2) from A2 and [K2, K) from A3 [M, lda3]
    int K1;           // split point (K when A2 == nullptr)
    const f16* A3;    // conv only (stride 1, no upsample; K1, K2, K multiples of 64)
    int lda3;
    int K2;           // (K when A3 == nullptr)
    int Bn, Hin, Win, Cin, Ho, Wo, stride, upsample;  // conv geometry
    // Sub-pixel form of a 3x3 conv (pad 1) over the 2x nearest upsampling of A
    // (subpix = 1; upsample = 0, stride 1, A the [Bn, Hin, Win, Cin] input, Ho = 2 Hin,
    // Wo = 2 Win, Cin % 64 == 0): output pixel (2y + py, 2x + px) only sees input rows
    // y + py - 1 + {0, 1} and columns x + px - 1 + {0, 1}, so each of the four phases
    // (py, px) is a 2x2 conv of the input with summed taps (fold_subpix_launch): Wt is
    // [4 phases][N][4 taps * Cin], K = 4 Cin, and GEMM row m = phase * (M / 4) + input
    // pixel, stored at its output pixel.  M / 4 must be a multiple of the tile rows
    // (the planner's choice); no residual, fp16 output, no split-K reduce launch.
    int subpix;
    // B operand: W [N, K] row-major
    const f16* Wt;
    // epilogue
    const f16* bias;    // [N] or null
    const float* bias2; // [N] fp32 or null (time projection broadcast)
    const f16* res;     // [M, ldr] residual or null
    int ldr;
    void* C;            // output
    int ldc;            // row stride of C in elements (after GEGLU: N/2 columns)
    int out_mode;
    // when set (the narrow-output conv only): the output pointer is read from this device
    // word at launch time instead of C, so a captured graph can write to a buffer that
    // changes between replays
    void* const* c_ind;
    int hw_out;         // OUT_F32_NCHW: pixels per image
    int geglu;
    int act;            // activation on the final value (after bias, GEGLU, residual): ACT_*
    // split-K (set by gemm_launch).  fixup: each block of a tile stores its fp32
    // partial tile into the tile's slots and the last of them to arrive (per-tile
    // counter) sums the slots and runs the epilogue.  Otherwise the blocks store
    // [splits, M, N] fp32 partials and a reduce kernel runs the epilogue.
    float* partial;     // fixup: [tiles, splits, MT * NT] fp32 (null: no split)
    unsigned* tile_cnt; // fixup: [tiles] arrival counters, zero on entry and left zero
    int fixup;
    int splits;
    int n_major;        // tile order (set by gemm_launch): N-major when W is the larger operand
    int k_per_split;    // multiple of the K tile
    // Optional per-channel statistics of the stored fp16 output, for a GroupNorm that
    // reads it: stats[b][n] += (sum, sum of squares) over the rows m of image
    // b = m / stats_hw.  Must be zero on entry.  fp16 output, no GEGLU, N % 8 == 0,
    // stats_hw >= 64 and gemm_stats_supported(stats_hw).  The planner then splits K
    // only with the in-kernel sum (the reduce launch keeps no statistics).
    double* stats;
    int stats_hw;
    // Optional LayerNorm between two GEMMs.  Producer: row_part[n / 64][m] = (sum, sum of
    // squares) of row m of the stored fp16 output over columns [n, n + 64) (fp32
    // [N / 64][M][2], every entry written; fp16 output, no GEGLU, N % 64 == 0).
    // Consumer (dense A from one source, fp16 output, N % 8 == 0, K % 64 == 0,
    // K <= 1280): ln_part holds those partials of A ([K / 64][M][2]), and the epilogue
    // computes
    //   C[m, n] = rstd_m * (sum_k A[m, k] W[n, k] - mean_m * ln_colsum[n]) + bias...
    // (eps ln_eps), the LayerNorm's affine folded into W and the bias (fold_ln_launch).
    // With either, the planner splits K only with the in-kernel sum.
    float* row_part;
    const float* ln_part;
    const float* ln_colsum;  // [N]: sum_k W[n, k] of the fp16 W
    float ln_eps;
};

// Whether a GEMM can produce output statistics for images of `hw` rows (some tile
// shape keeps each tile within two images).
bool gemm_stats_supported(int hw);

// Picks the tile shape and split-K factor; returns the workspace bytes the launch
// needs (0 if none).  `ws` may be null when the return value is 0.  A split launch
// uses the first gemm_counter_bytes() of the workspace as tile counters: they must
// be zero before the first launch on a workspace and every launch leaves them zero.
size_t gemm_counter_bytes();
size_t gemm_workspace_bytes(const GemmArgs& a);
const char* gemm_kernel_name(const GemmArgs& a);  // tile variant the launch will use
hipError_t gemm_launch(GemmArgs a, float* ws, hipStream_t s);
// Sum a.splits fp32 partials [splits][M][N] at a.partial and run the epilogue.
hipError_t splitk_reduce_launch(const GemmArgs& a, double bytes, hipStream_t s);
// Sub-pixel weights of a 3x3 conv that follows a 2x nearest upsampling (GemmArgs::subpix):
// w3 [Cout][3][3][Cin] -> w4 [4 phases][Cout][2][2][Cin], phase = 2 py + px.  Tap (ty, tx)
// of phase (py, px) is the fp32 sum of the 3x3 taps (ky, kx) with ty = (py + ky + 1) / 2 - py
// and tx = (px + kx + 1) / 2 - px (upsampled row 2y + py - 1 + ky is input row
// y + py - 1 + ty), rounded to fp16 once.
hipError_t fold_subpix_launch(const f16* w3, f16* w4, int Cout, int Cin, hipStream_t s);

// y[n] = act_out( sum_k act_in(x[k]) * W[n,k] + bias[n] ), fp32 in/out, W fp16 [N,K].
// act: 0 none, 1 SiLU.  nvec vectors: x [nvec][K] -> y [nvec][N], up to 4 per launch
// sharing each weight read; every vector's result equals its own nvec = 1 call.
hipError_t gemv_launch(const float* x, const f16* W, const f16* bias, float* y, int N, int K,
                       int act_in, int act_out, hipStream_t s, int nvec = 1);

// ----------------------------------------------------------------- attention
struct AttnArgs {
    const f16* q; const f16* k; const f16* v; f16* o;
    int B, heads, Sq, Sk, d;
    int ldq, ldk, ldv, ldo;
    float scale;
    int causal;  // query i attends keys 0..i only (Sq == Sk; the CLIP text encoder)
    int q_log2;  // q already holds q * scale * log2 e (the projection folded it in)
    // Optional workspace (attention_workspace_bytes; its first gemm_counter_bytes() zero on
    // entry and left zero, as the GEMM's): with it, a shared-tile launch whose blocks would
    // leave a partly filled last round splits the keys in two and merges the halves.
    float* ws;
    int kpart;  // (set by attention_launch)
};
hipError_t attention_launch(const AttnArgs& a, hipStream_t s);
// Workspace bytes attention_launch uses for these arguments when given one (0: none).
size_t attention_workspace_bytes(const AttnArgs& a);

// ----------------------------------------------------------------- norms
// GroupNorm accumulator: fp64 [B][G][2] (sum, sum of squares); must be zero on
// entry (zero_launch).  C = C1 + C2 <= 2560, G <= 32.
size_t groupnorm_acc_bytes(int B, int G);
hipError_t groupnorm_launch(const f16* x, const f16* x2, int C1, int C2, const f16* gamma,
                            const f16* beta, f16* y, int B, int HW, int G, float eps, int silu,
                            double* acc, hipStream_t s);
// GroupNorm apply from per-channel statistics produced by the GEMMs that wrote x and
// x2 (GemmArgs::stats: [B][C1][2] and [B][C2][2] fp64 sums and sums of squares).
hipError_t groupnorm_apply_stats_launch(const f16* x, const f16* x2, int C1, int C2, const double* st1,
                                        const double* st2, const f16* gamma, const f16* beta, f16* y,
                                        int B, int HW, int G, float eps, int silu, hipStream_t s);
// Clear `bytes` (rounded up to 16) with a fill kernel (graph-safe, no memset node).
hipError_t zero_launch(void* p, size_t bytes, hipStream_t s);
hipError_t layernorm_launch(const f16* x, const f16* gamma, const f16* beta, f16* y, int T, int C,
                            float eps, hipStream_t s);

// ----------------------------------------------------------------- elementwise
// NCHW fp32 [Bsrc,C,H,W] -> NHWC fp16 [B,H,W,Cpad]; batch b reads source b % Bsrc,
// channels >= C are zero.  tanh_clamp: each value becomes 3 tanh(x / 3) first (the
// TAESD decoder's input clamp).
hipError_t nchw_to_nhwc_launch(const float* src, f16* dst, int B, int Bsrc, int C, int Cpad, int HW,
                               hipStream_t s, int tanh_clamp = 0);
// The VAE decoder's input stage: NHWC fp16 [B,H,W,8] = post_quant_conv(z * inv_scale)
// (w [4][4], bias [4]) from the NCHW fp32 latent [B,4,H,W]; channels 4..7 zero.
hipError_t vae_stage_launch(const float* z, const f16* w, const f16* bias, f16* y, int B, int HW, float inv_scale,
                            hipStream_t s);
// p[r][j] = fp16(softmax_j(scale * s[r][:])) for an fp32 [rows][n] score matrix.
hipError_t softmax_rows_launch(const float* s, f16* p, int rows, int n, float scale, hipStream_t st);
// The UNet forward's inputs in one launch: latent NCHW fp32 [B,C,H,W] -> NHWC fp16
// [B,H,W,Cpad], context fp32 -> fp16 (nctx values), ntemb time-projection floats copied
// to temb_dst (ntemb 0: none).  The same launch clears zero_bytes (rounded up to 16) at
// the 16-byte aligned zero_dst and, when out_slot is set, stores out_ptr there.
hipError_t stage_in_launch(const float* lat, const float* ctx, const float* temb, f16* lat16, f16* ctx16,
                           float* temb_dst, int B, int C, int Cpad, int HW, int64_t nctx, int ntemb,
                           hipStream_t s, void* zero_dst = nullptr, size_t zero_bytes = 0,
                           void** out_slot = nullptr, void* out_ptr = nullptr);
// Token + position embedding: out[b*S + i][:] = tok[ids[b*S + i]][:] + pos[i][:] (fp16,
// summed in fp32), ids clamped to [0, vocab).  C % 8 == 0.
hipError_t embed_launch(const int32_t* ids, const f16* tok, const f16* pos, f16* out, int B, int S, int C,
                        int vocab, hipStream_t s);
// fp32 -> fp16 copy
hipError_t f32_to_f16_launch(const float* src, f16* dst, int64_t n, hipStream_t s);
hipError_t f16_to_f32_launch(const f16* src, float* dst, int64_t n, hipStream_t s);
hipError_t silu_launch(const f16* x, f16* y, int64_t n, hipStream_t s);
hipError_t add_launch(const f16* a, const f16* b, f16* y, int64_t n, hipStream_t s);
hipError_t add_bias_launch(f16* y, const f16* bias, int64_t n, int C, hipStream_t s);
hipError_t geglu_launch(const f16* g, f16* y, int T, int C2, hipStream_t s);

struct LcmCoeffs {
    float guidance;
    const float* guidance_dev;  // if set, the guidance scale is read from device memory
    double sqrt_alpha, sqrt_beta, c_skip, c_out, sqrt_alpha_prev, sqrt_beta_prev;
    int last;
    int cond_only;  // eps = cond (a step without CFG: eps2 holds only the cond half)
};
// p[0, n) = v (graph-safe fill kernel)
hipError_t fill_f32_launch(float* p, float v, int64_t n, hipStream_t s);
// eps2: [2, n] (cond, uncond) fp32; x: [n] fp32 updated in place; noise [n] or null.
// If unet_in != null, also writes the next UNet input NHWC fp16 [2, HW, Cpad]
// (x duplicated into both CFG slots, C channels of HW pixels).
hipError_t lcm_step_launch(float* x, const float* eps2, const float* noise, int64_t n,
                           LcmCoeffs c, f16* unet_in, int C, int HW, int Cpad, hipStream_t s);

// Seeded fp16 N(mean, std) generator (same specification as the oracle's gen.c).
// Layout descriptors map device index -> canonical (diffusers) index.
enum GenLayout { GL_PLAIN = 0, GL_CONV_OHWI = 1, GL_GEGLU_PERM = 2 };
struct GenDesc {
    uint64_t key;
    int64_t n;         // device elements
    int layout;
    int co, ci, kh, kw, ci_pad;  // GL_CONV_OHWI: canonical [co,ci,kh,kw] -> device [co,kh,kw,ci_pad]
    int half_rows, cols;         // GL_GEGLU_PERM: canonical [2*half_rows, cols]
    double mean, stdv;
    int constant;      // 1: fill `mean` (no randomness)
};
hipError_t gen_launch(f16* dst, const GenDesc& g, hipStream_t s);

// Transformer output fold (init time): wcat [C, 5C] = [Wp.Wf | Wp], bcat [C] = Wp.bf + bp,
// for proj_out (Wp [C, C], bp) after the feed-forward output (Wf [C, 4C], bf).  C % 16 == 0.
hipError_t fold_ffout_launch(const f16* Wp, const f16* bp, const f16* Wf, const f16* bf, f16* wcat, f16* bcat,
                             int C, hipStream_t s);
// LayerNorm affine folded into the Linear that reads it (init time): Wf[n, k] =
// gamma[k] W[n, k] c_n (fp16), bf[n] = c_n (b[n] + sum_k beta[k] W[n, k]) (b may be
// null), sf[n] = sum_k Wf[n, k] (GemmArgs::ln_colsum), with c_n = oscale for the first
// nscale rows (an attention query projection that also applies the softmax's
// scale * log2 e) and 1 for the others.
hipError_t fold_ln_launch(const f16* W, const f16* b, const f16* gamma, const f16* beta, f16* Wf, float* bf,
                          float* sf, int N, int K, hipStream_t s, float oscale = 1.f, int nscale = 0);
// Resnet shortcut fold (init time): wcat [Co, 9 Ci2 + Cs] = [conv2 (OHWI) | shortcut],
// bcat = b2 + bs, for conv2 over Ci2 channels and a 1x1 shortcut over Cs channels.
hipError_t fold_shortcut_launch(const f16* w2, const f16* b2, const f16* ws, const f16* bs, f16* wcat, f16* bcat,
                                int Co, int Ci2, int Cs, hipStream_t s);
// n fp32 N(0,1) values of the same generator (element i from key, no fp16 rounding).
hipError_t gen_normal_f32_launch(float* dst, int64_t n, uint64_t key, hipStream_t s);

// Calibration (k_probe.hip): `blocks` x 8 waves of register-only f16 MFMA, `iters` x 16 per
// wave; clk[0] / clk[1] = shader-clock / 100 MHz real-time ticks of block 0's loop; sink
// >= 512 floats (never written in practice).  A 16-byte streaming copy of `bytes`.
hipError_t mfma_probe_launch(float* sink, long long* clk, int blocks, int iters, hipStream_t s);
hipError_t copy_probe_launch(const void* src, void* dst, size_t bytes, hipStream_t s);

uint64_t fnv1a64(const char* s);
uint64_t splitmix64(uint64_t x);

}  // namespace sdu
