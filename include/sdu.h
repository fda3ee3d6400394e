/*
 * sdu.h -- C ABI of the MI355X (gfx950) SD1.5 UNet engine.
 *
 * Drop-in for the reference's Vulkan engine boundary: the JNI entry points of
 * app/src/main/cpp/vk_engine.cpp (declared in sd/VulkanBench.kt:22-27) and the
 * op-level interface of its `namespace unet` (vk_engine.cpp:487-790), without the
 * JVM.  Plain pointers and sizes only; no C++ or torch types cross this line.
 *
 * Conventions
 *  - Every entry point returns an int status (SDU_OK == 0, negative on error) and
 *    never throws; sdu_last_error() returns the message of the last failure.
 *  - One sdu_ctx owns one HIP stream, the resident fp16 weights and an activation
 *    arena.  A context is not thread-safe: call it from one thread at a time
 *    (the reference runs every call on one GpuThread, GenerateViewModel.kt:31).
 *  - Host-buffer entry points are synchronous.  *_device entry points enqueue on
 *    the context stream and return; sdu_synchronize() waits.
 *  - Host tensors at the UNet boundary are float32 NCHW, as the reference's JNI
 *    byte arrays are (vk_engine.cpp:874-887).  Inside, activations are fp16 NHWC.
 */
#ifndef SDU_H
#define SDU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sdu_ctx sdu_ctx;
typedef struct sdu_tensor sdu_tensor;

enum sdu_status {
    SDU_OK = 0,
    SDU_ERR_DEVICE = -1,     /* device init failed (unetInit's -1, vk_engine.cpp:801) */
    SDU_ERR_NOT_INIT = -2,   /* no context (unetSelfTest's -2, vk_engine.cpp:813)     */
    SDU_ERR_ARG = -3,        /* bad pointer, size or shape                            */
    SDU_ERR_WEIGHT = -4,     /* missing / short weight file or unknown weight name    */
    SDU_ERR_IO = -5,         /* file could not be read                                */
    SDU_ERR_OOM = -6,        /* device allocation failed                              */
    SDU_ERR_HIP = -7         /* a HIP runtime call failed                             */
};

enum sdu_dtype { SDU_F16 = 1, SDU_F32 = 2 };

/* sdu_init flags */
#define SDU_INIT_RANDOM_AFFINE 0x1 /* seeded weights: biases/betas N(0,.02), gammas N(1,.02) */
#define SDU_INIT_NO_WEIGHTS    0x2 /* op-level use only: no UNet weights are created      */

/* ---------------------------------------------------------------- lifecycle */

/* unetInit (vk_engine.cpp:796-808).  weights_dir == NULL: seeded random-init
 * weights (conv/linear fp16(N(0,0.02)), norm gamma 1 / beta 0, biases 0).
 * Otherwise every tensor is read from <dir>/<diffusers key>.bin, raw fp16 LE, the
 * reference's unet_w/ layout (Linear stored [in,out]); a missing or short file is
 * an error (SDU_ERR_WEIGHT), not a silent zero tensor as in vk_engine.cpp:500-505. */
int sdu_init(sdu_ctx** out, const char* weights_dir, uint64_t seed, int flags);
/* unetRelease (vk_engine.cpp:915-926).  NULL is accepted. */
int sdu_release(sdu_ctx* ctx);
const char* sdu_last_error(const sdu_ctx* ctx);
int sdu_synchronize(sdu_ctx* ctx);

/* Replace / read one UNet weight, given in its canonical diffusers layout
 * (conv [Co,Ci,kh,kw], Linear [out,in]) as float32 host data (rounded to fp16).
 * Synchronous; the next forward uses it.  Weights the engine keeps in a derived
 * form (a transformer's feed-forward output folded with its proj_out, its LayerNorm
 * affines folded into the projections that read them, a resnet's conv2 with its 1x1
 * shortcut) are recomputed from their sources by this call. */
int sdu_set_weight(sdu_ctx* ctx, const char* name, const float* data, int64_t numel);
int sdu_get_weight(sdu_ctx* ctx, const char* name, float* out, int64_t numel);
/* Number of UNet parameters (859,520,964 for SD1.5) and of named tensors. */
int sdu_param_count(sdu_ctx* ctx, int64_t* n_params, int64_t* n_tensors);

/* ------------------------------------------------------------ UNet forward */

/* unetForward (vk_engine.cpp:875-887), generalised to explicit shapes.
 * lat [B,4,H,W], temb [320] (sinusoid-projected timestep, shared by the batch as
 * tembp is, vk_engine.cpp:715-717), ctx [B,L,768]  ->  out [B,4,H,W].
 * H, W multiples of 8; 1 <= B <= 64; 1 <= L <= 256. */
int sdu_forward(sdu_ctx* ctx, const float* lat, const float* temb, const float* ctx_emb,
                int B, int H, int W, int L, float* out);

/* unetForward2 (vk_engine.cpp:891-913): one latent shared by the cond and uncond
 * slots (B=2), ctx = [cond; uncond]; out = [cond eps | uncond eps], each [4,H,W]. */
int sdu_forward_cfg(sdu_ctx* ctx, const float* lat, const float* temb, const float* cond,
                    const float* uncond, int H, int W, int L, float* out);

/* Full LCM + batch-CFG denoise (VulkanUnetPipeline.kt:63-97 with
 * LcmScheduler.kt:56-82) on the device: lat [4,H,W] -> out [4,H,W].
 * noise [steps-1,4,H,W] is the injected per-step noise (the reference draws it
 * from its RNG at :87).  guidance is the CFG scale (u + s (c - u)). */
int sdu_denoise_lcm(sdu_ctx* ctx, const float* lat, const float* cond, const float* uncond,
                    int H, int W, int L, int steps, float guidance, const float* noise,
                    float* out);

/* timeProj (VulkanUnetPipeline.kt:36-46): the 320-d timestep embedding the forward
 * takes as temb, out = [cos(t f_i) (160) | sin(t f_i) (160)], f_i = exp(-ln(1e4) i/160),
 * evaluated in float64 and rounded to float32.  0 <= t <= 100000; needs no context. */
int sdu_time_proj(int t, float* out);

/* Device-resident variants for throughput runs: every pointer is device memory
 * (same layouts and dtypes as above).  Enqueued on the context stream; the first
 * call for a shape records a HIP graph, later calls replay it. */
int sdu_forward_device(sdu_ctx* ctx, const float* d_lat, const float* d_temb,
                       const float* d_ctx, int B, int H, int W, int L, float* d_out);
int sdu_denoise_lcm_device(sdu_ctx* ctx, const float* d_lat, const float* d_cond,
                           const float* d_uncond, int H, int W, int L, int steps,
                           float guidance, const float* d_noise, float* d_out);

/* Device LCM denoise with the generation options of TpuUnetPipeline.kt:82-112
 * (replaces its host loop over tpuForward / LcmScheduler.step):
 *  - cfg_steps in [0, steps]: steps 0 .. cfg_steps-1 run the batch-CFG forward (B=2,
 *    eps = u + guidance (c - u)); the later steps run one B=1 forward on cond and use
 *    its eps directly (:94-99).  guidance <= 1 disables CFG on every step (:97).
 *    cfg_steps = steps is sdu_denoise_lcm_device.
 *  - d_noise: [steps-1,4,H,W] fp32 device noise, or NULL to draw it on the device:
 *    element i = float(sqrt(-2 ln u1) cos(2 pi u2)) of the seeded generator with
 *    key = fnv1a64("lcm.noise") ^ splitmix64(noise_seed) (:100 draws it from its own
 *    RNG; the stream differs, the distribution is the same).
 * Each (H, W, L, steps, CFG pattern) records its own HIP graph, where the CFG pattern
 * is the number of batch-CFG steps (0 when guidance <= 1); the guidance value is read
 * by the graph from device memory written before each replay, so any number of
 * guidance values share one graph.  A non-finite guidance is SDU_ERR_ARG.  A context
 * keeps at most 16 planned shapes (forward and denoise) and evicts the least recently
 * used one to plan another. */
int sdu_denoise_lcm_ex(sdu_ctx* ctx, const float* d_lat, const float* d_cond,
                       const float* d_uncond, int H, int W, int L, int steps, float guidance,
                       int cfg_steps, const float* d_noise, uint64_t noise_seed, float* d_out);

/* Latent decoder: replaces vaeDecode (VulkanUnetPipeline.kt:55-61), the LiteRT export of
 * diffusers AutoencoderTiny("madebyollin/taesd").decode (tools/export_taesd.py:52-54, contract
 * at :2).  sdu_taesd_init creates the decoder's weights: from weights_dir (one raw fp16 file
 * per diffusers key, decoder.layers.<i>..., as the UNet's weight directory) or, when
 * weights_dir is NULL, seeded (conv weights N(0, 0.04); biases 0, or N(0, .02) with
 * SDU_INIT_RANDOM_AFFINE).  Decode: fp32 latent [B,4,H,W] -> fp32 image [B,3,8H,8W] in
 * about [-1, 1] (B 1..16, H and W 8..128), one captured graph per shape. */
int sdu_taesd_init(sdu_ctx* ctx, const char* weights_dir, uint64_t seed, int flags);
int sdu_taesd_decode(sdu_ctx* ctx, const float* lat, int B, int H, int W, float* img);
int sdu_taesd_decode_device(sdu_ctx* ctx, const float* d_lat, int B, int H, int W, float* d_img);

/* Full VAE decoder: replaces vaeDecode with gpu_vae.tflite (VulkanUnetPipeline.kt:55-61;
 * contract GpuMonoPipeline.kt:26, latents [1,4,64,64] -> image [1,3,512,512] in [-1, 1]), the
 * LiteRT export of the SD1.5 AutoencoderKL decoder applied as vae.decode(z / 0.18215)
 * (tools/export_taesd.py:53).  sdu_vae_init creates the decoder's weights: from weights_dir
 * (one raw fp16 file per diffusers key, post_quant_conv.* and decoder.*, Linear [in, out])
 * or, when weights_dir is NULL, seeded (conv weights N(0, 0.02), the attention's Linear
 * weights N(0, 0.1); norms gamma 1 / beta 0 and biases 0, or the affine mode).  Decode: fp32
 * UNet latent [B,4,H,W] -> fp32 image [B,3,8H,8W] (B 1..4, H and W >= 8, H * W <= 96 * 96),
 * one captured graph per shape. */
int sdu_vae_init(sdu_ctx* ctx, const char* weights_dir, uint64_t seed, int flags);
int sdu_vae_decode(sdu_ctx* ctx, const float* lat, int B, int H, int W, float* img);
int sdu_vae_decode_device(sdu_ctx* ctx, const float* d_lat, int B, int H, int W, float* d_img);

/* Text encoder: replaces clipContext (VulkanUnetPipeline.kt:48-53), the LiteRT export of SD1.5's
 * CLIP text encoder (CLIPTextModel): int32 token ids [B,77] -> fp32 last hidden state
 * [B,77,768], the UNet's context (B 1..64).  Weights from weights_dir (text_model.* keys,
 * Linear [in, out]) or seeded (Linear and embeddings N(0, 0.02); LayerNorm gamma 1, beta 0,
 * biases 0, or the affine mode). */
int sdu_clip_init(sdu_ctx* ctx, const char* weights_dir, uint64_t seed, int flags);
int sdu_clip_encode(sdu_ctx* ctx, const int32_t* ids, int B, float* out);
int sdu_clip_encode_device(sdu_ctx* ctx, const int32_t* d_ids, int B, float* d_out);

/* End-to-end image: VulkanUnetPipeline.generate (VulkanUnetPipeline.kt:63-97).  CLIP of the
 * prompt and empty-prompt ids in one batch, an initial latent N(0, 1) drawn on the device from
 * `seed`, the LCM denoise of sdu_denoise_lcm_ex (steps, guidance, cfg_steps, noise from
 * `seed`), then the full VAE decoder (sdu_vae_init) when it was initialised, else the TAESD
 * decoder.  image: fp32 [3, 8H, 8W] in about [-1, 1] (toBitmap, :99-109, maps (x + 1) *
 * 127.5).  Needs sdu_clip_init and sdu_vae_init or sdu_taesd_init. */
int sdu_generate(sdu_ctx* ctx, const int32_t* cond_ids, const int32_t* uncond_ids, int H, int W,
                 int steps, float guidance, int cfg_steps, uint64_t seed, float* image);

/* unetSelfTest (vk_engine.cpp:811-851): reads fixture_dir/IN_lat.bin (fp16 [4,64,64]),
 * IN_ctx.bin (fp16 [77,768]), IN_temb_proj.bin (fp16 [320]) and OUT_y.bin (fp16),
 * runs B=1 and B=2 (same input in both slots) and returns the largest
 * relErr_L1 = sum|ref-got| / sum|ref| over the three outputs; negative on error. */
double sdu_selftest(sdu_ctx* ctx, const char* fixture_dir);

/* The legs of unetSelfTest (vk_engine.cpp:811-851) one by one:
 *  - relerr_b1: the B=1 forward vs OUT_y (:818-821);
 *  - relerr_b2[2]: both images of the B=2 run with the input in both slots (:823-839);
 *  - ctx_sens: when fixture_dir holds IN_cond.bin, IN_unc.bin (fp16 [77,768]) and
 *    IN_temb999.bin (fp16 [320]), the mean |eps_cond - eps_unc| of two B=1 forwards of
 *    IN_lat under those contexts (:840-849; the reference logs it next to its PyTorch
 *    value), else -1. */
typedef struct sdu_selftest_report {
    double relerr_b1;
    double relerr_b2[2];
    double ctx_sens;
} sdu_selftest_report;
int sdu_selftest_ex(sdu_ctx* ctx, const char* fixture_dir, sdu_selftest_report* out);

/* unetProfile (vk_engine.cpp:854-872): one eager forward in which every kernel
 * launch is timed on its own: it carries a start and a stop HIP event that record the
 * kernel's own execution on the context stream (hipExtLaunchKernelGGL), and runs once.
 * Entries are accumulated per op category (e.g. "conv3x3") and per kernel ("k:" +
 * kernel name, e.g. "k:gemm_kernel<128,128,2,2,64,2>"); total_ms sums the categories. */
/* The GPU's practical ceilings, measured like the reference's micro-benchmarks
 * (VulkanBench.kt:10-19, benchMatmul / benchSilu ...) time single shaders: dense f16 MFMA
 * from registers on every CU (TFLOP/s, and the shader clock during that load), and a
 * 16-byte streaming device copy of copy_mib MiB (read + write GB/s).  Allocates and frees
 * 2 x copy_mib MiB; takes about 0.1 s. */
typedef struct sdu_calibration {
    double mfma_tflops;
    double mfma_clock_ghz;
    double copy_gbs;
} sdu_calibration;
int sdu_calibrate(sdu_ctx* ctx, int copy_mib, sdu_calibration* out);

typedef struct sdu_prof_entry {
    char name[48];
    int calls;
    double ms;      /* summed kernel time */
    double flops;   /* algorithmic FLOPs over those calls */
    double bytes;   /* algorithmic HBM bytes over those calls */
} sdu_prof_entry;
int sdu_profile(sdu_ctx* ctx, int B, int H, int W, int L, sdu_prof_entry* out,
                int max_entries, int* n_entries, double* total_ms);
/* Kernel timing of op-level calls, the counterpart of the reference's per-shader
 * micro-benchmarks (VulkanBench.kt:66-126 over vk_engine.cpp:226-420, :1017-1218, which
 * time one shader at fixed shapes).  enable = 1 opens a window: every kernel that the
 * op-level entry points (sdu_matmul, sdu_conv2d, sdu_conv2d_groupnorm, sdu_groupnorm,
 * sdu_groupnorm_noalloc, sdu_layernorm, sdu_attention(_ex), sdu_geglu, sdu_silu, sdu_add,
 * sdu_add_bias, sdu_lcm_step) launch from then on carries its own start / stop events, as
 * in sdu_profile.  enable = 0 closes the window: synchronises the stream and returns the
 * entries accumulated per op ("matmul", ...) and per kernel ("k:" + kernel name), with
 * total_ms summing the ops.  UNet / TAESD / CLIP calls made meanwhile are not timed.
 * Closing a window that was not opened is SDU_ERR_ARG. */
int sdu_profile_ops(sdu_ctx* ctx, int enable, sdu_prof_entry* out, int max_entries, int* n_entries,
                    double* total_ms);

/* ------------------------------------------------------------- tensors */

int sdu_tensor_alloc(sdu_ctx* ctx, int dtype, int ndim, const int64_t* shape, sdu_tensor** out);
int sdu_tensor_free(sdu_ctx* ctx, sdu_tensor* t);
int sdu_tensor_upload(sdu_ctx* ctx, sdu_tensor* t, const void* host, size_t bytes);
int sdu_tensor_download(sdu_ctx* ctx, const sdu_tensor* t, void* host, size_t bytes);
void* sdu_tensor_device_ptr(const sdu_tensor* t);
size_t sdu_tensor_bytes(const sdu_tensor* t);

/* ---------------------------------------------------------------- ops
 * The reference's `namespace unet` ops (vk_engine.cpp:547-613) with explicit
 * batch and shapes instead of the global gB.  fp16 tensors unless stated,
 * activations NHWC ([B, H*W, C] row-major = tokens x channels). */

/* groupnorm / groupnorm_silu (vk_engine.cpp:548-549): per-image statistics over
 * `groups` channel groups.  x2 (may be NULL) is a second source concatenated
 * along channels (C = C1 + C2) -- the up-path skip concat (vk_engine.cpp:678-688)
 * without materialising it.  gamma/beta fp16 [C]. */
int sdu_groupnorm(sdu_ctx* ctx, const sdu_tensor* x, const sdu_tensor* x2, const sdu_tensor* gamma,
                  const sdu_tensor* beta, sdu_tensor* y, int B, int HW, int C1, int C2,
                  int groups, float eps, int silu);

/* sdu_groupnorm without any device allocation.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments and results as
 * sdu_groupnorm, but the statistics accumulators live in a fixed 32 KiB device array of
 * the library (B <= 64 images x groups <= 32; larger is SDU_ERR_ARG) instead of the
 * context's allocated workspace, and the call makes no hipMalloc / hipFree.  Every call
 * on one device shares that array (cleared by a fill kernel at the start of each call):
 * calls that overlap on one device, from several streams or contexts, race. */
int sdu_groupnorm_noalloc(sdu_ctx* ctx, const sdu_tensor* x, const sdu_tensor* x2,
                          const sdu_tensor* gamma, const sdu_tensor* beta, sdu_tensor* y, int B,
                          int HW, int C1, int C2, int groups, float eps, int silu);

/* LN (vk_engine.cpp:652): y[t,:] = LN(x[t,:]) over C. */
int sdu_layernorm(sdu_ctx* ctx, const sdu_tensor* x, const sdu_tensor* gamma, const sdu_tensor* beta,
                  sdu_tensor* y, int T, int C, float eps);

/* Epilogue flags for sdu_matmul / sdu_conv2d */
#define SDU_EPI_GEGLU   0x1 /* w rows interleaved per 32 (a,b); y[:, N/2] = a * gelu_erf(b)   */
#define SDU_EPI_OUT_F32 0x2 /* y is float32                                                    */
#define SDU_EPI_RELU    0x4 /* y = max(y, 0) after bias and residual (TAESD decoder convs)     */
#define SDU_EPI_QUICK_GELU 0x8 /* y = y * sigmoid(1.702 y) after bias (CLIP text encoder fc1)   */

/* matmul (vk_engine.cpp:612-613) with fused epilogue:
 * y[M,N] = a[M,K] . w[N,K]^T (+ bias[N]) (+ residual[M,N]).
 * a2 (may be NULL) supplies columns [K1, K) of a (a = [a | a2], K1 = K - K2):
 * the 1x1 shortcut over a concatenated input.  y must not overlap a, a2, w or bias;
 * residual may be y itself (an in-place add) but must not otherwise overlap it
 * (SDU_ERR_ARG). */
int sdu_matmul(sdu_ctx* ctx, const sdu_tensor* a, const sdu_tensor* a2, const sdu_tensor* w,
               const sdu_tensor* bias, const sdu_tensor* residual, sdu_tensor* y,
               int M, int N, int K, int K2, int flags);

/* conv (vk_engine.cpp:578-608) as implicit GEMM: x NHWC [B,H,W,Ci], w [Co,k,k,Ci]
 * (k = 1 or 3, pad k/2), stride 1 or 2, optional nearest-2x upsample of the input
 * (upsample(), vk_engine.cpp:693-697).  y NHWC [B,Ho,Wo,Co] (+bias[Co])
 * (+ temb[Co] float32 broadcast, the resnet's time projection, :630)
 * (+ residual NHWC [B,Ho,Wo,Co]).  y must not overlap x, w, bias or temb; residual
 * may be y itself but must not otherwise overlap it (SDU_ERR_ARG). */
int sdu_conv2d(sdu_ctx* ctx, const sdu_tensor* x, const sdu_tensor* w, const sdu_tensor* bias,
               const sdu_tensor* temb, const sdu_tensor* residual, sdu_tensor* y, int B, int H,
               int W, int Ci, int Co, int ksize, int stride, int upsample, int flags);

/* A 3x3 conv (stride 1, no upsample; as sdu_conv2d with ksize 3) followed by the
 * groupnorm / groupnorm_silu of its output (vk_engine.cpp:626-631, the resnet's conv1 ->
 * norm2 step), in the engine's fused form: the conv's epilogue adds the per-channel sums
 * and sums of squares of its stored fp16 output (fp32 per tile, fp64 across tiles) and the
 * GroupNorm forms each group's mean and variance from them.  No separate counterpart in
 * the reference's op list: it exposes the path the UNet takes for its 64x64-level
 * GroupNorms to op-level callers and tests.  y NHWC [B,H,W,Co] (the conv output) and
 * gn_y NHWC [B,H,W,Co] (its GroupNorm); gamma/beta fp16 [Co]; H*W = 64 or >= 128 (a
 * 128-row output tile spans at most two images), Co % 8 == 0, groups <= 32 and
 * Co % groups == 0; other shapes are SDU_ERR_ARG.  y follows sdu_conv2d's overlap
 * rules and must not overlap gamma or beta either; gn_y may be y itself or any input of
 * the conv, but not gamma, beta or a shifted view of y (SDU_ERR_ARG). */
int sdu_conv2d_groupnorm(sdu_ctx* ctx, const sdu_tensor* x, const sdu_tensor* w, const sdu_tensor* bias,
                         const sdu_tensor* temb, const sdu_tensor* residual, sdu_tensor* y,
                         const sdu_tensor* gamma, const sdu_tensor* beta, sdu_tensor* gn_y, int B, int H,
                         int W, int Ci, int Co, int groups, float eps, int silu);

/* ATTN / ATTN_BIG (vk_engine.cpp:655, :663): per image b and head h,
 * o = softmax(q k^T * scale) v.  q rows b*Sq+i, k/v rows b*Sk+j, head h at column
 * h*d; ldq/ldk/ldv/ldo are row strides in elements.  d in {8,...,160}, d % 8 == 0. */
int sdu_attention(sdu_ctx* ctx, const sdu_tensor* q, const sdu_tensor* k, const sdu_tensor* v,
                  sdu_tensor* o, int B, int heads, int Sq, int Sk, int d, int ldq, int ldk,
                  int ldv, int ldo, float scale);
/* sdu_attention with flags: SDU_ATTN_CAUSAL masks key j > query i (Sq == Sk), the causal
 * self-attention of the CLIP text encoder behind VulkanUnetPipeline.kt:48-53.
 * SDU_ATTN_Q_LOG2 (no counterpart in the reference): q already holds q * scale * log2(e),
 * as the UNet's query projections write it (the softmax factor folded into their
 * weights), so o = softmax_2(q k^T) v; scale must still be > 0 and is otherwise unused.
 * Heads whose size is not a multiple of 16 then carry the softmax's running reference in
 * a spare MFMA dimension (one floating-point operation less per score). */
#define SDU_ATTN_CAUSAL 0x1
#define SDU_ATTN_Q_LOG2 0x2
int sdu_attention_ex(sdu_ctx* ctx, const sdu_tensor* q, const sdu_tensor* k, const sdu_tensor* v,
                     sdu_tensor* o, int B, int heads, int Sq, int Sk, int d, int ldq, int ldk,
                     int ldv, int ldo, float scale, int flags);

/* GEGLU (geglu_f32.comp): y[t,c] = g[t,c] * gelu_erf(g[t,C2+c]). */
int sdu_geglu(sdu_ctx* ctx, const sdu_tensor* g, sdu_tensor* y, int T, int C2);
/* SILU (silu_f32.comp), ADD (add_f32.comp) and AB/AB2 (addbias_f32.comp,
 * addbias2_f32.comp; y[i] += b[i % C]) on n elements. */
int sdu_silu(sdu_ctx* ctx, const sdu_tensor* x, sdu_tensor* y, int64_t n);
int sdu_add(sdu_ctx* ctx, const sdu_tensor* a, const sdu_tensor* b, sdu_tensor* y, int64_t n);
int sdu_add_bias(sdu_ctx* ctx, sdu_tensor* y, const sdu_tensor* bias, int64_t n, int C);

/* LcmScheduler.step (LcmScheduler.kt:56-82) fused with the CFG combine
 * (VulkanUnetPipeline.kt:86).  float32 tensors: x [n] (updated in place),
 * eps2 [2, n] (cond then uncond), noise [n] (NULL on the last step).
 * The coefficients come from the schedule of `steps` steps at step `idx`. */
int sdu_lcm_step(sdu_ctx* ctx, sdu_tensor* x, const sdu_tensor* eps2, const sdu_tensor* noise,
                 int64_t n, int steps, int idx, float guidance);

#ifdef __cplusplus
}
#endif
#endif /* SDU_H */
