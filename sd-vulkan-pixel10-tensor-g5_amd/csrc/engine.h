// Host-side engine state shared by runtime.cpp, unet.cpp and capi.cpp.
#pragma once

#include "sdu_internal.h"
#include "../../include/sdu.h"

#include <map>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

namespace sdu {

enum WKind { WK_CONV = 0, WK_LINEAR = 1, WK_NORM_W = 2, WK_NORM_B = 3, WK_BIAS = 4, WK_EMBED = 5 };

// One named UNet parameter.  `dev` points into the weight pool; the device layout
// is described by (layout, ci_pad): conv weights are [Co, kh, kw, Ci_pad] (the
// K dimension of the implicit GEMM is tap-major, channel-minor), Linear weights
// [out, in], the GEGLU projection row-interleaved per 32 (a, b).
struct WeightRec {
    std::string name;
    std::vector<int64_t> shape;  // canonical (diffusers) shape
    int kind = 0;
    int layout = GL_PLAIN;
    int ci_pad = 0;
    f16* dev = nullptr;
    int64_t dev_n = 0;
    int64_t numel() const {
        int64_t n = 1;
        for (auto s : shape) n *= s;
        return n;
    }
};

// Bump arena with stack marks.  In sizing mode it hands out no memory and only
// records the high-water mark.
struct Arena {
    char* base = nullptr;
    size_t cap = 0, top = 0, high = 0;
    bool sizing = false;
    void* alloc(size_t bytes) {
        size_t off = (top + 255) & ~(size_t)255;
        top = off + ((bytes + 255) & ~(size_t)255);
        if (top > high) high = top;
        if (sizing) return nullptr;
        return base + off;
    }
    size_t mark() const { return top; }
    void release(size_t m) { top = m; }
};

// Shapes of one UNet instance: per-resnet / per-transformer channel counts and
// offsets into the fused time-projection and cross-K/V weight blocks.
struct ResDesc {
    std::string pf;
    int cin, cout, cin1;  // cin1: channels from the first source (concat split)
    int tproj_off;
    // cin != cout: conv2 and the 1x1 shortcut folded into one GEMM (fold_weights)
    f16* w2sc = nullptr;  // [cout, 9 cout + cin] = [conv2 | shortcut]
    f16* b2sc = nullptr;  // [cout] = b2 + bs
};
// Attention heads of every SD1.5 transformer (head size C / 8), and the factor
// scale * log2 e = log2 e / sqrt(C / 8) that the query projections fold in.
static const int kUnetHeads = 8;
inline float attn_qscale(int C) { return 1.4426950408889634f / sqrtf((float)(C / kUnetHeads)); }

// A 3x3 conv after a 2x nearest upsampling, with its sub-pixel weights (GemmArgs::subpix;
// fold_weights): [4 phases][C][2][2][C]
struct UpDesc {
    std::string pf;  // the conv's prefix
    int c;
    f16* w4 = nullptr;
};

struct XfDesc {
    std::string pf;
    int c;
    int kv_off;  // column offset of this block's K in the fused cross K/V output
    // feed-forward output and proj_out folded into one GEMM over [g | t] (fold_weights)
    f16* w_out = nullptr;  // [C, 5C] = [Wp.Wf | Wp]
    f16* b_out = nullptr;  // [C] = Wp.bf + bp
    // LayerNorms norm1 / norm2 / norm3 folded into the GEMMs that read them (the QKV
    // projection, the cross-attention query, the GEGLU projection): fp16 W' = W.diag(gamma),
    // fp32 bias' = b + W.beta and column sums of W' (GemmArgs::ln_colsum).  The query rows
    // of w_qkv and all of w_q2 also carry the softmax factor attn_qscale(C): the attention
    // reads Q in log2 units (AttnArgs::q_log2).
    f16* w_qkv = nullptr;  // [3C, C]
    f16* w_q2 = nullptr;   // [C, C]
    f16* w_ff = nullptr;   // [8C, C]
    float *b_qkv = nullptr, *s_qkv = nullptr, *b_q2 = nullptr, *s_q2 = nullptr, *b_ff = nullptr, *s_ff = nullptr;
};

struct ProfAcc {
    int calls = 0;
    double ms = 0, flops = 0, bytes = 0;
};

struct FwdState;  // per-shape graph state (unet.cpp)
struct AuxState;  // per-shape graph state of an auxiliary network (taesd.cpp, clip.cpp)

// The weights and planned graphs of an auxiliary network: the TAESD latent decoder or
// the CLIP text encoder.  Its own fp16 pool, in the device layouts its kernels read,
// registered and loaded like the UNet's (same seeded generator, same weight-file format).
struct AuxNet {
    int kind = 0;  // AUX_TAESD | AUX_CLIP | AUX_VAE
    f16* pool = nullptr;
    size_t pool_bytes = 0;
    std::vector<WeightRec> weights;
    std::unordered_map<std::string, int> widx;
    std::vector<char> contig;  // placed right after the previous tensor (fused q/k/v blocks)
    std::vector<AuxState*> states;  // owned, LRU-capped
    uint64_t use_clock = 0;
    // TAESD: conv_out with the output affine y = 2 x - 1 folded in (2 W fp16, 2 b - 1 fp32)
    f16* w_out2 = nullptr;
    float* b_out2 = nullptr;
    // VAE: [conv2 | shortcut] weights and biases of the two width-changing resnets, and the
    // attention's fp32 to_out bias with to_v's folded in
    f16* w2sc[2] = {nullptr, nullptr};
    f16* b2sc[2] = {nullptr, nullptr};
    float* b_attn_out = nullptr;
    // VAE / TAESD: sub-pixel weights of the convs after each 2x upsampling (GemmArgs::subpix)
    f16* w4[3] = {nullptr, nullptr, nullptr};
    int add(const std::string& name, std::vector<int64_t> shape, int kind, int layout = GL_PLAIN, int ci_pad = 0,
            bool follows = false);
    const WeightRec* w(const std::string& name) const {
        auto it = widx.find(name);
        return it == widx.end() ? nullptr : &weights[it->second];
    }
    f16* wd(const std::string& name) const {
        const WeightRec* r = w(name);
        return r ? r->dev : nullptr;
    }
};
enum AuxKind { AUX_TAESD = 1, AUX_CLIP = 2, AUX_VAE = 3 };

struct Ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    uint64_t seed = 0;
    int flags = 0;

    // weights
    f16* wpool = nullptr;
    size_t wpool_bytes = 0, wpool_top = 0;
    std::vector<WeightRec> weights;
    std::unordered_map<std::string, int> widx;
    // fused blocks
    f16* w_tproj = nullptr;   // [sum Cout, 1280]
    f16* b_tproj = nullptr;   // [sum Cout]
    int tproj_total = 0;
    f16* w_kv = nullptr;      // [sum 2C, 768]
    int kv_total = 0;
    std::vector<ResDesc> resnets;
    std::vector<XfDesc> xfs;
    std::vector<UpDesc> ups;
    std::map<std::string, int> res_by_pf, xf_by_pf;

    // op-level tensors and per-shape forward state
    std::vector<FwdState*> fwd;  // owned; freed by free_fwd_states (LRU-capped)
    uint64_t use_clock = 0;
    float* op_ws = nullptr;     // scratch for op-level calls
    size_t op_ws_bytes = 0;

    // auxiliary networks (created on demand by sdu_taesd_init / sdu_clip_init)
    AuxNet* taesd = nullptr;
    AuxNet* clip = nullptr;
    AuxNet* vae = nullptr;

    // profiling
    bool profiling = false;
    std::map<std::string, ProfAcc> prof;

    const WeightRec* w(const std::string& name) const {
        auto it = widx.find(name);
        return it == widx.end() ? nullptr : &weights[it->second];
    }
    f16* wd(const std::string& name) const {
        const WeightRec* r = w(name);
        return r ? r->dev : nullptr;
    }
};

struct sdu_tensor_impl {
    void* ptr = nullptr;
    size_t bytes = 0;
    int dtype = SDU_F16;
    std::vector<int64_t> shape;
};

// runtime.cpp
int build_inventory(Ctx& c);                       // fills weights / descs and allocates the pool
int init_weights_seeded(Ctx& c);
int init_weights_dir(Ctx& c, const std::string& dir);
int set_weight_canonical(Ctx& c, const WeightRec& r, const float* data);
// Recompute the folded weights (transformer output, resnet conv2 + shortcut) from
// the loaded ones (all blocks, or the one whose prefix `name` starts with); synchronous.
int fold_weights(Ctx& c, const std::string& name = std::string());
int get_weight_canonical(Ctx& c, const WeightRec& r, float* out);
// One tensor: seeded values (conv / linear / embedding N(0, wstd); norms and biases per the
// init mode), or read from <dir>/<name>.bin (raw fp16, Linear stored [in, out]).
int gen_weight(Ctx& c, const WeightRec& r, uint64_t seed, bool affine, double wstd);
int load_weight_file(Ctx& c, const WeightRec& r, const std::string& dir);
// Allocate an auxiliary network's pool for its registered tensors and place them.
int aux_alloc(Ctx& c, AuxNet& n, size_t extra_bytes);
void aux_free(AuxNet* n);
int ensure_op_ws(Ctx& c, size_t bytes);
int set_err(Ctx* c, int code, const std::string& msg);

// taesd.cpp: latent [B, 4, H, W] fp32 -> image [B, 3, 8H, 8W] fp32 in about [-1, 1]
int taesd_create(Ctx& c, const char* weights_dir, uint64_t seed, int flags);
int taesd_decode_device(Ctx& c, const float* d_lat, int B, int H, int W, float* d_img);
// vae.cpp: UNet latent [B, 4, H, W] fp32 -> image [B, 3, 8H, 8W] fp32 in about [-1, 1]
int vae_create(Ctx& c, const char* weights_dir, uint64_t seed, int flags);
int vae_decode_device(Ctx& c, const float* d_lat, int B, int H, int W, float* d_img);
// clip.cpp: token ids [B, 77] -> last hidden state [B, 77, 768] fp32
int clip_create(Ctx& c, const char* weights_dir, uint64_t seed, int flags);
int clip_encode_device(Ctx& c, const int32_t* d_ids, int B, float* d_out);

// unet.cpp
int unet_forward_host(Ctx& c, const float* lat, const float* temb, const float* ctx, int B, int H,
                      int W, int L, float* out);
int unet_forward_device(Ctx& c, const float* d_lat, const float* d_temb, const float* d_ctx, int B,
                        int H, int W, int L, float* d_out);
int unet_denoise_device(Ctx& c, const float* d_lat, const float* d_cond, const float* d_uncond,
                        int H, int W, int L, int steps, float guidance, int cfg_steps,
                        const float* d_noise, uint64_t noise_seed, float* d_out);
int unet_profile(Ctx& c, int B, int H, int W, int L);
// timeProj (VulkanUnetPipeline.kt:36-46): out[320] = [cos(t f_i) | sin(t f_i)]
void time_proj_host(int t, float* out);
void free_fwd_states(Ctx& c);

}  // namespace sdu

struct sdu_ctx {
    sdu::Ctx c;
    // op-level kernel timing (sdu_profile_ops): an EventTimer of graph.h while enabled
    void* op_timer = nullptr;
};
struct sdu_tensor {
    sdu::sdu_tensor_impl t;
};
