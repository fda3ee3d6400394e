// SD1.5 VAE decoder on the HIP kernels: UNet latent [B, 4, H, W] -> image [B, 3, 8H, 8W].
//
// Replaces the reference's LiteRT full VAE (gpu_vae.tflite, VulkanUnetPipeline.kt:55-61,
// contract GpuMonoPipeline.kt:26: latents [1,4,64,64] -> image [1,3,512,512] in [-1, 1];
// the reference's own full-VAE call is vae.decode(z / scaling_factor),
// tools/export_taesd.py:53).  The network is diffusers' AutoencoderKL decoder with the
// SD1.5 configuration (block_out_channels 128, 256, 512, 512; 32 groups, eps 1e-6):
//   post_quant_conv(z / 0.18215) -> conv_in 4->512 -> mid (resnet, attention, resnet)
//   -> 4 up blocks of 3 resnets (512, 512, 256, 128 channels), the first three followed
//      by nearest 2x upsampling and a 3x3 conv -> GroupNorm + SiLU -> conv_out 128->3
// Every conv is the implicit-GEMM conv with its bias and residual in the epilogue (the
// resnets' 1x1 shortcuts as extra K columns of conv2, the upsampling in the next conv's
// index math), GroupNorm statistics come from the producing conv's epilogue above 32x32
// pixels, and the mid block's single-head attention (d = 512, beyond the fused attention
// kernel's head sizes) runs as GEMMs: S = Q K^T in fp32, a row softmax, O = P V, then
// to_out with the residual.  The latent scaling and post_quant_conv form the input
// stage; conv_out writes fp32 NCHW directly.
#include "graph.h"

#include <cmath>
#include <cstring>
#include <vector>

namespace sdu {

static const int kCh[4] = {128, 256, 512, 512};  // block_out_channels
static const int kTop = 512;
static const float kEpsVae = 1e-6f, kScaling = 0.18215f;
// seeded random init, as the oracle's vae_ref: conv weights N(0, 0.02), the attention's
// Linear weights N(0, 0.1)
static const double kConvStd = 0.02, kLinStd = 0.1;
static const int kMaxHW = 96 * 96;  // the attention's fp32 score matrix is HW^2 per image

struct UpStage {
    int cin, cout;
    bool up;
};
static std::vector<UpStage> up_plan() {
    std::vector<UpStage> v;
    int prev = kCh[3];
    for (int i = 0; i < 4; ++i) {
        const int c = kCh[3 - i];
        v.push_back({prev, c, i < 3});
        prev = c;
    }
    return v;
}

static std::string resnet_pf(int blk, int j) {
    return blk < 0 ? "decoder.mid_block.resnets." + std::to_string(j)
                   : "decoder.up_blocks." + std::to_string(blk) + ".resnets." + std::to_string(j);
}
static const char* kAttn = "decoder.mid_block.attentions.0";

static void add_conv3(AuxNet& n, const std::string& pf, int cin, int cout, int ci_pad = 0) {
    n.add(pf + ".weight", {cout, cin, 3, 3}, WK_CONV, GL_CONV_OHWI, ci_pad ? ci_pad : cin);
    n.add(pf + ".bias", {cout}, WK_BIAS);
}
static void add_norm(AuxNet& n, const std::string& pf, int c) {
    n.add(pf + ".weight", {c}, WK_NORM_W);
    n.add(pf + ".bias", {c}, WK_NORM_B);
}
static void add_resnet(AuxNet& n, const std::string& pf, int cin, int cout) {
    add_norm(n, pf + ".norm1", cin);
    add_conv3(n, pf + ".conv1", cin, cout);
    add_norm(n, pf + ".norm2", cout);
    add_conv3(n, pf + ".conv2", cout, cout);
    if (cin != cout) {
        n.add(pf + ".conv_shortcut.weight", {cout, cin, 1, 1}, WK_CONV);
        n.add(pf + ".conv_shortcut.bias", {cout}, WK_BIAS);
    }
}

static void vae_register(AuxNet& n) {
    n.add("post_quant_conv.weight", {4, 4, 1, 1}, WK_CONV);
    n.add("post_quant_conv.bias", {4}, WK_BIAS);
    add_conv3(n, "decoder.conv_in", 4, kTop, 8);
    add_resnet(n, resnet_pf(-1, 0), kTop, kTop);
    add_norm(n, std::string(kAttn) + ".group_norm", kTop);
    for (const char* l : {".to_q", ".to_k", ".to_v", ".to_out.0"}) {
        n.add(kAttn + std::string(l) + ".weight", {kTop, kTop}, WK_LINEAR);
        n.add(kAttn + std::string(l) + ".bias", {kTop}, WK_BIAS);
    }
    add_resnet(n, resnet_pf(-1, 1), kTop, kTop);
    const std::vector<UpStage> plan = up_plan();
    for (int i = 0; i < 4; ++i) {
        for (int j = 0; j < 3; ++j) add_resnet(n, resnet_pf(i, j), j == 0 ? plan[i].cin : plan[i].cout, plan[i].cout);
        if (plan[i].up) {
            const std::string u = "decoder.up_blocks." + std::to_string(i) + ".upsamplers.0.conv";
            add_conv3(n, u, plan[i].cout, plan[i].cout);
        }
    }
    add_norm(n, "decoder.conv_norm_out", kCh[0]);
    add_conv3(n, "decoder.conv_out", kCh[0], 3);
}

// Extra pool space after the registered tensors: the two width-changing resnets'
// [conv2 | shortcut] weights and summed biases, and the fp32 to_out bias with to_v's bias
// folded in (bo + Wo bv: the rows of the softmax sum to 1, so P (V + bv) = P V + bv).
struct VaeExtra {
    size_t w2sc_off[2], b2sc_off[2], bout_off, w4_off[3], bytes;
};
static VaeExtra extra_layout() {
    VaeExtra x{};
    size_t top = 0;
    auto take = [&](size_t b) { const size_t o = top; top += (b + 255) / 256 * 256; return o; };
    const int co[2] = {kCh[1], kCh[0]}, ci[2] = {kCh[2], kCh[1]};
    for (int k = 0; k < 2; ++k) {
        x.w2sc_off[k] = take((size_t)co[k] * (9 * co[k] + ci[k]) * 2);
        x.b2sc_off[k] = take((size_t)co[k] * 2);
    }
    x.bout_off = take((size_t)kTop * 4);
    // the upsampling convs' sub-pixel weights [4][C][2][2][C]
    const std::vector<UpStage> plan = up_plan();
    for (int i = 0; i < 3; ++i) x.w4_off[i] = take((size_t)16 * plan[i].cout * plan[i].cout * 2);
    x.bytes = top;
    return x;
}

static int vae_fold(Ctx& c, AuxNet& n) {
    const VaeExtra x = extra_layout();
    char* base = (char*)n.pool + (n.pool_bytes - x.bytes);
    hipError_t e;
    for (int k = 0; k < 2; ++k) {
        const int blk = k + 2, co = kCh[1 - k], ci = kCh[2 - k];
        const std::string pf = resnet_pf(blk, 0);
        n.w2sc[k] = (f16*)(base + x.w2sc_off[k]);
        n.b2sc[k] = (f16*)(base + x.b2sc_off[k]);
        if ((e = fold_shortcut_launch(n.wd(pf + ".conv2.weight"), n.wd(pf + ".conv2.bias"),
                                      n.wd(pf + ".conv_shortcut.weight"), n.wd(pf + ".conv_shortcut.bias"), n.w2sc[k],
                                      n.b2sc[k], co, co, ci, c.stream)))
            return hip_fail(c, e, "vae fold");
    }
    // bo + Wo bv on the host (fp32)
    const std::string a = kAttn;
    std::vector<f16> wo((size_t)kTop * kTop), bv(kTop), bo(kTop);
    if ((e = hipStreamSynchronize(c.stream)) ||
        (e = hipMemcpy(wo.data(), n.wd(a + ".to_out.0.weight"), wo.size() * 2, hipMemcpyDeviceToHost)) ||
        (e = hipMemcpy(bv.data(), n.wd(a + ".to_v.bias"), kTop * 2, hipMemcpyDeviceToHost)) ||
        (e = hipMemcpy(bo.data(), n.wd(a + ".to_out.0.bias"), kTop * 2, hipMemcpyDeviceToHost)))
        return hip_fail(c, e, "vae fold");
    std::vector<float> bout(kTop);
    for (int o = 0; o < kTop; ++o) {
        double acc = (float)bo[o];
        for (int k = 0; k < kTop; ++k) acc += (double)(float)wo[(size_t)o * kTop + k] * (float)bv[k];
        bout[o] = (float)acc;
    }
    n.b_attn_out = (float*)(base + x.bout_off);
    if ((e = hipMemcpy(n.b_attn_out, bout.data(), kTop * 4, hipMemcpyHostToDevice)))
        return hip_fail(c, e, "vae fold");
    const std::vector<UpStage> plan = up_plan();
    for (int i = 0; i < 3; ++i) {
        n.w4[i] = (f16*)(base + x.w4_off[i]);
        const std::string u = "decoder.up_blocks." + std::to_string(i) + ".upsamplers.0.conv.weight";
        if ((e = fold_subpix_launch(n.wd(u), n.w4[i], plan[i].cout, plan[i].cout, c.stream)))
            return hip_fail(c, e, "vae fold");
    }
    if ((e = hipStreamSynchronize(c.stream))) return hip_fail(c, e, "vae fold");
    return SDU_OK;
}

int vae_create(Ctx& c, const char* weights_dir, uint64_t seed, int flags) {
    AuxNet* n = new AuxNet();
    n->kind = AUX_VAE;
    vae_register(*n);
    const VaeExtra x = extra_layout();
    int st = aux_alloc(c, *n, x.bytes);
    if (st) { aux_free(n); return st; }
    const bool affine = (flags & SDU_INIT_RANDOM_AFFINE) != 0;
    for (const WeightRec& r : n->weights) {
        st = weights_dir ? load_weight_file(c, r, weights_dir)
                         : gen_weight(c, r, seed, affine, r.kind == WK_LINEAR ? kLinStd : kConvStd);
        if (st) { aux_free(n); return st; }
    }
    if ((st = vae_fold(c, *n))) { aux_free(n); return st; }
    aux_free(c.vae);
    c.vae = n;
    return SDU_OK;
}

static f16* conv(Exec& E, AuxNet& n, const std::string& pf, Act x, int H, int W, int cin, int cout, int ups,
                 Act* out_act, const f16* w4 = nullptr) {
    const int Ho = ups ? 2 * H : H, Wo = ups ? 2 * W : W;
    f16* y = E.alloc<f16>((size_t)E.B * Ho * Wo * cout);
    GemmArgs a = conv3_args(x.p, E.B, H, W, cin, cout, 1, ups, n.wd(pf + ".weight"), y);
    // after the 2x upsampling: the sub-pixel form where each phase's pixels fill whole tiles
    if (ups && w4 && cin % 64 == 0 && (E.B * H * W) % 64 == 0) {
        a.upsample = 0;
        a.subpix = 1;
        a.K = 4 * cin;
        a.Wt = w4;
    }
    a.bias = n.wd(pf + ".bias");
    want_stats(E, a, Ho * Wo);
    gemm(E, "vae_conv3x3", a);
    *out_act = Act{y, a.stats};
    return y;
}

// ResnetBlock2D without time embedding: shortcut(x) + conv2(SiLU(GN2(conv1(SiLU(GN1(x))))))
static Act resnet(Exec& E, AuxNet& n, const std::string& pf, Act x, int H, int W, int cin, int cout, int sc) {
    const int M = E.B * H * W, HW = H * W;
    f16* out = E.alloc<f16>((size_t)M * cout);
    const size_t mk = E.ar->mark();
    f16* h = E.alloc<f16>((size_t)M * cin);
    group_norm_op(E, x, Act{nullptr, nullptr}, cin, 0, n.wd(pf + ".norm1.weight"), n.wd(pf + ".norm1.bias"), h, HW, 1,
                  kEpsVae);
    Act hc;
    conv(E, n, pf + ".conv1", Act{h, nullptr}, H, W, cin, cout, 0, &hc);
    f16* h2 = E.alloc<f16>((size_t)M * cout);
    group_norm_op(E, hc, Act{nullptr, nullptr}, cout, 0, n.wd(pf + ".norm2.weight"), n.wd(pf + ".norm2.bias"), h2, HW,
                  1, kEpsVae);
    GemmArgs a = conv3_args(h2, E.B, H, W, cout, cout, 1, 0, n.wd(pf + ".conv2.weight"), out);
    a.bias = n.wd(pf + ".conv2.bias");
    if (cin != cout) {
        // the 1x1 shortcut over the block's input as extra K columns: A = [im2col(h2) | x]
        a.Wt = n.w2sc[sc];
        a.bias = n.b2sc[sc];
        a.K1 = 9 * cout;
        a.A2 = x.p; a.lda2 = cin;
        a.K = a.K1 + cin;
    } else {
        a.res = x.p; a.ldr = cout;
    }
    want_stats(E, a, HW);
    gemm(E, "vae_conv3x3", a);
    E.ar->release(mk);
    return Act{out, a.stats};
}

// The mid block's attention: x + to_out(softmax(q k^T / sqrt(512)) v) over the HW tokens
// of each image, q / k / v = to_q / to_k / to_v of GroupNorm(x), one head of 512.
static Act attention(Exec& E, AuxNet& n, Act x, int H, int W) {
    const int C = kTop, HW = H * W, M = E.B * HW;
    const std::string a = kAttn;
    f16* out = E.alloc<f16>((size_t)M * C);
    const size_t mk = E.ar->mark();
    f16* g = E.alloc<f16>((size_t)M * C);
    group_norm_op(E, x, Act{nullptr, nullptr}, C, 0, n.wd(a + ".group_norm.weight"), n.wd(a + ".group_norm.bias"), g,
                  HW, 0, kEpsVae);
    f16* q = E.alloc<f16>((size_t)M * C);
    f16* k = E.alloc<f16>((size_t)M * C);
    for (int i = 0; i < 2; ++i) {
        GemmArgs ga = dense_args(g, C, M, C, C, n.wd(a + (i ? ".to_k.weight" : ".to_q.weight")), i ? k : q, C);
        ga.bias = n.wd(a + (i ? ".to_k.bias" : ".to_q.bias"));
        gemm(E, "vae_linear", ga);
    }
    f16* vt = E.alloc<f16>((size_t)C * HW);    // V^T of one image (to_v's bias is in to_out's)
    float* s = E.alloc<float>((size_t)HW * HW);  // scores of one image
    f16* p = E.alloc<f16>((size_t)HW * HW);
    f16* o = E.alloc<f16>((size_t)M * C);
    const float scale = 1.0f / sqrtf((float)C);
    for (int b = 0; b < E.B; ++b) {
        const size_t t0 = (size_t)b * HW * C;
        gemm(E, "vae_linear", dense_args(n.wd(a + ".to_v.weight"), C, C, HW, C, g + t0, vt, HW));
        GemmArgs sa = dense_args(q + t0, C, HW, HW, C, k + t0, s, HW);
        sa.out_mode = OUT_F32;
        gemm(E, "vae_attn_scores", sa);
        E.run("vae_attn_softmax", [&] { return softmax_rows_launch(s, p, HW, HW, scale, E.s); });
        gemm(E, "vae_attn_pv", dense_args(p, HW, HW, C, HW, vt, o + t0, C));
    }
    GemmArgs oa = dense_args(o, C, M, C, C, n.wd(a + ".to_out.0.weight"), out, C);
    oa.bias2 = n.b_attn_out;
    oa.res = x.p; oa.ldr = C;
    want_stats(E, oa, HW);
    gemm(E, "vae_linear", oa);
    E.ar->release(mk);
    return Act{out, oa.stats};
}

static void vae_body(Exec& E, AuxNet& n, AuxState& S) {
    const int B = S.key[0];
    int h = S.key[1], w = S.key[2];
    // GroupNorm accumulators (2 per resnet, the attention's, conv_norm_out) and the
    // statistics pool of the GEMM outputs GroupNorms read, cleared by one fill kernel
    const size_t n_gn = 2 * 14 + 2;
    const size_t acc_n = n_gn * groupnorm_acc_bytes(B, 32) / sizeof(double);
    const size_t st_n = (size_t)B * 40 * kTop * 2;
    E.gn_acc = E.alloc<double>(acc_n + st_n);
    E.st_next = E.gn_acc + acc_n;
    E.st_end = E.st_next + st_n;
    {
        void* pool = E.gn_acc;
        E.run("vae_io", [&] { return zero_launch(pool, (acc_n + st_n) * sizeof(double), E.s); });
    }
    f16* x0 = E.alloc<f16>((size_t)B * h * w * 8);
    E.run("vae_io", [&] {
        return vae_stage_launch((const float*)S.in, n.wd("post_quant_conv.weight"), n.wd("post_quant_conv.bias"), x0,
                                B, h * w, 1.0f / kScaling, E.s);
    });
    Act x;
    conv(E, n, "decoder.conv_in", Act{x0, nullptr}, h, w, 8, kTop, 0, &x);
    x = resnet(E, n, resnet_pf(-1, 0), x, h, w, kTop, kTop, -1);
    x = attention(E, n, x, h, w);
    x = resnet(E, n, resnet_pf(-1, 1), x, h, w, kTop, kTop, -1);
    const std::vector<UpStage> plan = up_plan();
    for (int i = 0; i < 4; ++i) {
        for (int j = 0; j < 3; ++j) {
            const int cin = j == 0 ? plan[i].cin : plan[i].cout;
            x = resnet(E, n, resnet_pf(i, j), x, h, w, cin, plan[i].cout, cin != plan[i].cout ? i - 2 : -1);
        }
        if (plan[i].up) {
            conv(E, n, "decoder.up_blocks." + std::to_string(i) + ".upsamplers.0.conv", x, h, w, plan[i].cout,
                 plan[i].cout, 1, &x, n.w4[i]);
            h *= 2;
            w *= 2;
        }
    }
    f16* g = E.alloc<f16>((size_t)B * h * w * kCh[0]);
    group_norm_op(E, x, Act{nullptr, nullptr}, kCh[0], 0, n.wd("decoder.conv_norm_out.weight"),
                  n.wd("decoder.conv_norm_out.bias"), g, h * w, 1, kEpsVae);
    GemmArgs a = conv3_args(g, B, h, w, kCh[0], 3, 1, 0, n.wd("decoder.conv_out.weight"), S.out);
    a.bias = n.wd("decoder.conv_out.bias");
    a.out_mode = OUT_F32_NCHW;
    a.ldc = 3;
    a.hw_out = h * w;
    gemm(E, "vae_conv3x3", a);
}

int vae_decode_device(Ctx& c, const float* d_lat, int B, int H, int W, float* d_img) {
    if (!c.vae) return set_err(&c, SDU_ERR_WEIGHT, "no VAE decoder (sdu_vae_init)");
    if (B < 1 || B > 4 || H < 8 || W < 8 || H * W > kMaxHW)
        return set_err(&c, SDU_ERR_ARG, "VAE decode: B in 1..4, H and W >= 8, H * W <= 96 * 96");
    const size_t in_b = (size_t)B * 4 * H * W * 4, out_b = (size_t)B * 3 * 64 * H * W * 4;
    int st = 0;
    AuxState* S = aux_state(c, *c.vae, {B, H, W}, B, in_b, out_b, vae_body, &st);
    if (!S) return st;
    hipError_t e;
    if ((e = hipMemcpyAsync(S->in, d_lat, in_b, hipMemcpyDeviceToDevice, c.stream)) ||
        (e = hipGraphLaunch(S->exec, c.stream)) ||
        (e = hipMemcpyAsync(d_img, S->out, out_b, hipMemcpyDeviceToDevice, c.stream)))
        return hip_fail(c, e, "vae decode");
    return SDU_OK;
}

}  // namespace sdu
