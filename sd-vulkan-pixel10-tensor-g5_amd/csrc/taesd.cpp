// TAESD latent decoder on the HIP kernels: latent [B, 4, H, W] -> image [B, 3, 8H, 8W].
//
// Replaces the reference's LiteRT VAE / TAESD decoder (VulkanUnetPipeline.kt:55-61,
// exported from diffusers AutoencoderTiny in tools/export_taesd.py:52-54; contract
// [1,4,64,64] -> [1,3,512,512] in [-1, 1], tools/export_taesd.py:2).  The network
// (diffusers DecoderTiny, num_blocks (3, 3, 3, 1), 64 channels):
//   3 tanh(x / 3) -> conv 4->64 + ReLU -> {3 blocks, upsample 2x, conv} x 3 -> block
//   -> conv 64->3 -> 2 y - 1,   block(x) = ReLU(conv(ReLU(conv(ReLU(conv(x))))) + x)
// Every conv is the implicit-GEMM conv with its bias, residual and ReLU fused into the
// epilogue; the nearest upsampling is folded into the following conv's index math; the
// clamp is applied while converting the latent to NHWC fp16; the output affine is folded
// into conv_out (2 W, 2 b - 1), which writes fp32 NCHW directly.
#include "graph.h"

#include <cstring>
#include <vector>

namespace sdu {

static const int kCh = 64;
// (blocks, upsample after) per stage, as the decoder's layer list
static const int kStageBlocks[4] = {3, 3, 3, 1};
// seeded random init: conv weights N(0, 0.04), as the oracle's taesd_ref.CONV_STD
static const double kConvStd = 0.04;

// decoder.layers index of each element, in order: conv_in, relu, blocks / upsample + conv,
// conv_out (the Sequential indices of diffusers' DecoderTiny)
struct Plan {
    int conv_in = 0;
    std::vector<std::vector<int>> blocks;  // per stage
    std::vector<int> up_conv;              // per upsampling stage
    int conv_out = 0;
    Plan() {
        int i = 2;
        for (int s = 0; s < 4; ++s) {
            blocks.emplace_back();
            for (int b = 0; b < kStageBlocks[s]; ++b) blocks.back().push_back(i++);
            if (s < 3) {
                ++i;  // nn.Upsample
                up_conv.push_back(i++);
            } else {
                conv_out = i++;
            }
        }
    }
};

static std::string L(int i) { return "decoder.layers." + std::to_string(i); }

static void taesd_register(AuxNet& n) {
    const Plan p;
    n.add(L(p.conv_in) + ".weight", {kCh, 4, 3, 3}, WK_CONV, GL_CONV_OHWI, 8);
    n.add(L(p.conv_in) + ".bias", {kCh}, WK_BIAS);
    for (int s = 0; s < 4; ++s) {
        for (int b : p.blocks[s])
            for (int j : {0, 2, 4}) {
                const std::string pf = L(b) + ".conv." + std::to_string(j);
                n.add(pf + ".weight", {kCh, kCh, 3, 3}, WK_CONV, GL_CONV_OHWI, kCh);
                n.add(pf + ".bias", {kCh}, WK_BIAS);
            }
        if (s < 3) n.add(L(p.up_conv[s]) + ".weight", {kCh, kCh, 3, 3}, WK_CONV, GL_CONV_OHWI, kCh);
    }
    n.add(L(p.conv_out) + ".weight", {3, kCh, 3, 3}, WK_CONV, GL_CONV_OHWI, kCh);
    n.add(L(p.conv_out) + ".bias", {3}, WK_BIAS);
}

// conv_out with y = 2 x - 1 folded in: 2 W (exact in fp16), fp32 bias 2 b - 1
static int fold_out(Ctx& c, AuxNet& n) {
    const Plan p;
    const WeightRec* w = n.w(L(p.conv_out) + ".weight");
    const WeightRec* b = n.w(L(p.conv_out) + ".bias");
    std::vector<f16> hw((size_t)w->dev_n), hb((size_t)b->dev_n);
    hipError_t e;
    if ((e = hipStreamSynchronize(c.stream)) || (e = hipMemcpy(hw.data(), w->dev, hw.size() * 2, hipMemcpyDeviceToHost)) ||
        (e = hipMemcpy(hb.data(), b->dev, hb.size() * 2, hipMemcpyDeviceToHost)))
        return hip_fail(c, e, "taesd fold");
    for (f16& v : hw) v = (f16)(2.0f * (float)v);
    float bf[3];
    for (int i = 0; i < 3; ++i) bf[i] = 2.0f * (float)hb[i] - 1.0f;
    if ((e = hipMemcpy(n.w_out2, hw.data(), hw.size() * 2, hipMemcpyHostToDevice)) ||
        (e = hipMemcpy(n.b_out2, bf, sizeof bf, hipMemcpyHostToDevice)))
        return hip_fail(c, e, "taesd fold");
    for (int s = 0; s < 3; ++s)
        if ((e = fold_subpix_launch(n.wd(L(p.up_conv[s]) + ".weight"), n.w4[s], kCh, kCh, c.stream)))
            return hip_fail(c, e, "taesd fold");
    if ((e = hipStreamSynchronize(c.stream))) return hip_fail(c, e, "taesd fold");
    return SDU_OK;
}

int taesd_create(Ctx& c, const char* weights_dir, uint64_t seed, int flags) {
    AuxNet* n = new AuxNet();
    n->kind = AUX_TAESD;
    taesd_register(*n);
    // extra pool space: conv_out with the output affine, its fp32 bias, and the upsampling
    // convs' sub-pixel weights [4][64][2][2][64]
    const size_t wout_n = 3 * 9 * kCh, wout_b = (wout_n * 2 + 255) / 256 * 256, w4_b = 16 * kCh * kCh * 2;
    const size_t extra_b = wout_b + 256 + 3 * w4_b;
    int st = aux_alloc(c, *n, extra_b);
    if (st) { aux_free(n); return st; }
    char* extra = (char*)n->pool + (n->pool_bytes - extra_b);
    n->w_out2 = (f16*)extra;
    n->b_out2 = (float*)(extra + wout_b);
    for (int s = 0; s < 3; ++s) n->w4[s] = (f16*)(extra + wout_b + 256 + s * w4_b);
    const bool affine = (flags & SDU_INIT_RANDOM_AFFINE) != 0;
    for (const WeightRec& r : n->weights) {
        st = weights_dir ? load_weight_file(c, r, weights_dir) : gen_weight(c, r, seed, affine, kConvStd);
        if (st) { aux_free(n); return st; }
    }
    if ((st = fold_out(c, *n))) { aux_free(n); return st; }
    aux_free(c.taesd);
    c.taesd = n;
    return SDU_OK;
}

static void conv(Exec& E, const f16* x, int B, int h, int w, int cin, int ups, const f16* W, const f16* bias,
                 const f16* res, f16* y, const f16* w4 = nullptr) {
    GemmArgs a = conv3_args(x, B, h, w, cin, kCh, 1, ups, W, y);
    // after the 2x upsampling: the sub-pixel form where each phase's pixels fill whole tiles
    if (ups && w4 && (B * h * w) % 64 == 0) {
        a.upsample = 0;
        a.subpix = 1;
        a.K = 4 * cin;
        a.Wt = w4;
    }
    a.bias = bias;
    a.res = res;
    a.ldr = kCh;
    a.act = ACT_RELU;
    if (ups) a.act = ACT_NONE;  // the upsampling stages' conv has neither bias nor activation
    gemm(E, "taesd_conv", a);
}

static void taesd_body(Exec& E, AuxNet& n, AuxState& S) {
    const Plan p;
    const int B = S.key[0];
    int h = S.key[1], w = S.key[2];
    f16* x = E.alloc<f16>((size_t)B * h * w * 8);
    E.run("taesd_io", [&] { return nchw_to_nhwc_launch((const float*)S.in, x, B, B, 4, 8, h * w, E.s, 1); });
    auto act = [&](int hh, int ww) { return E.alloc<f16>((size_t)B * hh * ww * kCh); };
    f16 *cur = act(h, w), *t1 = act(h, w), *t2 = act(h, w), *nxt = act(h, w);
    conv(E, x, B, h, w, 8, 0, n.wd(L(p.conv_in) + ".weight"), n.wd(L(p.conv_in) + ".bias"), nullptr, cur);
    for (int s = 0; s < 4; ++s) {
        for (int b : p.blocks[s]) {
            const std::string pf = L(b) + ".conv.";
            conv(E, cur, B, h, w, kCh, 0, n.wd(pf + "0.weight"), n.wd(pf + "0.bias"), nullptr, t1);
            conv(E, t1, B, h, w, kCh, 0, n.wd(pf + "2.weight"), n.wd(pf + "2.bias"), nullptr, t2);
            conv(E, t2, B, h, w, kCh, 0, n.wd(pf + "4.weight"), n.wd(pf + "4.bias"), cur, nxt);  // fuse(conv + x)
            std::swap(cur, nxt);
        }
        if (s < 3) {
            f16* up = act(2 * h, 2 * w);
            conv(E, cur, B, h, w, kCh, 1, n.wd(L(p.up_conv[s]) + ".weight"), nullptr, nullptr, up, n.w4[s]);
            h *= 2;
            w *= 2;
            cur = up;
            t1 = act(h, w);
            t2 = act(h, w);
            nxt = act(h, w);
        }
    }
    GemmArgs a = conv3_args(cur, B, h, w, kCh, 3, 1, 0, n.w_out2, S.out);
    a.bias2 = n.b_out2;
    a.out_mode = OUT_F32_NCHW;
    a.ldc = 3;
    a.hw_out = h * w;
    gemm(E, "taesd_conv", a);
}

int taesd_decode_device(Ctx& c, const float* d_lat, int B, int H, int W, float* d_img) {
    if (!c.taesd) return set_err(&c, SDU_ERR_WEIGHT, "no TAESD decoder (sdu_taesd_init)");
    if (B < 1 || B > 16 || H < 8 || W < 8 || H > 128 || W > 128)
        return set_err(&c, SDU_ERR_ARG, "TAESD decode: B in 1..16, H and W in 8..128");
    const size_t in_b = (size_t)B * 4 * H * W * 4, out_b = (size_t)B * 3 * 64 * H * W * 4;
    int st = 0;
    AuxState* S = aux_state(c, *c.taesd, {B, H, W}, B, in_b, out_b, taesd_body, &st);
    if (!S) return st;
    hipError_t e;
    if ((e = hipMemcpyAsync(S->in, d_lat, in_b, hipMemcpyDeviceToDevice, c.stream)) ||
        (e = hipGraphLaunch(S->exec, c.stream)) ||
        (e = hipMemcpyAsync(d_img, S->out, out_b, hipMemcpyDeviceToDevice, c.stream)))
        return hip_fail(c, e, "taesd decode");
    return SDU_OK;
}

}  // namespace sdu
