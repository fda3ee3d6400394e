// CLIP text encoder on the HIP kernels: token ids [B, 77] -> last hidden state [B, 77, 768].
//
// Replaces the reference's LiteRT text encoder (VulkanUnetPipeline.kt:48-53: int[77] ->
// [1, 77, 768], the UNet's cross-attention context), an export of SD1.5's text_encoder
// (CLIP ViT-L/14 text tower: 12 pre-LayerNorm layers of width 768, 12 heads, quick-GELU MLP
// of 3072, causal self-attention, final LayerNorm).  Per layer:
//   h = LN1(x); qkv = h Wqkv^T + b (one GEMM over the fused q/k/v weight);
//   x += out_proj(causal_attention(q, k, v));  h = LN2(x);
//   x += fc2(quick_gelu(fc1(h)))                (quick-GELU in fc1's epilogue)
// with the residual adds in the GEMM epilogues (in place on x), activations fp16.
#include "graph.h"

namespace sdu {

static const int kSeq = 77, kHid = 768, kLayers = 12, kHeads = 12, kFfn = 3072, kVocab = 49408;
static const float kLnEps = 1e-5f;
static const std::string kPf = "text_model.";

static std::string layer(int i) { return kPf + "encoder.layers." + std::to_string(i); }

static void clip_register(AuxNet& n) {
    n.add(kPf + "embeddings.token_embedding.weight", {kVocab, kHid}, WK_EMBED);
    n.add(kPf + "embeddings.position_embedding.weight", {kSeq, kHid}, WK_EMBED);
    for (int i = 0; i < kLayers; ++i) {
        const std::string a = layer(i) + ".self_attn.";
        // q, k, v weights and biases each contiguous: one [3C, C] weight, one [3C] bias
        n.add(a + "q_proj.weight", {kHid, kHid}, WK_LINEAR);
        n.add(a + "k_proj.weight", {kHid, kHid}, WK_LINEAR, GL_PLAIN, 0, true);
        n.add(a + "v_proj.weight", {kHid, kHid}, WK_LINEAR, GL_PLAIN, 0, true);
        n.add(a + "q_proj.bias", {kHid}, WK_BIAS);
        n.add(a + "k_proj.bias", {kHid}, WK_BIAS, GL_PLAIN, 0, true);
        n.add(a + "v_proj.bias", {kHid}, WK_BIAS, GL_PLAIN, 0, true);
        n.add(a + "out_proj.weight", {kHid, kHid}, WK_LINEAR);
        n.add(a + "out_proj.bias", {kHid}, WK_BIAS);
        n.add(layer(i) + ".layer_norm1.weight", {kHid}, WK_NORM_W);
        n.add(layer(i) + ".layer_norm1.bias", {kHid}, WK_NORM_B);
        n.add(layer(i) + ".mlp.fc1.weight", {kFfn, kHid}, WK_LINEAR);
        n.add(layer(i) + ".mlp.fc1.bias", {kFfn}, WK_BIAS);
        n.add(layer(i) + ".mlp.fc2.weight", {kHid, kFfn}, WK_LINEAR);
        n.add(layer(i) + ".mlp.fc2.bias", {kHid}, WK_BIAS);
        n.add(layer(i) + ".layer_norm2.weight", {kHid}, WK_NORM_W);
        n.add(layer(i) + ".layer_norm2.bias", {kHid}, WK_NORM_B);
    }
    n.add(kPf + "final_layer_norm.weight", {kHid}, WK_NORM_W);
    n.add(kPf + "final_layer_norm.bias", {kHid}, WK_NORM_B);
}

int clip_create(Ctx& c, const char* weights_dir, uint64_t seed, int flags) {
    AuxNet* n = new AuxNet();
    n->kind = AUX_CLIP;
    clip_register(*n);
    int st = aux_alloc(c, *n, 0);
    if (st) { aux_free(n); return st; }
    const bool affine = (flags & SDU_INIT_RANDOM_AFFINE) != 0;
    for (const WeightRec& r : n->weights) {
        st = weights_dir ? load_weight_file(c, r, weights_dir) : gen_weight(c, r, seed, affine, 0.02);
        if (st) { aux_free(n); return st; }
    }
    hipError_t e = hipStreamSynchronize(c.stream);
    if (e != hipSuccess) { aux_free(n); return hip_fail(c, e, "clip weights"); }
    aux_free(c.clip);
    c.clip = n;
    return SDU_OK;
}

static void clip_body(Exec& E, AuxNet& n, AuxState& S) {
    const int B = S.key[0], T = B * kSeq, C = kHid;
    f16* x = E.alloc<f16>((size_t)T * C);
    f16* h = E.alloc<f16>((size_t)T * C);
    f16* qkv = E.alloc<f16>((size_t)T * 3 * C);
    f16* at = E.alloc<f16>((size_t)T * C);
    f16* f = E.alloc<f16>((size_t)T * kFfn);
    E.run("clip_embed", [&] {
        return embed_launch((const int32_t*)S.in, n.wd(kPf + "embeddings.token_embedding.weight"),
                            n.wd(kPf + "embeddings.position_embedding.weight"), x, B, kSeq, C, kVocab, E.s);
    });
    auto ln = [&](const f16* in, const std::string& pf, f16* out) {
        E.run("clip_ln", [&] {
            return layernorm_launch(in, n.wd(pf + ".weight"), n.wd(pf + ".bias"), out, T, C, kLnEps, E.s);
        });
    };
    for (int i = 0; i < kLayers; ++i) {
        const std::string pf = layer(i), a = pf + ".self_attn.";
        ln(x, pf + ".layer_norm1", h);
        {
            GemmArgs g = dense_args(h, C, T, 3 * C, C, n.wd(a + "q_proj.weight"), qkv, 3 * C);
            g.bias = n.wd(a + "q_proj.bias");
            gemm(E, "clip_linear", g);
        }
        AttnArgs aa{qkv, qkv + C, qkv + 2 * C, at, B, kHeads, kSeq, kSeq, C / kHeads, 3 * C, 3 * C, 3 * C, C,
                    1.0f / sqrtf((float)(C / kHeads)), 1};
        E.run("clip_attn", [&] { return attention_launch(aa, E.s); });
        {
            GemmArgs g = dense_args(at, C, T, C, C, n.wd(a + "out_proj.weight"), x, C);
            g.bias = n.wd(a + "out_proj.bias");
            g.res = x;
            g.ldr = C;
            gemm(E, "clip_linear", g);
        }
        ln(x, pf + ".layer_norm2", h);
        {
            GemmArgs g = dense_args(h, C, T, kFfn, C, n.wd(pf + ".mlp.fc1.weight"), f, kFfn);
            g.bias = n.wd(pf + ".mlp.fc1.bias");
            g.act = ACT_QUICK_GELU;
            gemm(E, "clip_linear", g);
        }
        {
            GemmArgs g = dense_args(f, kFfn, T, C, kFfn, n.wd(pf + ".mlp.fc2.weight"), x, C);
            g.bias = n.wd(pf + ".mlp.fc2.bias");
            g.res = x;
            g.ldr = C;
            gemm(E, "clip_linear", g);
        }
    }
    ln(x, kPf + "final_layer_norm", h);
    E.run("clip_io", [&] { return f16_to_f32_launch(h, (float*)S.out, (int64_t)T * C, E.s); });
}

int clip_encode_device(Ctx& c, const int32_t* d_ids, int B, float* d_out) {
    if (!c.clip) return set_err(&c, SDU_ERR_WEIGHT, "no CLIP text encoder (sdu_clip_init)");
    if (B < 1 || B > 64) return set_err(&c, SDU_ERR_ARG, "CLIP encode: B in 1..64");
    const size_t in_b = (size_t)B * kSeq * 4, out_b = (size_t)B * kSeq * kHid * 4;
    int st = 0;
    AuxState* S = aux_state(c, *c.clip, {B}, B, in_b, out_b, clip_body, &st);
    if (!S) return st;
    hipError_t e;
    if ((e = hipMemcpyAsync(S->in, d_ids, in_b, hipMemcpyDeviceToDevice, c.stream)) ||
        (e = hipGraphLaunch(S->exec, c.stream)) ||
        (e = hipMemcpyAsync(d_out, S->out, out_b, hipMemcpyDeviceToDevice, c.stream)))
        return hip_fail(c, e, "clip encode");
    return SDU_OK;
}

}  // namespace sdu
