// SD1.5 UNet graph on the HIP kernels: blocks, full forward, LCM denoise loop.
//
// Restates runGraph (vk_engine.cpp:711-790) and its blocks (:623-697) over NHWC
// fp16 activations.  Each forward is planned once per shape: a sizing pass runs
// the graph without launching to size the activation arena and workspaces, then
// the real pass is captured into a HIP graph and replayed on later calls (the
// reference records one command buffer per forward, :714, :783-788).
#include "graph.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace sdu {

static const int kGroups = 32;
static const float kEps = 1e-5f;  // GN and LN (vk_engine.cpp:548-549, :652)
static const int kLatC = 4, kLatCpad = 8, kCtxDim = 768;

// ------------------------------------------------------------------ execution

thread_local KernelTimer* g_kernel_timer = nullptr;
thread_local hipEvent_t g_launch_ev0 = nullptr, g_launch_ev1 = nullptr;


static void groupnorm(Exec& E, Act x, Act x2, int C1, int C2, const f16* g, const f16* b, f16* y, int HW,
                      int silu) {
    group_norm_op(E, x, x2, C1, C2, g, b, y, HW, silu, kEps);
}

static void attention(Exec& E, const char* cat, const f16* q, const f16* k, const f16* v, f16* o,
                      int Sq, int Sk, int C, int ldq, int ldk, int ldv) {
    // q comes from a projection with the softmax factor folded in (attn_qscale); the GEMM
    // workspace serves a key-split launch
    AttnArgs a{q, k, v, o, E.B, kUnetHeads, Sq, Sk, C / kUnetHeads, ldq, ldk, ldv, C,
               1.0f / sqrtf((float)(C / kUnetHeads)), 0, 1, E.gemm_ws, 0};
    const size_t ws = attention_workspace_bytes(a);
    if (ws > E.gemm_ws_need) E.gemm_ws_need = ws;
    char shape[64];
    snprintf(shape, sizeof shape, "Sq=%d Sk=%d d=%d", Sq, Sk, C / kUnetHeads);
    E.run(cat, [&] { return attention_launch(a, E.s); }, shape);
}

// ------------------------------------------------------------------ blocks

struct Fwd {
    int B, H, W, L;
};

static const f16* W(Exec& E, const std::string& n) { return E.c.wd(n); }

// ResNet block (vk_engine.cpp:623-637).  x2 != null: input is concat(x, x2).
static Act resnet(Exec& E, const ResDesc& r, Act x, Act x2, int H, int Wd, const float* tproj) {
    const int B = E.B, M = B * H * Wd, HW = H * Wd;
    f16* out = E.alloc<f16>((size_t)M * r.cout);
    const size_t mk = E.ar->mark();
    f16* h = E.alloc<f16>((size_t)M * r.cin);
    groupnorm(E, x, x2, r.cin1, r.cin - r.cin1, W(E, r.pf + ".norm1.weight"), W(E, r.pf + ".norm1.bias"),
              h, HW, 1);
    f16* hc = E.alloc<f16>((size_t)M * r.cout);
    Act hca{hc, nullptr};
    {
        GemmArgs a = conv3_args(h, B, H, Wd, r.cin, r.cout, 1, 0, W(E, r.pf + ".conv1.weight"), hc);
        a.bias = W(E, r.pf + ".conv1.bias");
        a.bias2 = tproj + r.tproj_off;  // + time_emb_proj(silu(temb)) broadcast (:627-630)
        want_stats(E, a, HW);
        hca.st = a.stats;
        gemm(E, "conv3x3", a);
    }
    f16* h2 = E.alloc<f16>((size_t)M * r.cout);
    groupnorm(E, hca, Act{nullptr, nullptr}, r.cout, 0, W(E, r.pf + ".norm2.weight"),
              W(E, r.pf + ".norm2.bias"), h2, HW, 1);
    Act o{out, nullptr};
    {
        GemmArgs a = conv3_args(h2, B, H, Wd, r.cout, r.cout, 1, 0, W(E, r.pf + ".conv2.weight"), out);
        a.bias = W(E, r.pf + ".conv2.bias");
        if (r.cin != r.cout) {
            // the 1x1 shortcut over the (possibly concatenated) input (:634) is extra K
            // columns of conv2: A = [im2col(h2) | x | x2], W = [conv2 | shortcut]
            a.Wt = r.w2sc;
            a.bias = r.b2sc;
            a.K1 = 9 * r.cout;
            a.A2 = x.p; a.lda2 = r.cin1;
            a.K2 = a.K1 + r.cin1;
            if (x2.p) { a.A3 = x2.p; a.lda3 = r.cin - r.cin1; }
            a.K = a.K1 + r.cin;
        } else {
            a.res = x.p; a.ldr = r.cout;
        }
        want_stats(E, a, HW);
        o.st = a.stats;
        gemm(E, "conv3x3", a);
    }
    E.ar->release(mk);
    return o;
}

// Spatial transformer (vk_engine.cpp:640-675).  kv: fused cross K/V [B*L, kv_total].
static Act transformer(Exec& E, const XfDesc& t, Act xa, int H, int Wd, const f16* kv, int L) {
    const f16* x = xa.p;
    const int B = E.B, HW = H * Wd, M = B * HW, C = t.c;
    const std::string b = t.pf + ".transformer_blocks.0";
    f16* out = E.alloc<f16>((size_t)M * C);
    const size_t mk = E.ar->mark();
    // 64-column partial row sums / sums of squares of the token stream tt before norm1,
    // norm2, norm3 (GemmArgs::row_part)
    const size_t np = (size_t)(C / 64) * M * 2;
    float* rp = E.alloc<float>(3 * np);
    f16* g = E.alloc<f16>((size_t)M * C);
    groupnorm(E, xa, Act{nullptr, nullptr}, C, 0, W(E, t.pf + ".norm.weight"), W(E, t.pf + ".norm.bias"), g,
              HW, 0);
    f16* tt = E.alloc<f16>((size_t)M * C);  // token stream [B*HW, C] (no T_CH transpose: NHWC)
    {
        GemmArgs a = dense_args(g, C, M, C, C, W(E, t.pf + ".proj_in.weight"), tt, C);
        a.bias = W(E, t.pf + ".proj_in.bias");
        a.row_part = rp;
        gemm(E, "conv1x1", a);
    }
    f16* qkv = E.alloc<f16>((size_t)M * 3 * C);
    f16* at = E.alloc<f16>((size_t)M * C);
    // Each LayerNorm (norm1, norm2, norm3) runs inside the GEMMs around it: the GEMM
    // that writes the token stream tt keeps its row statistics, and the GEMM that
    // reads it takes tt as A with the folded weight / bias / column sums (fold_weights).
    auto ln_gemm = [&](f16* out, int N, int ldo, const f16* w, const float* bias, const float* colsum,
                       const float* part) {
        GemmArgs a = dense_args(tt, C, M, N, C, w, out, ldo);
        a.bias2 = bias;
        a.ln_part = part;
        a.ln_colsum = colsum;
        a.ln_eps = kEps;
        return a;
    };
    // self-attention
    gemm(E, "linear", ln_gemm(qkv, 3 * C, 3 * C, t.w_qkv, t.b_qkv, t.s_qkv, rp));
    attention(E, "attn_self", qkv, qkv + C, qkv + 2 * C, at, HW, HW, C, 3 * C, 3 * C, 3 * C);
    {
        GemmArgs a = dense_args(at, C, M, C, C, W(E, b + ".attn1.to_out.0.weight"), tt, C);
        a.bias = W(E, b + ".attn1.to_out.0.bias");
        a.res = tt; a.ldr = C;
        a.row_part = rp + np;
        gemm(E, "linear", a);
    }
    // cross-attention: K/V of this block are columns [kv_off, kv_off + 2C) of kv
    gemm(E, "linear", ln_gemm(qkv, C, C, t.w_q2, t.b_q2, t.s_q2, rp + np));
    const int ldkv = E.c.kv_total;
    attention(E, "attn_cross", qkv, kv + t.kv_off, kv + t.kv_off + C, at, HW, L, C, C, ldkv, ldkv);
    {
        GemmArgs a = dense_args(at, C, M, C, C, W(E, b + ".attn2.to_out.0.weight"), tt, C);
        a.bias = W(E, b + ".attn2.to_out.0.bias");
        a.res = tt; a.ldr = C;
        a.row_part = rp + 2 * np;
        gemm(E, "linear", a);
    }
    // GEGLU feed-forward: proj (+bias, GEGLU in the epilogue).  Its output projection
    // (+bias, +residual t) and proj_out (+bias, +residual x) are one GEMM over the
    // two-source A = [ff | t] with the folded weight [Wp.Wf | Wp] (fold_weights):
    // out = Wp.(t + Wf.ff + bf) + bp + x.
    f16* ff = E.alloc<f16>((size_t)M * 4 * C);
    {
        GemmArgs a = ln_gemm(ff, 8 * C, 4 * C, t.w_ff, t.b_ff, t.s_ff, rp + 2 * np);
        a.geglu = 1;
        gemm(E, "linear_geglu", a);
    }
    Act o{out, nullptr};
    {
        GemmArgs a = dense_args(ff, 4 * C, M, C, 5 * C, t.w_out, out, C);
        a.A2 = tt; a.lda2 = C; a.K1 = 4 * C;
        a.bias = t.b_out;
        a.res = x; a.ldr = C;
        want_stats(E, a, HW);
        o.st = a.stats;
        gemm(E, "linear_out", a);
    }
    E.ar->release(mk);
    return o;
}

static Act conv3_block(Exec& E, const std::string& pf, const f16* x, int H, int Wd, int Cin, int Cout,
                       int stride, int ups) {
    GemmArgs a = conv3_args(x, E.B, H, Wd, Cin, Cout, stride, ups, W(E, pf + ".weight"), nullptr);
    // after a 2x nearest upsampling: the sub-pixel form (4 taps per output pixel instead of 9)
    // where each phase's input pixels fill whole tiles
    if (ups && Cin % 64 == 0 && (E.B * H * Wd) % 64 == 0)
        for (const UpDesc& u : E.c.ups)
            if (u.pf == pf && u.c == Cin && Cout == Cin) {
                a.upsample = 0;
                a.subpix = 1;
                a.K = 4 * Cin;
                a.Wt = u.w4;
            }
    f16* y = E.alloc<f16>((size_t)a.M * Cout);
    a.C = y;
    a.bias = W(E, pf + ".bias");
    want_stats(E, a, a.Ho * a.Wo);
    gemm(E, "conv3x3", a);
    return Act{y, a.stats};
}

// time MLP (vk_engine.cpp:716-717) + every resnet's time_emb_proj(silu(temb)) in
// one GEMV over the fused projection block.  Returns tproj [tproj_total] fp32.
// n time embeddings at once (temb320 [n][320] -> [n][tproj_total]): the steps of a
// denoise share each weight read.
static float* time_embed(Exec& E, const float* temb320, int n = 1) {
    Ctx& c = E.c;
    float* t1 = E.alloc<float>((size_t)n * 1280);
    float* temb = E.alloc<float>((size_t)n * 1280);
    float* tproj = E.alloc<float>((size_t)n * c.tproj_total);
    E.run("time_mlp", [&] {
        return gemv_launch(temb320, c.wd("time_embedding.linear_1.weight"), c.wd("time_embedding.linear_1.bias"),
                           t1, 1280, 320, 0, 1, E.s, n);
    });
    E.run("time_mlp", [&] {
        return gemv_launch(t1, c.wd("time_embedding.linear_2.weight"), c.wd("time_embedding.linear_2.bias"),
                           temb, 1280, 1280, 0, 0, E.s, n);
    });
    E.run("time_mlp", [&] {
        return gemv_launch(temb, c.w_tproj, c.b_tproj, tproj, c.tproj_total, 1280, 1, 0, E.s, n);
    });
    return tproj;
}

// All 16 transformers' attn2 to_k / to_v in one GEMM: [B*L, 768] x [kv_total, 768]^T.
static f16* cross_kv(Exec& E, const f16* ctx16, int L) {
    Ctx& c = E.c;
    const int M = E.B * L;
    f16* kv = E.alloc<f16>((size_t)M * c.kv_total);
    gemm(E, "cross_kv", dense_args(ctx16, kCtxDim, M, c.kv_total, kCtxDim, c.w_kv, kv, c.kv_total));
    return kv;
}

// UNet body: lat NHWC fp16 [B,H,W,8] -> eps fp32 NCHW [B,4,H,W] (vk_engine.cpp:711-790).
// tproj_pre: the time projections of this forward when already computed (a denoise
// computes every step's at once); otherwise they are formed here from temb320.
// out_ind: when set, conv_out reads its output pointer from this device word (written
// before each replay) instead of writing to `out`.
static void unet_core(Exec& E, const Fwd& F, const f16* lat, const float* temb320, const f16* kv,
                      float* out, const float* tproj_pre = nullptr, void* const* out_ind = nullptr) {
    Ctx& c = E.c;
    const size_t mk0 = E.ar->mark();
    // GroupNorm accumulators of this forward (2 per resnet, 1 per transformer, conv_norm_out)
    // for GroupNorms that compute their own statistics, then the pool of per-channel
    // statistics of the GEMM outputs that GroupNorms read (conv1 and conv2 of every
    // resnet, every transformer's proj_out, conv_in and the 6 resampling convs);
    // one clear for both.
    const size_t n_gn = 2 * c.resnets.size() + c.xfs.size() + 1;
    const size_t acc_n = n_gn * groupnorm_acc_bytes(E.B, kGroups) / sizeof(double);
    size_t st_ch = 7 * 1280;
    for (const ResDesc& r : c.resnets) st_ch += 2 * r.cout;
    for (const XfDesc& t : c.xfs) st_ch += t.c;
    const size_t st_n = (size_t)E.B * st_ch * 2;
    E.gn_acc = E.alloc<double>(acc_n + st_n);
    E.st_next = E.gn_acc + acc_n;
    E.st_end = E.st_next + st_n;
    if (E.stats_outside) {
        E.stats_pool = E.gn_acc;
        E.stats_bytes = (acc_n + st_n) * sizeof(double);
    } else {
        void* p = E.gn_acc;
        E.run("groupnorm", [&] { return zero_launch(p, (acc_n + st_n) * sizeof(double), E.s); });
    }
    const float* tproj = tproj_pre ? tproj_pre : time_embed(E, temb320);
    int H = F.H, Wd = F.W;
    struct Skip { Act a; int ch; };
    std::vector<Skip> skips;
    Act x = conv3_block(E, "conv_in", lat, H, Wd, kLatCpad, 320, 1, 0);
    skips.push_back({x, 320});
    static const int bo[4] = {320, 640, 1280, 1280};
    static const int uo[4] = {1280, 1280, 640, 320};
    char pf[96];
    int cprev = 320;
    for (int i = 0; i < 4; ++i) {
        for (int r = 0; r < 2; ++r) {
            snprintf(pf, sizeof pf, "down_blocks.%d.resnets.%d", i, r);
            x = resnet(E, c.resnets[c.res_by_pf[pf]], x, Act{nullptr, nullptr}, H, Wd, tproj);
            if (i < 3) {
                snprintf(pf, sizeof pf, "down_blocks.%d.attentions.%d", i, r);
                x = transformer(E, c.xfs[c.xf_by_pf[pf]], x, H, Wd, kv, F.L);
            }
            skips.push_back({x, bo[i]});
        }
        cprev = bo[i];
        if (i < 3) {
            snprintf(pf, sizeof pf, "down_blocks.%d.downsamplers.0.conv", i);
            x = conv3_block(E, pf, x.p, H, Wd, bo[i], bo[i], 2, 0);
            H /= 2; Wd /= 2;
            skips.push_back({x, bo[i]});
        }
    }
    x = resnet(E, c.resnets[c.res_by_pf["mid_block.resnets.0"]], x, Act{nullptr, nullptr}, H, Wd, tproj);
    x = transformer(E, c.xfs[c.xf_by_pf["mid_block.attentions.0"]], x, H, Wd, kv, F.L);
    x = resnet(E, c.resnets[c.res_by_pf["mid_block.resnets.1"]], x, Act{nullptr, nullptr}, H, Wd, tproj);
    for (int i = 0; i < 4; ++i) {
        for (int r = 0; r < 3; ++r) {
            const Skip sk = skips.back();
            skips.pop_back();
            snprintf(pf, sizeof pf, "up_blocks.%d.resnets.%d", i, r);
            const ResDesc& rd = c.resnets[c.res_by_pf[pf]];
            x = resnet(E, rd, x, sk.a, H, Wd, tproj);  // concat(prev, skip) read in place
            cprev = uo[i];
            if (i > 0) {
                snprintf(pf, sizeof pf, "up_blocks.%d.attentions.%d", i, r);
                x = transformer(E, c.xfs[c.xf_by_pf[pf]], x, H, Wd, kv, F.L);
            }
        }
        if (i < 3) {
            snprintf(pf, sizeof pf, "up_blocks.%d.upsamplers.0.conv", i);
            x = conv3_block(E, pf, x.p, H, Wd, uo[i], uo[i], 1, 1);
            H *= 2; Wd *= 2;
        }
    }
    (void)cprev;
    const int M = E.B * H * Wd;
    f16* gn = E.alloc<f16>((size_t)M * 320);
    groupnorm(E, x, Act{nullptr, nullptr}, 320, 0, c.wd("conv_norm_out.weight"), c.wd("conv_norm_out.bias"), gn,
              H * Wd, 1);
    GemmArgs a = conv3_args(gn, E.B, H, Wd, 320, kLatC, 1, 0, c.wd("conv_out.weight"), out);
    a.bias = c.wd("conv_out.bias");
    a.out_mode = OUT_F32_NCHW;
    a.ldc = kLatC;
    a.hw_out = H * Wd;
    a.c_ind = out_ind;
    gemm(E, "conv3x3", a);
    E.ar->release(mk0);
}

// ------------------------------------------------------------------ LCM schedule

struct LcmSched {
    std::vector<int> timesteps;
    std::vector<double> ac;
    // LcmScheduler.kt:25-46
    explicit LcmSched(int steps) {
        const int n_train = 1000, n_orig = 50;
        ac.resize(n_train);
        double acc = 1.0;
        const double b0 = 0.00085, b1 = 0.0120;
        for (int i = 0; i < n_train; ++i) {
            const double s = std::sqrt(b0) + (std::sqrt(b1) - std::sqrt(b0)) * i / (n_train - 1);
            acc *= 1.0 - s * s;
            ac[i] = acc;
        }
        const int k = n_train / n_orig;
        std::vector<int> rev(n_orig);
        for (int j = 0; j < n_orig; ++j) rev[j] = (n_orig - j) * k - 1;
        for (int j = 0; j < steps; ++j) timesteps.push_back(rev[(int)std::floor((double)j * n_orig / steps)]);
    }
    // LcmScheduler.kt:57-68
    LcmCoeffs coeffs(int idx, float guidance) const {
        const int steps = (int)timesteps.size();
        const int t = timesteps[idx];
        const double a_t = ac[t], st = t * 10.0, sd2 = 0.25;
        LcmCoeffs c{};
        c.guidance = guidance;
        c.sqrt_alpha = std::sqrt(a_t);
        c.sqrt_beta = std::sqrt(1.0 - a_t);
        c.c_skip = sd2 / (st * st + sd2);
        c.c_out = st / std::sqrt(st * st + sd2);
        c.last = idx == steps - 1;
        const double ap = c.last ? 1.0 : ac[timesteps[idx + 1]];
        c.sqrt_alpha_prev = std::sqrt(ap);
        c.sqrt_beta_prev = std::sqrt(1.0 - ap);
        return c;
    }
};

// sinusoid of VulkanUnetPipeline.kt:36-46 in float64
void time_proj_host(int t, float* out) {
    for (int i = 0; i < 160; ++i) {
        const double a = t * std::exp(-std::log(10000.0) * i / 160.0);
        out[i] = (float)std::cos(a);
        out[160 + i] = (float)std::sin(a);
    }
}

// ------------------------------------------------------------------ planned state

struct FwdState {
    int kind;  // 0 forward, 1 denoise
    Fwd f;
    int steps = 0;
    // denoise: steps [0, cfg_steps) run batch CFG, the rest cond only (0 when the
    // guidance scale is <= 1).  The scale itself is not part of the graph: the CFG
    // combine reads it from d_guidance, written before each replay.
    int cfg_steps = 0;
    float* d_guidance = nullptr;
    uint64_t last_use = 0;  // LRU order of the planned states
    char* arena = nullptr;
    size_t arena_bytes = 0;
    float* gemm_ws = nullptr;
    float* in_lat = nullptr;   // forward: [B,4,H,W]; denoise: [4,H,W]
    float* in_temb = nullptr;  // forward: [320]; denoise: [steps, 320]
    float* in_ctx = nullptr;   // [B, L, 768]
    float* in_noise = nullptr; // denoise: [steps-1, 4, H, W]
    float* out = nullptr;      // forward: [B,4,H,W]; denoise: [4,H,W]
    // forward: the graph's fp16 inputs (arena), filled before each replay by one
    // stage_in launch from the caller's buffers
    f16* lat16 = nullptr;      // [B,H,W,8]
    f16* ctx16 = nullptr;      // [B,L,768]
    // forward: the statistics pool the staging launch clears before each replay, and the
    // device word holding the output pointer that conv_out reads (set by that launch)
    void* stats_pool = nullptr;
    size_t stats_bytes = 0;
    void** out_slot = nullptr;
    hipGraphExec_t exec = nullptr;
};

static void body(Exec& E, FwdState& S) {
    const Fwd& F = S.f;
    const int HW = F.H * F.W;
    if (S.kind == 0) {
        // the first two allocations, so every run of the body (sizing, capture, profile)
        // places them at the same arena offsets
        S.lat16 = E.alloc<f16>((size_t)F.B * HW * kLatCpad);
        S.ctx16 = E.alloc<f16>((size_t)F.B * F.L * kCtxDim);
        const f16* kv = cross_kv(E, S.ctx16, F.L);
        // the graph: statistics cleared and output pointer set by the staging launch
        // before each replay; the eager profiling pass clears them itself and writes to
        // the state's own output
        E.stats_outside = E.timer == nullptr;
        unet_core(E, F, S.lat16, S.in_temb, kv, S.out, nullptr, E.timer ? nullptr : S.out_slot);
        if (E.stats_outside) {
            S.stats_pool = E.stats_pool;
            S.stats_bytes = E.stats_bytes;
        }
        return;
    }
    // denoise: x (fp32 [4,H,W]) lives in `out`; B = 2 (cond, uncond)
    const int64_t n = (int64_t)kLatC * HW;
    f16* lat = E.alloc<f16>((size_t)2 * HW * kLatCpad);
    f16* ctx16 = E.alloc<f16>((size_t)2 * F.L * kCtxDim);
    float* eps2 = E.alloc<float>((size_t)2 * n);
    E.run("io", [&] {
        hipError_t e = hipMemcpyAsync(S.out, S.in_lat, n * sizeof(float), hipMemcpyDeviceToDevice, E.s);
        if (e != hipSuccess) return e;
        return nchw_to_nhwc_launch(S.in_lat, lat, 2, 1, kLatC, kLatCpad, HW, E.s);
    });
    E.run("io", [&] { return f32_to_f16_launch(S.in_ctx, ctx16, (int64_t)2 * F.L * kCtxDim, E.s); });
    const f16* kv = cross_kv(E, ctx16, F.L);  // context is fixed across steps
    // every step's time MLP and resnet time projections in one pass
    const float* tproj_all = time_embed(E, S.in_temb, S.steps);
    LcmSched sched(S.steps);
    for (int i = 0; i < S.steps; ++i) {
        // TpuUnetPipeline.kt:94-99: CFG on the first cfg_steps steps, then one forward on
        // cond alone (its image 0: slot 0 of the input, the first L rows of K/V)
        const bool cfg = i < S.cfg_steps;
        E.B = cfg ? 2 : 1;
        Fwd Fi = F;
        Fi.B = E.B;
        unet_core(E, Fi, lat, nullptr, kv, eps2, tproj_all + (size_t)i * E.c.tproj_total);
        E.B = 2;
        LcmCoeffs co = sched.coeffs(i, 0.f);
        co.guidance_dev = S.d_guidance;
        co.cond_only = !cfg;
        const float* nz = co.last ? nullptr : S.in_noise + (size_t)i * n;
        f16* next = co.last ? nullptr : lat;
        E.run("lcm_step", [&] {
            return lcm_step_launch(S.out, eps2, nz, n, co, next, kLatC, HW, kLatCpad, E.s);
        });
    }
}

static void free_state(FwdState* S) {
    if (!S) return;
    if (S->exec) hipGraphExecDestroy(S->exec);
    hipFree(S->arena);
    hipFree(S->gemm_ws);
    hipFree(S->in_lat);
    hipFree(S->in_temb);
    hipFree(S->in_ctx);
    hipFree(S->in_noise);
    hipFree(S->out);
    hipFree(S->d_guidance);
    hipFree(S->out_slot);
}

void free_fwd_states(Ctx& c) {
    for (FwdState* s : c.fwd) {
        free_state(s);
        delete s;
    }
    c.fwd.clear();
}


// Plan a state: size (dry run), allocate, and capture the graph.
static int plan_state(Ctx& c, FwdState& S) {
    const int B = S.kind == 0 ? S.f.B : 2;
    const int HW = S.f.H * S.f.W;
    Arena ar;
    ar.sizing = true;
    Exec dry{c, c.stream, &ar, B};
    dry.dry = true;
    body(dry, S);
    S.arena_bytes = ar.high;
    auto mal = [&](void** p, size_t bytes) { return hipMalloc(p, bytes < 256 ? 256 : bytes); };
    hipError_t e;
    if ((e = mal((void**)&S.arena, S.arena_bytes)) != hipSuccess) return set_err(&c, SDU_ERR_OOM, "arena allocation failed");
    if ((e = mal((void**)&S.gemm_ws, dry.gemm_ws_need)) != hipSuccess) return set_err(&c, SDU_ERR_OOM, "gemm workspace");
    // split-K tile counters start at zero (each launch leaves them zero)
    if (dry.gemm_ws_need && (e = zero_launch(S.gemm_ws, gemm_counter_bytes(), c.stream)) != hipSuccess)
        return hip_fail(c, e, "gemm workspace");
    const size_t lat_n = (size_t)(S.kind == 0 ? B : 1) * kLatC * HW;
    if ((e = mal((void**)&S.in_lat, lat_n * 4)) != hipSuccess) return set_err(&c, SDU_ERR_OOM, "staging");
    if ((e = mal((void**)&S.in_temb, (size_t)(S.kind == 0 ? 1 : S.steps) * 320 * 4)) != hipSuccess) return set_err(&c, SDU_ERR_OOM, "staging");
    if ((e = mal((void**)&S.in_ctx, (size_t)B * S.f.L * kCtxDim * 4)) != hipSuccess) return set_err(&c, SDU_ERR_OOM, "staging");
    if (S.kind == 1 && (e = mal((void**)&S.in_noise, (size_t)(S.steps > 1 ? S.steps - 1 : 1) * kLatC * HW * 4)) != hipSuccess)
        return set_err(&c, SDU_ERR_OOM, "staging");
    if ((e = mal((void**)&S.out, lat_n * 4)) != hipSuccess) return set_err(&c, SDU_ERR_OOM, "staging");
    if (S.kind == 1 && (e = mal((void**)&S.d_guidance, 4)) != hipSuccess) return set_err(&c, SDU_ERR_OOM, "staging");
    if (S.kind == 0 && (e = mal((void**)&S.out_slot, sizeof(void*))) != hipSuccess)
        return set_err(&c, SDU_ERR_OOM, "staging");
    if (S.kind == 1) {
        LcmSched sched(S.steps);
        std::vector<float> te((size_t)S.steps * 320);
        for (int i = 0; i < S.steps; ++i) time_proj_host(sched.timesteps[i], te.data() + (size_t)i * 320);
        if ((e = hipMemcpy(S.in_temb, te.data(), te.size() * 4, hipMemcpyHostToDevice)) != hipSuccess)
            return hip_fail(c, e, "temb upload");
    }
    // capture
    ar.sizing = false;
    ar.base = S.arena;
    ar.cap = S.arena_bytes;
    ar.top = ar.high = 0;
    Exec E{c, c.stream, &ar, B};
    E.gemm_ws = S.gemm_ws;
    hipGraph_t g = nullptr;
    if ((e = hipStreamBeginCapture(c.stream, hipStreamCaptureModeThreadLocal)) != hipSuccess)
        return hip_fail(c, e, "begin capture");
    body(E, S);
    hipError_t ec = hipStreamEndCapture(c.stream, &g);
    if (E.err != hipSuccess) { if (g) hipGraphDestroy(g); return hip_fail(c, E.err, "kernel launch during capture"); }
    if (ec != hipSuccess) return hip_fail(c, ec, "end capture");
    e = hipGraphInstantiate(&S.exec, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(c, e, "graph instantiate");
    return SDU_OK;
}

// At most kMaxStates planned states (arena, workspace, staging and graph each) are
// kept per context; planning another evicts the least recently used one.
static const size_t kMaxStates = 16;

static FwdState* get_state(Ctx& c, int kind, int B, int H, int W, int L, int steps, int cfg_steps, int* st) {
    for (FwdState* s : c.fwd)
        if (s->kind == kind && s->f.B == B && s->f.H == H && s->f.W == W && s->f.L == L &&
            s->steps == steps && s->cfg_steps == cfg_steps) {
            s->last_use = ++c.use_clock;
            return s;
        }
    if (c.fwd.size() >= kMaxStates) {
        // the evicted state's graph may still be running on the stream
        hipError_t e = hipStreamSynchronize(c.stream);
        if (e != hipSuccess) { *st = hip_fail(c, e, "evict state"); return nullptr; }
        auto lru = std::min_element(c.fwd.begin(), c.fwd.end(),
                                    [](const FwdState* a, const FwdState* b) { return a->last_use < b->last_use; });
        free_state(*lru);
        delete *lru;
        c.fwd.erase(lru);
    }
    std::unique_ptr<FwdState> S(new FwdState());
    S->kind = kind;
    S->f = Fwd{B, H, W, L};
    S->steps = steps;
    S->cfg_steps = cfg_steps;
    *st = plan_state(c, *S);
    if (*st) { free_state(S.get()); return nullptr; }
    S->last_use = ++c.use_clock;
    c.fwd.push_back(S.release());
    return c.fwd.back();
}

static int check_shape(Ctx& c, int B, int H, int W, int L) {
    if (B < 1 || B > 64 || H < 8 || W < 8 || H % 8 || W % 8 || L < 1 || L > 256 || (int64_t)H * W > 65536)
        return set_err(&c, SDU_ERR_ARG, "unsupported shape (B in 1..64, H/W multiples of 8, L in 1..256)");
    if (!c.wpool) return set_err(&c, SDU_ERR_WEIGHT, "context has no UNet weights (SDU_INIT_NO_WEIGHTS)");
    return SDU_OK;
}

// A forward state's inputs into its graph's fp16 buffers, in one launch (temb NULL: the
// time projection is already in S.in_temb), which also clears the forward's statistics
// pool and points the graph's output at `out`.
static hipError_t stage_inputs(Ctx& c, const FwdState& S, const float* lat, const float* temb, const float* ctx,
                               float* out) {
    const Fwd& F = S.f;
    return stage_in_launch(lat, ctx, temb, S.lat16, S.ctx16, S.in_temb, F.B, kLatC, kLatCpad, F.H * F.W,
                           (int64_t)F.B * F.L * kCtxDim, temb ? 320 : 0, c.stream, S.stats_pool, S.stats_bytes,
                           S.out_slot, out);
}

int unet_forward_device(Ctx& c, const float* d_lat, const float* d_temb, const float* d_ctx, int B, int H,
                        int W, int L, float* d_out) {
    int st = check_shape(c, B, H, W, L);
    if (st) return st;
    FwdState* S = get_state(c, 0, B, H, W, L, 0, 0, &st);
    if (!S) return st;
    hipError_t e;
    if ((e = stage_inputs(c, *S, d_lat, d_temb, d_ctx, d_out)) || (e = hipGraphLaunch(S->exec, c.stream)))
        return hip_fail(c, e, "forward");
    return SDU_OK;
}

int unet_forward_host(Ctx& c, const float* lat, const float* temb, const float* ctx, int B, int H, int W,
                      int L, float* out) {
    int st = check_shape(c, B, H, W, L);
    if (st) return st;
    FwdState* S = get_state(c, 0, B, H, W, L, 0, 0, &st);
    if (!S) return st;
    const size_t lat_b = (size_t)B * kLatC * H * W * 4;
    hipError_t e;
    if ((e = hipMemcpyAsync(S->in_lat, lat, lat_b, hipMemcpyHostToDevice, c.stream)) ||
        (e = hipMemcpyAsync(S->in_temb, temb, 320 * 4, hipMemcpyHostToDevice, c.stream)) ||
        (e = hipMemcpyAsync(S->in_ctx, ctx, (size_t)B * L * kCtxDim * 4, hipMemcpyHostToDevice, c.stream)) ||
        (e = stage_inputs(c, *S, S->in_lat, nullptr, S->in_ctx, S->out)) || (e = hipGraphLaunch(S->exec, c.stream)) ||
        (e = hipMemcpyAsync(out, S->out, lat_b, hipMemcpyDeviceToHost, c.stream)) ||
        (e = hipStreamSynchronize(c.stream)))
        return hip_fail(c, e, "forward");
    return SDU_OK;
}

int unet_denoise_device(Ctx& c, const float* d_lat, const float* d_cond, const float* d_uncond, int H,
                        int W, int L, int steps, float guidance, int cfg_steps, const float* d_noise,
                        uint64_t noise_seed, float* d_out) {
    int st = check_shape(c, 2, H, W, L);
    if (st) return st;
    if (steps < 1 || steps > 50) return set_err(&c, SDU_ERR_ARG, "steps must be in 1..50");
    if (cfg_steps < 0 || cfg_steps > steps) return set_err(&c, SDU_ERR_ARG, "cfg_steps must be in 0..steps");
    if (!std::isfinite(guidance)) return set_err(&c, SDU_ERR_ARG, "guidance must be finite");
    if (!(guidance > 1.f)) cfg_steps = 0;  // no CFG on any step (TpuUnetPipeline.kt:97)
    FwdState* S = get_state(c, 1, 2, H, W, L, steps, cfg_steps, &st);
    if (!S) return st;
    const size_t n = (size_t)kLatC * H * W;
    const size_t cb = (size_t)L * kCtxDim * 4;
    hipError_t e;
    if ((e = hipMemcpyAsync(S->in_lat, d_lat, n * 4, hipMemcpyDeviceToDevice, c.stream)) ||
        (e = hipMemcpyAsync(S->in_ctx, d_cond, cb, hipMemcpyDeviceToDevice, c.stream)) ||
        (e = hipMemcpyAsync((char*)S->in_ctx + cb, d_uncond, cb, hipMemcpyDeviceToDevice, c.stream)))
        return hip_fail(c, e, "denoise");
    if (steps > 1) {
        // caller's noise, or N(0,1) drawn on the device from noise_seed
        e = d_noise ? hipMemcpyAsync(S->in_noise, d_noise, (size_t)(steps - 1) * n * 4, hipMemcpyDeviceToDevice,
                                     c.stream)
                    : gen_normal_f32_launch(S->in_noise, (int64_t)(steps - 1) * n,
                                            fnv1a64("lcm.noise") ^ splitmix64(noise_seed), c.stream);
        if (e != hipSuccess) return hip_fail(c, e, "denoise");
    }
    if ((e = fill_f32_launch(S->d_guidance, guidance, 1, c.stream)) ||
        (e = hipGraphLaunch(S->exec, c.stream)) ||
        (e = hipMemcpyAsync(d_out, S->out, n * 4, hipMemcpyDeviceToDevice, c.stream)))
        return hip_fail(c, e, "denoise");
    return SDU_OK;
}

// Eager forward with every kernel timed on its own (unetProfile,
// vk_engine.cpp:854-872): each launch carries its own start / stop events
// (hipExtLaunchKernelGGL on the engine stream) and runs once.
int unet_profile(Ctx& c, int B, int H, int W, int L) {
    int st = check_shape(c, B, H, W, L);
    if (st) return st;
    FwdState* S = get_state(c, 0, B, H, W, L, 0, 0, &st);
    if (!S) return st;
    hipError_t e = hipStreamSynchronize(c.stream);
    if (e != hipSuccess) return hip_fail(c, e, "profile");
    Arena ar;
    ar.base = S->arena;
    ar.cap = S->arena_bytes;
    EventTimer timer;
    timer.s = c.stream;
    Exec E{c, c.stream, &ar, B};
    E.gemm_ws = S->gemm_ws;
    E.timer = &timer;
    struct Install {
        explicit Install(KernelTimer* t) { g_kernel_timer = t; }
        ~Install() { g_kernel_timer = nullptr; }
    };
    {
        Install guard(&timer);
        body(E, *S);
    }
    e = hipStreamSynchronize(c.stream);
    if (E.err != hipSuccess) e = E.err;
    c.prof.clear();
    // SDU_PROFILE_DUMP=<path>: also write one CSV line per kernel launch
    FILE* dump = nullptr;
    if (const char* path = getenv("SDU_PROFILE_DUMP")) {
        dump = fopen(path, "w");
        if (dump) fprintf(dump, "category,kernel,shape,flops,bytes,ms\n");
    }
    for (ProfRec& r : timer.recs) {
        float ms = 0.f;
        if (e == hipSuccess) hipEventElapsedTime(&ms, r.e0, r.e1);
        hipEventDestroy(r.e0);
        hipEventDestroy(r.e1);
        if (dump) fprintf(dump, "%s,\"%s\",\"%s\",%.0f,%.0f,%.5f\n", r.cat.c_str(), r.kern.c_str(), r.shape.c_str(),
                          r.flops, r.bytes, ms);
        for (const std::string& key : {r.cat, std::string("k:") + r.kern}) {
            ProfAcc& a = c.prof[key];
            a.calls += 1;
            a.ms += ms;
            a.flops += r.flops;
            a.bytes += r.bytes;
        }
    }
    if (dump) fclose(dump);
    if (e != hipSuccess) return hip_fail(c, e, "profile");
    return SDU_OK;
}

}  // namespace sdu
