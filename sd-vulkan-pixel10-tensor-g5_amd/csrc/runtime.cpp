// Weight inventory, device weight pool and weight loading.
//
// The reference loads each tensor lazily by diffusers key from <dir>/<key>.bin
// (raw fp16, Linear stored [in,out]) and expands it to fp32 on the device
// (vk_engine.cpp:497-508).  Here every tensor is resident fp16 in one pool,
// created at init, in the layout its kernel reads:
//   conv 3x3        [Co, 3, 3, Ci]   (implicit-GEMM K = tap-major, channel-minor)
//   conv 1x1/Linear [out, in]
//   GEGLU proj      [8C, C] with rows interleaved per 32 (hidden, gate) so one
//                   GEMM tile holds both halves of its output columns
// and three fused blocks so one launch serves many layers:
//   * attn1 to_q/to_k/to_v of a transformer   -> one [3C, C] QKV weight,
//   * attn2 to_k/to_v of all 16 transformers  -> one [sum 2C, 768] weight
//     (the context is shared, so all cross K/V come from one GEMM per forward),
//   * time_emb_proj of all 22 resnets         -> one [sum Cout, 1280] weight.
#include "engine.h"

#include <cstdio>
#include <cstring>
#include <algorithm>
#include <fstream>

namespace sdu {

int set_err(Ctx* c, int code, const std::string& msg) {
    if (c) c->err = msg;
    return code;
}

namespace {

const int kBlockOut[4] = {320, 640, 1280, 1280};
const int kUpOut[4] = {1280, 1280, 640, 320};
const int kCtxDim = 768, kTembIn = 320, kTembDim = 1280;

struct Builder {
    Ctx& c;
    // pending device sizes; pointers are fixed after the pool is allocated
    std::vector<int64_t> dev_off;  // element offset into the pool, -1: fused (set later)

    int add(const std::string& name, std::vector<int64_t> shape, int kind, int layout = GL_PLAIN,
            int ci_pad = 0) {
        WeightRec r;
        r.name = name;
        r.shape = std::move(shape);
        r.kind = kind;
        r.layout = layout;
        r.ci_pad = ci_pad;
        if (layout == GL_CONV_OHWI)
            r.dev_n = r.shape[0] * r.shape[2] * r.shape[3] * ci_pad;
        else
            r.dev_n = r.numel();
        c.widx[name] = (int)c.weights.size();
        c.weights.push_back(r);
        dev_off.push_back(-2);  // -2: own allocation
        return (int)c.weights.size() - 1;
    }
    void conv3(const std::string& pf, int cin, int cout, int ci_pad = 0) {
        add(pf + ".weight", {cout, cin, 3, 3}, WK_CONV, GL_CONV_OHWI, ci_pad ? ci_pad : cin);
        add(pf + ".bias", {cout}, WK_BIAS);
    }
    void conv1(const std::string& pf, int cin, int cout) {
        add(pf + ".weight", {cout, cin, 1, 1}, WK_CONV);
        add(pf + ".bias", {cout}, WK_BIAS);
    }
    void norm(const std::string& pf, int ch) {
        add(pf + ".weight", {ch}, WK_NORM_W);
        add(pf + ".bias", {ch}, WK_NORM_B);
    }
    void resnet(const std::string& pf, int cin, int cout, int cin1) {
        ResDesc d{pf, cin, cout, cin1, c.tproj_total};
        c.res_by_pf[pf] = (int)c.resnets.size();
        c.resnets.push_back(d);
        c.tproj_total += cout;
        norm(pf + ".norm1", cin);
        conv3(pf + ".conv1", cin, cout);
        int w = add(pf + ".time_emb_proj.weight", {cout, kTembDim}, WK_LINEAR);
        int b = add(pf + ".time_emb_proj.bias", {cout}, WK_BIAS);
        dev_off[w] = dev_off[b] = -1;  // fused time-projection block
        norm(pf + ".norm2", cout);
        conv3(pf + ".conv2", cout, cout);
        if (cin != cout) conv1(pf + ".conv_shortcut", cin, cout);
    }
    void transformer(const std::string& pf, int ch) {
        XfDesc d{pf, ch, c.kv_total};
        c.xf_by_pf[pf] = (int)c.xfs.size();
        c.xfs.push_back(d);
        c.kv_total += 2 * ch;
        const std::string b = pf + ".transformer_blocks.0";
        norm(pf + ".norm", ch);
        conv1(pf + ".proj_in", ch, ch);
        norm(b + ".norm1", ch);
        int q = add(b + ".attn1.to_q.weight", {ch, ch}, WK_LINEAR);
        add(b + ".attn1.to_k.weight", {ch, ch}, WK_LINEAR);
        add(b + ".attn1.to_v.weight", {ch, ch}, WK_LINEAR);
        dev_off[q] = -3;  // QKV block allocated at to_q, k/v follow contiguously
        dev_off[q + 1] = dev_off[q + 2] = -4;
        add(b + ".attn1.to_out.0.weight", {ch, ch}, WK_LINEAR);
        add(b + ".attn1.to_out.0.bias", {ch}, WK_BIAS);
        norm(b + ".norm2", ch);
        add(b + ".attn2.to_q.weight", {ch, ch}, WK_LINEAR);
        int k2 = add(b + ".attn2.to_k.weight", {ch, kCtxDim}, WK_LINEAR);
        int v2 = add(b + ".attn2.to_v.weight", {ch, kCtxDim}, WK_LINEAR);
        dev_off[k2] = dev_off[v2] = -1;  // fused cross K/V block
        add(b + ".attn2.to_out.0.weight", {ch, ch}, WK_LINEAR);
        add(b + ".attn2.to_out.0.bias", {ch}, WK_BIAS);
        norm(b + ".norm3", ch);
        add(b + ".ff.net.0.proj.weight", {8 * ch, ch}, WK_LINEAR, GL_GEGLU_PERM);
        add(b + ".ff.net.0.proj.bias", {8 * ch}, WK_BIAS, GL_GEGLU_PERM);
        add(b + ".ff.net.2.weight", {ch, 4 * ch}, WK_LINEAR);
        add(b + ".ff.net.2.bias", {ch}, WK_BIAS);
        conv1(pf + ".proj_out", ch, ch);
    }
};

}  // namespace

// Walk the graph in runGraph order (vk_engine.cpp:711-790) and register every
// parameter; then allocate the pool and place each tensor.
int build_inventory(Ctx& c) {
    Builder bd{c, {}};
    c.weights.clear();
    c.widx.clear();
    c.resnets.clear();
    c.xfs.clear();
    c.ups.clear();
    c.tproj_total = c.kv_total = 0;

    bd.add("time_embedding.linear_1.weight", {kTembDim, kTembIn}, WK_LINEAR);
    bd.add("time_embedding.linear_1.bias", {kTembDim}, WK_BIAS);
    bd.add("time_embedding.linear_2.weight", {kTembDim, kTembDim}, WK_LINEAR);
    bd.add("time_embedding.linear_2.bias", {kTembDim}, WK_BIAS);
    bd.conv3("conv_in", 4, 320, 8);
    std::vector<int> skips = {320};
    int cprev = 320;
    char pf[96];
    for (int i = 0; i < 4; ++i) {
        const int cout = kBlockOut[i];
        for (int r = 0; r < 2; ++r) {
            snprintf(pf, sizeof pf, "down_blocks.%d.resnets.%d", i, r);
            bd.resnet(pf, r == 0 ? cprev : cout, cout, r == 0 ? cprev : cout);
            if (i < 3) {
                snprintf(pf, sizeof pf, "down_blocks.%d.attentions.%d", i, r);
                bd.transformer(pf, cout);
            }
            skips.push_back(cout);
        }
        cprev = cout;
        if (i < 3) {
            snprintf(pf, sizeof pf, "down_blocks.%d.downsamplers.0.conv", i);
            bd.conv3(pf, cout, cout);
            skips.push_back(cout);
        }
    }
    bd.resnet("mid_block.resnets.0", 1280, 1280, 1280);
    bd.transformer("mid_block.attentions.0", 1280);
    bd.resnet("mid_block.resnets.1", 1280, 1280, 1280);
    cprev = 1280;
    for (int i = 0; i < 4; ++i) {
        const int cout = kUpOut[i];
        for (int r = 0; r < 3; ++r) {
            const int cs = skips.back();
            skips.pop_back();
            snprintf(pf, sizeof pf, "up_blocks.%d.resnets.%d", i, r);
            bd.resnet(pf, cprev + cs, cout, cprev);
            cprev = cout;
            if (i > 0) {
                snprintf(pf, sizeof pf, "up_blocks.%d.attentions.%d", i, r);
                bd.transformer(pf, cout);
            }
        }
        if (i < 3) {
            snprintf(pf, sizeof pf, "up_blocks.%d.upsamplers.0.conv", i);
            bd.conv3(pf, cout, cout);
            c.ups.push_back({pf, cout});
        }
    }
    bd.norm("conv_norm_out", 320);
    bd.conv3("conv_out", 320, 4);

    // ---- pool layout (element offsets, 128-element = 256-byte aligned)
    auto align = [](int64_t n) { return (n + 127) & ~(int64_t)127; };
    // a transformer's folded weights, in this order: w_out, b_out, w_qkv, w_q2, w_ff
    // (fp16), then b_qkv, s_qkv, b_q2, s_q2, b_ff, s_ff (fp32, two halves each)
    auto xf_fold = [&](int64_t ch, XfDesc* xd, f16* base) {
        int64_t o = 0;
        auto h = [&](int64_t n) { f16* p = base ? base + o : nullptr; o += align(n); return p; };
        auto f = [&](int64_t n) { return (float*)h(2 * n); };
        f16* w_out = h(5 * ch * ch);
        f16* b_out = h(ch);
        f16* w_qkv = h(3 * ch * ch);
        f16* w_q2 = h(ch * ch);
        f16* w_ff = h(8 * ch * ch);
        float* b_qkv = f(3 * ch);
        float* s_qkv = f(3 * ch);
        float* b_q2 = f(ch);
        float* s_q2 = f(ch);
        float* b_ff = f(8 * ch);
        float* s_ff = f(8 * ch);
        if (xd) {
            xd->w_out = w_out; xd->b_out = b_out; xd->w_qkv = w_qkv; xd->w_q2 = w_q2; xd->w_ff = w_ff;
            xd->b_qkv = b_qkv; xd->s_qkv = s_qkv; xd->b_q2 = b_q2; xd->s_q2 = s_q2; xd->b_ff = b_ff;
            xd->s_ff = s_ff;
        }
        return o;
    };
    int64_t top = 0;
    const int64_t off_tproj_w = top; top += align((int64_t)c.tproj_total * kTembDim);
    const int64_t off_tproj_b = top; top += align(c.tproj_total);
    const int64_t off_kv = top; top += align((int64_t)c.kv_total * kCtxDim);
    std::vector<int64_t> off(c.weights.size(), 0);
    for (size_t i = 0; i < c.weights.size(); ++i) {
        const int64_t d = bd.dev_off[i];
        if (d == -2) { off[i] = top; top += align(c.weights[i].dev_n); }
        else if (d == -3) { off[i] = top; top += align(3 * c.weights[i].dev_n); }
    }
    std::vector<int64_t> off_fold(c.xfs.size()), off_rfold(c.resnets.size(), -1);
    for (size_t i = 0; i < c.xfs.size(); ++i) {
        const int64_t ch = c.xfs[i].c;
        off_fold[i] = top;
        top += xf_fold(ch, nullptr, nullptr);
    }
    for (size_t i = 0; i < c.resnets.size(); ++i) {
        const ResDesc& rd = c.resnets[i];
        if (rd.cin == rd.cout) continue;
        off_rfold[i] = top;
        top += align((int64_t)rd.cout * (9 * rd.cout + rd.cin)) + align(rd.cout);
    }
    std::vector<int64_t> off_up(c.ups.size());
    for (size_t i = 0; i < c.ups.size(); ++i) {
        off_up[i] = top;
        top += align(16 * (int64_t)c.ups[i].c * c.ups[i].c);
    }
    c.wpool_bytes = (size_t)top * sizeof(f16);
    hipError_t e = hipMalloc(&c.wpool, c.wpool_bytes);
    if (e != hipSuccess) return set_err(&c, SDU_ERR_OOM, "weight pool allocation failed");
    f16* P = c.wpool;
    c.w_tproj = P + off_tproj_w;
    c.b_tproj = P + off_tproj_b;
    c.w_kv = P + off_kv;
    for (size_t i = 0; i < c.weights.size(); ++i) {
        WeightRec& r = c.weights[i];
        const int64_t d = bd.dev_off[i];
        if (d == -2 || d == -3) r.dev = P + off[i];
        else if (d == -4) r.dev = c.weights[i - 1].dev + c.weights[i - 1].dev_n;  // k after q, v after k
    }
    for (size_t i = 0; i < c.resnets.size(); ++i) {
        ResDesc& rd = c.resnets[i];
        c.weights[c.widx[rd.pf + ".time_emb_proj.weight"]].dev = c.w_tproj + (int64_t)rd.tproj_off * kTembDim;
        c.weights[c.widx[rd.pf + ".time_emb_proj.bias"]].dev = c.b_tproj + rd.tproj_off;
        if (off_rfold[i] >= 0) {
            rd.w2sc = P + off_rfold[i];
            rd.b2sc = rd.w2sc + align((int64_t)rd.cout * (9 * rd.cout + rd.cin));
        }
    }
    for (size_t i = 0; i < c.xfs.size(); ++i) {
        XfDesc& xd = c.xfs[i];
        const std::string b = xd.pf + ".transformer_blocks.0";
        c.weights[c.widx[b + ".attn2.to_k.weight"]].dev = c.w_kv + (int64_t)xd.kv_off * kCtxDim;
        c.weights[c.widx[b + ".attn2.to_v.weight"]].dev = c.w_kv + (int64_t)(xd.kv_off + xd.c) * kCtxDim;
        xf_fold(xd.c, &xd, P + off_fold[i]);
    }
    for (size_t i = 0; i < c.ups.size(); ++i) c.ups[i].w4 = P + off_up[i];
    return SDU_OK;
}

int fold_weights(Ctx& c, const std::string& name) {
    for (const ResDesc& rd : c.resnets) {
        if (rd.cin == rd.cout) continue;
        if (!name.empty() && name.compare(0, rd.pf.size() + 1, rd.pf + ".") != 0) continue;
        hipError_t e = fold_shortcut_launch(c.wd(rd.pf + ".conv2.weight"), c.wd(rd.pf + ".conv2.bias"),
                                            c.wd(rd.pf + ".conv_shortcut.weight"), c.wd(rd.pf + ".conv_shortcut.bias"),
                                            rd.w2sc, rd.b2sc, rd.cout, rd.cout, rd.cin, c.stream);
        if (e != hipSuccess) return set_err(&c, SDU_ERR_HIP, std::string("weight fold: ") + hipGetErrorString(e));
    }
    for (const UpDesc& u : c.ups) {
        if (!name.empty() && name.compare(0, u.pf.size() + 1, u.pf + ".") != 0) continue;
        hipError_t e = fold_subpix_launch(c.wd(u.pf + ".weight"), u.w4, u.c, u.c, c.stream);
        if (e != hipSuccess) return set_err(&c, SDU_ERR_HIP, std::string("weight fold: ") + hipGetErrorString(e));
    }
    for (const XfDesc& xd : c.xfs) {
        if (!name.empty() && name.compare(0, xd.pf.size() + 1, xd.pf + ".") != 0) continue;
        const std::string b = xd.pf + ".transformer_blocks.0";
        const int C = xd.c;
        hipError_t e = fold_ffout_launch(c.wd(xd.pf + ".proj_out.weight"), c.wd(xd.pf + ".proj_out.bias"),
                                         c.wd(b + ".ff.net.2.weight"), c.wd(b + ".ff.net.2.bias"), xd.w_out,
                                         xd.b_out, C, c.stream);
        // to_q, to_k, to_v are consecutive [C, C] blocks of the pool: one [3C, C] weight
        if (e == hipSuccess)
            e = fold_ln_launch(c.wd(b + ".attn1.to_q.weight"), nullptr, c.wd(b + ".norm1.weight"),
                               c.wd(b + ".norm1.bias"), xd.w_qkv, xd.b_qkv, xd.s_qkv, 3 * C, C, c.stream,
                               attn_qscale(C), C);
        if (e == hipSuccess)
            e = fold_ln_launch(c.wd(b + ".attn2.to_q.weight"), nullptr, c.wd(b + ".norm2.weight"),
                               c.wd(b + ".norm2.bias"), xd.w_q2, xd.b_q2, xd.s_q2, C, C, c.stream,
                               attn_qscale(C), C);
        if (e == hipSuccess)
            e = fold_ln_launch(c.wd(b + ".ff.net.0.proj.weight"), c.wd(b + ".ff.net.0.proj.bias"),
                               c.wd(b + ".norm3.weight"), c.wd(b + ".norm3.bias"), xd.w_ff, xd.b_ff, xd.s_ff,
                               8 * C, C, c.stream);
        if (e != hipSuccess) return set_err(&c, SDU_ERR_HIP, std::string("weight fold: ") + hipGetErrorString(e));
    }
    hipError_t e = hipStreamSynchronize(c.stream);
    if (e != hipSuccess) return set_err(&c, SDU_ERR_HIP, hipGetErrorString(e));
    return SDU_OK;
}

// device element index -> canonical element index (-1: padding)
static int64_t dev_to_canon_index(const WeightRec& r, int64_t i) {
    if (r.layout == GL_CONV_OHWI) {
        const int kh = (int)r.shape[2], kw = (int)r.shape[3], ci = (int)r.shape[1];
        const int c = (int)(i % r.ci_pad);
        int64_t q = i / r.ci_pad;
        const int kx = (int)(q % kw); q /= kw;
        const int ky = (int)(q % kh);
        const int64_t o = q / kh;
        if (c >= ci) return -1;
        return ((o * ci + c) * kh + ky) * kw + kx;
    }
    if (r.layout == GL_GEGLU_PERM) {
        const int64_t cols = r.shape.size() > 1 ? r.shape[1] : 1;
        const int64_t half = r.shape[0] / 2;
        const int64_t row = i / cols, col = i % cols;
        const int64_t blk = row / 64, w = row % 64;
        const int64_t cr = (w < 32) ? blk * 32 + w : half + blk * 32 + (w - 32);
        return cr * cols + col;
    }
    return i;
}

int gen_weight(Ctx& c, const WeightRec& r, uint64_t seed, bool affine, double wstd) {
    GenDesc g{};
    g.key = fnv1a64(r.name.c_str()) ^ splitmix64(seed);
    g.n = r.dev_n;
    g.layout = r.layout;
    if (r.layout == GL_CONV_OHWI) {
        g.co = (int)r.shape[0]; g.ci = (int)r.shape[1]; g.kh = (int)r.shape[2];
        g.kw = (int)r.shape[3]; g.ci_pad = r.ci_pad;
    } else if (r.layout == GL_GEGLU_PERM) {
        g.half_rows = (int)(r.shape[0] / 2);
        g.cols = r.shape.size() > 1 ? (int)r.shape[1] : 1;
    }
    if (r.kind == WK_CONV || r.kind == WK_LINEAR || r.kind == WK_EMBED) { g.mean = 0.0; g.stdv = wstd; }
    else if (!affine) { g.constant = 1; g.mean = (r.kind == WK_NORM_W) ? 1.0 : 0.0; }
    else { g.mean = (r.kind == WK_NORM_W) ? 1.0 : 0.0; g.stdv = 0.02; }
    hipError_t e = gen_launch(r.dev, g, c.stream);
    if (e != hipSuccess) return set_err(&c, SDU_ERR_HIP, std::string("weight generator: ") + hipGetErrorString(e));
    return SDU_OK;
}

int init_weights_seeded(Ctx& c) {
    const bool affine = (c.flags & SDU_INIT_RANDOM_AFFINE) != 0;
    for (const WeightRec& r : c.weights) {
        int st = gen_weight(c, r, c.seed, affine, 0.02);
        if (st) return st;
    }
    return fold_weights(c);
}

// canonical fp16 bits -> device layout, upload
static int upload_canonical_f16(Ctx& c, const WeightRec& r, const uint16_t* canon) {
    std::vector<uint16_t> dev((size_t)r.dev_n);
    for (int64_t i = 0; i < r.dev_n; ++i) {
        const int64_t ci = dev_to_canon_index(r, i);
        dev[(size_t)i] = ci < 0 ? 0 : canon[ci];
    }
    hipError_t e = hipMemcpy(r.dev, dev.data(), dev.size() * 2, hipMemcpyHostToDevice);
    if (e != hipSuccess) return set_err(&c, SDU_ERR_HIP, hipGetErrorString(e));
    return SDU_OK;
}

int load_weight_file(Ctx& c, const WeightRec& r, const std::string& dir) {
    const std::string path = dir + "/" + r.name + ".bin";
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) return set_err(&c, SDU_ERR_WEIGHT, "weight missing: " + path);
    const int64_t sz = (int64_t)f.tellg();
    const int64_t n = r.numel();
    if (sz != n * 2)
        return set_err(&c, SDU_ERR_WEIGHT, "weight size mismatch: " + path + " has " + std::to_string(sz) +
                                               " bytes, expected " + std::to_string(n * 2));
    std::vector<uint16_t> raw((size_t)n);
    f.seekg(0);
    if (!f.read((char*)raw.data(), n * 2)) return set_err(&c, SDU_ERR_IO, "read failed: " + path);
    std::vector<uint16_t> canon;
    const uint16_t* src = raw.data();
    if (r.kind == WK_LINEAR) {
        // the reference stores Linear weights [in, out] (vk_engine.cpp:653, :629)
        const int64_t out = r.shape[0], in = r.shape[1];
        canon.resize((size_t)n);
        for (int64_t i = 0; i < in; ++i)
            for (int64_t o = 0; o < out; ++o) canon[(size_t)(o * in + i)] = raw[(size_t)(i * out + o)];
        src = canon.data();
    }
    return upload_canonical_f16(c, r, src);
}

int init_weights_dir(Ctx& c, const std::string& dir) {
    for (const WeightRec& r : c.weights) {
        int st = load_weight_file(c, r, dir);
        if (st) return st;
    }
    return fold_weights(c);
}

int AuxNet::add(const std::string& name, std::vector<int64_t> shape, int kind, int layout, int ci_pad,
                bool follows) {
    WeightRec r;
    r.name = name;
    r.shape = std::move(shape);
    r.kind = kind;
    r.layout = layout;
    r.ci_pad = ci_pad;
    r.dev_n = layout == GL_CONV_OHWI ? r.shape[0] * r.shape[2] * r.shape[3] * ci_pad : r.numel();
    widx[name] = (int)weights.size();
    weights.push_back(r);
    contig.push_back(follows ? 1 : 0);
    return (int)weights.size() - 1;
}

int aux_alloc(Ctx& c, AuxNet& n, size_t extra_bytes) {
    auto align = [](int64_t v) { return (v + 127) & ~(int64_t)127; };
    std::vector<int64_t> off(n.weights.size());
    int64_t top = 0;
    for (size_t i = 0; i < n.weights.size(); ++i) {
        if (n.contig[i] && i > 0) {
            off[i] = off[i - 1] + n.weights[i - 1].dev_n;
            top = std::max(top, align(off[i] + n.weights[i].dev_n));
        } else {
            off[i] = top;
            top += align(n.weights[i].dev_n);
        }
    }
    n.pool_bytes = (size_t)top * sizeof(f16) + extra_bytes;
    if (hipMalloc(&n.pool, n.pool_bytes) != hipSuccess) return set_err(&c, SDU_ERR_OOM, "weight pool allocation failed");
    for (size_t i = 0; i < n.weights.size(); ++i) n.weights[i].dev = n.pool + off[i];
    return SDU_OK;
}

int set_weight_canonical(Ctx& c, const WeightRec& r, const float* data) {
    std::vector<uint16_t> h((size_t)r.numel());
    for (size_t i = 0; i < h.size(); ++i) {
        f16 v = (f16)data[i];
        memcpy(&h[i], &v, 2);
    }
    return upload_canonical_f16(c, r, h.data());
}

int get_weight_canonical(Ctx& c, const WeightRec& r, float* out) {
    std::vector<uint16_t> dev((size_t)r.dev_n);
    hipError_t e = hipMemcpy(dev.data(), r.dev, dev.size() * 2, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return set_err(&c, SDU_ERR_HIP, hipGetErrorString(e));
    for (int64_t i = 0; i < r.dev_n; ++i) {
        const int64_t ci = dev_to_canon_index(r, i);
        if (ci < 0) continue;
        f16 v;
        memcpy(&v, &dev[(size_t)i], 2);
        out[ci] = (float)v;
    }
    return SDU_OK;
}

int ensure_op_ws(Ctx& c, size_t bytes) {
    if (bytes <= c.op_ws_bytes) return SDU_OK;
    if (c.op_ws) {
        hipStreamSynchronize(c.stream);
        hipFree(c.op_ws);
        c.op_ws = nullptr;
        c.op_ws_bytes = 0;
    }
    if (hipMalloc(&c.op_ws, bytes) != hipSuccess) return set_err(&c, SDU_ERR_OOM, "op workspace allocation failed");
    c.op_ws_bytes = bytes;
    return SDU_OK;
}

}  // namespace sdu
