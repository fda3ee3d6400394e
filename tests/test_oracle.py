"""CPU tests that pin the oracle (no GPU).

* reference fixtures app/src/main/assets/rb|tf (real SD1.5 block I/O exported from
  PyTorch, VulkanBench.kt:39-64) -- run only where /root/reference is mounted;
* closed forms (time projection, LCM schedule constants, consistency of the LCM
  update), brute-force loops on tiny inputs, structural invariants of the graph
  (parameter count, op census of tools/op_coverage_report.md:51);
* mutation checks: plausible mistakes planted in the oracle must fail a check.
"""
import math
import os

import numpy as np
import pytest
import torch

from conftest import REFERENCE, rel_err_l1
from oracle import lcm, unet_ref as U, weights as Wt

ASSETS = os.path.join(REFERENCE, "app/src/main/assets")
need_ref = pytest.mark.skipif(not os.path.isdir(ASSETS), reason="reference fixtures not mounted")


def _ld(d, n, shape=None):
    a = np.fromfile(os.path.join(ASSETS, d, n + ".bin"), dtype="<f2").astype(np.float32)
    return torch.from_numpy(a.reshape(shape) if shape else a)


def _rb_params():
    C = 320
    pf = "rb"
    p = {pf + ".norm1.weight": _ld("rb", "norm1_w"), pf + ".norm1.bias": _ld("rb", "norm1_b"),
         pf + ".conv1.weight": _ld("rb", "conv1_w", (C, C, 3, 3)), pf + ".conv1.bias": _ld("rb", "conv1_b"),
         pf + ".time_emb_proj.weight": _ld("rb", "tproj_w", (C, 1280)),
         pf + ".time_emb_proj.bias": _ld("rb", "tproj_b"),
         pf + ".norm2.weight": _ld("rb", "norm2_w"), pf + ".norm2.bias": _ld("rb", "norm2_b"),
         pf + ".conv2.weight": _ld("rb", "conv2_w", (C, C, 3, 3)), pf + ".conv2.bias": _ld("rb", "conv2_b")}
    return p


def _tf_params(linear_in_out=True):
    """tf/ Linear files are [in, out] (the engine's layout); ``linear_in_out=False``
    plants the mistake of reading them as [out, in]."""
    C = 320
    pf, b = "tf", "tf.transformer_blocks.0"

    def io(n, i, o):
        a = _ld("tf", n, (i, o))
        return a.T.contiguous() if linear_in_out else a.reshape(o, i)

    t = {pf + ".norm.weight": _ld("tf", "gn_w"), pf + ".norm.bias": _ld("tf", "gn_b"),
         pf + ".proj_in.weight": _ld("tf", "pin_w", (C, C, 1, 1)), pf + ".proj_in.bias": _ld("tf", "pin_b"),
         pf + ".proj_out.weight": _ld("tf", "pout_w", (C, C, 1, 1)), pf + ".proj_out.bias": _ld("tf", "pout_b")}
    for i, (n, nb) in enumerate([("n1_w", "n1_b"), ("n2_w", "n2_b"), ("n3_w", "n3_b")]):
        t[f"{b}.norm{i + 1}.weight"] = _ld("tf", n)
        t[f"{b}.norm{i + 1}.bias"] = _ld("tf", nb)
    t[b + ".attn1.to_q.weight"] = io("q1", C, C)
    t[b + ".attn1.to_k.weight"] = io("k1", C, C)
    t[b + ".attn1.to_v.weight"] = io("v1", C, C)
    t[b + ".attn1.to_out.0.weight"] = io("o1", C, C)
    t[b + ".attn1.to_out.0.bias"] = _ld("tf", "o1_b")
    t[b + ".attn2.to_q.weight"] = io("q2", C, C)
    t[b + ".attn2.to_k.weight"] = io("k2", 768, C)
    t[b + ".attn2.to_v.weight"] = io("v2", 768, C)
    t[b + ".attn2.to_out.0.weight"] = io("o2", C, C)
    t[b + ".attn2.to_out.0.bias"] = _ld("tf", "o2_b")
    t[b + ".ff.net.0.proj.weight"] = io("geglu", C, 8 * C)
    t[b + ".ff.net.0.proj.bias"] = _ld("tf", "geglu_b")
    t[b + ".ff.net.2.weight"] = io("ffout", 4 * C, C)
    t[b + ".ff.net.2.bias"] = _ld("tf", "ffout_b")
    return t


# ------------------------------------------------------------------ fixtures


@need_ref
def test_resnet_block_matches_reference_fixture():
    """rb/y.bin = diffusers ResnetBlock2D(down_blocks.0.resnets.0) output (fp16)."""
    p = _rb_params()
    x = _ld("rb", "x", (1, 320, 64, 64))
    temb = _ld("rb", "temb", (1280,))
    with torch.no_grad():
        got = U.resnet(p, "rb", x, temb)
    e = rel_err_l1(got, _ld("rb", "y"))
    assert e < 5e-4, e  # measured 2.31e-4: the fixture's fp16 rounding floor
    # rb/tproj_wT is the [in,out] copy of the diffusers [out,in] weight
    assert torch.equal(_ld("rb", "tproj_wT", (1280, 320)), p["rb.time_emb_proj.weight"].T)


@need_ref
def test_transformer_block_matches_reference_fixture():
    """tf/y.bin = diffusers Transformer2DModel(down_blocks.0.attentions.0) output."""
    x = _ld("tf", "x", (1, 320, 64, 64))
    ctx = _ld("tf", "ctx", (1, 77, 768))
    with torch.no_grad():
        got = U.transformer(_tf_params(), "tf", x, ctx)
    e = rel_err_l1(got, _ld("tf", "y"))
    assert e < 5e-4, e  # measured 2.60e-4


@need_ref
def test_fixture_checks_catch_planted_mistakes():
    """Mistakes planted in the oracle must break the fixture match."""
    x = _ld("tf", "x", (1, 320, 64, 64))
    ctx = _ld("tf", "ctx", (1, 77, 768))
    y = _ld("tf", "y")
    with torch.no_grad():
        wrong_layout = U.transformer(_tf_params(linear_in_out=False), "tf", x, ctx)
    assert rel_err_l1(wrong_layout, y) > 0.1
    # GEGLU halves swapped (gate <-> hidden)
    orig = U.geglu
    try:
        U.geglu = lambda g: orig(torch.cat([g[..., g.shape[-1] // 2:], g[..., :g.shape[-1] // 2]], -1))
        with torch.no_grad():
            swapped = U.transformer(_tf_params(), "tf", x, ctx)
    finally:
        U.geglu = orig
    assert rel_err_l1(swapped, y) > 1e-2
    # ResNet: time embedding without the SiLU
    p = _rb_params()
    xr = _ld("rb", "x", (1, 320, 64, 64))
    temb = _ld("rb", "temb", (1280,))
    orig_silu = U.silu
    try:
        calls = {"n": 0}

        def silu_skip_temb(t):
            calls["n"] += 1
            return t if t.dim() == 1 else orig_silu(t)
        U.silu = silu_skip_temb
        with torch.no_grad():
            bad = U.resnet(p, "rb", xr, temb)
    finally:
        U.silu = orig_silu
    assert rel_err_l1(bad, _ld("rb", "y")) > 1e-3


# ------------------------------------------------------------------ closed forms


def test_time_proj_closed_form():
    """VulkanUnetPipeline.kt:36-46: cos(t f_i) | sin(t f_i), f_i = 1e4^(-i/160)."""
    tp = lcm.time_proj(999)
    assert tp.shape == (320,)
    assert abs(tp[0] - math.cos(999.0)) < 1e-7 and abs(tp[160] - math.sin(999.0)) < 1e-7
    f1 = 10000.0 ** (-1 / 160)
    assert abs(tp[1] - math.cos(999 * f1)) < 1e-6
    np.testing.assert_allclose(tp[:3], [0.9996499, 0.802681, -0.278114], atol=2e-6)
    np.testing.assert_allclose(tp[160:163], [-0.0264608, 0.5964086, -0.9605481], atol=2e-6)
    assert np.all(lcm.time_proj(0)[:160] == 1) and np.all(lcm.time_proj(0)[160:] == 0)


def test_lcm_schedule_constants():
    """LcmScheduler.kt:25-46 -- timesteps and alphas_cumprod (closed form)."""
    s = lcm.LcmSchedule(4)
    assert s.timesteps == [999, 759, 499, 259]
    ac = [s.alphas_cumprod[t] for t in s.timesteps]
    np.testing.assert_allclose(ac, [0.0046600985, 0.0522129283, 0.2776696505, 0.6589755269], rtol=1e-8)
    # scaled-linear betas: product form from the definition
    betas = np.linspace(0.00085 ** 0.5, 0.012 ** 0.5, 1000, dtype=np.float64) ** 2
    np.testing.assert_allclose(s.alphas_cumprod, np.cumprod(1 - betas), rtol=1e-12)
    c = s.coeffs(0)
    st = 9990.0
    assert abs(c["c_skip"] - 0.25 / (st * st + 0.25)) < 1e-18
    assert abs(c["c_out"] - st / math.sqrt(st * st + 0.25)) < 1e-15
    assert lcm.LcmSchedule(1).timesteps == [999]
    assert lcm.LcmSchedule(8).timesteps[:3] == [999, 879, 759]


def test_lcm_step_recovers_clean_sample():
    """If x = sqrt(a) x0 + sqrt(1-a) eps and the model predicts eps exactly, the
    x0 estimate is exact, so the last step returns c_out x0 + c_skip x."""
    s = lcm.LcmSchedule(4)
    rng = np.random.default_rng(0)
    x0 = rng.standard_normal(1000)
    eps = rng.standard_normal(1000)
    for idx in range(4):
        c = s.coeffs(idx)
        x = c["sqrt_alpha"] * x0 + c["sqrt_beta"] * eps
        noise = rng.standard_normal(1000)
        out = s.step(idx, x.astype(np.float32), eps.astype(np.float32), noise.astype(np.float32))
        den = c["c_out"] * x0 + c["c_skip"] * x
        ref = den if c["last"] else c["sqrt_alpha_prev"] * den + c["sqrt_beta_prev"] * noise
        np.testing.assert_allclose(out, ref, rtol=2e-4, atol=2e-5)


def test_cfg_combine():
    c = np.array([1.0, 2.0], np.float32)
    u = np.array([0.5, -1.0], np.float32)
    np.testing.assert_array_equal(lcm.cfg_combine(c, u, 1.0), c)
    np.testing.assert_array_equal(lcm.cfg_combine(c, u, 0.0), u)
    np.testing.assert_allclose(lcm.cfg_combine(c, u, 8.0), u + 8 * (c - u))


# ------------------------------------------------------------------ brute force


def test_conv2d_brute_force():
    rng = np.random.default_rng(1)
    for stride, ups in ((1, False), (2, False), (1, True)):
        x = rng.standard_normal((2, 3, 5, 6)).astype(np.float32)
        w = rng.standard_normal((4, 3, 3, 3)).astype(np.float32)
        b = rng.standard_normal(4).astype(np.float32)
        xin = x.repeat(2, 2).repeat(2, 3) if ups else x
        got = (U.conv2d(U.upsample2x(torch.from_numpy(x)), torch.from_numpy(w), torch.from_numpy(b))
               if ups else U.conv2d(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b),
                                    stride=stride, pad=1)).numpy()
        B, C, H, W = xin.shape
        Ho, Wo = (H + 2 - 3) // stride + 1, (W + 2 - 3) // stride + 1
        ref = np.zeros((B, 4, Ho, Wo))
        for bb in range(B):
            for o in range(4):
                for oy in range(Ho):
                    for ox in range(Wo):
                        s = b[o]
                        for ci in range(C):
                            for ky in range(3):
                                for kx in range(3):
                                    iy, ix = oy * stride + ky - 1, ox * stride + kx - 1
                                    if 0 <= iy < H and 0 <= ix < W:
                                        s += xin[bb, ci, iy, ix] * w[o, ci, ky, kx]
                        ref[bb, o, oy, ox] = s
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_group_norm_brute_force():
    """groupnorm_silu.comp:13-31 statistics per (image, group)."""
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((2, 8, 3, 5)) * 3 + 1).astype(np.float32)
    g = rng.standard_normal(8).astype(np.float32)
    b = rng.standard_normal(8).astype(np.float32)
    got = U.group_norm(torch.from_numpy(x), torch.from_numpy(g), torch.from_numpy(b), groups=4,
                       act_silu=True).numpy()
    ref = np.empty_like(x, dtype=np.float64)
    for bb in range(2):
        for gi in range(4):
            sl = x[bb, gi * 2:(gi + 1) * 2].astype(np.float64)
            m, v = sl.mean(), ((sl - sl.mean()) ** 2).mean()
            for c in range(gi * 2, gi * 2 + 2):
                z = (x[bb, c] - m) / math.sqrt(v + 1e-5) * g[c] + b[c]
                ref[bb, c] = z / (1 + np.exp(-z))
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_layer_norm_and_geglu_brute_force():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((3, 16)) * 2 + 0.5).astype(np.float32)
    g = rng.standard_normal(16).astype(np.float32)
    b = rng.standard_normal(16).astype(np.float32)
    got = U.layer_norm(torch.from_numpy(x), torch.from_numpy(g), torch.from_numpy(b)).numpy()
    for t in range(3):
        m = x[t].astype(np.float64).mean()
        v = ((x[t] - m) ** 2).mean()
        np.testing.assert_allclose(got[t], (x[t] - m) / math.sqrt(v + 1e-5) * g + b, rtol=1e-5, atol=1e-5)
    gg = rng.standard_normal((2, 8)).astype(np.float32)
    out = U.geglu(torch.from_numpy(gg)).numpy()
    for t in range(2):
        for c in range(4):
            a, bb = gg[t, c], gg[t, 4 + c]
            assert abs(out[t, c] - a * 0.5 * bb * (1 + math.erf(bb / math.sqrt(2)))) < 1e-6


def test_attention_brute_force():
    """Two-pass softmax per query, as the reference's CPU check (vk_engine.cpp:1095-1103)."""
    rng = np.random.default_rng(4)
    B, Sq, Sk, heads, d = 2, 5, 7, 2, 4
    q = rng.standard_normal((B, Sq, heads * d)).astype(np.float32)
    k = rng.standard_normal((B, Sk, heads * d)).astype(np.float32)
    v = rng.standard_normal((B, Sk, heads * d)).astype(np.float32)
    got = U.attention(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), heads, q_chunk=2).numpy()
    for b in range(B):
        for h in range(heads):
            for i in range(Sq):
                s = [float(np.dot(q[b, i, h * d:(h + 1) * d], k[b, j, h * d:(h + 1) * d])) / math.sqrt(d)
                     for j in range(Sk)]
                m = max(s)
                p = [math.exp(x - m) for x in s]
                den = sum(p)
                o = sum(p[j] * v[b, j, h * d:(h + 1) * d] for j in range(Sk)) / den
                np.testing.assert_allclose(got[b, i, h * d:(h + 1) * d], o, rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------ structure


def test_parameter_inventory():
    ps = Wt.param_specs()
    assert sum(p.numel for p in ps) == 859_520_964  # SD1.5 UNet2DConditionModel
    assert len(ps) == 686
    assert len({p.name for p in ps}) == len(ps)
    assert Wt.skip_channels() == [320, 320, 320, 320, 640, 640, 640, 1280, 1280, 1280, 1280, 1280]


def test_op_census_matches_reference_report():
    """tools/op_coverage_report.md:51: FULLY_CONNECTED x184, CONV_2D x98, BATCH_MATMUL x64."""
    seen = {"linear": 0, "conv": 0, "bmm": 0}
    lin, conv, att = U.linear, U.conv2d, U.attention

    def c_lin(*a, **k):
        seen["linear"] += 1
        return lin(*a, **k)

    def c_conv(*a, **k):
        seen["conv"] += 1
        return conv(*a, **k)

    def c_att(*a, **k):
        seen["bmm"] += 2
        return att(*a, **k)
    names = {p.name: p for p in Wt.param_specs()}
    p = {n: torch.zeros(s.shape) for n, s in names.items()}
    try:
        U.linear, U.conv2d, U.attention = c_lin, c_conv, c_att
        with torch.no_grad():
            U.unet_forward(p, np.zeros((1, 4, 8, 8), np.float32), np.zeros(320, np.float32),
                           np.zeros((1, 77, 768), np.float32))
    finally:
        U.linear, U.conv2d, U.attention = lin, conv, att
    assert seen == {"linear": 184, "conv": 98, "bmm": 64}


def test_batch_duplicate_and_context_sensitivity():
    """B=2 with the same input in both slots gives identical images
    (vk_engine.cpp:823-839); different contexts give different eps (:840-849)."""
    w = Wt.generate(7, names=None)
    p = U.to_torch(w)
    lat = Wt.gauss("t.lat", (1, 4, 16, 16), 1, fp16=False)
    ctx = Wt.gauss("t.ctx", (2, 77, 768), 1, fp16=False)
    tp = lcm.time_proj(999)
    with torch.no_grad():
        y2 = U.unet_forward(p, np.concatenate([lat, lat]), tp, np.stack([ctx[0], ctx[0]])).numpy()
        yc = U.unet_forward(p, np.concatenate([lat, lat]), tp, ctx).numpy()
    # torch's CPU kernels may block the two images differently: equal to fp32 rounding
    assert rel_err_l1(y2[1], y2[0]) < 1e-6
    assert np.abs(yc[0] - yc[1]).mean() > 1e-4


# ------------------------------------------------------------------ generator


def test_generator_distribution_and_determinism():
    a = Wt.gauss("x.weight", (200_000,), 5, 0.0, 0.02)
    b = Wt.gauss("x.weight", (200_000,), 5, 0.0, 0.02)
    c = Wt.gauss("x.weight", (200_000,), 6, 0.0, 0.02)
    d = Wt.gauss("y.weight", (200_000,), 5, 0.0, 0.02)
    assert np.array_equal(a, b) and not np.array_equal(a, c) and not np.array_equal(a, d)
    assert abs(a.mean()) < 3e-4 and abs(a.std() - 0.02) < 3e-4
    # fp16-representable
    assert np.array_equal(a, a.astype(np.float16).astype(np.float32))
    # tails of a normal: P(|z| > 3) = 0.27%
    frac = (np.abs(a) > 0.06).mean()
    assert 0.0020 < frac < 0.0034
    # Box-Muller from the documented hash: element 0 recomputed in Python
    key = Wt.tensor_key("x.weight", 5)

    def mix(x):
        x = (x + 0x9E3779B97F4A7C15) & (2**64 - 1)
        x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & (2**64 - 1)
        x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & (2**64 - 1)
        return x ^ (x >> 31)
    h = 0xCBF29CE484222325  # fnv1a64 of the tensor name
    for ch in b"x.weight":
        h = ((h ^ ch) * 0x100000001B3) & (2**64 - 1)
    assert h ^ mix(5) == key
    for i in (0, 1, 12345):
        h1, h2 = mix((key + 2 * i) & (2**64 - 1)), mix((key + 2 * i + 1) & (2**64 - 1))
        u1 = ((h1 >> 11) + 1) * 2.0 ** -53
        u2 = (h2 >> 11) * 2.0 ** -53
        z = math.sqrt(-2 * math.log(u1)) * math.cos(2 * math.pi * u2)
        assert np.float32(np.float16(np.float32(0.02 * z))) == a[i]
