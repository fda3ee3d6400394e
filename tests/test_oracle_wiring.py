"""CPU checks that pin the oracle's graph wiring (no GPU).

The block functions of oracle/unet_ref.py are pinned by the reference's rb/ and tf/
fixtures and by brute force (test_oracle.py).  The choices made only at graph level
are pinned here, each by weights or inputs whose result the mathematics fixes, and
each check is shown to fail on a plausible mistake planted in a copy of the oracle:

* the SiLU between time_embedding.linear_1 and linear_2 (vk_engine.cpp:716-717);
* the up-path concat: previous output first, then the LIFO skip
  (vk_engine.cpp:678-688 used at :752-753; skips pushed at :720-742);
* the SiLU on conv_norm_out before conv_out (vk_engine.cpp:781-782);
* the GroupNorm census: 45 GroupNorm+SiLU and 16 plain GroupNorm per forward
  (groupnorm_silu at :625, :631, :781; groupnorm at :643);
* the CFG orientation u + s (c - u), the timestep sequence and the per-step noise of
  the denoise loop (VulkanUnetPipeline.kt:79-90);
* the downsample / upsample blocks (:689-697) against explicit loops.
"""
import math

import numpy as np
import pytest
import torch

from conftest import rel_err_l1
from oracle import lcm, unet_ref as U, weights as Wt

SILU_MIN = -0.2784645427610738  # min_z z / (1 + e^-z), at z = -1.2784645...


@pytest.fixture(scope="module")
def params():
    return U.to_torch(Wt.generate(7))


def _small_inputs(H=8, W=8, seed=3):
    lat = Wt.gauss("t.lat", (1, 4, H, W), seed, fp16=False)
    ctx = Wt.gauss("t.ctx", (1, 77, 768), seed, fp16=False)
    return lat, lcm.time_proj(999), ctx


class Recorder:
    """Wraps the oracle's block functions to record, in call order, each block's
    prefix, inputs and output while unet_forward runs."""

    NAMES = ("resnet", "transformer", "downsample", "upsample")

    def __init__(self):
        self.log = []
        self.orig = {}

    def __enter__(self):
        for n in self.NAMES:
            f = getattr(U, n)
            self.orig[n] = f

            def wrap(*a, _f=f, _n=n, **k):
                out = _f(*a, **k)
                # (kind, prefix, x, extra, out): resnet(p, pf, x, temb), transformer(p, pf, x, ctx)
                self.log.append((_n, a[1], a[2], a[3] if len(a) > 3 else None, out))
                return out
            setattr(U, n, wrap)
        return self

    def __exit__(self, *exc):
        for n, f in self.orig.items():
            setattr(U, n, f)


# ------------------------------------------------------------------ time MLP


def _time_mlp_params(v):
    """linear_1 maps e_0 to v (column 0 = v, zero bias); linear_2 = -I (zero bias)."""
    w1 = torch.zeros(1280, 320)
    w1[:, 0] = torch.from_numpy(v)
    return {"time_embedding.linear_1.weight": w1, "time_embedding.linear_1.bias": torch.zeros(1280),
            "time_embedding.linear_2.weight": -torch.eye(1280), "time_embedding.linear_2.bias": torch.zeros(1280)}


def _silu64(v):
    return np.array([x / (1.0 + math.exp(-x)) for x in v.astype(np.float64)])


def _time_mlp_check(fn):
    """fn(p, temb_proj) must give -silu(v) for e_0 in: SiLU between the two linears."""
    v = np.linspace(-4.0, 4.0, 1280).astype(np.float32)
    e0 = np.zeros(320, np.float32)
    e0[0] = 1.0
    with torch.no_grad():
        got = fn(_time_mlp_params(v), torch.from_numpy(e0)).numpy()
    return np.abs(got - (-_silu64(v))).max() < 1e-6


def test_time_mlp_silu_between_linears():
    """vk_engine.cpp:716-717: MM(320->1280)+bias, SILU, MM(1280->1280)+bias."""
    assert _time_mlp_check(U.time_mlp)
    L = U.linear
    # planted: no SiLU / SiLU after linear_2 / SiLU on the input
    no_silu = lambda p, t: L(L(t, p["time_embedding.linear_1.weight"], p["time_embedding.linear_1.bias"]),
                             p["time_embedding.linear_2.weight"], p["time_embedding.linear_2.bias"])
    silu_after = lambda p, t: U.silu(no_silu(p, t))
    silu_before = lambda p, t: no_silu(p, U.silu(t))
    for bad in (no_silu, silu_after, silu_before):
        assert not _time_mlp_check(bad)


def test_forward_feeds_time_mlp_to_every_resnet(params):
    """unet_forward passes time_mlp(temb_proj) to all 22 resnets (vk_engine.cpp:716-717,
    :627): with the constructed time MLP, every resnet receives -silu(v)."""
    v = np.linspace(-4.0, 4.0, 1280).astype(np.float32)
    p = dict(params)
    p.update(_time_mlp_params(v))
    lat, _, ctx = _small_inputs()
    e0 = np.zeros(320, np.float32)
    e0[0] = 1.0
    with Recorder() as rec, torch.no_grad():
        U.unet_forward(p, lat, e0, ctx)
    tembs = [e for k, _, _, e, _ in rec.log if k == "resnet"]
    assert len(tembs) == 22
    for t in tembs:
        assert np.abs(t.numpy() - (-_silu64(v))).max() < 1e-6


# ------------------------------------------------------------------ skip concat


def _down_skips(log):
    """Skip tensors in push order (vk_engine.cpp:720-742): conv_in's output (the first
    resnet's input), then every down resnet / transformer output and downsample output."""
    first = next(x for k, pf, x, _, _ in log if k == "resnet")
    skips = [first]
    for k, pf, x, _, out in log:
        if pf.startswith("down_blocks") and (k in ("downsample",) or
                                             (k == "resnet" and pf.startswith("down_blocks.3")) or
                                             k == "transformer"):
            skips.append(out)
    return skips


def _concat_ok(log):
    skips = _down_skips(log)
    assert [s.shape[1] for s in skips] == Wt.skip_channels()
    ups = [i for i, (k, pf, *_r) in enumerate(log) if k == "resnet" and pf.startswith("up_blocks")]
    assert len(ups) == 12
    for j, i in enumerate(ups):
        x_in, prev = log[i][2], log[i - 1][4]
        skip = skips[len(skips) - 1 - j]
        cp = prev.shape[1]
        if x_in.shape[1] != cp + skip.shape[1]:
            return False
        if not (torch.equal(x_in[:, :cp], prev) and torch.equal(x_in[:, cp:], skip)):
            return False
    return True


def test_up_path_concat_is_previous_then_lifo_skip(params):
    """Each up resnet's input is cat(previous output, skip) with skips popped LIFO
    (vk_engine.cpp:721, :748-753).  Checked channel block by channel block, exactly;
    a planted skip-first concat fails."""
    lat, temb, ctx = _small_inputs()
    with Recorder() as rec, torch.no_grad():
        U.unet_forward(params, lat, temb, ctx)
    assert _concat_ok(rec.log)
    # planted: skip first.  The channel counts then differ from the weights of most
    # up resnets, so only the first (1280 + 1280 channels) runs; its input must fail.
    orig_cat = torch.cat
    orig_res = U.resnet

    class Stop(Exception):
        pass

    def cat_swapped(ts, dim=0):
        if dim == 1 and len(ts) == 2:
            return orig_cat([ts[1], ts[0]], dim=1)
        return orig_cat(ts, dim=dim)
    seen = []

    def res_first_up(p, pf, x, temb):
        if pf.startswith("up_blocks"):
            seen.append(x)
            raise Stop()
        return orig_res(p, pf, x, temb)
    try:
        torch.cat = cat_swapped
        U.resnet = res_first_up
        with Recorder() as rec2, torch.no_grad():
            with pytest.raises(Stop):
                U.unet_forward(params, lat, temb, ctx)
    finally:
        torch.cat = orig_cat
        U.resnet = orig_res
    mid = [r for r in rec.log if r[1] == "mid_block.resnets.1"][0][4]
    assert len(seen) == 1 and not torch.equal(seen[0][:, :1280], mid)
    del rec2


def test_up_concat_weight_semantics(params):
    """The weight files index the concat's input channels prev-first (diffusers'
    cat([hidden, res_hidden])).  With up_blocks.0.resnets.0's conv2 zeroed and its 1x1
    shortcut = [I | 0], the block returns its previous input (the mid block's output)
    exactly; a planted skip-first concat returns the skip instead and fails."""
    pf = "up_blocks.0.resnets.0"
    p = dict(params)
    p[pf + ".conv2.weight"] = torch.zeros_like(p[pf + ".conv2.weight"])
    p[pf + ".conv2.bias"] = torch.zeros(1280)
    sc = torch.zeros(1280, 2560, 1, 1)
    sc[:, :1280, 0, 0] = torch.eye(1280)
    p[pf + ".conv_shortcut.weight"] = sc
    p[pf + ".conv_shortcut.bias"] = torch.zeros(1280)
    lat, temb, ctx = _small_inputs(seed=4)

    def run():
        with Recorder() as rec, torch.no_grad():
            U.unet_forward(p, lat, temb, ctx)
        i = next(i for i, r in enumerate(rec.log) if r[1] == pf)
        return rec.log[i][4], rec.log[i - 1][4]  # block output, mid block output

    out, mid = run()
    assert torch.equal(out, mid)
    # planted: skip first
    orig_cat = torch.cat
    try:
        def cat_swapped(ts, dim=0):
            if dim == 1 and len(ts) == 2:
                return orig_cat([ts[1], ts[0]], dim=1)
            return orig_cat(ts, dim=dim)
        torch.cat = cat_swapped
        out_bad, mid_bad = run()
    finally:
        torch.cat = orig_cat
    assert not torch.equal(out_bad, mid_bad)


# ------------------------------------------------------------------ conv_norm_out


def _conv_out_probe(p):
    """conv_out = centre taps: out0 = y0, out1 = -y0, out2 = y5, out3 = 0 (y = the
    normalised, activated input of conv_out)."""
    w = torch.zeros(4, 320, 3, 3)
    w[0, 0, 1, 1] = 1.0
    w[1, 0, 1, 1] = -1.0
    w[2, 5, 1, 1] = 1.0
    q = dict(p)
    q["conv_out.weight"] = w
    q["conv_out.bias"] = torch.zeros(4)
    return q


def test_conv_norm_out_has_silu(params):
    """vk_engine.cpp:781: GN_SILU before conv_out.  Every output of the centre-tap
    probe is a SiLU value, so it is >= min(SiLU) = -0.27846; without the SiLU the
    normalised values (zero mean, unit variance per group) go far below."""
    q = _conv_out_probe(params)
    lat, temb, ctx = _small_inputs(16, 16, seed=5)
    with torch.no_grad():
        y = U.unet_forward(q, lat, temb, ctx).numpy()
    assert y[:, 0].min() >= SILU_MIN - 1e-6 and y[:, 2].min() >= SILU_MIN - 1e-6
    assert y[:, 1].max() <= -SILU_MIN + 1e-6
    assert np.all(y[:, 3] == 0)
    assert y[:, 0].min() < 0  # some inputs are negative: the bound is attained from above
    orig = U.group_norm

    def gn_no_silu_at_end(x, g, b, groups=U.GN_GROUPS, eps=U.EPS, act_silu=False):
        if x.shape[1] == 320 and g is q["conv_norm_out.weight"]:
            act_silu = False
        return orig(x, g, b, groups, eps, act_silu)
    try:
        U.group_norm = gn_no_silu_at_end
        with torch.no_grad():
            bad = U.unet_forward(q, lat, temb, ctx).numpy()
    finally:
        U.group_norm = orig
    assert bad[:, 0].min() < SILU_MIN - 0.5


def test_groupnorm_census():
    """61 GroupNorms per forward: 45 with SiLU (two per resnet and conv_norm_out,
    vk_engine.cpp:625, :631, :781) and 16 plain (one per transformer, :643)."""
    seen = {True: 0, False: 0}
    orig = U.group_norm

    def count(x, g, b, groups=U.GN_GROUPS, eps=U.EPS, act_silu=False):
        seen[bool(act_silu)] += 1
        return orig(x, g, b, groups, eps, act_silu)
    p = {s.name: torch.zeros(s.shape) for s in Wt.param_specs()}
    for s in Wt.param_specs():
        if s.kind == "norm_w":
            p[s.name] = torch.ones(s.shape)
    try:
        U.group_norm = count
        with torch.no_grad():
            U.unet_forward(p, np.zeros((1, 4, 8, 8), np.float32), np.zeros(320, np.float32),
                           np.zeros((1, 77, 768), np.float32))
    finally:
        U.group_norm = orig
    assert seen == {True: 45, False: 16}


# ------------------------------------------------------------------ denoise loop


def _fake_model(calls):
    """A stand-in UNet for the loop: eps of image i = mean(ctx[i]) everywhere, so cond
    (ctx 1) gives 1 and uncond (ctx 0) gives 0; records (latent pair, temb)."""
    def f(p, lat, temb, ctx):
        calls.append((np.asarray(lat).copy(), np.asarray(temb).copy()))
        m = ctx.reshape(ctx.shape[0], -1).mean(1)
        return torch.from_numpy(np.asarray(lat, np.float32)) * 0 + m[:, None, None, None]
    return f


def _denoise_expect(lat, guidance, noise, steps=4):
    """The loop's closed form for eps = 0 + s (1 - 0) = s at every step."""
    sched = lcm.LcmSchedule(steps)
    x = lat.astype(np.float64)
    for idx in range(steps):
        c = sched.coeffs(idx)
        x0 = (x - c["sqrt_beta"] * guidance) / c["sqrt_alpha"]
        den = c["c_out"] * x0 + c["c_skip"] * x
        x = den if c["last"] else c["sqrt_alpha_prev"] * den + c["sqrt_beta_prev"] * noise[idx]
        x = x.astype(np.float32).astype(np.float64)
    return x


def test_denoise_loop_cfg_orientation_and_noise():
    """VulkanUnetPipeline.kt:79-90: per step t in [999, 759, 499, 259], the latent in
    both slots with temb = timeProj(t), eps = u + s (c - u) with slot 0 = cond, and
    noise[idx] added after step idx (none after the last)."""
    steps, g = 4, 8.0
    rng = np.random.default_rng(0)
    lat = rng.standard_normal((4, 8, 8)).astype(np.float32)
    noise = np.stack([np.full((4, 8, 8), i + 1.0, np.float32) for i in range(steps - 1)])
    cond, unc = np.ones((77, 768), np.float32), np.zeros((77, 768), np.float32)
    orig = U.unet_forward
    calls = []
    try:
        U.unet_forward = _fake_model(calls)
        got = U.denoise_lcm(None, lat, cond, unc, steps, g, noise)
        calls_ok = list(calls)
        # planted: cond / uncond swapped in the combine
        orig_cfg = lcm.cfg_combine
        lcm.cfg_combine = lambda c, u, s: orig_cfg(u, c, s)
        try:
            bad = U.denoise_lcm(None, lat, cond, unc, steps, g, noise)
        finally:
            lcm.cfg_combine = orig_cfg
    finally:
        U.unet_forward = orig
    exp = _denoise_expect(lat, g, noise)
    assert rel_err_l1(got, exp) < 1e-6
    assert rel_err_l1(bad, exp) > 1e-2
    ts = [999, 759, 499, 259]
    assert len(calls_ok) == steps
    for (both, temb), t in zip(calls_ok, ts):
        assert np.array_equal(both[0], both[1])
        assert np.array_equal(temb, lcm.time_proj(t))
    # noise at the wrong step (planted: reversed) changes the result
    bad2 = _denoise_expect(lat, g, noise[::-1])
    assert rel_err_l1(got, bad2) > 1e-3


# ------------------------------------------------------------------ resampling blocks


def _conv_loop(x, w, b, stride):
    B, C, H, W = x.shape
    Co = w.shape[0]
    Ho, Wo = (H - 1) // stride + 1, (W - 1) // stride + 1
    y = np.zeros((B, Co, Ho, Wo))
    for bb in range(B):
        for o in range(Co):
            for oy in range(Ho):
                for ox in range(Wo):
                    s = float(b[o])
                    for ky in range(3):
                        for kx in range(3):
                            iy, ix = oy * stride + ky - 1, ox * stride + kx - 1
                            if 0 <= iy < H and 0 <= ix < W:
                                s += float(np.dot(x[bb, :, iy, ix], w[o, :, ky, kx]))
                    y[bb, o, oy, ox] = s
    return y


def test_resampling_blocks_brute_force():
    """downsample = conv3x3 stride 2 pad 1 (vk_engine.cpp:689-692); upsample = nearest
    2x then conv3x3 (:693-697; upsample_f32.comp:5-11: out[y,x] = in[y/2, x/2])."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((2, 3, 5, 6)).astype(np.float32)
    w = rng.standard_normal((4, 3, 3, 3)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    p = {"d.conv.weight": torch.from_numpy(w), "d.conv.bias": torch.from_numpy(b)}
    with torch.no_grad():
        dn = U.downsample(p, "d", torch.from_numpy(x)).numpy()
        up = U.upsample(p, "d", torch.from_numpy(x)).numpy()
    np.testing.assert_allclose(dn, _conv_loop(x, w, b, 2), rtol=1e-5, atol=1e-5)
    xu = np.empty((2, 3, 10, 12), np.float32)
    for yy in range(10):
        for xx in range(12):
            xu[:, :, yy, xx] = x[:, :, yy // 2, xx // 2]
    np.testing.assert_allclose(up, _conv_loop(xu, w, b, 1), rtol=1e-5, atol=1e-5)


def test_rel_err_l1_closed_form():
    """relErr_L1 = sum|ref - got| / sum|ref| (vk_engine.cpp:698-704, run_ref.py:46)."""
    ref = np.array([1.0, -2.0, 3.0, -4.0])
    got = np.array([1.5, -2.0, 2.0, -4.0])
    assert abs(U.rel_err_l1(got, ref) - 1.5 / 10.0) < 1e-15
    assert U.rel_err_l1(ref, ref) == 0.0
