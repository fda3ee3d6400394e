"""Full-graph parity of the HIP UNet engine against the CPU oracle.

Identical seeded random-init weights are generated on both sides independently
(device generator vs oracle/gen.c, checked equal below) and identical inputs are
fed to both.  Acceptance: relErr_L1 = sum|got-ref| / sum|ref| <= 3e-3 (the
tools/run_ref.py:46 and vk_engine.cpp:698-704 metric).
"""
import os

import numpy as np
import pytest
import torch

from conftest import rel_err_l1, say
from oracle import lcm, unet_ref as U, weights as Wt

pytestmark = pytest.mark.gpu
TOL = 3e-3


def inputs(B, H, W, L=77, seed=11):
    lat = Wt.gauss("input.latent", (B, 4, H, W), seed, fp16=False)
    ctx = Wt.gauss("input.context", (B, L, 768), seed, fp16=False)
    return lat, lcm.time_proj(999), ctx


def oracle_forward(p, lat, temb, ctx):
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    with torch.inference_mode():
        return U.unet_forward(p, lat, temb, ctx).numpy()


def test_generator_matches_oracle(unet_engine):
    """Device generator == oracle generator, bit for bit, across every layout
    (conv OHWI with channel padding, GEGLU row interleave, fused QKV / cross-K/V /
    time-projection blocks)."""
    names = ["conv_in.weight", "conv_in.bias", "time_embedding.linear_1.weight",
             "down_blocks.0.resnets.0.conv1.weight", "down_blocks.0.resnets.0.time_emb_proj.weight",
             "up_blocks.3.resnets.2.time_emb_proj.weight",
             "down_blocks.0.attentions.0.transformer_blocks.0.attn1.to_k.weight",
             "down_blocks.0.attentions.0.transformer_blocks.0.attn1.to_v.weight",
             "up_blocks.1.attentions.2.transformer_blocks.0.attn2.to_v.weight",
             "mid_block.attentions.0.transformer_blocks.0.ff.net.0.proj.weight",
             "up_blocks.3.resnets.0.conv_shortcut.weight", "conv_out.weight",
             "up_blocks.0.upsamplers.0.conv.weight", "conv_norm_out.weight"]
    specs = {p.name: p for p in Wt.param_specs()}
    for n in names:
        say(f"weight {n}")
        got = unet_engine.get_weight(n, specs[n].shape)
        ref = Wt.param_value(specs[n], 1234)
        assert np.array_equal(got, ref), n
    assert unet_engine.param_count() == (859_520_964, 686)


def test_forward_b2_64(unet_engine, oracle_weights):
    """B=2 (cond + uncond stacked), 64x64, fp16: the benchmarked configuration."""
    lat, temb, ctx = inputs(2, 64, 64)
    say("forward B=2 64x64")
    got = unet_engine.forward(lat, temb, ctx)
    ref = oracle_forward(oracle_weights, lat, temb, ctx)
    e = rel_err_l1(got, ref)
    say(f"relErr B=2 64x64 = {e:.3e}")
    assert np.isfinite(got).all()
    assert e <= TOL
    # graph replay is deterministic
    assert np.array_equal(unet_engine.forward(lat, temb, ctx), got)


def test_forward_b1_64(unet_engine, oracle_weights):
    lat, temb, ctx = inputs(1, 64, 64, seed=12)
    say("forward B=1 64x64")
    got = unet_engine.forward(lat, temb, ctx)
    e = rel_err_l1(got, oracle_forward(oracle_weights, lat, temb, ctx))
    say(f"relErr B=1 64x64 = {e:.3e}")
    assert e <= TOL


def test_forward_cfg_slots(unet_engine, oracle_weights):
    """unetForward2 semantics (vk_engine.cpp:891-913): one latent in both slots,
    [cond; uncond] contexts.  Same context in both slots -> identical images
    (vk_engine.cpp:823-839); different contexts -> different eps (:840-849)."""
    lat, temb, ctx = inputs(2, 32, 32, seed=13)
    say("forward_cfg 32x32")
    same = unet_engine.forward_cfg(lat[0], temb, ctx[0], ctx[0])
    assert np.array_equal(same[0], same[1])
    both = unet_engine.forward_cfg(lat[0], temb, ctx[0], ctx[1])
    ref = oracle_forward(oracle_weights, np.stack([lat[0], lat[0]]), temb, ctx)
    assert rel_err_l1(both, ref) <= TOL
    d_gpu = np.abs(both[0] - both[1]).mean()
    d_ref = np.abs(ref[0] - ref[1]).mean()
    say(f"ctx sensitivity gpu={d_gpu:.4e} oracle={d_ref:.4e}")
    assert d_gpu > 0 and abs(d_gpu - d_ref) / d_ref < 0.05


def test_forward_affine_small():
    """Random biases / norm affines (so every bias and affine path carries signal)."""
    import sdu
    eng = sdu.Engine(seed=99, flags=sdu.SDU_INIT_RANDOM_AFFINE)
    try:
        p = U.to_torch(Wt.generate(99, mode="affine"))
        lat, temb, ctx = inputs(2, 16, 24, L=40, seed=14)  # non-square, short context
        temb = lcm.time_proj(259)
        say("forward affine B=2 16x24 L=40")
        got = eng.forward(lat, temb, ctx)
        e = rel_err_l1(got, oracle_forward(p, lat, temb, ctx))
        say(f"relErr affine = {e:.3e}")
        assert e <= TOL
    finally:
        eng.release()


def test_forward_b3_24(unet_engine, oracle_weights):
    """Odd batch and a latent whose levels (576, 144, 36, 9 pixels per image) are not
    multiples of the GEMM row tiles; every level's GroupNorms compute their own
    statistics."""
    lat, temb, ctx = inputs(3, 24, 24, seed=17)
    say("forward B=3 24x24")
    got = unet_engine.forward(lat, temb, ctx)
    e = rel_err_l1(got, oracle_forward(oracle_weights, lat, temb, ctx))
    say(f"relErr B=3 24x24 = {e:.3e}")
    assert e <= TOL


def test_forward_b3_40(unet_engine, oracle_weights):
    """Odd batch at 40x40: the first level (1600 pixels per image) takes GroupNorm
    statistics from the GEMM epilogues, and its 128-row tiles straddle two images
    (1600 = 12.5 x 128), so the epilogue's second-image slot is used."""
    lat, temb, ctx = inputs(3, 40, 40, seed=18)
    say("forward B=3 40x40")
    got = unet_engine.forward(lat, temb, ctx)
    e = rel_err_l1(got, oracle_forward(oracle_weights, lat, temb, ctx))
    say(f"relErr B=3 40x40 = {e:.3e}")
    assert e <= TOL


def test_forward_b2_72x56(unet_engine, oracle_weights):
    """Non-square latent whose levels are 72x56, 36x28, 18x14 and 9x7: the first level
    (4032 pixels, 31.5 row tiles per image) takes its GroupNorm statistics from the GEMM
    epilogues, the bottom level has an odd 63 pixels, and the up path's 2x upsamples must
    land back on 18x14 and 36x28."""
    lat, temb, ctx = inputs(2, 72, 56, seed=19)
    say("forward B=2 72x56")
    got = unet_engine.forward(lat, temb, ctx)
    e = rel_err_l1(got, oracle_forward(oracle_weights, lat, temb, ctx))
    say(f"relErr B=2 72x56 = {e:.3e}")
    assert e <= TOL


@pytest.mark.slow
def test_forward_b2_96(unet_engine, oracle_weights):
    """96x96 latent: 9216-token self-attention at hd 40."""
    lat, temb, ctx = inputs(2, 96, 96, seed=15)
    say("forward B=2 96x96")
    got = unet_engine.forward(lat, temb, ctx)
    e = rel_err_l1(got, oracle_forward(oracle_weights, lat, temb, ctx))
    say(f"relErr B=2 96x96 = {e:.3e}")
    assert e <= TOL


def test_set_weight_refolds(unet_engine, oracle_weights):
    """Folded weights: a transformer's feed-forward output and proj_out run as one
    GEMM, and so do a resnet's conv2 and 1x1 shortcut; the convs after the 2x
    upsamplings run on sub-pixel weights folded from theirs (at a 32x32 latent the 8->16
    and 16->32 upsamplings take that form).  Setting any of their source tensors through
    sdu_set_weight refolds them: the forward matches the oracle run with the same new
    weights."""
    pf = "up_blocks.3.attentions.1"
    rpf = "up_blocks.3.resnets.1"
    names = [pf + ".transformer_blocks.0.ff.net.2.weight", pf + ".transformer_blocks.0.ff.net.2.bias",
             pf + ".proj_out.weight", pf + ".proj_out.bias",
             rpf + ".conv2.weight", rpf + ".conv2.bias", rpf + ".conv_shortcut.weight", rpf + ".conv_shortcut.bias",
             "up_blocks.1.upsamplers.0.conv.weight", "up_blocks.2.upsamplers.0.conv.weight"]
    specs = {p.name: p for p in Wt.param_specs()}
    rng = np.random.default_rng(5)
    p2 = dict(oracle_weights)
    orig = {}
    try:
        for n in names:
            shape = specs[n].shape
            v = (rng.standard_normal(shape) * 0.05).astype(np.float16).astype(np.float32)
            orig[n] = unet_engine.get_weight(n, shape)
            unet_engine.set_weight(n, v)
            p2[n] = torch.from_numpy(v)
        lat, temb, ctx = inputs(1, 32, 32, seed=17)
        say("forward B=1 32x32 after set_weight on folded sources")
        got = unet_engine.forward(lat, temb, ctx)
        e = rel_err_l1(got, oracle_forward(p2, lat, temb, ctx))
        e_old = rel_err_l1(got, oracle_forward(oracle_weights, lat, temb, ctx))
        say(f"relErr new weights = {e:.3e}, vs old weights = {e_old:.3e}")
        assert e <= TOL
        assert e_old > max(TOL, 5 * e)  # the change is visible in the output
    finally:
        for n, v in orig.items():
            unet_engine.set_weight(n, v)


def test_set_weight_refolds_layernorm(unet_engine, oracle_weights):
    """The transformer LayerNorms (norm1 / norm2 / norm3) run inside the GEMMs that
    read them (row statistics from the A tiles, affine folded into the weights).
    Non-trivial scales and shifts and new projection weights, set through
    sdu_set_weight, refold: the forward matches the oracle with the same weights, at
    C = 320, 640 and 1280 (mid block: 16 tokens, rows past M in every tile)."""
    blocks = ["up_blocks.3.attentions.2.transformer_blocks.0", "down_blocks.1.attentions.0.transformer_blocks.0",
              "mid_block.attentions.0.transformer_blocks.0"]
    sufs = ["norm1.weight", "norm1.bias", "norm2.weight", "norm2.bias", "norm3.weight", "norm3.bias",
            "attn1.to_k.weight", "attn2.to_q.weight", "ff.net.0.proj.weight", "ff.net.0.proj.bias"]
    specs = {p.name: p for p in Wt.param_specs()}
    rng = np.random.default_rng(6)
    p2 = dict(oracle_weights)
    orig = {}
    try:
        for b in blocks:
            for sfx in sufs:
                n = b + "." + sfx
                shape = specs[n].shape
                if sfx.startswith("norm") and sfx.endswith(".weight"):
                    v = 1.0 + 0.5 * rng.standard_normal(shape)
                elif sfx.startswith("norm"):
                    v = 0.5 * rng.standard_normal(shape)
                else:
                    v = 0.05 * rng.standard_normal(shape)
                v = v.astype(np.float16).astype(np.float32)
                orig[n] = unet_engine.get_weight(n, shape)
                unet_engine.set_weight(n, v)
                p2[n] = torch.from_numpy(v)
        lat, temb, ctx = inputs(1, 32, 32, seed=18)
        say("forward B=1 32x32 after set_weight on LayerNorm-folded sources")
        got = unet_engine.forward(lat, temb, ctx)
        e = rel_err_l1(got, oracle_forward(p2, lat, temb, ctx))
        e_old = rel_err_l1(got, oracle_forward(oracle_weights, lat, temb, ctx))
        say(f"relErr new weights = {e:.3e}, vs old weights = {e_old:.3e}")
        assert e <= TOL
        assert e_old > max(TOL, 5 * e)
    finally:
        for n, v in orig.items():
            unet_engine.set_weight(n, v)


def test_forward_b16_matches_pairs(unet_engine, oracle_weights):
    """B=16 throughput batch (8 prompts x CFG), every image with its own latent and
    context: each pair of the B=16 output must reproduce a B=2 forward of that pair
    alone (an index mix-up between images -- attention grid, cross-K/V rows b*L,
    statistics slots -- would pull in another pair's data), and the first and last
    pairs are compared with the oracle directly (vk_engine.cpp:542, :823-839)."""
    lat, temb, ctx = inputs(16, 64, 64, seed=16)
    say("forward B=16 64x64 (distinct pairs)")
    y16 = unet_engine.forward(lat, temb, ctx)
    assert np.isfinite(y16).all()
    for i in range(8):
        sl = slice(2 * i, 2 * i + 2)
        y2 = unet_engine.forward(lat[sl], temb, ctx[sl])
        e = rel_err_l1(y16[sl], y2)
        say(f"B=16 pair {i} vs its own B=2 forward: {e:.2e}")
        assert e <= TOL  # tile / split-K plans differ with M: fp16 rounding differs
        # and the pairs really differ from each other
        if i:
            assert rel_err_l1(y16[sl], y16[0:2]) > 0.1
    for i in (0, 7):
        sl = slice(2 * i, 2 * i + 2)
        e = rel_err_l1(y16[sl], oracle_forward(oracle_weights, lat[sl], temb, ctx[sl]))
        say(f"B=16 pair {i} vs oracle: {e:.3e}")
        assert e <= TOL


def _denoise_inputs(H, W, steps):
    lat = Wt.gauss("input.latent", (4, H, W), 21, fp16=False)
    cond = Wt.gauss("input.cond", (77, 768), 21, fp16=False)
    unc = Wt.gauss("input.uncond", (77, 768), 21, fp16=False)
    noise = Wt.gauss("input.noise", (steps - 1, 4, H, W), 21, fp16=False)
    return lat, cond, unc, noise


def test_denoise_loop_matches_host_loop(unet_engine):
    """The on-device loop (graph of 4 forwards + fused CFG/LCM kernels, cross K/V
    computed once) equals a host loop over the engine's own batch-CFG forward and
    the oracle's float64 LcmSchedule.step, bit for bit."""
    steps, g, H, W = 4, 8.0, 32, 32
    lat, cond, unc, noise = _denoise_inputs(H, W, steps)
    dev = unet_engine.denoise_lcm(lat, cond, unc, steps, g, noise)
    sched = lcm.LcmSchedule(steps)
    x = lat.copy()
    for idx, t in enumerate(sched.timesteps):
        both = unet_engine.forward_cfg(x, lcm.time_proj(t), cond, unc)
        eps = lcm.cfg_combine(both[0], both[1], g)
        x = sched.step(idx, x, eps, None if idx == steps - 1 else noise[idx])
    assert np.array_equal(dev, x)


def _denoise_ex(eng, lat, cond, unc, steps, g, cfg_steps, noise, seed=0):
    import sdu
    H, W = lat.shape[1:]
    d = [eng.upload(a) for a in (lat, cond, unc)]
    dn = eng.upload(noise) if noise is not None else None
    out = eng.tensor((4, H, W), sdu.SDU_F32)
    eng.denoise_lcm_ex(d[0].ptr, d[1].ptr, d[2].ptr, H, W, cond.shape[0], steps, g, cfg_steps,
                       dn.ptr if dn is not None else None, seed, out.ptr)
    return out.numpy()


def test_denoise_cfg_first_steps(unet_engine):
    """CFG on the first cfg_steps steps only (TpuUnetPipeline.kt:94-99): the device
    loop against a host loop of the engine's own forwards -- batch CFG for the first
    two steps, then B=1 on cond with eps used as is -- and the oracle's float64 step.
    The B=1 steps of the device loop take cond's K/V rows from the B=2 cross-K/V GEMM,
    whose tile plan differs from a B=1 forward's, so the bar is relErr, not equality."""
    steps, g, H, W, k = 4, 8.0, 32, 32, 2
    lat, cond, unc, noise = _denoise_inputs(H, W, steps)
    say(f"denoise LCM cfg_steps={k}")
    dev = _denoise_ex(unet_engine, lat, cond, unc, steps, g, k, noise)
    sched = lcm.LcmSchedule(steps)
    x = lat.copy()
    for idx, t in enumerate(sched.timesteps):
        if idx < k:
            both = unet_engine.forward_cfg(x, lcm.time_proj(t), cond, unc)
            eps = lcm.cfg_combine(both[0], both[1], g)
        else:
            eps = unet_engine.forward(x[None], lcm.time_proj(t), cond[None])[0]
        x = sched.step(idx, x, eps, None if idx == steps - 1 else noise[idx])
    e = rel_err_l1(dev, x)
    say(f"  relErr vs host loop {e:.2e}")
    assert e <= 1e-3
    # cfg_steps = steps is the batch-CFG loop
    full = _denoise_ex(unet_engine, lat, cond, unc, steps, g, steps, noise)
    assert np.array_equal(full, unet_engine.denoise_lcm(lat, cond, unc, steps, g, noise))
    # guidance <= 1 disables CFG on every step: the same as cfg_steps = 0
    a = _denoise_ex(unet_engine, lat, cond, unc, steps, 1.0, steps, noise)
    b = _denoise_ex(unet_engine, lat, cond, unc, steps, g, 0, noise)
    assert np.array_equal(a, b)
    assert rel_err_l1(a, full) > 1e-2  # and it is a different result


def test_denoise_guidance_shares_one_graph(unet_engine):
    """The guidance scale is read by the denoise graph from device memory, so every
    value > 1 replays the same graph: after a run at 8.0, a run at 3.0 equals the host
    loop at 3.0 bit for bit, and sweeping many values allocates nothing new.  A NaN or
    infinite guidance is rejected."""
    import sdu
    steps, H, W = 4, 32, 32
    lat, cond, unc, noise = _denoise_inputs(H, W, steps)
    _denoise_ex(unet_engine, lat, cond, unc, steps, 8.0, steps, noise)
    g = 3.0
    dev = _denoise_ex(unet_engine, lat, cond, unc, steps, g, steps, noise)
    sched = lcm.LcmSchedule(steps)
    x = lat.copy()
    for idx, tt in enumerate(sched.timesteps):
        both = unet_engine.forward_cfg(x, lcm.time_proj(tt), cond, unc)
        eps = lcm.cfg_combine(both[0], both[1], g)
        x = sched.step(idx, x, eps, None if idx == steps - 1 else noise[idx])
    assert np.array_equal(dev, x)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for gg in np.linspace(1.5, 12.0, 12):
        _denoise_ex(unet_engine, lat, cond, unc, steps, float(gg), steps, noise)
    torch.cuda.synchronize()
    grown = free0 - torch.cuda.mem_get_info()[0]
    say(f"device memory taken by 12 more guidance values: {grown / 2**20:.1f} MiB")
    assert grown < 64 * 2**20
    for bad in (float("nan"), float("inf")):
        with pytest.raises(sdu.SduError) as ex:
            _denoise_ex(unet_engine, lat, cond, unc, steps, bad, steps, noise)
        assert ex.value.code == sdu.SDU_ERR_ARG


def test_denoise_device_noise(unet_engine):
    """noise = NULL draws N(0,1) on the device from the seed (key
    fnv1a64("lcm.noise") ^ splitmix64(seed)); the oracle's generator with the same key
    gives the same noise, so the two runs agree."""
    steps, g, H, W = 4, 8.0, 32, 32
    lat, cond, unc, _ = _denoise_inputs(H, W, steps)
    seed = 77
    noise = Wt.gauss("lcm.noise", (steps - 1, 4, H, W), seed, fp16=False)
    assert abs(float(noise.mean())) < 0.05 and abs(float(noise.std()) - 1.0) < 0.05
    a = _denoise_ex(unet_engine, lat, cond, unc, steps, g, steps, None, seed)
    b = _denoise_ex(unet_engine, lat, cond, unc, steps, g, steps, noise)
    e = rel_err_l1(a, b)
    say(f"device noise vs oracle noise: relErr {e:.2e}")
    assert e <= 1e-6
    c = _denoise_ex(unet_engine, lat, cond, unc, steps, g, steps, None, seed + 1)
    assert rel_err_l1(a, c) > 1e-3


def _denoise_case(unet_engine, oracle_weights, H, W):
    """4-step LCM + CFG (guidance 8) vs the oracle loop with the same injected
    noise (VulkanUnetPipeline.kt:63-97, LcmScheduler.kt:56-82).

    Per step, the engine's forward on the oracle's own step input is held to the
    forward bar (3e-3).  The final latent is held to 1e-2: guidance 8 multiplies
    the difference of the cond and uncond errors, and each step feeds the next."""
    steps, g = 4, 8.0
    lat, cond, unc, noise = _denoise_inputs(H, W, steps)
    say(f"denoise LCM {steps} steps {H}x{W}")
    got = unet_engine.denoise_lcm(lat, cond, unc, steps, g, noise)
    trace = []
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    ref = U.denoise_lcm(oracle_weights, lat, cond, unc, steps, g, noise, trace=trace)
    sched = lcm.LcmSchedule(steps)
    for idx, (x_in, ec, eu, _) in enumerate(trace):
        both = unet_engine.forward_cfg(x_in, lcm.time_proj(sched.timesteps[idx]), cond, unc)
        e = rel_err_l1(both, np.stack([ec, eu]))
        say(f"  step {idx} (t={sched.timesteps[idx]}) teacher-forced eps relErr {e:.3e}")
        assert e <= TOL
    e = rel_err_l1(got, ref)
    say(f"relErr final latent {H}x{W} = {e:.3e}")
    assert e <= 1e-2


def test_denoise_lcm_32(unet_engine, oracle_weights):
    _denoise_case(unet_engine, oracle_weights, 32, 32)


@pytest.mark.slow
def test_denoise_lcm_64(unet_engine, oracle_weights):
    _denoise_case(unet_engine, oracle_weights, 64, 64)


def test_device_entry_point_matches_host(unet_engine):
    lat, temb, ctx = inputs(2, 32, 32, seed=17)
    host = unet_engine.forward(lat, temb, ctx)
    e = unet_engine
    tl, tt, tc = e.upload(lat), e.upload(temb), e.upload(ctx)
    to = e.tensor(lat.shape, 2)
    e.forward_device(tl.ptr, tt.ptr, tc.ptr, 2, 32, 32, 77, to.ptr)
    e.sync()
    assert np.array_equal(to.numpy(), host)


def _write_unet_w(d, seed):
    """The reference's on-device unet_w/ layout: <diffusers key>.bin raw fp16,
    Linear weights stored [in, out] (vk_engine.cpp:497-505, README.md:293)."""
    for p in Wt.param_specs():
        v = Wt.param_value(p, seed, "affine")
        if p.kind == "linear":
            v = v.T
        np.ascontiguousarray(v).astype("<f2").tofile(os.path.join(d, p.name + ".bin"))


def test_weights_dir_loader(tmp_path, unet_engine):
    """Weights read from a unet_w/ directory equal the seeded generator's, so the
    forward equals that of a seeded context bit for bit; a missing or short file
    is an error, not a silent zero tensor."""
    import sdu
    d = str(tmp_path)
    say("writing unet_w/")
    _write_unet_w(d, 5)
    lat, temb, ctx = inputs(2, 16, 16, seed=18)
    a = sdu.Engine(weights_dir=d)
    try:
        specs = {p.name: p for p in Wt.param_specs()}
        for n in ("down_blocks.1.attentions.0.transformer_blocks.0.ff.net.0.proj.weight",
                  "down_blocks.1.attentions.0.transformer_blocks.0.attn2.to_k.weight",
                  "time_embedding.linear_2.weight", "conv_in.weight"):
            assert np.array_equal(a.get_weight(n, specs[n].shape), Wt.param_value(specs[n], 5, "affine"))
        ya = a.forward(lat, temb, ctx)
    finally:
        a.release()
    b = sdu.Engine(seed=5, flags=sdu.SDU_INIT_RANDOM_AFFINE)
    try:
        assert np.array_equal(b.forward(lat, temb, ctx), ya)
    finally:
        b.release()
    os.remove(os.path.join(d, "mid_block.resnets.1.conv2.bias.bin"))
    with pytest.raises(sdu.SduError) as ex:
        sdu.Engine(weights_dir=d)
    assert ex.value.code == sdu.SDU_ERR_WEIGHT and "mid_block.resnets.1.conv2.bias" in str(ex.value)
    np.zeros(3, "<f2").tofile(os.path.join(d, "mid_block.resnets.1.conv2.bias.bin"))
    with pytest.raises(sdu.SduError) as ex:
        sdu.Engine(weights_dir=d)
    assert ex.value.code == sdu.SDU_ERR_WEIGHT


def test_selftest_protocol(tmp_path, unet_engine, oracle_weights):
    """unetSelfTest (vk_engine.cpp:811-851) with fixtures written by the oracle."""
    import sdu
    lat, temb, ctx = inputs(1, 64, 64, seed=19)
    lat16 = lat.astype(np.float16)
    ctx16 = ctx.astype(np.float16)
    tp16 = temb.astype(np.float16)
    ref = oracle_forward(oracle_weights, lat16.astype(np.float32), tp16.astype(np.float32),
                         ctx16.astype(np.float32))
    d = str(tmp_path)
    lat16.tofile(os.path.join(d, "IN_lat.bin"))
    ctx16.tofile(os.path.join(d, "IN_ctx.bin"))
    tp16.tofile(os.path.join(d, "IN_temb_proj.bin"))
    ref.astype(np.float16).tofile(os.path.join(d, "OUT_y.bin"))
    e = unet_engine.selftest(d)
    say(f"selftest relErr = {e:.3e}")
    assert 0 <= e <= TOL
    assert unet_engine.selftest(str(tmp_path / "missing")) < 0
    r = unet_engine.selftest_report(d)
    assert max(r["relerr_b1"], *r["relerr_b2"]) == e and r["ctx_sens"] == -1.0
    # context-sensitivity leg (vk_engine.cpp:840-849): IN_cond / IN_unc at IN_temb999,
    # mean |eps_cond - eps_unc| of two B=1 forwards, against the oracle's value
    cond = Wt.gauss("input.cond", (77, 768), 19, fp16=True)
    unc = Wt.gauss("input.uncond", (77, 768), 19, fp16=True)
    t999 = lcm.time_proj(999).astype(np.float16)
    cond.astype(np.float16).tofile(os.path.join(d, "IN_cond.bin"))
    unc.astype(np.float16).tofile(os.path.join(d, "IN_unc.bin"))
    t999.tofile(os.path.join(d, "IN_temb999.bin"))
    ec = oracle_forward(oracle_weights, lat16.astype(np.float32), t999.astype(np.float32), cond[None])
    eu = oracle_forward(oracle_weights, lat16.astype(np.float32), t999.astype(np.float32), unc[None])
    d_ref = float(np.abs(ec - eu).mean())
    r = unet_engine.selftest_report(d)
    say(f"ctx sensitivity engine {r['ctx_sens']:.4e} oracle {d_ref:.4e}")
    assert d_ref > 0 and abs(r["ctx_sens"] - d_ref) / d_ref < 0.05
    # a context-sensitivity set with a short file is an error, not a silent zero
    np.zeros(3, np.float16).tofile(os.path.join(d, "IN_unc.bin"))
    with pytest.raises(sdu.SduError):
        unet_engine.selftest_report(d)
