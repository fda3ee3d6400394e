"""GPU parity of the TAESD decoder, the CLIP text encoder and the end-to-end image path
(through the C ABI) against the CPU oracles, plus the kernel features they add: the ReLU /
quick-GELU GEMM epilogue and causal attention.

Tolerances as the UNet path: relErr_L1 <= 1e-3 per GEMM / conv op, <= 2e-3 for attention,
<= 3e-3 for whole networks (fp16 activations against the fp32 oracle).
"""
import os

import numpy as np
import pytest
import torch

from conftest import rel_err_l1, say
from oracle import clip_ref, taesd_ref, weights

pytestmark = pytest.mark.gpu


def r16(shape, seed, scale=1.0, mean=0.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape) * scale + mean).astype(np.float16).astype(np.float32)


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def quick_gelu(x):
    return x * torch.sigmoid(1.702 * x)


# ------------------------------------------------------------------ epilogue activations


@pytest.mark.parametrize("M,N,K,act", [
    (154, 3072, 768, "quick_gelu"),   # CLIP fc1 at B=2
    (77, 2304, 768, None),            # CLIP fused QKV at B=1
    (300, 512, 320, "relu"),
])
def test_matmul_activation(op_engine, M, N, K, act):
    import sdu
    say(f"matmul act={act} M={M} N={N} K={K}")
    e = op_engine
    a, w, b = r16((M, K), 1), r16((N, K), 2, 0.05), r16((N,), 3, 0.5)
    flags = {"relu": sdu.SDU_EPI_RELU, "quick_gelu": sdu.SDU_EPI_QUICK_GELU, None: 0}[act]
    ty = e.tensor((M, N))
    e.matmul(e.upload(a.astype(np.float16)), e.upload(w.astype(np.float16)), ty, M, N, K,
             bias=e.upload(b.astype(np.float16)), flags=flags)
    ref = t(a) @ t(w).T + t(b)
    ref = {"relu": torch.relu, "quick_gelu": quick_gelu, None: lambda x: x}[act](ref).numpy()
    got = ty.numpy().astype(np.float32)
    assert rel_err_l1(got, ref) < 1e-3
    assert np.abs(got - ref).max() < 2e-2


@pytest.mark.parametrize("B,H,W,ups", [(1, 16, 16, 0), (2, 12, 20, 0), (1, 8, 8, 1)])
def test_conv_relu_residual(op_engine, B, H, W, ups):
    """The TAESD block's last conv: y = ReLU(conv(x) + b + res) (and the upsampling conv)."""
    import sdu
    say(f"conv relu+res B={B} {H}x{W} ups={ups}")
    e, C = op_engine, 64
    Ho, Wo = (2 * H, 2 * W) if ups else (H, W)
    x = r16((B, H, W, C), 4)
    w = r16((C, 3, 3, C), 5, 0.04)
    b = r16((C,), 6, 0.2)
    res = r16((B, Ho, Wo, C), 7)
    ty = e.tensor((B, Ho, Wo, C))
    e.conv2d(e.upload(x.astype(np.float16)), e.upload(w.astype(np.float16)), ty, B, H, W, C, C, 3, 1, bool(ups),
             bias=e.upload(b.astype(np.float16)), residual=e.upload(res.astype(np.float16)), flags=sdu.SDU_EPI_RELU)
    xin = t(x).permute(0, 3, 1, 2)
    if ups:
        xin = torch.nn.functional.interpolate(xin, scale_factor=2, mode="nearest")
    ref = torch.nn.functional.conv2d(xin, t(w).permute(0, 3, 1, 2), t(b), padding=1)
    ref = torch.relu(ref + t(res).permute(0, 3, 1, 2)).permute(0, 2, 3, 1).numpy()
    got = ty.numpy().astype(np.float32)
    assert rel_err_l1(got, ref) < 1e-3
    assert np.abs(got - ref).max() < 2e-2


# ------------------------------------------------------------------ causal attention


@pytest.mark.parametrize("B,heads,S,d", [(2, 12, 77, 64), (1, 2, 200, 64), (1, 1, 33, 40), (3, 4, 5, 64)])
def test_attention_causal(op_engine, B, heads, S, d):
    import sdu
    say(f"causal attention B={B} heads={heads} S={S} d={d}")
    e = op_engine
    C = heads * d
    q, k, v = r16((B, S, C), 8), r16((B, S, C), 9), r16((B, S, C), 10)
    to = e.tensor((B, S, C))
    scale = d ** -0.5
    e.attention_ex(e.upload(q.astype(np.float16)), e.upload(k.astype(np.float16)), e.upload(v.astype(np.float16)),
                   to, B, heads, S, S, d, C, C, C, C, scale, sdu.SDU_ATTN_CAUSAL)
    got = to.numpy().astype(np.float32)
    qh = t(q).view(B, S, heads, d).transpose(1, 2)
    kh = t(k).view(B, S, heads, d).transpose(1, 2)
    vh = t(v).view(B, S, heads, d).transpose(1, 2)
    s = (qh @ kh.transpose(-1, -2)) * scale
    s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    ref = (torch.softmax(s, -1) @ vh).transpose(1, 2).reshape(B, S, C).numpy()
    assert rel_err_l1(got, ref) < 2e-3
    assert np.abs(got - ref).max() < 2e-2
    # the first query sees only itself
    np.testing.assert_allclose(got[:, 0], v[:, 0], rtol=2e-3, atol=2e-3)


def test_attention_causal_rejects_cross(op_engine):
    import sdu
    e = op_engine
    x = e.tensor((1, 8, 64))
    with pytest.raises(sdu.SduError):
        e.attention_ex(x, x, x, x, 1, 1, 8, 4, 64, 64, 64, 64, 64, 0.125, sdu.SDU_ATTN_CAUSAL)


# ------------------------------------------------------------------ TAESD decoder


@pytest.fixture(scope="module")
def taesd_engine():
    import sdu
    eng = sdu.Engine(flags=sdu.SDU_INIT_NO_WEIGHTS)
    eng.taesd_init(seed=77, flags=sdu.SDU_INIT_RANDOM_AFFINE)
    yield eng
    eng.release()


@pytest.mark.parametrize("B,H,W", [(1, 16, 16), (2, 8, 12), (1, 64, 64)])
def test_taesd_decode_matches_oracle(taesd_engine, B, H, W):
    say(f"taesd decode B={B} {H}x{W}")
    z = (np.random.default_rng(B * 100 + H).standard_normal((B, 4, H, W)) * 1.5).astype(np.float32)
    got = taesd_engine.taesd_decode(z)
    p = taesd_ref.generate(77, "affine")
    with torch.inference_mode():
        ref = taesd_ref.decode(p, z).numpy()
    assert got.shape == (B, 3, 8 * H, 8 * W)
    # compared before the output affine y = 2 x - 1: its constant -1 would dilute the
    # error of the network itself
    err = rel_err_l1(got + 1.0, ref + 1.0)
    say(f"  relErr_L1 of y + 1 {err:.2e} (of y {rel_err_l1(got, ref):.2e})")
    assert err < 3e-3
    # replay of the captured graph is deterministic
    np.testing.assert_array_equal(taesd_engine.taesd_decode(z), got)


def test_taesd_weights_dir(tmp_path, taesd_engine):
    """Weights written in the weight-directory format load to the same decoder."""
    import sdu
    p = taesd_ref.generate(77, "affine")
    for name, v in p.items():
        v.astype(np.float16).tofile(os.path.join(tmp_path, name + ".bin"))
    z = np.random.default_rng(3).standard_normal((1, 4, 8, 8)).astype(np.float32)
    eng = sdu.Engine(flags=sdu.SDU_INIT_NO_WEIGHTS)
    try:
        eng.taesd_init(str(tmp_path))
        np.testing.assert_array_equal(eng.taesd_decode(z), taesd_engine.taesd_decode(z))
        os.remove(os.path.join(tmp_path, "decoder.layers.18.bias.bin"))
        with pytest.raises(sdu.SduError) as ei:
            eng.taesd_init(str(tmp_path))
        assert ei.value.code == sdu.SDU_ERR_WEIGHT
    finally:
        eng.release()


# ------------------------------------------------------------------ CLIP text encoder


@pytest.fixture(scope="module")
def clip_engine():
    import sdu
    eng = sdu.Engine(flags=sdu.SDU_INIT_NO_WEIGHTS)
    eng.clip_init(seed=99, flags=sdu.SDU_INIT_RANDOM_AFFINE)
    yield eng
    eng.release()


def _ids(B, seed):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, clip_ref.VOCAB, size=(B, 77)).astype(np.int32)
    ids[:, 0] = 49406          # start token
    ids[:, 20:] = 49407        # end token, padded to 77 as ClipTokenizer.kt does
    return ids


@pytest.fixture(scope="module")
def clip_oracle_weights():
    return clip_ref.generate(99, "affine")


@pytest.mark.parametrize("B", [1, 2, 5])
def test_clip_encode_matches_oracle(clip_engine, clip_oracle_weights, B):
    say(f"clip encode B={B}")
    ids = _ids(B, B)
    got = clip_engine.clip_encode(ids)
    with torch.inference_mode():
        ref = clip_ref.encode(clip_oracle_weights, ids).numpy()
    err = rel_err_l1(got, ref)
    say(f"  relErr_L1 {err:.2e}")
    assert err < 3e-3
    np.testing.assert_array_equal(clip_engine.clip_encode(ids), got)


def test_clip_causality(clip_engine):
    """Changing token j changes only the hidden states of positions >= j."""
    ids = _ids(1, 7)
    a = clip_engine.clip_encode(ids)
    ids2 = ids.copy()
    ids2[0, 10] = 123
    b = clip_engine.clip_encode(ids2)
    np.testing.assert_array_equal(a[0, :10], b[0, :10])
    assert np.abs(a[0, 10:] - b[0, 10:]).max() > 1e-3


# ------------------------------------------------------------------ end to end


def test_generate_is_the_device_chain(unet_engine):
    """sdu_generate equals CLIP -> LCM denoise -> TAESD run one by one through the ABI with
    the same seeds: the initial latent is the generator's 'lcm.latent' stream, which the
    oracle's generator reproduces up to host / device libm rounding (hence a relErr bar,
    not equality), and the noise is drawn on the device from the same seed in both."""
    import sdu
    eng = unet_engine
    eng.clip_init(seed=5)
    eng.taesd_init(seed=6)
    H = W = 16
    cond, unc = _ids(1, 11)[0], _ids(1, 12)[0]
    unc[1:] = 49407
    seed, steps, guidance = 42, 4, 8.0
    img = eng.generate(cond, unc, H, W, steps, guidance, steps, seed)
    assert img.shape == (3, 8 * H, 8 * W) and np.isfinite(img).all()
    ctx = eng.clip_encode(np.stack([cond, unc]))
    lat = weights.gauss("lcm.latent", (4, H, W), seed, fp16=False)
    d_lat, d_c, d_u = eng.upload(lat), eng.upload(ctx[0]), eng.upload(ctx[1])
    d_x = eng.tensor((4, H, W), sdu.SDU_F32)
    eng.denoise_lcm_ex(d_lat.ptr, d_c.ptr, d_u.ptr, H, W, 77, steps, guidance, steps, None, seed, d_x.ptr)
    eng.sync()
    img2 = eng.taesd_decode(d_x.numpy()[None])[0]
    err = rel_err_l1(img2, img)
    say(f"generate vs chain relErr {err:.2e}")
    assert err <= 1e-4
    np.testing.assert_array_equal(eng.generate(cond, unc, H, W, steps, guidance, steps, seed), img)
    assert rel_err_l1(eng.generate(cond, unc, H, W, steps, guidance, steps, seed + 1), img) > 1e-3


# ------------------------------------------------------------------ calibration


def test_calibrate_sane(op_engine):
    """sdu_calibrate reports the box's MFMA ceiling, the shader clock under it and a copy
    rate; each within what an MI355X can physically do (2.5 PF/s, 2.4 GHz, 8 TB/s)."""
    c = op_engine.calibrate(64)
    say(f"calibration {c}")
    assert 300.0 < c["mfma_tflops"] <= 2600.0
    assert 0.5 < c["mfma_clock_ghz"] <= 2.5
    assert 500.0 < c["copy_gbs"] <= 8200.0
