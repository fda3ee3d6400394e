"""Pinning the SD1.5 VAE decoder oracle (oracle/vae_ref.py) on the CPU.

The reference decodes with a LiteRT export of diffusers' AutoencoderKL (gpu_vae.tflite,
VulkanUnetPipeline.kt:55-61; the full-VAE call at tools/export_taesd.py:53) and ships no
VAE weights or decoded fixtures, so the restatement is pinned by:
  * the parameter inventory: 49,490,179 decoder parameters (the published size of the SD1.5
    VAE decoder) plus post_quant_conv's 20, with the shortcut convs where the up path
    changes width and no upsampler after the last block;
  * GroupNorm against a per-group brute-force loop at a variance comparable to its eps
    (1e-6, not 1e-5);
  * the mid-block attention against a per-token brute-force loop: one head of all C
    channels, softmax scale 1 / sqrt(C), the residual added;
  * resnets built from identity taps: the shortcut applied to the block's input, SiLU after
    both GroupNorms;
  * a passthrough decoder (identity taps, zero residual branches but one constant): the
    latent scaling 1 / 0.18215, three nearest 2x upsamplings and the SiLU after
    conv_norm_out fix the output in closed form.
Each check is shown to fail on a planted mistake.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import vae_ref as V


def _tt(a):
    return torch.as_tensor(np.asarray(a), dtype=torch.float32)


def _gn_brute(x, w, b, groups, eps):
    """GroupNorm by explicit loops over images and groups (float64)."""
    x = np.asarray(x, np.float64)
    B, C = x.shape[:2]
    y = np.empty_like(x)
    cg = C // groups
    for i in range(B):
        for g in range(groups):
            sl = x[i, g * cg:(g + 1) * cg]
            m = sl.sum() / sl.size
            v = ((sl - m) ** 2).sum() / sl.size
            y[i, g * cg:(g + 1) * cg] = (sl - m) / math.sqrt(v + eps)
    return y * np.asarray(w).reshape(1, C, 1, 1) + np.asarray(b).reshape(1, C, 1, 1)


def _silu(x):
    return x / (1.0 + np.exp(-x))


def test_inventory():
    ps = V.param_specs()
    n = {p.name: p for p in ps}
    assert len(n) == len(ps)
    assert sum(p.numel for p in ps if p.name.startswith("decoder.")) == 49_490_179
    assert sum(p.numel for p in ps if p.name.startswith("post_quant_conv.")) == 20
    assert n["decoder.up_blocks.2.resnets.0.conv_shortcut.weight"].shape == (256, 512, 1, 1)
    assert n["decoder.up_blocks.3.resnets.0.conv_shortcut.weight"].shape == (128, 256, 1, 1)
    assert not any("conv_shortcut" in k for k in n if k.startswith(("decoder.up_blocks.0", "decoder.up_blocks.1",
                                                                      "decoder.mid_block")))
    assert "decoder.up_blocks.3.upsamplers.0.conv.weight" not in n
    assert n["decoder.up_blocks.2.upsamplers.0.conv.weight"].shape == (256, 256, 3, 3)
    assert n["decoder.mid_block.attentions.0.to_out.0.weight"].shape == (512, 512)


def test_decode_shape():
    p = V.generate(5, "affine")
    z = np.random.default_rng(0).standard_normal((2, 4, 2, 3)).astype(np.float32)
    y = V.decode(p, z)
    assert tuple(y.shape) == (2, 3, 16, 24)
    assert torch.isfinite(y).all()


def test_group_norm_brute_force(monkeypatch):
    rng = np.random.default_rng(1)
    # variance about 1e-6 per group: the epsilon is a third of the denominator
    # (one offset per group of two channels, so the group's variance is the 1e-6 part)
    off = rng.standard_normal((1, 32, 1, 1)).repeat(2, axis=1)
    x = (1e-3 * rng.standard_normal((2, 64, 3, 5)) + off).astype(np.float32)
    w = rng.standard_normal(64).astype(np.float32)
    b = rng.standard_normal(64).astype(np.float32)
    ref = _gn_brute(x, w, b, 32, 1e-6)
    got = V.group_norm(_tt(x), _tt(w), _tt(b)).numpy()
    np.testing.assert_allclose(got, ref, rtol=2e-3, atol=2e-3)
    # planted: the UNet's eps 1e-5
    monkeypatch.setattr(V, "EPS", 1e-5)
    bad = V.group_norm(_tt(x), _tt(w), _tt(b), eps=V.EPS).numpy()
    assert np.abs(bad - ref).max() > 0.1


def _attn_brute(p, pf, x):
    """Single-head attention over tokens by explicit per-query loops (float64)."""
    B, C, H, W = x.shape
    h = _gn_brute(x, p[pf + ".group_norm.weight"], p[pf + ".group_norm.bias"], 32, 1e-6)
    out = np.array(x, np.float64)
    for i in range(B):
        t = h[i].reshape(C, H * W).T
        q = t @ np.asarray(p[pf + ".to_q.weight"], np.float64).T + p[pf + ".to_q.bias"]
        k = t @ np.asarray(p[pf + ".to_k.weight"], np.float64).T + p[pf + ".to_k.bias"]
        v = t @ np.asarray(p[pf + ".to_v.weight"], np.float64).T + p[pf + ".to_v.bias"]
        o = np.zeros_like(q)
        for r in range(H * W):
            s = np.array([q[r] @ k[j] for j in range(H * W)]) / math.sqrt(C)
            e = np.exp(s - s.max())
            o[r] = (e / e.sum()) @ v
        o = o @ np.asarray(p[pf + ".to_out.0.weight"], np.float64).T + p[pf + ".to_out.0.bias"]
        out[i] += o.T.reshape(C, H, W)
    return out


def _attn_params(C, seed):
    rng = np.random.default_rng(seed)
    pf = "a"
    p = {pf + ".group_norm.weight": 1 + 0.1 * rng.standard_normal(C), pf + ".group_norm.bias": 0.1 * rng.standard_normal(C)}
    for lin in ("to_q", "to_k", "to_v", "to_out.0"):
        p[f"{pf}.{lin}.weight"] = 0.3 * rng.standard_normal((C, C))
        p[f"{pf}.{lin}.bias"] = 0.1 * rng.standard_normal(C)
    return pf, {k: np.asarray(v, np.float32) for k, v in p.items()}


def test_attention_brute_force():
    C = 64
    pf, p = _attn_params(C, 2)
    x = np.random.default_rng(3).standard_normal((2, C, 3, 4)).astype(np.float32)
    ref = _attn_brute(p, pf, x)
    pt = {k: _tt(v) for k, v in p.items()}
    got = V.attention(pt, pf, _tt(x)).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-3, atol=1e-3)
    # planted: 8 heads of C / 8 (the UNet's layout), and a dropped residual
    t = V.group_norm(_tt(x), pt[pf + ".group_norm.weight"], pt[pf + ".group_norm.bias"])
    t = t.reshape(2, C, 12).transpose(1, 2)
    q, k, v = (F.linear(t, pt[f"{pf}.{n}.weight"], pt[f"{pf}.{n}.bias"]) for n in ("to_q", "to_k", "to_v"))
    qh, kh, vh = (u.reshape(2, 12, 8, C // 8).transpose(1, 2) for u in (q, k, v))
    o = torch.softmax(qh @ kh.transpose(-1, -2) / math.sqrt(C // 8), -1) @ vh
    o = F.linear(o.transpose(1, 2).reshape(2, 12, C), pt[pf + ".to_out.0.weight"], pt[pf + ".to_out.0.bias"])
    multi = (_tt(x) + o.transpose(1, 2).reshape(2, C, 3, 4)).numpy()
    assert np.abs(multi - ref).max() > 0.05
    assert np.abs((got - x) - ref).max() > 0.5  # without the residual


def _tap(co, ci, pairs, k=3):
    w = np.zeros((co, ci, k, k), np.float32)
    for o, i in pairs:
        w[o, i, k // 2, k // 2] = 1.0
    return w


def _resnet_params(pf, cin, cout):
    return {q.name: np.zeros(q.shape, np.float32) for q in V._resnet_specs(pf, cin, cout)}


def test_resnet_shortcut_and_silus():
    rng = np.random.default_rng(4)
    cin, cout = 64, 32
    pf = "r"
    p = _resnet_params(pf, cin, cout)
    for n in ("norm1", "norm2"):
        p[f"{pf}.{n}.weight"] = np.ones(p[f"{pf}.{n}.weight"].shape, np.float32)
    p[pf + ".conv1.weight"] = _tap(cout, cin, [(c, c) for c in range(cout)])
    p[pf + ".conv2.weight"] = _tap(cout, cout, [(c, c) for c in range(cout)])
    p[pf + ".conv_shortcut.weight"] = _tap(cout, cin, [(c, c + 1) for c in range(cout)], k=1)
    x = rng.standard_normal((1, cin, 4, 5)).astype(np.float32)
    g1 = _silu(_gn_brute(x, p[pf + ".norm1.weight"], p[pf + ".norm1.bias"], 32, 1e-6))[:, :cout]
    g2 = _silu(_gn_brute(g1, p[pf + ".norm2.weight"], p[pf + ".norm2.bias"], 32, 1e-6))
    expected = x[:, 1:cout + 1] + g2  # shortcut: input channel c + 1 -> output c
    got = V.resnet({k: _tt(v) for k, v in p.items()}, pf, _tt(x)).numpy()
    np.testing.assert_allclose(got, expected, rtol=2e-3, atol=2e-3)
    # planted: the residual dropped; no SiLU after norm1
    assert np.abs(g2 - got).max() > 0.5
    g1b = _gn_brute(x, p[pf + ".norm1.weight"], p[pf + ".norm1.bias"], 32, 1e-6)[:, :cout]
    bad2 = x[:, 1:cout + 1] + _silu(_gn_brute(g1b, p[pf + ".norm2.weight"], p[pf + ".norm2.bias"], 32, 1e-6))
    assert np.abs(bad2 - got).max() > 0.05


def _passthrough(c_add):
    """Identity taps on channel 0 from the latent to conv_out, every residual branch zero
    except the last resnet's conv2 bias (c_add on channel 0), conv_norm_out gamma 1."""
    p = {q.name: np.zeros(q.shape, np.float32) for q in V.param_specs()}
    top = V.BLOCK_OUT[-1]
    p["post_quant_conv.weight"] = _tap(4, 4, [(c, c) for c in range(4)], k=1)
    p["decoder.conv_in.weight"] = _tap(top, 4, [(0, 0)])
    for i, cin, cout, up in V.up_plan():
        if cin != cout:
            p[f"decoder.up_blocks.{i}.resnets.0.conv_shortcut.weight"] = _tap(cout, cin, [(0, 0)], k=1)
        if up:
            p[f"decoder.up_blocks.{i}.upsamplers.0.conv.weight"] = _tap(cout, cout, [(0, 0)])
    p["decoder.up_blocks.3.resnets.2.conv2.bias"][0] = c_add
    p["decoder.conv_norm_out.weight"][:] = 1.0
    p["decoder.conv_out.weight"] = _tap(3, V.BLOCK_OUT[0], [(o, 0) for o in range(3)])
    return p


def _passthrough_expected(z, c_add, scale=V.SCALING, silu=True):
    B, _, H, W = z.shape
    h0 = (z[:, 0] / scale).repeat(8, axis=1).repeat(8, axis=2) + c_add  # channel 0
    x = np.zeros((B, V.BLOCK_OUT[0], 8 * H, 8 * W), np.float64)
    x[:, 0] = h0
    g = _gn_brute(x, np.ones(V.BLOCK_OUT[0]), np.zeros(V.BLOCK_OUT[0]), 32, 1e-6)[:, 0]
    g = _silu(g) if silu else g
    return np.repeat(g[:, None], 3, axis=1)


def test_passthrough_scaling_upsampling_final_silu():
    z = np.random.default_rng(5).standard_normal((1, 4, 2, 3)).astype(np.float32)
    c_add = 3.0
    got = V.decode(_passthrough(c_add), z).numpy()
    ref = _passthrough_expected(z, c_add)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)
    # every 8x8 block constant (nearest, not bilinear, upsampling)
    blocks = got.reshape(1, 3, 2, 8, 3, 8)
    assert np.ptp(blocks, axis=(3, 5)).max() < 1e-6
    # planted: no latent scaling; no SiLU after conv_norm_out
    assert np.abs(_passthrough_expected(z, c_add, scale=1.0) - got).max() > 0.05
    assert np.abs(_passthrough_expected(z, c_add, silu=False) - got).max() > 0.05
