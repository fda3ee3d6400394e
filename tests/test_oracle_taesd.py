"""Pinning the TAESD decoder oracle (oracle/taesd_ref.py) on the CPU.

The reference decodes with a LiteRT export of diffusers' AutoencoderTiny
(tools/export_taesd.py:52-54) and ships no TAESD weights or decoded fixtures, so the
restatement is pinned by constructed weights whose output the mathematics fixes:
  * all weights zero but conv_out's bias b: the image is 2 b - 1 everywhere (output affine);
  * identity taps through every conv, zero block convs: the image is
    2 ReLU(3 tanh(z / 3)) - 1 upsampled 8x by pixel replication (clamp, the three nearest
    upsamplings, the identity residual of every block);
  * a block whose last conv is zero passes its (non-negative) input through unchanged,
    whatever its first two convs hold (the residual).
Each check is shown to fail on a planted mistake.
"""
import numpy as np
import pytest
import torch

from oracle import taesd_ref as T


def _zero_params():
    return {p.name: np.zeros(p.shape, np.float32) for p in T.param_specs()}


def _identity_tap(co, ci, pairs):
    w = np.zeros((co, ci, 3, 3), np.float32)
    for o, i in pairs:
        w[o, i, 1, 1] = 1.0
    return w


def test_inventory_and_shape():
    ps = T.param_specs()
    # conv_in 2,368 + 10 blocks x 3 x 36,928 + 3 upsampling convs x 36,864 + conv_out 1,731
    assert sum(p.numel for p in ps) == 1_222_531
    p = T.generate(3)
    z = np.random.default_rng(0).standard_normal((2, 4, 8, 12)).astype(np.float32)
    y = T.decode(p, z)
    assert tuple(y.shape) == (2, 3, 64, 96)
    assert torch.isfinite(y).all()


def test_output_affine():
    p = _zero_params()
    out = f"decoder.layers.{T.layer_plan()[-1][1]}"
    p[out + ".bias"] = np.array([0.25, -0.5, 1.0], np.float32)
    z = np.random.default_rng(1).standard_normal((1, 4, 8, 8)).astype(np.float32)
    y = T.decode(p, z).numpy()
    np.testing.assert_allclose(y[0, :, 0, 0], [-0.5, -2.0, 1.0], atol=0)
    assert np.ptp(y, axis=(2, 3)).max() == 0.0


def _passthrough_params():
    """conv_in passes latent channel 0 to channel 0, the upsampling convs are identity,
    conv_out reads channel 0 into all three outputs; every block conv is zero."""
    p = _zero_params()
    for kind, i in T.layer_plan():
        pf = f"decoder.layers.{i}"
        if kind == "conv_in":
            p[pf + ".weight"] = _identity_tap(T.CH, T.LATENT_C, [(0, 0)])
        elif kind == "conv_nobias":
            p[pf + ".weight"] = _identity_tap(T.CH, T.CH, [(c, c) for c in range(T.CH)])
        elif kind == "conv_out":
            p[pf + ".weight"] = _identity_tap(T.OUT_C, T.CH, [(o, 0) for o in range(T.OUT_C)])
    return p


def _passthrough_expected(z):
    v = np.maximum(3.0 * np.tanh(z[:, 0] / 3.0), 0.0)
    v = v.repeat(8, axis=1).repeat(8, axis=2)
    return 2.0 * v - 1.0


def test_clamp_upsampling_and_residual_wiring(monkeypatch):
    p = _passthrough_params()
    z = (np.random.default_rng(2).standard_normal((1, 4, 8, 8)) * 4.0).astype(np.float32)
    want = _passthrough_expected(z)
    got = T.decode(p, z).numpy()
    for c in range(3):
        np.testing.assert_allclose(got[:, c], want, rtol=1e-6, atol=1e-6)

    # planted mistakes, each must break the check
    with monkeypatch.context() as mp:
        mp.setattr(T, "clamp", lambda x: x)
        bad = T.decode(p, z).numpy()
        assert np.abs(bad[:, 0] - want).max() > 0.1, "missing clamp not detected"

    def block_without_skip(pp, pf, x):
        h = torch.relu(T._conv(x, pp[pf + ".conv.0.weight"], pp[pf + ".conv.0.bias"]))
        h = torch.relu(T._conv(h, pp[pf + ".conv.2.weight"], pp[pf + ".conv.2.bias"]))
        return torch.relu(T._conv(h, pp[pf + ".conv.4.weight"], pp[pf + ".conv.4.bias"]))

    with monkeypatch.context() as mp:
        mp.setattr(T, "block", block_without_skip)
        bad = T.decode(p, z).numpy()
        assert np.abs(bad[:, 0] - want).max() > 0.5, "missing residual not detected"

    orig_plan = T.layer_plan

    def plan_two_upsamplings():
        out, dropped = [], False
        for kind, i in orig_plan():
            if kind == "upsample" and not dropped:
                dropped = True
                continue
            out.append((kind, i))
        return out

    with monkeypatch.context() as mp:
        mp.setattr(T, "layer_plan", plan_two_upsamplings)
        bad = T.decode(p, z)
        assert tuple(bad.shape[-2:]) != tuple(want.shape[-2:]), "upsampling count not detected"


def test_block_residual_ignores_first_convs():
    """A block with a zero last conv returns ReLU(x) = x for x >= 0, whatever convs 0 and 2 hold."""
    p = T.generate(5, "affine")
    pf = "decoder.layers.2"
    p[pf + ".conv.4.weight"] = np.zeros_like(p[pf + ".conv.4.weight"])
    p[pf + ".conv.4.bias"] = np.zeros_like(p[pf + ".conv.4.bias"])
    x = torch.relu(torch.randn(1, T.CH, 6, 6, generator=torch.Generator().manual_seed(0)))
    pt = {k: torch.as_tensor(v) for k, v in p.items()}
    np.testing.assert_array_equal(T.block(pt, pf, x).numpy(), x.numpy())
