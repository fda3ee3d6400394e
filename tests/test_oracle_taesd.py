"""Pinning the TAESD decoder oracle (oracle/taesd_ref.py) on the CPU.

The reference decodes with a LiteRT export of diffusers' AutoencoderTiny
(tools/export_taesd.py:52-54) and ships no TAESD weights or decoded fixtures, so the
restatement is pinned by constructed weights whose output the mathematics fixes:
  * all weights zero but conv_out's bias b: the image is 2 b - 1 everywhere (output affine);
  * identity taps through every conv, zero block convs: the image is
    2 ReLU(3 tanh(z / 3)) - 1 upsampled 8x by pixel replication (clamp, the three nearest
    upsamplings, the identity residual of every block);
  * a block whose last conv is zero passes its (non-negative) input through unchanged,
    whatever its first two convs hold (the residual);
  * a block with identity-tap convs and biases -1, 2, 0 on one channel gives
    ReLU(ReLU(2 - ReLU(x - 1)) + x) (both inner ReLUs);
  * conv_in negating the latent, with a first block that maps x to x + 3 ReLU(-x),
    gives 2 ReLU(-3 tanh(z / 3)) - 1 only with the ReLU after conv_in.
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


def _block_relu_params():
    """Weights of one block whose inner ReLUs each change its output: on channel 0,
    conv.0 = x - 1, conv.2 = 2 - h1, conv.4 = h2 (identity taps, biases -1, 2, 0); every
    other tap and channel zero, so the other channels pass through the residual."""
    p = T.generate(9, "affine")
    pf = "decoder.layers.2"
    for j, (wt, b) in zip((0, 2, 4), ((1.0, -1.0), (-1.0, 2.0), (1.0, 0.0))):
        w = np.zeros((T.CH, T.CH, 3, 3), np.float32)
        w[0, 0, 1, 1] = wt
        bias = np.zeros(T.CH, np.float32)
        bias[0] = b
        p[f"{pf}.conv.{j}.weight"] = w
        p[f"{pf}.conv.{j}.bias"] = bias
    return {k: torch.as_tensor(v) for k, v in p.items()}, pf


def test_block_inner_relus():
    """Block(x) = ReLU(conv4(ReLU(conv2(ReLU(conv0(x))))) + x), channel 0 in closed form:
    ReLU(ReLU(2 - ReLU(x - 1)) + x) for x >= 0 (the block input follows a ReLU).  x runs
    over 0 .. 5, so each inner ReLU is active on part of the range."""
    pt, pf = _block_relu_params()
    xs = np.linspace(0.0, 5.0, 36, dtype=np.float32).reshape(6, 6)
    x = torch.zeros(1, T.CH, 6, 6)
    x[0, 0] = torch.as_tensor(xs)
    x[0, 1:] = torch.relu(torch.randn(T.CH - 1, 6, 6, generator=torch.Generator().manual_seed(1)))
    relu = lambda v: np.maximum(v, 0.0)
    want0 = relu(relu(2.0 - relu(xs - 1.0)) + xs)
    got = T.block(pt, pf, x).numpy()
    np.testing.assert_allclose(got[0, 0], want0, rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(got[0, 1:], x[0, 1:].numpy())

    # planted mistakes: each missing inner ReLU breaks the closed form
    def no_first_relu(pp, pf, x):
        h = T._conv(x, pp[pf + ".conv.0.weight"], pp[pf + ".conv.0.bias"])
        h = torch.relu(T._conv(h, pp[pf + ".conv.2.weight"], pp[pf + ".conv.2.bias"]))
        h = T._conv(h, pp[pf + ".conv.4.weight"], pp[pf + ".conv.4.bias"])
        return torch.relu(h + x)

    def no_second_relu(pp, pf, x):
        h = torch.relu(T._conv(x, pp[pf + ".conv.0.weight"], pp[pf + ".conv.0.bias"]))
        h = T._conv(h, pp[pf + ".conv.2.weight"], pp[pf + ".conv.2.bias"])
        h = T._conv(h, pp[pf + ".conv.4.weight"], pp[pf + ".conv.4.bias"])
        return torch.relu(h + x)

    for bad_block in (no_first_relu, no_second_relu):
        bad = bad_block(pt, pf, x).numpy()
        assert np.abs(bad[0, 0] - want0).max() > 0.5, f"{bad_block.__name__} not detected"


def test_conv_in_relu():
    """conv_in maps latent channel 0 to v = -clamp(z0) on channel 0; the first block's convs
    give F(x) = 3 ReLU(-x) on channel 0, which is zero for the ReLU'd input x = ReLU(v).
    With the ReLU after conv_in the image is 2 ReLU(-3 tanh(z0 / 3)) - 1 replicated 8x;
    without it, F(v) + v = -2v > 0 wherever v < 0 leaks through the first block."""
    p = _passthrough_params()
    p["decoder.layers.0.weight"] = -p["decoder.layers.0.weight"]
    pf = "decoder.layers.2"
    for j, wt in zip((0, 2, 4), (-1.0, 1.0, 3.0)):
        p[f"{pf}.conv.{j}.weight"] = _identity_tap(T.CH, T.CH, [(0, 0)]) * wt
    z = (np.random.default_rng(4).standard_normal((1, 4, 8, 8)) * 4.0).astype(np.float32)
    v = np.maximum(-3.0 * np.tanh(z[:, 0] / 3.0), 0.0).repeat(8, axis=1).repeat(8, axis=2)
    want = 2.0 * v - 1.0
    got = T.decode(p, z).numpy()
    for c in range(3):
        np.testing.assert_allclose(got[:, c], want, rtol=1e-6, atol=1e-6)

    orig_plan = T.layer_plan

    def plan_without_conv_in_relu():
        return [(k, i) for k, i in orig_plan() if k != "relu"]

    import unittest.mock as um
    with um.patch.object(T, "layer_plan", plan_without_conv_in_relu):
        bad = T.decode(p, z).numpy()
    assert np.abs(bad[:, 0] - want).max() > 0.5, "missing conv_in ReLU not detected"
