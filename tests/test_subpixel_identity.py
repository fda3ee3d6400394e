"""The identity behind the engine's sub-pixel upsampling convs (GemmArgs::subpix,
fold_subpix_kernel): a 3x3 conv (pad 1) over the 2x nearest upsampling of X equals, for
each output phase (py, px), a 2x2 conv of X at rows y + py - 1 + ty and columns
x + px - 1 + tx whose tap (ty, tx) is the sum of the 3x3 taps (ky, kx) with
ty = (py + ky + 1) // 2 - py and tx = (px + kx + 1) // 2 - px.  Checked in float64
against the direct conv of the upsampled image (torch's nearest interpolation and
conv2d), with ragged sizes so the zero padding at every border is exercised; a planted
wrong tap map fails."""
import numpy as np
import torch
import torch.nn.functional as F


def subpixel_weights(w3, tap_map):
    co, ci = w3.shape[:2]
    w4 = np.zeros((4, co, ci, 2, 2))
    for ph in range(4):
        py, px = ph >> 1, ph & 1
        for ky in range(3):
            for kx in range(3):
                w4[ph, :, :, tap_map(py, ky), tap_map(px, kx)] += w3[:, :, ky, kx]
    return w4


def subpixel_conv(x, w4):
    b, ci, h, w = x.shape
    co = w4.shape[1]
    out = np.zeros((b, co, 2 * h, 2 * w))
    xp = np.pad(x, ((0, 0), (0, 0), (1, 1), (1, 1)))
    for ph in range(4):
        py, px = ph >> 1, ph & 1
        for ty in range(2):
            for tx in range(2):
                # input row y + py - 1 + ty is padded row y + py + ty
                patch = xp[:, :, py + ty:py + ty + h, px + tx:px + tx + w]
                out[:, :, py::2, px::2] += np.einsum("bchw,oc->bohw", patch, w4[ph, :, :, ty, tx])
    return out


def direct(x, w3):
    u = F.interpolate(torch.from_numpy(x), scale_factor=2, mode="nearest")
    return F.conv2d(u, torch.from_numpy(w3), padding=1).numpy()


def test_subpixel_form_equals_upsample_conv():
    rng = np.random.default_rng(5)
    for (b, ci, co, h, w) in [(2, 3, 4, 5, 7), (1, 5, 2, 1, 6), (3, 2, 3, 4, 4)]:
        x = rng.standard_normal((b, ci, h, w))
        w3 = rng.standard_normal((co, ci, 3, 3))
        got = subpixel_conv(x, subpixel_weights(w3, lambda p, k: (p + k + 1) // 2 - p))
        np.testing.assert_allclose(got, direct(x, w3), rtol=1e-12, atol=1e-12)


def test_planted_tap_map_fails():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((1, 2, 4, 5))
    w3 = rng.standard_normal((3, 2, 3, 3))
    bad = subpixel_conv(x, subpixel_weights(w3, lambda p, k: min(k, 1)))  # ignores the phase
    assert np.abs(bad - direct(x, w3)).max() > 1e-3
