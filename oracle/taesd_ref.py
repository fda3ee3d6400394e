"""CPU fp32 restatement of the TAESD latent decoder (test infrastructure only).

The reference decodes the final latent with a LiteRT model exported from diffusers'
``AutoencoderTiny.from_pretrained("madebyollin/taesd")`` (tools/export_taesd.py:52-54,
contract stated at :2: ``[1,4,64,64] -> [1,3,512,512]``, output in [-1, 1]; consumed by
``VulkanUnetPipeline.kt:55-61`` / ``toBitmap`` at :99-109).  That model is a third-party
dependency absent from the reference tree (diffusers, no pinned version in the reference;
TAESD by madebyollin), so this module restates its published decoder, diffusers
``DecoderTiny`` with the default AutoencoderTiny configuration:

    x = 3 tanh(x / 3)                                   (input clamp)
    conv3x3(4 -> 64) + ReLU
    3 x Block(64), upsample x2 (nearest), conv3x3(64 -> 64, no bias)
    3 x Block(64), upsample x2, conv3x3 (no bias)
    3 x Block(64), upsample x2, conv3x3 (no bias)
    1 x Block(64), conv3x3(64 -> 3)
    y = 2 x - 1                                          ([0, 1] -> [-1, 1])

    Block(x) = ReLU(conv(ReLU(conv(ReLU(conv(x))))) + x)   (AutoencoderTinyBlock, 64 -> 64)

Parameter names are the diffusers keys of ``AutoencoderTiny.decoder``
(``decoder.layers.<i>...``, Sequential indices of the layer list above).

Parity against the reference is unpinned: the reference ships neither TAESD weights nor
decoded fixtures.  The restatement is pinned by constructed-weight checks
(tests/test_oracle_taesd.py) that fix the wiring: the clamp, every residual, the three
upsamplings and the output affine.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import weights as _w

LATENT_C = 4
CH = 64
OUT_C = 3
# (number of blocks, upsample after) per stage: num_blocks=(3, 3, 3, 1)
STAGES = ((3, True), (3, True), (3, True), (1, False))
# seeded random init: conv weights N(0, CONV_STD) (activations neither vanish nor explode
# through 30 ReLU convs with residuals), biases 0 (baseline) or N(0, 0.02) (affine)
CONV_STD = 0.04


def layer_plan():
    """[(kind, index)] of decoder.layers in order: conv_in, relu, blocks, upsample, conv..."""
    plan = [("conv_in", 0), ("relu", 1)]
    i = 2
    for nb, up in STAGES:
        for _ in range(nb):
            plan.append(("block", i))
            i += 1
        if up:
            plan.append(("upsample", i))
            i += 1
            plan.append(("conv_nobias", i))
            i += 1
        else:
            plan.append(("conv_out", i))
            i += 1
    return plan


def param_specs():
    """All decoder parameters (name, canonical shape, kind) in layer order."""
    ps = []
    for kind, i in layer_plan():
        pf = f"decoder.layers.{i}"
        if kind == "conv_in":
            ps += [_w.Param(pf + ".weight", (CH, LATENT_C, 3, 3), "conv"), _w.Param(pf + ".bias", (CH,), "bias")]
        elif kind == "block":
            for j in (0, 2, 4):
                ps += [_w.Param(f"{pf}.conv.{j}.weight", (CH, CH, 3, 3), "conv"),
                       _w.Param(f"{pf}.conv.{j}.bias", (CH,), "bias")]
        elif kind == "conv_nobias":
            ps += [_w.Param(pf + ".weight", (CH, CH, 3, 3), "conv")]
        elif kind == "conv_out":
            ps += [_w.Param(pf + ".weight", (OUT_C, CH, 3, 3), "conv"), _w.Param(pf + ".bias", (OUT_C,), "bias")]
    return ps


def generate(seed: int, mode: str = "baseline"):
    """Seeded decoder weights {name: float32 ndarray}, fp16-representable values."""
    if mode not in ("baseline", "affine"):
        raise ValueError(mode)
    out = {}
    for p in param_specs():
        if p.kind == "conv":
            out[p.name] = _w.gauss(p.name, p.shape, seed, 0.0, CONV_STD)
        elif mode == "baseline":
            out[p.name] = np.zeros(p.shape, np.float32)
        else:
            out[p.name] = _w.gauss(p.name, p.shape, seed, 0.0, 0.02)
    return out


def _conv(x, w, b):
    return F.conv2d(x, w, b, padding=1)


def block(p, pf, x):
    """AutoencoderTinyBlock(64, 64): ReLU(conv(ReLU(conv(ReLU(conv(x))))) + x)."""
    h = F.relu(_conv(x, p[pf + ".conv.0.weight"], p[pf + ".conv.0.bias"]))
    h = F.relu(_conv(h, p[pf + ".conv.2.weight"], p[pf + ".conv.2.bias"]))
    h = _conv(h, p[pf + ".conv.4.weight"], p[pf + ".conv.4.bias"])
    return F.relu(h + x)


def clamp(x):
    """DecoderTiny's input clamp: 3 tanh(x / 3)."""
    return torch.tanh(x / 3.0) * 3.0


def decode(p, z):
    """z: [B, 4, H, W] latent (numpy or torch) -> image [B, 3, 8H, 8W] in fp32, ~[-1, 1]."""
    p = {k: torch.as_tensor(np.asarray(v), dtype=torch.float32) for k, v in p.items()}
    x = clamp(torch.as_tensor(np.asarray(z), dtype=torch.float32))
    for kind, i in layer_plan():
        pf = f"decoder.layers.{i}"
        if kind == "conv_in":
            x = _conv(x, p[pf + ".weight"], p[pf + ".bias"])
        elif kind == "relu":
            x = F.relu(x)
        elif kind == "block":
            x = block(p, pf, x)
        elif kind == "upsample":
            x = F.interpolate(x, scale_factor=2, mode="nearest")
        elif kind == "conv_nobias":
            x = _conv(x, p[pf + ".weight"], None)
        elif kind == "conv_out":
            x = _conv(x, p[pf + ".weight"], p[pf + ".bias"])
    return x * 2.0 - 1.0
