"""CPU fp32 restatement of the Stable Diffusion 1.5 VAE decoder (test infrastructure only).

The reference's Vulkan pipeline decodes the final latent with a LiteRT model,
``gpu_vae.tflite`` (``VulkanUnetPipeline.kt:55-61``, contract ``vae: latents[1,4,64,64] ->
image[1,3,512,512]`` in [-1, 1] as stated for the same asset in ``GpuMonoPipeline.kt:26``),
exported from diffusers' ``AutoencoderKL`` of the SD1.5 checkpoint; the reference's own
full-VAE call is ``pipe.vae.decode(z / pipe.vae.config.scaling_factor).sample``
(``tools/export_taesd.py:53``).  The model and its exporter are third-party (diffusers, no
pinned version in the reference) and absent from the tree, so this module restates the
published decoder with the SD1.5 configuration (block_out_channels (128, 256, 512, 512),
layers_per_block 2, 32 groups, GroupNorm eps 1e-6, scaling_factor 0.18215):

    h = post_quant_conv(z / 0.18215)                       1x1, 4 -> 4
    h = conv_in(h)                                         3x3, 4 -> 512
    h = resnet(h); h = attention(h); h = resnet(h)         mid block at 512 channels
    4 up blocks (512, 512, 256, 128 channels), each 3 resnets, then (not the last)
        nearest 2x upsampling and a 3x3 conv
    h = conv_out(SiLU(GroupNorm(h)))                       3x3, 128 -> 3

    resnet(x) = shortcut(x) + conv2(SiLU(GN2(conv1(SiLU(GN1(x))))))
                (shortcut: a 1x1 conv where the channel count changes, else identity)
    attention(x) = x + to_out(softmax(q k^T / sqrt(512)) v),  q, k, v = to_q / to_k / to_v of
                GroupNorm(x) over the H*W tokens, one head of 512

Parameter names are the diffusers keys of ``AutoencoderKL`` (``post_quant_conv.*`` and
``decoder.*``).  The inventory holds 49,490,179 decoder parameters plus the 20 of
post_quant_conv, the published size of the SD1.5 VAE decoder.

Parity against the reference is unpinned: the reference ships neither VAE weights nor
decoded fixtures.  The restatement is pinned by that parameter count and by
constructed-weight checks (tests/test_oracle_vae.py) that fix the scaling, the GroupNorm
epsilon, the single-head attention and its residual, the shortcuts, the nearest
upsampling and the final SiLU, each shown to fail on a planted mistake.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from . import weights as _w

LATENT_C = 4
OUT_C = 3
SCALING = 0.18215
BLOCK_OUT = (128, 256, 512, 512)
LAYERS = 2  # per encoder block; the decoder's up blocks hold LAYERS + 1 resnets
GROUPS = 32
EPS = 1e-6
# seeded random init: conv weights N(0, CONV_STD), the attention's Linear weights
# N(0, LINEAR_STD) (sharp enough for the softmax to matter), norms and biases per mode
CONV_STD = 0.02
LINEAR_STD = 0.1


def up_plan():
    """[(block, in channels, out channels, upsample)] of decoder.up_blocks in order."""
    rev = tuple(reversed(BLOCK_OUT))
    plan, prev = [], rev[0]
    for i, c in enumerate(rev):
        plan.append((i, prev, c, i < len(rev) - 1))
        prev = c
    return plan


def _resnet_specs(pf, cin, cout):
    P = _w.Param
    ps = [P(pf + ".norm1.weight", (cin,), "norm_w"), P(pf + ".norm1.bias", (cin,), "norm_b"),
          P(pf + ".conv1.weight", (cout, cin, 3, 3), "conv"), P(pf + ".conv1.bias", (cout,), "bias"),
          P(pf + ".norm2.weight", (cout,), "norm_w"), P(pf + ".norm2.bias", (cout,), "norm_b"),
          P(pf + ".conv2.weight", (cout, cout, 3, 3), "conv"), P(pf + ".conv2.bias", (cout,), "bias")]
    if cin != cout:
        ps += [P(pf + ".conv_shortcut.weight", (cout, cin, 1, 1), "conv"), P(pf + ".conv_shortcut.bias", (cout,), "bias")]
    return ps


def param_specs():
    """All decoder parameters (name, canonical shape, kind) in graph order."""
    P = _w.Param
    top = BLOCK_OUT[-1]
    ps = [P("post_quant_conv.weight", (LATENT_C, LATENT_C, 1, 1), "conv"),
          P("post_quant_conv.bias", (LATENT_C,), "bias"),
          P("decoder.conv_in.weight", (top, LATENT_C, 3, 3), "conv"), P("decoder.conv_in.bias", (top,), "bias")]
    ps += _resnet_specs("decoder.mid_block.resnets.0", top, top)
    a = "decoder.mid_block.attentions.0"
    ps += [P(a + ".group_norm.weight", (top,), "norm_w"), P(a + ".group_norm.bias", (top,), "norm_b")]
    for lin in ("to_q", "to_k", "to_v", "to_out.0"):
        ps += [P(f"{a}.{lin}.weight", (top, top), "linear"), P(f"{a}.{lin}.bias", (top,), "bias")]
    ps += _resnet_specs("decoder.mid_block.resnets.1", top, top)
    for i, cin, cout, up in up_plan():
        for j in range(LAYERS + 1):
            ps += _resnet_specs(f"decoder.up_blocks.{i}.resnets.{j}", cin if j == 0 else cout, cout)
        if up:
            u = f"decoder.up_blocks.{i}.upsamplers.0.conv"
            ps += [P(u + ".weight", (cout, cout, 3, 3), "conv"), P(u + ".bias", (cout,), "bias")]
    c0 = BLOCK_OUT[0]
    ps += [P("decoder.conv_norm_out.weight", (c0,), "norm_w"), P("decoder.conv_norm_out.bias", (c0,), "norm_b"),
           P("decoder.conv_out.weight", (OUT_C, c0, 3, 3), "conv"), P("decoder.conv_out.bias", (OUT_C,), "bias")]
    return ps


def generate(seed: int, mode: str = "baseline"):
    """Seeded decoder weights {name: float32 ndarray}, fp16-representable values."""
    if mode not in ("baseline", "affine"):
        raise ValueError(mode)
    out = {}
    for p in param_specs():
        if p.kind == "conv":
            out[p.name] = _w.gauss(p.name, p.shape, seed, 0.0, CONV_STD)
        elif p.kind == "linear":
            out[p.name] = _w.gauss(p.name, p.shape, seed, 0.0, LINEAR_STD)
        elif mode == "baseline":
            out[p.name] = np.full(p.shape, 1.0 if p.kind == "norm_w" else 0.0, np.float32)
        else:
            out[p.name] = _w.gauss(p.name, p.shape, seed, 1.0 if p.kind == "norm_w" else 0.0, 0.02)
    return out


def group_norm(x, w, b, eps=EPS):
    """GroupNorm(32) over (channels of the group, H, W) per image, biased variance."""
    B, C = x.shape[:2]
    xg = x.reshape(B, GROUPS, -1)
    mean = xg.mean(-1, keepdim=True)
    var = ((xg - mean) ** 2).mean(-1, keepdim=True)
    y = ((xg - mean) / torch.sqrt(var + eps)).reshape(x.shape)
    return y * w.reshape(1, C, 1, 1) + b.reshape(1, C, 1, 1)


def resnet(p, pf, x):
    """ResnetBlock2D without time embedding (eps 1e-6, output scale 1)."""
    h = F.silu(group_norm(x, p[pf + ".norm1.weight"], p[pf + ".norm1.bias"]))
    h = F.conv2d(h, p[pf + ".conv1.weight"], p[pf + ".conv1.bias"], padding=1)
    h = F.silu(group_norm(h, p[pf + ".norm2.weight"], p[pf + ".norm2.bias"]))
    h = F.conv2d(h, p[pf + ".conv2.weight"], p[pf + ".conv2.bias"], padding=1)
    if pf + ".conv_shortcut.weight" in p:
        x = F.conv2d(x, p[pf + ".conv_shortcut.weight"], p[pf + ".conv_shortcut.bias"])
    return x + h


def attention(p, pf, x):
    """The mid block's self-attention over the H*W tokens: one head of C, residual added."""
    B, C, H, W = x.shape
    h = group_norm(x, p[pf + ".group_norm.weight"], p[pf + ".group_norm.bias"])
    t = h.reshape(B, C, H * W).transpose(1, 2)  # [B, HW, C]
    q = F.linear(t, p[pf + ".to_q.weight"], p[pf + ".to_q.bias"])
    k = F.linear(t, p[pf + ".to_k.weight"], p[pf + ".to_k.bias"])
    v = F.linear(t, p[pf + ".to_v.weight"], p[pf + ".to_v.bias"])
    s = torch.matmul(q, k.transpose(1, 2)) / math.sqrt(C)
    o = torch.matmul(torch.softmax(s, dim=-1), v)
    o = F.linear(o, p[pf + ".to_out.0.weight"], p[pf + ".to_out.0.bias"])
    return x + o.transpose(1, 2).reshape(B, C, H, W)


def upsample(x):
    """Nearest-neighbour 2x: out[y, x] = in[y // 2, x // 2]."""
    return F.interpolate(x, scale_factor=2, mode="nearest")


def decode(p, z):
    """z: [B, 4, H, W] UNet latent (numpy or torch) -> image [B, 3, 8H, 8W] fp32, ~[-1, 1]."""
    p = {k: torch.as_tensor(np.asarray(v), dtype=torch.float32) for k, v in p.items()}
    h = torch.as_tensor(np.asarray(z), dtype=torch.float32) / SCALING
    h = F.conv2d(h, p["post_quant_conv.weight"], p["post_quant_conv.bias"])
    h = F.conv2d(h, p["decoder.conv_in.weight"], p["decoder.conv_in.bias"], padding=1)
    h = resnet(p, "decoder.mid_block.resnets.0", h)
    h = attention(p, "decoder.mid_block.attentions.0", h)
    h = resnet(p, "decoder.mid_block.resnets.1", h)
    for i, _cin, _cout, up in up_plan():
        for j in range(LAYERS + 1):
            h = resnet(p, f"decoder.up_blocks.{i}.resnets.{j}", h)
        if up:
            u = f"decoder.up_blocks.{i}.upsamplers.0.conv"
            h = F.conv2d(upsample(h), p[u + ".weight"], p[u + ".bias"], padding=1)
    h = F.silu(group_norm(h, p["decoder.conv_norm_out.weight"], p["decoder.conv_norm_out.bias"]))
    return F.conv2d(h, p["decoder.conv_out.weight"], p["decoder.conv_out.bias"], padding=1)
