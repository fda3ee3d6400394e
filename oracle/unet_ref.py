"""fp32 torch restatement of the reference engine's UNet path (CPU oracle).

Test infrastructure only: the HIP engine is checked against these functions,
never routed through them.  Tensors are NCHW float32; weights are a dict
``{diffusers key: tensor}`` in canonical layouts (conv ``[Co,Ci,kh,kw]``,
Linear ``[out,in]``).  Each function cites the reference code it restates.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from . import lcm as _lcm
from .weights import BLOCK_OUT

GN_GROUPS = 32
EPS = 1e-5  # vk_engine.cpp:548-549, :652 (GN and LN both use 1e-5)
HEADS = 8


def _t(x):
    return x if isinstance(x, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(x))


# ---------------------------------------------------------------------------
# ops


def silu(x):
    """silu_f32.comp: x / (1 + exp(-x))."""
    return x * torch.sigmoid(x)


def group_norm(x, gamma, beta, groups=GN_GROUPS, eps=EPS, act_silu=False):
    """Per-image GroupNorm, optional SiLU (groupnorm_f32.comp:12-28,
    groupnorm_silu.comp:13-31)."""
    y = F.group_norm(x, groups, gamma, beta, eps)
    return silu(y) if act_silu else y


def layer_norm(x, gamma, beta, eps=EPS):
    """Per-token LayerNorm over channels (layernorm_f32.comp:9-17)."""
    return F.layer_norm(x, (x.shape[-1],), gamma, beta, eps)


def linear(x, w, b=None):
    """``y = x @ W^T + b`` with W in ``[out,in]`` (the reference's ``matmul`` with
    its ``[in,out]`` operand, vk_engine.cpp:612-613)."""
    return F.linear(x, w, b)


def conv2d(x, w, b=None, stride=1, pad=None):
    """Direct conv (vk_engine.cpp:578-608 dispatch; CPU check :1157-1161)."""
    k = w.shape[-1]
    if pad is None:
        pad = k // 2
    return F.conv2d(x, w, b, stride=stride, padding=pad)


def upsample2x(x):
    """Nearest 2x per image (upsample_f32.comp:5-11)."""
    return F.interpolate(x, scale_factor=2.0, mode="nearest")


def gelu_erf(x):
    """Exact-erf GELU (geglu_f32.comp:6-9 approximates the same function)."""
    return 0.5 * x * (1.0 + torch.erf(x / math.sqrt(2.0)))


def geglu(g):
    """``a * gelu(b)`` with a = first half, b = second half (geglu_f32.comp:10-14)."""
    c2 = g.shape[-1] // 2
    return g[..., :c2] * gelu_erf(g[..., c2:])


def attention(q, k, v, heads, q_chunk=2048):
    """softmax(Q K^T d^-1/2) V per head and image (attention_f32.comp:20-69).

    q: [B, Sq, C], k/v: [B, Sk, C]; returns [B, Sq, C].  Two-pass softmax in fp32,
    chunked over queries to bound memory."""
    B, Sq, C = q.shape
    Sk = k.shape[1]
    d = C // heads
    scale = 1.0 / math.sqrt(d)
    qh = q.reshape(B, Sq, heads, d).permute(0, 2, 1, 3)
    kh = k.reshape(B, Sk, heads, d).permute(0, 2, 3, 1)
    vh = v.reshape(B, Sk, heads, d).permute(0, 2, 1, 3)
    out = torch.empty(B, heads, Sq, d, dtype=q.dtype)
    for s0 in range(0, Sq, q_chunk):
        s = torch.matmul(qh[:, :, s0:s0 + q_chunk], kh) * scale
        p = torch.softmax(s, dim=-1)
        out[:, :, s0:s0 + q_chunk] = torch.matmul(p, vh)
    return out.permute(0, 2, 1, 3).reshape(B, Sq, C)


# ---------------------------------------------------------------------------
# blocks


def time_mlp(p, temb_proj):
    """linear_1 + bias, SiLU, linear_2 + bias (vk_engine.cpp:716-717)."""
    t = silu(linear(temb_proj, p["time_embedding.linear_1.weight"], p["time_embedding.linear_1.bias"]))
    return linear(t, p["time_embedding.linear_2.weight"], p["time_embedding.linear_2.bias"])


def resnet(p, pf, x, temb):
    """ResNet block (vk_engine.cpp:623-637); ``temb`` [1280] shared by the batch
    (or [B,1280])."""
    h = group_norm(x, p[pf + ".norm1.weight"], p[pf + ".norm1.bias"], act_silu=True)
    h = conv2d(h, p[pf + ".conv1.weight"], p[pf + ".conv1.bias"])
    tp = linear(silu(temb), p[pf + ".time_emb_proj.weight"], p[pf + ".time_emb_proj.bias"])
    if tp.dim() == 1:
        tp = tp[None]
    h = h + tp[:, :, None, None]
    h = group_norm(h, p[pf + ".norm2.weight"], p[pf + ".norm2.bias"], act_silu=True)
    h = conv2d(h, p[pf + ".conv2.weight"], p[pf + ".conv2.bias"])
    if (pf + ".conv_shortcut.weight") in p:
        x = conv2d(x, p[pf + ".conv_shortcut.weight"], p[pf + ".conv_shortcut.bias"], pad=0)
    return x + h


def transformer(p, pf, x, ctx, heads=HEADS):
    """Spatial transformer (vk_engine.cpp:640-675).  x: [B,C,H,W]; ctx: [B,L,768]."""
    B, C, H, W = x.shape
    b = pf + ".transformer_blocks.0"
    g = group_norm(x, p[pf + ".norm.weight"], p[pf + ".norm.bias"])
    t = conv2d(g, p[pf + ".proj_in.weight"], p[pf + ".proj_in.bias"], pad=0)
    t = t.reshape(B, C, H * W).transpose(1, 2)  # T_CH: [B, HW, C]
    h = layer_norm(t, p[b + ".norm1.weight"], p[b + ".norm1.bias"])
    q = linear(h, p[b + ".attn1.to_q.weight"])
    k = linear(h, p[b + ".attn1.to_k.weight"])
    v = linear(h, p[b + ".attn1.to_v.weight"])
    a = attention(q, k, v, heads)
    t = t + linear(a, p[b + ".attn1.to_out.0.weight"], p[b + ".attn1.to_out.0.bias"])
    h = layer_norm(t, p[b + ".norm2.weight"], p[b + ".norm2.bias"])
    q = linear(h, p[b + ".attn2.to_q.weight"])
    k = linear(ctx, p[b + ".attn2.to_k.weight"])
    v = linear(ctx, p[b + ".attn2.to_v.weight"])
    a = attention(q, k, v, heads)
    t = t + linear(a, p[b + ".attn2.to_out.0.weight"], p[b + ".attn2.to_out.0.bias"])
    h = layer_norm(t, p[b + ".norm3.weight"], p[b + ".norm3.bias"])
    ff = geglu(linear(h, p[b + ".ff.net.0.proj.weight"], p[b + ".ff.net.0.proj.bias"]))
    t = t + linear(ff, p[b + ".ff.net.2.weight"], p[b + ".ff.net.2.bias"])
    t = t.transpose(1, 2).reshape(B, C, H, W)  # T_HC
    return x + conv2d(t, p[pf + ".proj_out.weight"], p[pf + ".proj_out.bias"], pad=0)


def downsample(p, pf, x):
    """conv3x3 stride 2 pad 1 (vk_engine.cpp:689-692)."""
    return conv2d(x, p[pf + ".conv.weight"], p[pf + ".conv.bias"], stride=2, pad=1)


def upsample(p, pf, x):
    """nearest 2x then conv3x3 (vk_engine.cpp:693-697)."""
    return conv2d(upsample2x(x), p[pf + ".conv.weight"], p[pf + ".conv.bias"])


def unet_forward(p, lat, temb_proj, ctx):
    """Full UNet forward (vk_engine.cpp:711-790).

    lat: [B,4,H,W]; temb_proj: [320] (shared by the batch, as ``tembp`` is) or
    [B,320]; ctx: [B,L,768].  Returns eps [B,4,H,W]."""
    lat, temb_proj, ctx = _t(lat).float(), _t(temb_proj).float(), _t(ctx).float()
    temb = time_mlp(p, temb_proj)
    x = conv2d(lat, p["conv_in.weight"], p["conv_in.bias"])
    skips = [x]
    cprev = 320
    for i in range(4):  # vk_engine.cpp:723-742
        cout = BLOCK_OUT[i]
        for r in range(2):
            x = resnet(p, f"down_blocks.{i}.resnets.{r}", x, temb)
            if i < 3:
                x = transformer(p, f"down_blocks.{i}.attentions.{r}", x, ctx)
            skips.append(x)
        cprev = cout
        if i < 3:
            x = downsample(p, f"down_blocks.{i}.downsamplers.0", x)
            skips.append(x)
    x = resnet(p, "mid_block.resnets.0", x, temb)  # :744-746
    x = transformer(p, "mid_block.attentions.0", x, ctx)
    x = resnet(p, "mid_block.resnets.1", x, temb)
    for i in range(4):  # :748-779
        for r in range(3):
            x = torch.cat([x, skips.pop()], dim=1)  # concat(prev, skip), :678-688
            x = resnet(p, f"up_blocks.{i}.resnets.{r}", x, temb)
            if i > 0:
                x = transformer(p, f"up_blocks.{i}.attentions.{r}", x, ctx)
        if i < 3:
            x = upsample(p, f"up_blocks.{i}.upsamplers.0", x)
    del cprev
    x = group_norm(x, p["conv_norm_out.weight"], p["conv_norm_out.bias"], act_silu=True)  # :781
    return conv2d(x, p["conv_out.weight"], p["conv_out.bias"])  # :782


def denoise_lcm(p, lat, cond, uncond, steps=4, guidance=8.0, noise=None, trace=None):
    """4-step LCM + batch-CFG loop (VulkanUnetPipeline.kt:63-97).

    lat: [4,H,W] float32; cond/uncond: [L,768]; noise: [steps-1,4,H,W] injected
    noise (the reference draws it from its RNG, :87).  Returns the final latent.
    ``trace`` (a list) receives (latent_in, cond_eps, uncond_eps, latent_out) per step."""
    sched = _lcm.LcmSchedule(steps)
    ctx = torch.stack([_t(cond).float(), _t(uncond).float()])
    x = np.asarray(lat, np.float32)
    for idx, t in enumerate(sched.timesteps):
        x_in = x.copy()
        temb = torch.from_numpy(_lcm.time_proj(t))
        both = torch.from_numpy(np.stack([x, x]))
        with torch.no_grad():
            eps2 = unet_forward(p, both, temb, ctx).numpy()
        eps = _lcm.cfg_combine(eps2[0], eps2[1], guidance)
        nz = None if idx == steps - 1 else noise[idx]
        x = sched.step(idx, x, eps, nz)
        if trace is not None:
            trace.append((x_in, eps2[0].copy(), eps2[1].copy(), x.copy()))
    return x


# ---------------------------------------------------------------------------
# metric


def rel_err_l1(got, ref) -> float:
    """sum|ref - got| / sum|ref| (vk_engine.cpp:698-704; run_ref.py:46)."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    return float(np.abs(ref - got).sum() / (np.abs(ref).sum() + 1e-30))


def to_torch(weights: dict):
    return {k: torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32)) for k, v in weights.items()}
