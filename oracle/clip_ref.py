"""CPU fp32 restatement of the SD1.5 CLIP text encoder (test infrastructure only).

The reference encodes the 77 token ids of a prompt with a LiteRT export of SD1.5's
``text_encoder`` (``VulkanUnetPipeline.kt:48-53``: int[77] -> [1, 77, 768], read as the
UNet's cross-attention context; tokens from ``ClipTokenizer.kt``).  That encoder is
diffusers' ``CLIPTextModel`` (openai/clip-vit-large-patch14 text tower, transformers), a
third-party dependency absent from the reference tree.  This module restates its published
algorithm with that configuration:

    x = token_embedding[ids] + position_embedding[0..76]
    12 x { x = x + out_proj(causal_attention(LN1(x)));  x = x + fc2(quick_gelu(fc1(LN2(x)))) }
    last_hidden_state = final_layer_norm(x)

attention: 12 heads of 64, q scaled by 64^-0.5, key j > query i masked; LayerNorm eps
1e-5; quick_gelu(x) = x * sigmoid(1.702 x).  Names are the diffusers checkpoint keys
(``text_model.*``).

The restatement is pinned against transformers' own ``CLIPTextModel`` built from the same
configuration and weights (tests/test_oracle_clip.py); against the reference it is
unpinned (no CLIP weights or encoded fixtures ship with it).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import weights as _w

VOCAB = 49408
SEQ = 77
HIDDEN = 768
LAYERS = 12
HEADS = 12
FFN = 3072
EPS = 1e-5
PREFIX = "text_model."


def param_specs(vocab=VOCAB, hidden=HIDDEN, layers=LAYERS, ffn=FFN, seq=SEQ):
    """All encoder parameters (name, canonical shape, kind); Linear [out, in]."""
    ps = [_w.Param(PREFIX + "embeddings.token_embedding.weight", (vocab, hidden), "embed"),
          _w.Param(PREFIX + "embeddings.position_embedding.weight", (seq, hidden), "embed")]
    for i in range(layers):
        pf = f"{PREFIX}encoder.layers.{i}"
        for n in ("q_proj", "k_proj", "v_proj", "out_proj"):
            ps += [_w.Param(f"{pf}.self_attn.{n}.weight", (hidden, hidden), "linear"),
                   _w.Param(f"{pf}.self_attn.{n}.bias", (hidden,), "bias")]
        ps += [_w.Param(f"{pf}.layer_norm1.weight", (hidden,), "norm_w"),
               _w.Param(f"{pf}.layer_norm1.bias", (hidden,), "norm_b"),
               _w.Param(f"{pf}.mlp.fc1.weight", (ffn, hidden), "linear"),
               _w.Param(f"{pf}.mlp.fc1.bias", (ffn,), "bias"),
               _w.Param(f"{pf}.mlp.fc2.weight", (hidden, ffn), "linear"),
               _w.Param(f"{pf}.mlp.fc2.bias", (hidden,), "bias"),
               _w.Param(f"{pf}.layer_norm2.weight", (hidden,), "norm_w"),
               _w.Param(f"{pf}.layer_norm2.bias", (hidden,), "norm_b")]
    ps += [_w.Param(PREFIX + "final_layer_norm.weight", (hidden,), "norm_w"),
           _w.Param(PREFIX + "final_layer_norm.bias", (hidden,), "norm_b")]
    return ps


def generate(seed: int, mode: str = "baseline", **cfg):
    """Seeded weights {name: float32 ndarray}: Linear / embedding N(0, 0.02); LayerNorm
    gamma 1 / beta 0 and biases 0 (baseline) or gamma N(1, .02), beta / bias N(0, .02)
    (affine).  Values are fp16-representable."""
    if mode not in ("baseline", "affine"):
        raise ValueError(mode)
    out = {}
    for p in param_specs(**cfg):
        if p.kind in ("linear", "embed"):
            out[p.name] = _w.gauss(p.name, p.shape, seed, 0.0, 0.02)
        elif mode == "baseline":
            out[p.name] = (np.ones if p.kind == "norm_w" else np.zeros)(p.shape, np.float32)
        elif p.kind == "norm_w":
            out[p.name] = _w.gauss(p.name, p.shape, seed, 1.0, 0.02)
        else:
            out[p.name] = _w.gauss(p.name, p.shape, seed, 0.0, 0.02)
    return out


def quick_gelu(x):
    return x * torch.sigmoid(1.702 * x)


def causal_attention(q, k, v, heads):
    """q, k, v: [B, S, C] -> [B, S, C]; head h = columns [h*d, (h+1)*d)."""
    B, S, C = q.shape
    d = C // heads
    q = q.view(B, S, heads, d).transpose(1, 2) * (d ** -0.5)
    k = k.view(B, S, heads, d).transpose(1, 2)
    v = v.view(B, S, heads, d).transpose(1, 2)
    s = q @ k.transpose(-1, -2)
    mask = torch.triu(torch.ones(S, S, dtype=torch.bool), diagonal=1)
    s = s.masked_fill(mask, float("-inf"))
    o = torch.softmax(s, dim=-1) @ v
    return o.transpose(1, 2).reshape(B, S, C)


def encode(p, ids, heads=HEADS):
    """ids: int [B, S] token ids -> last_hidden_state [B, S, C] (fp32 torch tensor)."""
    p = {k: torch.as_tensor(np.asarray(v), dtype=torch.float32) for k, v in p.items()}
    ids = torch.as_tensor(np.asarray(ids), dtype=torch.long)
    B, S = ids.shape
    tok = p[PREFIX + "embeddings.token_embedding.weight"]
    pos = p[PREFIX + "embeddings.position_embedding.weight"]
    C = tok.shape[1]
    x = tok[ids.clamp(0, tok.shape[0] - 1)] + pos[:S][None]
    i = 0
    while f"{PREFIX}encoder.layers.{i}.layer_norm1.weight" in p:
        pf = f"{PREFIX}encoder.layers.{i}"

        def lin(name, t):
            return F.linear(t, p[f"{pf}.{name}.weight"], p[f"{pf}.{name}.bias"])

        h = F.layer_norm(x, (C,), p[pf + ".layer_norm1.weight"], p[pf + ".layer_norm1.bias"], EPS)
        a = causal_attention(lin("self_attn.q_proj", h), lin("self_attn.k_proj", h), lin("self_attn.v_proj", h), heads)
        x = x + lin("self_attn.out_proj", a)
        h = F.layer_norm(x, (C,), p[pf + ".layer_norm2.weight"], p[pf + ".layer_norm2.bias"], EPS)
        x = x + lin("mlp.fc2", quick_gelu(lin("mlp.fc1", h)))
        i += 1
    return F.layer_norm(x, (C,), p[PREFIX + "final_layer_norm.weight"], p[PREFIX + "final_layer_norm.bias"], EPS)
