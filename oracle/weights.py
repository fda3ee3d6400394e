"""Parameter inventory of the reference UNet graph and the seeded generator.

The inventory walks the graph in the order ``runGraph`` loads weights
(vk_engine.cpp:711-790, blocks at :623-697) and names every tensor by the
diffusers key the reference's ``W(name)`` loader reads (vk_engine.cpp:497-508).
Shapes are the canonical diffusers layouts: conv ``[Co, Ci, kh, kw]``, Linear
``[out, in]``.  (The reference's on-disk Linear files are ``[in, out]``; that
transpose belongs to the loader, not to the inventory.)

Generated values follow the specification in ``oracle/gen.c``.  Init modes:
  * ``"baseline"``: conv/linear weights fp16(N(0, 0.02)), norm gamma 1, beta 0,
    biases 0 -- the random-init rule of the benchmarked configurations;
  * ``"affine"``: as baseline, but biases and norm betas are fp16(N(0, 0.02)) and
    norm gammas fp16(N(1, 0.02)), so bias and affine paths carry signal in tests.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

CTX_DIM = 768
TEMB_IN = 320
TEMB_DIM = 1280
BLOCK_OUT = (320, 640, 1280, 1280)


@dataclass(frozen=True)
class Param:
    name: str
    shape: tuple
    kind: str  # conv | linear | norm_w | norm_b | bias

    @property
    def numel(self) -> int:
        n = 1
        for s in self.shape:
            n *= s
        return n


def _lib():
    """Load (building if needed) the oracle's C generator."""
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        src = os.path.join(_HERE, "gen.c")
        if not os.path.exists(path) or os.path.getmtime(path) < os.path.getmtime(src):
            subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
        lib = ctypes.CDLL(path)
        lib.oracle_fnv1a64.restype = ctypes.c_uint64
        lib.oracle_fnv1a64.argtypes = [ctypes.c_char_p]
        lib.oracle_tensor_key.restype = ctypes.c_uint64
        lib.oracle_tensor_key.argtypes = [ctypes.c_char_p, ctypes.c_uint64]
        for fn in (lib.oracle_gauss_fill, lib.oracle_gauss_fill_f32):
            fn.restype = None
            fn.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_double,
                           ctypes.c_double, ctypes.c_void_p]
        _LIB = lib
    return _LIB


def tensor_key(name: str, seed: int) -> int:
    return int(_lib().oracle_tensor_key(name.encode(), ctypes.c_uint64(seed & (2**64 - 1))))


def gauss(name: str, shape, seed: int, mean: float = 0.0, std: float = 1.0,
          fp16: bool = True) -> np.ndarray:
    """Seeded N(mean, std) tensor; fp16-rounded values (as float32) when ``fp16``."""
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, dtype=np.float32)
    fn = _lib().oracle_gauss_fill if fp16 else _lib().oracle_gauss_fill_f32
    fn(tensor_key(name, seed), n, mean, std, out.ctypes.data)
    return out.reshape(shape)


# ---------------------------------------------------------------------------
# inventory


def _resnet(pf: str, cin: int, cout: int):
    """ResNet block parameters (vk_engine.cpp:623-637)."""
    ps = [
        Param(pf + ".norm1.weight", (cin,), "norm_w"),
        Param(pf + ".norm1.bias", (cin,), "norm_b"),
        Param(pf + ".conv1.weight", (cout, cin, 3, 3), "conv"),
        Param(pf + ".conv1.bias", (cout,), "bias"),
        Param(pf + ".time_emb_proj.weight", (cout, TEMB_DIM), "linear"),
        Param(pf + ".time_emb_proj.bias", (cout,), "bias"),
        Param(pf + ".norm2.weight", (cout,), "norm_w"),
        Param(pf + ".norm2.bias", (cout,), "norm_b"),
        Param(pf + ".conv2.weight", (cout, cout, 3, 3), "conv"),
        Param(pf + ".conv2.bias", (cout,), "bias"),
    ]
    if cin != cout:
        ps += [Param(pf + ".conv_shortcut.weight", (cout, cin, 1, 1), "conv"),
               Param(pf + ".conv_shortcut.bias", (cout,), "bias")]
    return ps


def _transformer(pf: str, c: int):
    """Spatial transformer parameters (vk_engine.cpp:640-675)."""
    b = pf + ".transformer_blocks.0"
    return [
        Param(pf + ".norm.weight", (c,), "norm_w"),
        Param(pf + ".norm.bias", (c,), "norm_b"),
        Param(pf + ".proj_in.weight", (c, c, 1, 1), "conv"),
        Param(pf + ".proj_in.bias", (c,), "bias"),
        Param(b + ".norm1.weight", (c,), "norm_w"),
        Param(b + ".norm1.bias", (c,), "norm_b"),
        Param(b + ".attn1.to_q.weight", (c, c), "linear"),
        Param(b + ".attn1.to_k.weight", (c, c), "linear"),
        Param(b + ".attn1.to_v.weight", (c, c), "linear"),
        Param(b + ".attn1.to_out.0.weight", (c, c), "linear"),
        Param(b + ".attn1.to_out.0.bias", (c,), "bias"),
        Param(b + ".norm2.weight", (c,), "norm_w"),
        Param(b + ".norm2.bias", (c,), "norm_b"),
        Param(b + ".attn2.to_q.weight", (c, c), "linear"),
        Param(b + ".attn2.to_k.weight", (c, CTX_DIM), "linear"),
        Param(b + ".attn2.to_v.weight", (c, CTX_DIM), "linear"),
        Param(b + ".attn2.to_out.0.weight", (c, c), "linear"),
        Param(b + ".attn2.to_out.0.bias", (c,), "bias"),
        Param(b + ".norm3.weight", (c,), "norm_w"),
        Param(b + ".norm3.bias", (c,), "norm_b"),
        Param(b + ".ff.net.0.proj.weight", (8 * c, c), "linear"),
        Param(b + ".ff.net.0.proj.bias", (8 * c,), "bias"),
        Param(b + ".ff.net.2.weight", (c, 4 * c), "linear"),
        Param(b + ".ff.net.2.bias", (c,), "bias"),
        Param(pf + ".proj_out.weight", (c, c, 1, 1), "conv"),
        Param(pf + ".proj_out.bias", (c,), "bias"),
    ]


def _conv(pf: str, cin: int, cout: int, k: int = 3):
    return [Param(pf + ".weight", (cout, cin, k, k), "conv"),
            Param(pf + ".bias", (cout,), "bias")]


def param_specs():
    """All UNet parameters in graph order (vk_engine.cpp:716-782)."""
    ps = [
        Param("time_embedding.linear_1.weight", (TEMB_DIM, TEMB_IN), "linear"),
        Param("time_embedding.linear_1.bias", (TEMB_DIM,), "bias"),
        Param("time_embedding.linear_2.weight", (TEMB_DIM, TEMB_DIM), "linear"),
        Param("time_embedding.linear_2.bias", (TEMB_DIM,), "bias"),
    ]
    ps += _conv("conv_in", 4, 320)
    cprev = 320
    for i in range(4):
        cout = BLOCK_OUT[i]
        for r in range(2):
            ps += _resnet(f"down_blocks.{i}.resnets.{r}", cprev if r == 0 else cout, cout)
            if i < 3:
                ps += _transformer(f"down_blocks.{i}.attentions.{r}", cout)
        cprev = cout
        if i < 3:
            ps += _conv(f"down_blocks.{i}.downsamplers.0.conv", cout, cout)
    ps += _resnet("mid_block.resnets.0", 1280, 1280)
    ps += _transformer("mid_block.attentions.0", 1280)
    ps += _resnet("mid_block.resnets.1", 1280, 1280)
    skips = skip_channels()
    up_out = (1280, 1280, 640, 320)
    cprev = 1280
    for i in range(4):
        cout = up_out[i]
        for r in range(3):
            cs = skips.pop()
            ps += _resnet(f"up_blocks.{i}.resnets.{r}", cprev + cs, cout)
            cprev = cout
            if i > 0:
                ps += _transformer(f"up_blocks.{i}.attentions.{r}", cout)
        if i < 3:
            ps += _conv(f"up_blocks.{i}.upsamplers.0.conv", cout, cout)
    ps += [Param("conv_norm_out.weight", (320,), "norm_w"),
           Param("conv_norm_out.bias", (320,), "norm_b")]
    ps += _conv("conv_out", 320, 4)
    return ps


def skip_channels():
    """Channel counts of the 12 skip tensors in push order (vk_engine.cpp:720-742)."""
    sk = [320]
    for i in range(4):
        sk += [BLOCK_OUT[i]] * 2
        if i < 3:
            sk.append(BLOCK_OUT[i])
    return sk


def generate(seed: int, mode: str = "baseline", dtype=np.float32, names=None):
    """Generate the full weight dict {name: ndarray (canonical layout)}."""
    if mode not in ("baseline", "affine"):
        raise ValueError(mode)
    out = {}
    for p in param_specs():
        if names is not None and p.name not in names:
            continue
        out[p.name] = param_value(p, seed, mode).astype(dtype, copy=False)
    return out


def param_value(p: Param, seed: int, mode: str = "baseline") -> np.ndarray:
    if p.kind in ("conv", "linear"):
        return gauss(p.name, p.shape, seed, 0.0, 0.02)
    if mode == "baseline":
        if p.kind == "norm_w":
            return np.ones(p.shape, np.float32)
        return np.zeros(p.shape, np.float32)
    if p.kind == "norm_w":
        return gauss(p.name, p.shape, seed, 1.0, 0.02)
    return gauss(p.name, p.shape, seed, 0.0, 0.02)
