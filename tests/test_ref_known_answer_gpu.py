"""The reference's own micro-benchmark cases as parity cases (GPU, through the C ABI).

The reference's bench JNI functions (vk_engine.cpp:224-480, :1017-1218, driven by
VulkanBench.kt:66-126) fill their operands with deterministic integer patterns such as
((i*131+7) % 17) * 0.01 - 0.08 and check a few sampled outputs against an fp32 CPU
recomputation (relErr thresholds 0.02 / 0.03).  Here the same patterns and the same
shapes run through this engine's ops and are compared over every output element
with the fp32 oracle on the fp16-rounded operands (relErr_L1 <= 1e-3, attention
<= 2e-3), and with the reference's sampled check on the unrounded fp32 operands at the
reference's own thresholds.
"""
import math

import numpy as np
import pytest
import torch

from conftest import rel_err_l1, say
from oracle import unet_ref as U

pytestmark = pytest.mark.gpu


def pattern(n, mul, add, mod, scale, off):
    """((i*mul + add) % mod) * scale - off in float32 arithmetic, i = 0 .. n-1."""
    i = np.arange(n, dtype=np.uint64)
    k = ((i * np.uint64(mul) + np.uint64(add)) % np.uint64(mod)).astype(np.float32)
    return k * np.float32(scale) - np.float32(off)


def h(a):
    return a.astype(np.float16).astype(np.float32)


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def sampled_rel(got, ref_fn, idx):
    """The reference's check: sum |ref - got| / sum |ref| over sampled outputs."""
    se = sr = 0.0
    for ix in idx:
        r = ref_fn(ix)
        se += abs(r - float(got[ix]))
        sr += abs(r)
    return se / (sr + 1e-6)


# ----------------------------------------------------------------- matmul

# VulkanBench.kt:72-78 (mm) and :84-85 (split-K conv shapes at 16^2 / 8^2, M = Cout,
# N = tiles, K = 9 Cin); operands of benchMatmul / benchSplitK (vk_engine.cpp:235-236,
# :298-299): A [M,K] = ((i*131+7)%17)*0.01-0.08, B [K,N] = ((i*61+13)%19)*0.01-0.09.
@pytest.mark.parametrize("M,N,K", [
    (4096, 2560, 320),    # ff-proj
    (4096, 320, 1280),    # ff-out
    (2048, 2048, 2048),   # square
    (1280, 256, 11520),   # conv 16^2 as split K
    (1280, 64, 11520),    # conv 8^2 as split K
])
def test_reference_matmul_shapes(op_engine, M, N, K):
    say(f"reference matmul {M}x{N}x{K}")
    e = op_engine
    A = pattern(M * K, 131, 7, 17, 0.01, 0.08).reshape(M, K)
    Bm = pattern(K * N, 61, 13, 19, 0.01, 0.09).reshape(K, N)
    W = np.ascontiguousarray(Bm.T)  # the engine's [N, K] weight
    ta, tw = e.upload(A.astype(np.float16)), e.upload(W.astype(np.float16))
    ty = e.tensor((M, N), 2)
    e.matmul(ta, tw, ty, M, N, K, flags=2)
    got = ty.numpy()
    ref = (t(h(A)) @ t(h(Bm))).numpy()
    err = rel_err_l1(got, ref)
    say(f"  relErr {err:.2e}")
    assert err < 1e-3
    # the reference's sampled check (vk_engine.cpp:246-250) on the fp32 operands, < 0.02
    g = got.reshape(-1)
    idx = [((s * 97 + 3) % M) * N + (s * 53 + 11) % N for s in range(16)]
    assert sampled_rel(g, lambda ix: float(np.dot(A[ix // N].astype(np.float64), Bm[:, ix % N])), idx) < 0.02


# ----------------------------------------------------------------- conv 3x3

# VulkanBench.kt:88-92 (conv 320->320 @64^2, 640->640 @32^2, 1280->1280 @16^2);
# operands of benchConvGemm (vk_engine.cpp:1129-1130): X [Cin,H,W] =
# ((i*131+7)%17)*0.02-0.16, W [Cout,Cin,3,3] = ((i*61+13)%19)*0.02-0.18.
@pytest.mark.parametrize("Ci,Co,H", [(320, 320, 64), (640, 640, 32), (1280, 1280, 16)])
def test_reference_conv_shapes(op_engine, Ci, Co, H):
    say(f"reference conv {Ci}->{Co} @{H}^2")
    e = op_engine
    X = pattern(Ci * H * H, 131, 7, 17, 0.02, 0.16).reshape(1, Ci, H, H)
    Wc = pattern(Co * Ci * 9, 61, 13, 19, 0.02, 0.18).reshape(Co, Ci, 3, 3)
    tx = e.upload(h(X).transpose(0, 2, 3, 1).astype(np.float16))
    tw = e.upload(h(Wc).transpose(0, 2, 3, 1).astype(np.float16))
    ty = e.tensor((1, H, H, Co))
    e.conv2d(tx, tw, ty, 1, H, H, Ci, Co, ksize=3)
    got = ty.numpy().astype(np.float32).transpose(0, 3, 1, 2)
    ref = U.conv2d(t(h(X)), t(h(Wc))).numpy()
    err = rel_err_l1(got, ref)
    say(f"  relErr {err:.2e}")
    assert err < 1e-3


# ----------------------------------------------------------------- GroupNorm

# VulkanBench.kt:103-104 (groupnorm 320x64^2 and 1280x16^2, 32 groups); operands of
# benchGroupNorm (vk_engine.cpp:395-396): X [C,HW] = ((i*131+7)%29)*0.1-1.4 (fp16),
# gamma = 0.8 + 0.01 (c%7), beta = 0.05 (c%5) - 0.1; threshold 0.03 (:414).
@pytest.mark.parametrize("C,HW", [(320, 64 * 64), (1280, 16 * 16)])
def test_reference_groupnorm_shapes(op_engine, C, HW):
    say(f"reference groupnorm C={C} HW={HW}")
    e = op_engine
    X = h(pattern(C * HW, 131, 7, 29, 0.1, 1.4).reshape(C, HW))
    c = np.arange(C)
    gam = h((np.float32(0.8) + np.float32(0.01) * (c % 7).astype(np.float32)).astype(np.float32))
    bet = h((np.float32(0.05) * (c % 5).astype(np.float32) - np.float32(0.1)).astype(np.float32))
    tx = e.upload(np.ascontiguousarray(X.T).astype(np.float16))  # NHWC [HW, C]
    tg, tb = e.upload(gam.astype(np.float16)), e.upload(bet.astype(np.float16))
    ty = e.tensor((HW, C))
    e.groupnorm(tx, tg, tb, ty, 1, HW, C)
    got = ty.numpy().astype(np.float32).T
    ref = U.group_norm(t(X.reshape(1, C, HW, 1)), t(gam), t(bet)).numpy().reshape(C, HW)
    err = rel_err_l1(got, ref)
    say(f"  relErr {err:.2e}")
    assert err < 1e-3
    # the reference's check: 4 samples per group against fp64 group statistics
    G, cpg = 32, C // 32
    gs = cpg * HW
    se = sr = 0.0
    for gi in range(G):
        sl = X[gi * cpg:(gi + 1) * cpg].astype(np.float64)
        mean = sl.mean()
        inv = 1.0 / math.sqrt((sl * sl).mean() - mean * mean + 1e-5)
        for tt in range(4):
            j = (tt * 97 + gi) % gs
            ch, off = gi * cpg + j // HW, j % HW
            r = (X[ch, off] - mean) * inv * gam[ch] + bet[ch]
            se += abs(r - got[ch, off])
            sr += abs(r)
    assert se / (sr + 1e-6) < 0.03


# ----------------------------------------------------------------- attention

# VulkanBench.kt:107-118 (self 64^2 d40 h8, cross 4096x77 d40, d80 s1024, d160 s256);
# operands of benchAttention (vk_engine.cpp:1081-1083), layout [H, S, d]:
# Q = ((i*131+7)%23)*0.05-0.55, K = ((i*61+13)%19)*0.05-0.45, V = ((i*97+5)%17)*0.05-0.4.
@pytest.mark.parametrize("Sq,Sk,d", [(4096, 4096, 40), (4096, 77, 40), (1024, 1024, 80), (256, 256, 160)])
def test_reference_attention_shapes(op_engine, Sq, Sk, d):
    say(f"reference attention h8 Sq={Sq} Sk={Sk} d={d}")
    e = op_engine
    H = 8
    Q = h(pattern(H * Sq * d, 131, 7, 23, 0.05, 0.55).reshape(H, Sq, d))
    K = h(pattern(H * Sk * d, 61, 13, 19, 0.05, 0.45).reshape(H, Sk, d))
    V = h(pattern(H * Sk * d, 97, 5, 17, 0.05, 0.4).reshape(H, Sk, d))
    # the engine reads head h at column h*d of each token row: [S, H*d]
    tok = lambda a: np.ascontiguousarray(a.transpose(1, 0, 2).reshape(a.shape[1], H * d))
    tq, tk, tv = (e.upload(tok(a).astype(np.float16)) for a in (Q, K, V))
    to = e.tensor((Sq, H * d))
    e.attention(tq, tk, tv, to, 1, H, Sq, Sk, d, H * d, H * d, H * d, H * d, 1.0 / math.sqrt(d))
    got = to.numpy().astype(np.float32).reshape(Sq, H, d).transpose(1, 0, 2)
    ref = U.attention(t(tok(Q)[None]), t(tok(K)[None]), t(tok(V)[None]), H)[0].numpy()
    ref = ref.reshape(Sq, H, d).transpose(1, 0, 2)
    err = rel_err_l1(got, ref)
    say(f"  relErr {err:.2e}")
    assert err < 2e-3
    # the reference's check (vk_engine.cpp:1093-1104): 8 sampled (h, i, k), < 0.03
    se = sr = 0.0
    for s in range(8):
        hh, i, kk = s % H, (s * 53 + 1) % Sq, (s * 29 + 2) % d
        sc = K[hh].astype(np.float64) @ Q[hh, i].astype(np.float64) / math.sqrt(d)
        p = np.exp(sc - sc.max())
        r = float((p / p.sum()) @ V[hh, :, kk])
        se += abs(r - got[hh, i, kk])
        sr += abs(r)
    assert se / (sr + 1e-6) < 0.03


# ----------------------------------------------------------------- SiLU

def test_reference_silu_shape(op_engine):
    """VulkanBench.kt:102 (silu 320x64^2); benchSilu operand (vk_engine.cpp:373):
    ((i*131+7)%37)*0.1-1.8 (fp16), threshold 0.02 (:381)."""
    e = op_engine
    n = 320 * 64 * 64
    X = h(pattern(n, 131, 7, 37, 0.1, 1.8))
    tx = e.upload(X.astype(np.float16))
    ty = e.tensor((n,))
    e.silu(tx, ty, n)
    got = ty.numpy().astype(np.float32)
    ref = U.silu(t(X)).numpy()
    assert rel_err_l1(got, ref) < 1e-3
