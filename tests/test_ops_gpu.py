"""Per-op parity of the HIP kernels (through the C ABI) against the CPU oracle.

Inputs are fp16-representable; the oracle computes in fp32 on the same values.
Tolerances: fp16 storage of the output bounds the per-element error near 2^-11
relative, so relErr_L1 <= 1e-3 for GEMM / conv / norm kernels and <= 2e-3 for
attention (P is rounded to fp16 before the PV product), with max-abs guards.
"""
import math

import numpy as np
import pytest
import torch

from conftest import rel_err_l1, say
from oracle import lcm, unet_ref as U

pytestmark = pytest.mark.gpu


def r16(shape, seed, scale=1.0, mean=0.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape) * scale + mean).astype(np.float16).astype(np.float32)


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


# ------------------------------------------------------------------ GroupNorm


@pytest.mark.parametrize("B,H,W,C1,C2,silu", [
    (2, 64, 64, 320, 0, True),      # resnet norm at level 0 (C2 batch-CFG)
    (2, 64, 64, 320, 0, False),     # transformer input norm
    (2, 16, 16, 1280, 1280, True),  # up-path concat 2560 @16^2
    (1, 8, 8, 1280, 640, True),     # concat 1920 @8^2
    (2, 32, 32, 640, 320, True),    # concat 960 @32^2
    (3, 7, 9, 64, 0, True),         # ragged pixel count
    (16, 8, 8, 2560, 0, False),     # C > 2048 (two channel windows per block)
    (2, 64, 64, 640, 320, True),    # concat 960 @64^2: group slab too large for one block
    (1, 5, 5, 96, 0, False),        # 3 channels per group (odd): two-pass path
])
def test_groupnorm(op_engine, B, H, W, C1, C2, silu):
    say(f"groupnorm B={B} {H}x{W} C1={C1} C2={C2} silu={silu}")
    HW, C = H * W, C1 + C2
    x = r16((B, HW, C), 1, 2.0, 0.7)  # non-zero mean stresses the variance estimate
    g = r16((C,), 2, 0.3, 1.0)
    b = r16((C,), 3, 0.3)
    e = op_engine
    tx1 = e.upload(x[:, :, :C1].astype(np.float16))
    tx2 = e.upload(x[:, :, C1:].astype(np.float16)) if C2 else None
    tg, tb = e.upload(g.astype(np.float16)), e.upload(b.astype(np.float16))
    ty = e.tensor((B, HW, C))
    e.groupnorm(tx1, tg, tb, ty, B, HW, C1, C2, x2=tx2, silu=silu)
    got = ty.numpy().astype(np.float32)
    xn = t(x.transpose(0, 2, 1).reshape(B, C, H, W))
    ref = U.group_norm(xn, t(g), t(b), act_silu=silu).numpy().reshape(B, C, HW).transpose(0, 2, 1)
    assert rel_err_l1(got, ref) < 1e-3
    assert np.abs(got - ref).max() < 2e-2
    # second call on the same context (ticket counters must have reset)
    e.groupnorm(tx1, tg, tb, ty, B, HW, C1, C2, x2=tx2, silu=silu)
    assert np.array_equal(ty.numpy().astype(np.float32), got)


@pytest.mark.parametrize("B,H,W,C,silu", [(2, 32, 32, 640, True), (2, 16, 16, 1280, False)])
def test_groupnorm_large_mean(op_engine, B, H, W, C, silu):
    """Groups whose mean is 100x their spread (the single-kernel path sums x minus the
    group's first value in one pass; without the shift an fp32 one-pass variance of
    these values cancels to noise)."""
    say(f"groupnorm large mean B={B} {H}x{W} C={C}")
    HW = H * W
    x = r16((B, HW, C), 11, 1.0, 100.0)
    g = r16((C,), 2, 0.3, 1.0)
    b = r16((C,), 3, 0.3)
    e = op_engine
    tx = e.upload(x.astype(np.float16))
    tg, tb = e.upload(g.astype(np.float16)), e.upload(b.astype(np.float16))
    ty = e.tensor((B, HW, C))
    e.groupnorm(tx, tg, tb, ty, B, HW, C, 0, silu=silu)
    got = ty.numpy().astype(np.float32)
    xn = t(x.transpose(0, 2, 1).reshape(B, C, H, W)).double()
    ref = U.group_norm(xn, t(g).double(), t(b).double(), act_silu=silu).float().numpy()
    ref = ref.reshape(B, C, HW).transpose(0, 2, 1)
    assert rel_err_l1(got, ref) < 1e-3
    assert np.abs(got - ref).max() < 2e-2


@pytest.mark.parametrize("B,H,W,Ci,Co,mean,temb,res,silu", [
    (2, 64, 64, 320, 320, 0.0, True, False, True),    # resnet conv1 -> norm2 at 64x64
    (2, 64, 64, 320, 320, 100.0, False, False, True),  # output mean 100x its spread
    (3, 40, 40, 64, 640, 30.0, False, True, False),    # 1600-pixel images: tiles straddle two
    (1, 8, 8, 128, 320, 50.0, True, False, True),      # 64-pixel images
    # the UNet's smaller levels (split-K convs; the statistics from the in-kernel split sum)
    (2, 8, 8, 1280, 1280, 0.0, True, False, True),     # 8x8 resnet conv1 -> norm2
    (2, 16, 16, 1280, 1280, 30.0, False, True, False),  # 16x16 conv2 (+residual) -> GroupNorm
    (2, 32, 32, 640, 640, 100.0, True, False, True),   # 32x32, output mean 100x its spread
    (1, 32, 32, 640, 960, 0.0, False, True, True),     # 30 channels per group: 2 per thread
    (2, 16, 16, 640, 1920, 0.0, True, False, True),    # 60 channels per group: 4 per thread
    (1, 16, 16, 640, 2560, 10.0, False, False, True),  # 80 channels per group, 8 pixel rounds
    (3, 8, 8, 1280, 1280, 5.0, True, True, True),      # odd batch
])
def test_conv_groupnorm_epilogue_stats(op_engine, B, H, W, Ci, Co, mean, temb, res, silu):
    """The UNet's 64x64-level GroupNorm path: per-channel sums and sums of squares of the
    conv's stored fp16 output, kept by the GEMM epilogue (fp32 per tile, fp64 across tiles),
    then the GroupNorm from them.  The conv output is checked against the fp32 conv; the
    GroupNorm against an fp64 GroupNorm of the same fp16 conv output, so the check isolates
    the statistics.  A large output mean is the case where E[x^2] - mean^2 cancels.  The
    smaller shapes split K, so their statistics come from the in-kernel split sum's
    epilogue (60 and 80 channels per group, odd batch)."""
    say(f"conv+groupnorm B={B} {H}x{W} {Ci}->{Co} mean={mean} temb={temb} res={res} silu={silu}")
    e = op_engine
    HW = H * W
    x = r16((B, H, W, Ci), 31)
    w = r16((Co, Ci, 3, 3), 32, 1.0 / math.sqrt(Ci * 9))
    bb = r16((Co,), 33, 0.5, mean)
    tp = np.random.default_rng(34).standard_normal(Co).astype(np.float32)
    rr = r16((B, H, W, Co), 35)
    g = r16((Co,), 36, 0.3, 1.0)
    b = r16((Co,), 37, 0.3)
    tx = e.upload(x.astype(np.float16))
    tw = e.upload(w.transpose(0, 2, 3, 1).astype(np.float16))
    tb = e.upload(bb.astype(np.float16))
    tt = e.upload(tp) if temb else None
    tr = e.upload(rr.astype(np.float16)) if res else None
    tg, tbeta = e.upload(g.astype(np.float16)), e.upload(b.astype(np.float16))
    ty, tgn = e.tensor((B, H, W, Co)), e.tensor((B, H, W, Co))
    e.conv2d_groupnorm(tx, tw, ty, tg, tbeta, tgn, B, H, W, Ci, Co, bias=tb, temb=tt, residual=tr, silu=silu)
    ref = U.conv2d(t(x.transpose(0, 3, 1, 2)), t(w), t(bb), stride=1, pad=1)
    if temb:
        ref = ref + t(tp)[None, :, None, None]
    ref = ref.numpy().transpose(0, 2, 3, 1)
    if res:
        ref = ref + rr
    y = ty.numpy().astype(np.float32)
    assert rel_err_l1(y, ref) < 1e-3
    yn = t(y.reshape(B, HW, Co).transpose(0, 2, 1).reshape(B, Co, H, W)).double()
    gref = U.group_norm(yn, t(g).double(), t(b).double(), act_silu=silu).float().numpy()
    gref = gref.reshape(B, Co, HW).transpose(0, 2, 1).reshape(B, H, W, Co)
    got = tgn.numpy().astype(np.float32)
    assert rel_err_l1(got, gref) < 1e-3
    assert np.abs(got - gref).max() < 2e-2


# ------------------------------------------------------------------ LayerNorm


@pytest.mark.parametrize("T,C", [(8192, 320), (2048, 640), (512, 1280), (128, 1280), (5, 40)])
def test_layernorm(op_engine, T, C):
    say(f"layernorm T={T} C={C}")
    x = r16((T, C), 4, 3.0, -1.0)
    g = r16((C,), 5, 0.3, 1.0)
    b = r16((C,), 6, 0.3)
    e = op_engine
    tx, tg, tb = e.upload(x.astype(np.float16)), e.upload(g.astype(np.float16)), e.upload(b.astype(np.float16))
    ty = e.tensor((T, C))
    e.layernorm(tx, tg, tb, ty, T, C)
    ref = U.layer_norm(t(x), t(g), t(b)).numpy()
    got = ty.numpy().astype(np.float32)
    assert rel_err_l1(got, ref) < 1e-3
    assert np.abs(got - ref).max() < 2e-2


# ------------------------------------------------------------------ matmul


@pytest.mark.parametrize("M,N,K,K2,bias,res,geglu,f32", [
    (8192, 320, 320, 0, True, True, False, False),    # to_out with residual, level 0
    (8192, 960, 320, 0, False, False, False, False),  # fused QKV
    (8192, 2560, 320, 0, True, False, True, False),   # FF proj + GEGLU
    (8192, 320, 1280, 0, True, True, False, False),   # FF out
    (154, 2560, 768, 0, False, False, False, False),  # cross K/V (B=2 x 77 tokens)
    (128, 1280, 5120, 0, True, True, False, False),   # split-K (mid FF out)
    (128, 2560, 1280, 0, True, False, True, False),   # split-K with GEGLU (mid FF proj)
    (512, 1280, 2560, 1280, True, False, False, False),  # 1x1 shortcut over a concat
    (77, 64, 64, 0, True, False, False, True),        # ragged M, N <= 64 tile, fp32 out
    (100, 128, 128, 0, True, False, True, False),     # GEGLU with ragged M
    (64, 64, 8192, 0, True, True, False, False),      # one tile, many K splits
    (200, 384, 3000, 0, True, False, False, True),    # split-K, ragged M and K tail, fp32 out
    # few rows (the 8x8 level, batch 1 and 2): two sources along K, ragged M
    (128, 1280, 6400, 1280, True, True, False, False),  # mid FF out + proj_out over [g | t]
    (96, 320, 640, 0, True, True, False, True),          # ragged M, fp32 out
    (64, 1280, 1280, 0, False, True, False, False),      # M = 64
    (33, 64, 128, 0, True, False, True, False),          # ragged M, GEGLU
    # the 64x160 tile (16x16x32 MFMAs): ragged M with split K, and the 77-token cross K/V
    (8000, 320, 2880, 0, True, True, False, False),
    (154, 24960, 768, 0, False, False, False, False),
    (8192, 300, 2880, 0, True, False, False, True),  # N % 8 != 0: element-wise epilogue
    (8000, 312, 2880, 0, True, True, False, False),  # last N tile partly outside N
    # small dense GEMMs of the transformer blocks: ragged M, fp32 out, two K sources
    (8000, 320, 320, 0, True, True, False, False),
    (2048, 640, 640, 0, True, False, False, True),
    (8192, 320, 1600, 1280, True, True, False, False),
])
def test_matmul(op_engine, M, N, K, K2, bias, res, geglu, f32):
    say(f"matmul M={M} N={N} K={K} K2={K2} bias={bias} res={res} geglu={geglu} f32={f32}")
    e = op_engine
    a = r16((M, K), 7)
    w = r16((N, K), 8, 0.05)
    bb = r16((N,), 9, 0.5)
    Nout = N // 2 if geglu else N
    rr = r16((M, Nout), 10)
    K1 = K - K2
    ta = e.upload(a[:, :K1].astype(np.float16))
    ta2 = e.upload(a[:, K1:].astype(np.float16)) if K2 else None
    # GEGLU weights/bias are interleaved per 32 rows (hidden block, gate block)
    if geglu:
        perm = np.concatenate([np.concatenate([np.arange(j * 32, j * 32 + 32),
                                               N // 2 + np.arange(j * 32, j * 32 + 32)])
                               for j in range(N // 64)])
        wd, bd = w[perm], bb[perm]
    else:
        wd, bd = w, bb
    tw = e.upload(wd.astype(np.float16))
    tb = e.upload(bd.astype(np.float16)) if bias else None
    tr = e.upload(rr.astype(np.float16)) if res else None
    ty = e.tensor((M, Nout), 2 if f32 else 1)
    flags = (1 if geglu else 0) | (2 if f32 else 0)
    e.matmul(ta, tw, ty, M, N, K, bias=tb, residual=tr, a2=ta2, K2=K2, flags=flags)
    ref = U.linear(t(a), t(w), t(bb) if bias else None)
    if geglu:
        ref = U.geglu(ref)
    if res:
        ref = ref + t(rr)
    ref = ref.numpy()
    got = ty.numpy().astype(np.float32)
    assert rel_err_l1(got, ref) < 1e-3
    assert np.abs(got - ref).max() < 3e-2 * max(1.0, np.abs(ref).max() / 8)


def test_matmul_split_repeat(op_engine):
    """Split-K launches back to back: the per-tile arrival counters are left zero by
    each launch, and the tile sums run in a fixed order, so repeats are bit-identical."""
    say("matmul split-K repeat")
    e = op_engine
    outs = []
    for M, N, K in [(128, 1280, 5120), (64, 64, 8192), (128, 1280, 5120)]:
        a = r16((M, K), 21)
        w = r16((N, K), 22, 0.05)
        ta, tw = e.upload(a.astype(np.float16)), e.upload(w.astype(np.float16))
        ty = e.tensor((M, N))
        e.matmul(ta, tw, ty, M, N, K)
        e.matmul(ta, tw, ty, M, N, K)
        got = ty.numpy().astype(np.float32)
        assert rel_err_l1(got, U.linear(t(a), t(w), None).numpy()) < 1e-3
        outs.append(got)
    assert np.array_equal(outs[0], outs[2])


# ------------------------------------------------------------------ conv2d


@pytest.mark.parametrize("B,H,W,Ci,Co,k,stride,ups,temb,res", [
    (2, 64, 64, 320, 320, 3, 1, False, True, False),   # resnet conv1 @64^2 (+ time proj)
    (2, 64, 64, 320, 320, 3, 1, False, False, True),   # resnet conv2 (+ residual)
    (2, 64, 64, 320, 320, 3, 2, False, False, False),  # downsample
    (2, 8, 8, 1280, 1280, 3, 1, True, False, False),   # upsample (8 -> 16)
    (2, 8, 8, 1280, 1280, 3, 1, False, True, True),    # mid conv, split-K
    (2, 8, 8, 2560, 1280, 3, 1, False, False, False),  # K = 23040
    (2, 64, 64, 8, 320, 3, 1, False, False, False),    # conv_in (K = 72, tail tile)
    (2, 64, 64, 320, 4, 3, 1, False, False, False),    # conv_out (N = 4)
    (1, 5, 7, 16, 24, 3, 1, False, False, False),      # ragged
    (1, 5, 7, 16, 24, 3, 2, False, False, False),      # ragged stride 2
    (2, 32, 32, 640, 640, 1, 1, False, False, True),   # 1x1 proj
    (2, 16, 16, 1280, 1280, 3, 2, False, False, False),  # downsample to 8x8 (M = 128)
    (1, 8, 8, 640, 320, 3, 1, False, True, True),      # M = 64
    (1, 6, 10, 128, 96, 3, 1, False, False, True),     # ragged M = 60, Cin = 128
    # the 64x160 tile (16x16x32 MFMAs) with split K: ragged M = 8100, non-square image
    (1, 90, 90, 320, 320, 3, 1, False, True, True),
    (2, 62, 66, 320, 320, 3, 1, False, False, False),
    (1, 90, 90, 320, 312, 3, 1, False, True, True),    # last N tile partly outside N
    # odd and ragged images on the other paths
    (1, 5, 7, 64, 64, 3, 1, True, False, True),        # upsample 5x7 -> 10x14 (+ residual)
    (1, 33, 31, 320, 640, 3, 2, False, True, False),   # stride 2 over odd sizes -> 17x16
    (2, 17, 19, 640, 640, 3, 1, False, False, True),   # M = 646 at 640 channels
])
def test_conv2d(op_engine, B, H, W, Ci, Co, k, stride, ups, temb, res):
    say(f"conv2d B={B} {H}x{W} {Ci}->{Co} k={k} s={stride} ups={ups} temb={temb} res={res}")
    e = op_engine
    x = r16((B, H, W, Ci), 11)
    w = r16((Co, Ci, k, k), 12, 1.0 / math.sqrt(Ci * k * k))
    bb = r16((Co,), 13, 0.5)
    tp = np.random.default_rng(14).standard_normal(Co).astype(np.float32)
    Ho = 2 * H if ups else (H - 1) // stride + 1
    Wo = 2 * W if ups else (W - 1) // stride + 1
    rr = r16((B, Ho, Wo, Co), 15)
    tx = e.upload(x.astype(np.float16))
    tw = e.upload(w.transpose(0, 2, 3, 1).astype(np.float16))  # [Co, kh, kw, Ci]
    tb = e.upload(bb.astype(np.float16))
    tt = e.upload(tp) if temb else None
    tr = e.upload(rr.astype(np.float16)) if res else None
    ty = e.tensor((B, Ho, Wo, Co))
    e.conv2d(tx, tw, ty, B, H, W, Ci, Co, ksize=k, stride=stride, upsample=ups, bias=tb, temb=tt, residual=tr)
    xn = t(x.transpose(0, 3, 1, 2))
    if ups:
        xn = U.upsample2x(xn)
    ref = U.conv2d(xn, t(w), t(bb), stride=stride if not ups else 1, pad=k // 2)
    if temb:
        ref = ref + t(tp)[None, :, None, None]
    ref = ref.numpy().transpose(0, 2, 3, 1)
    if res:
        ref = ref + rr
    got = ty.numpy().astype(np.float32)
    assert got.shape == ref.shape
    assert rel_err_l1(got, ref) < 1e-3
    assert np.abs(got - ref).max() < 3e-2


@pytest.mark.parametrize("M,N,K", [
    (8192, 320, 320),    # the attention output projection's shape (residual loaded up front)
    (128, 1280, 5120),   # split K
])
def test_matmul_inplace_residual(op_engine, M, N, K):
    """residual = y: the transformer's in-place residual adds (t += attn . Wo^T + b)."""
    say(f"matmul in-place residual M={M} N={N} K={K}")
    e = op_engine
    a, w, bb, rr = r16((M, K), 51), r16((N, K), 52, 0.05), r16((N,), 53, 0.5), r16((M, N), 54)
    ty = e.upload(rr.astype(np.float16))
    e.matmul(e.upload(a.astype(np.float16)), e.upload(w.astype(np.float16)), ty, M, N, K,
             bias=e.upload(bb.astype(np.float16)), residual=ty)
    ref = (U.linear(t(a), t(w), t(bb)) + t(rr)).numpy()
    got = ty.numpy().astype(np.float32)
    assert rel_err_l1(got, ref) < 1e-3
    assert np.abs(got - ref).max() < 3e-2


def test_conv2d_inplace_residual_and_overlap_errors(op_engine):
    """A conv's residual may be its output; an output over the conv's or a matmul's own
    operands is an argument error (other tiles still read what it would overwrite)."""
    import sdu
    say("conv2d in-place residual; overlap errors")
    e = op_engine
    B, H, W, C = 2, 32, 32, 64
    x, w, rr = r16((B, H, W, C), 61), r16((C, C, 3, 3), 62, 1.0 / math.sqrt(9 * C)), r16((B, H, W, C), 63)
    tx = e.upload(x.astype(np.float16))
    tw = e.upload(w.transpose(0, 2, 3, 1).astype(np.float16))
    ty = e.upload(rr.astype(np.float16))
    e.conv2d(tx, tw, ty, B, H, W, C, C, residual=ty)
    ref = U.conv2d(t(x.transpose(0, 3, 1, 2)), t(w), None, stride=1, pad=1).numpy().transpose(0, 2, 3, 1) + rr
    got = ty.numpy().astype(np.float32)
    assert rel_err_l1(got, ref) < 1e-3
    with pytest.raises(sdu.SduError) as ex:
        e.conv2d(tx, tw, tx, B, H, W, C, C)  # y = x
    assert ex.value.code == sdu.SDU_ERR_ARG
    g, bt = e.upload(np.ones(C, np.float16)), e.upload(np.zeros(C, np.float16))
    with pytest.raises(sdu.SduError) as ex:
        e.conv2d_groupnorm(tx, tw, tx, g, bt, ty, B, H, W, C, C)  # conv output y = x
    assert ex.value.code == sdu.SDU_ERR_ARG
    ta = e.upload(r16((64, 64), 64).astype(np.float16))
    tw2 = e.upload(r16((64, 64), 65, 0.1).astype(np.float16))
    for y in (ta, tw2):
        with pytest.raises(sdu.SduError) as ex:
            e.matmul(ta, tw2, y, 64, 64, 64)  # y = a, y = w
        assert ex.value.code == sdu.SDU_ERR_ARG
    # an fp32 output over its own fp16 residual: a row's fp32 store would cover the
    # residual of two other rows, so even residual == y is an error with SDU_EPI_OUT_F32
    ty32 = e.tensor((B, H, W, C), sdu.SDU_F32)
    tr32 = e.upload(rr.astype(np.float16))
    with pytest.raises(sdu.SduError) as ex:
        e.conv2d(tx, tw, ty32, B, H, W, C, C, residual=ty32, flags=sdu.SDU_EPI_OUT_F32)
    assert ex.value.code == sdu.SDU_ERR_ARG
    tm32 = e.tensor((64, 64), sdu.SDU_F32)
    with pytest.raises(sdu.SduError) as ex:
        e.matmul(ta, tw2, tm32, 64, 64, 64, residual=tm32, flags=sdu.SDU_EPI_OUT_F32)
    assert ex.value.code == sdu.SDU_ERR_ARG
    # ... while an fp32 output with a separate fp16 residual is fine
    e.conv2d(tx, tw, ty32, B, H, W, C, C, residual=tr32, flags=sdu.SDU_EPI_OUT_F32)
    assert rel_err_l1(ty32.numpy(), ref) < 1e-3
    # the failed calls launched nothing: x still holds its input
    assert np.array_equal(tx.numpy(), x.astype(np.float16))


# ------------------------------------------------------------------ attention


@pytest.mark.parametrize("B,heads,Sq,Sk,d", [
    (2, 8, 4096, 4096, 40),   # level-0 self-attention
    (2, 8, 4096, 77, 40),     # level-0 cross-attention
    (2, 8, 1024, 1024, 80),
    (2, 8, 2304, 2304, 80),   # 96x96 level-1 self-attention: eight query waves per block
    (16, 8, 256, 256, 160),   # B=16 level-2 self-attention: shared K/V tiles, four waves
    (2, 8, 256, 256, 160),
    (2, 8, 64, 64, 160),      # mid block
    (2, 8, 256, 77, 160),
    (1, 2, 100, 37, 40),      # ragged query / key counts
    (1, 1, 1, 1, 8),          # single token
    (1, 3, 130, 200, 64),
    # other head sizes: the ones row of V^T (row sums) at dims 24, 56, 120; none at 96
    (1, 2, 70, 90, 24),
    (1, 1, 33, 65, 56),
    (1, 2, 40, 50, 96),
    (1, 1, 20, 30, 120),
    # the shared-tile kernel with ragged query and key counts (a last query block with
    # 2 valid queries; last key tiles with 6, 13 and 60 valid keys)
    (2, 8, 2050, 1030, 40),   # 128-key tiles (at most 512 blocks)
    (4, 8, 4000, 333, 40),    # 64-key tiles
    (4, 8, 1000, 700, 80),    # eight query waves per block
    # many shared-tile blocks (more than one round): ragged query count (last block with
    # 4 queries) and key count (last 64-key tile with 13)
    (8, 8, 4100, 333, 40),
    (4, 16, 2048, 200, 40),
    # keys split in two halves merged in-kernel (1.33 and 1.5 rounds of blocks; half a
    # round, with a ragged key count: halves of 1024 and 976 keys)
    (2, 8, 9216, 9216, 40),   # UNet 96x96 self-attention
    (3, 8, 2000, 1000, 40),
])
def test_attention(op_engine, B, heads, Sq, Sk, d):
    say(f"attention B={B} heads={heads} Sq={Sq} Sk={Sk} d={d}")
    e = op_engine
    C = heads * d
    q = r16((B, Sq, C), 16)
    k = r16((B, Sk, C), 17)
    v = r16((B, Sk, C), 18)
    tq, tk, tv = e.upload(q.astype(np.float16)), e.upload(k.astype(np.float16)), e.upload(v.astype(np.float16))
    to = e.tensor((B, Sq, C))
    e.attention(tq, tk, tv, to, B, heads, Sq, Sk, d, C, C, C, C, 1.0 / math.sqrt(d))
    got = to.numpy().astype(np.float32)
    ref = U.attention(t(q), t(k), t(v), heads).numpy()
    assert rel_err_l1(got, ref) < 2e-3
    assert np.abs(got - ref).max() < 2e-2


def test_attention_strided_rows(op_engine):
    """Row strides larger than heads*d (heads read in place from a fused buffer)."""
    e = op_engine
    B, heads, S, d = 2, 8, 256, 40
    C = heads * d
    buf = r16((B, S, 3 * C), 19)
    q, k, v = buf[..., :C], buf[..., C:2 * C], buf[..., 2 * C:]
    # emulate column windows with three buffers padded to row stride 3C
    pad = np.zeros((B, S, 3 * C), np.float32)
    tq = e.upload(np.concatenate([q, pad[..., :2 * C]], -1).astype(np.float16))
    tk = e.upload(np.concatenate([k, pad[..., :2 * C]], -1).astype(np.float16))
    tv = e.upload(np.concatenate([v, pad[..., :2 * C]], -1).astype(np.float16))
    to = e.tensor((B, S, 2 * C))
    e.attention(tq, tk, tv, to, B, heads, S, S, d, 3 * C, 3 * C, 3 * C, 2 * C, 1 / math.sqrt(d))
    got = to.numpy().astype(np.float32)[..., :C]
    ref = U.attention(t(q), t(k), t(v), heads).numpy()
    assert rel_err_l1(got, ref) < 2e-3


# Q pre-scaled by scale * log2 e (SDU_ATTN_Q_LOG2), as the UNet's query projections
# write it: o = softmax_2(q k^T) v = softmax(q' k^T / sqrt(d)) v with q' = q ln2 sqrt(d).
# Heads whose size leaves a spare MFMA dimension (8, 24, 40, 56) on the shared-tile kernel
# carry the softmax reference in that dimension; the others only drop the scale.
@pytest.mark.parametrize("B,heads,Sq,Sk,d", [
    (2, 8, 4096, 4096, 40),   # UNet 64x64 self-attention: 128-key tiles
    (2, 8, 2050, 1030, 40),   # ragged: last query block 2 queries, last key tile 6 keys
    (8, 8, 4100, 333, 40),    # 64-key tiles, more than one round of blocks
    (4, 8, 1100, 300, 24),    # reference dimension in the second k-step
    (4, 8, 1100, 300, 8),     # reference dimension in the first k-step
    (8, 8, 2048, 300, 56),    # four k-steps, dimension 56
    (1, 2, 100, 37, 40),      # key-split kernel (no reference dimension)
    (4, 8, 1000, 700, 80),    # eight-wave shared tiles (d a multiple of 16)
    (2, 8, 256, 256, 160),
    # keys split in two halves merged in-kernel, with the reference dimension
    (2, 8, 9216, 9216, 40),   # UNet 96x96 self-attention
    (3, 8, 2000, 1000, 40),
    (4, 16, 2048, 200, 40),
])
def test_attention_q_log2(op_engine, B, heads, Sq, Sk, d):
    import sdu
    say(f"attention q_log2 B={B} heads={heads} Sq={Sq} Sk={Sk} d={d}")
    e = op_engine
    C = heads * d
    qs = (r16((B, Sq, C), 24) * (math.log2(math.e) / math.sqrt(d))).astype(np.float16)
    k = r16((B, Sk, C), 25)
    v = r16((B, Sk, C), 26)
    tq, tk, tv = e.upload(qs), e.upload(k.astype(np.float16)), e.upload(v.astype(np.float16))
    to = e.tensor((B, Sq, C))
    e.attention_ex(tq, tk, tv, to, B, heads, Sq, Sk, d, C, C, C, C, 1.0 / math.sqrt(d), sdu.SDU_ATTN_Q_LOG2)
    got = to.numpy().astype(np.float32)
    qp = qs.astype(np.float32) * (math.log(2.0) * math.sqrt(d))
    ref = U.attention(t(qp), t(k), t(v), heads).numpy()
    assert rel_err_l1(got, ref) < 2e-3
    assert np.abs(got - ref).max() < 2e-2
    # bit-identical on a repeat (a key-split launch merges its halves in a fixed order)
    e.attention_ex(tq, tk, tv, to, B, heads, Sq, Sk, d, C, C, C, C, 1.0 / math.sqrt(d), sdu.SDU_ATTN_Q_LOG2)
    np.testing.assert_array_equal(to.numpy().astype(np.float32), got)


@pytest.mark.parametrize("B", [4, 16])  # 128-key tiles (256 blocks), 64-key tiles (1024)
def test_attention_q_log2_reference_moves(op_engine, B):
    """Score offsets per key range (log2 units) that move the softmax reference carried in
    the spare head dimension: the first tile far below zero (-3000), the next 10 higher
    (a move of more than 2^8 on the reference), keys 400-419 at +50 (a jump of 3000),
    the rest at +40 (no move), and a masked key tail (600 keys)."""
    import sdu
    say(f"attention q_log2 reference moves B={B}")
    e = op_engine
    heads, Sq, Sk, d = 8, 1024, 600, 40
    C = heads * d
    rng = np.random.default_rng(27)
    q = (0.5 * rng.standard_normal((B, Sq, heads, d))).astype(np.float16)
    k = (0.5 * rng.standard_normal((B, Sk, heads, d))).astype(np.float16)
    off = np.full(Sk, 40.0)
    off[:64] = -3000.0
    off[64:128] = -2990.0
    off[400:420] = 50.0
    q[..., 0] = 8.0
    k[..., 0] = (off / 8.0)[None, :, None]  # multiples of 1/8: exact in fp16
    v = r16((B, Sk, C), 28)
    q, k = q.reshape(B, Sq, C), k.reshape(B, Sk, C)
    tq, tk, tv = e.upload(q), e.upload(k), e.upload(v.astype(np.float16))
    to = e.tensor((B, Sq, C))
    e.attention_ex(tq, tk, tv, to, B, heads, Sq, Sk, d, C, C, C, C, 1.0 / math.sqrt(d), sdu.SDU_ATTN_Q_LOG2)
    got = to.numpy().astype(np.float32)
    qp = q.astype(np.float32) * (math.log(2.0) * math.sqrt(d))
    ref = U.attention(t(qp), t(k.astype(np.float32)), t(v), heads).numpy()
    assert np.isfinite(got).all()
    assert rel_err_l1(got, ref) < 2e-3
    assert np.abs(got - ref).max() < 2e-2


# ------------------------------------------------------------------ elementwise


@pytest.mark.parametrize("n", [3000, 1003, 5])  # 8-wide vectors; a 3-element tail; tail only
def test_elementwise_ops(op_engine, n):
    e = op_engine
    C = 40 if n % 40 == 0 else 1
    x = r16((n,), 20, 3.0)
    y = r16((n,), 21)
    b = r16((C,), 22)
    tx, ty, tb = e.upload(x.astype(np.float16)), e.upload(y.astype(np.float16)), e.upload(b.astype(np.float16))
    to = e.tensor((n,))
    e.silu(tx, to, n)
    np.testing.assert_allclose(to.numpy().astype(np.float32), U.silu(t(x)).numpy(), rtol=2e-3, atol=2e-3)
    e.add(tx, ty, to, n)
    np.testing.assert_allclose(to.numpy().astype(np.float32), x + y, rtol=2e-3, atol=2e-3)
    e.add_bias(ty, tb, n, C)
    np.testing.assert_allclose(ty.numpy().astype(np.float32), y + np.tile(b, n // C), rtol=2e-3, atol=2e-3)
    T, C2 = 50, 64
    g = r16((T, 2 * C2), 23, 2.0)
    tg = e.upload(g.astype(np.float16))
    tgo = e.tensor((T, C2))
    e.geglu(tg, tgo, T, C2)
    np.testing.assert_allclose(tgo.numpy().astype(np.float32), U.geglu(t(g)).numpy(), rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("steps", [4, 1, 8])
def test_lcm_step(op_engine, steps):
    """CFG combine + LcmScheduler.step on the device vs the float64 oracle."""
    e = op_engine
    n = 4 * 32 * 32
    rng = np.random.default_rng(24)
    sched = lcm.LcmSchedule(steps)
    x = rng.standard_normal(n).astype(np.float32)
    tx = e.upload(x)
    for idx in range(steps):
        eps2 = rng.standard_normal((2, n)).astype(np.float32)
        noise = rng.standard_normal(n).astype(np.float32)
        last = idx == steps - 1
        e.lcm_step(tx, e.upload(eps2), None if last else e.upload(noise), n, steps, idx, 8.0)
        eps = lcm.cfg_combine(eps2[0], eps2[1], 8.0)
        x = sched.step(idx, x, eps, None if last else noise)
        np.testing.assert_allclose(tx.numpy(), x, rtol=1e-6, atol=1e-6)


def test_op_argument_errors(op_engine):
    """Bad shapes come back as status codes, not faults (vk_engine.cpp has none)."""
    import sdu
    e = op_engine
    a = e.tensor((16, 16))
    with pytest.raises(sdu.SduError) as ex:
        e.matmul(a, a, a, 16, 16, 17)  # K not a multiple of 8
    assert ex.value.code == sdu.SDU_ERR_ARG
    with pytest.raises(sdu.SduError):
        e.matmul(a, a, a, 64, 64, 64)  # tensors too small
    with pytest.raises(sdu.SduError):
        e.attention(a, a, a, a, 1, 1, 4, 4, 168, 168, 168, 168, 168, 1.0)  # d > 160
    with pytest.raises(sdu.SduError):
        e.groupnorm(a, a, a, a, 1, 16, 12, 0)  # C not a multiple of 8
    # 100-pixel images (a 128-row tile spans three) with 3 channels per group (odd: no
    # single-kernel GroupNorm either)
    xs, ys, gs = e.tensor((1, 10, 10, 96)), e.tensor((1, 10, 10, 96)), e.tensor((1, 10, 10, 96))
    with pytest.raises(sdu.SduError) as ex:
        e.conv2d_groupnorm(xs, e.tensor((96, 3, 3, 96)), ys, e.tensor((96,)), e.tensor((96,)), gs,
                           1, 10, 10, 96, 96)
    assert ex.value.code == sdu.SDU_ERR_ARG
    with pytest.raises(sdu.SduError):
        e.forward(np.zeros((1, 4, 64, 64), np.float32), np.zeros(320, np.float32),
                  np.zeros((1, 77, 768), np.float32))  # context has no UNet weights
