"""sdu_groupnorm_noalloc (the entry point that allocates nothing) against
sdu_groupnorm, through the C ABI: two calls in a row, the second with a smaller
input, each equal to the allocating entry point's output to the per-op bar; sizes
beyond its fixed scratch are rejected.  GroupNorm bar: relErr_L1 <= 1e-3 against the
fp32 oracle (the allocating entry point's own test), here the two engine paths
against each other within one fp16 ulp."""
import numpy as np
import pytest
import torch

from conftest import rel_err_l1, say
from oracle import unet_ref as U

pytestmark = pytest.mark.gpu


def _case(e, B, H, W, C1, C2, silu, seed):
    import sdu
    HW, C = H * W, C1 + C2
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((B, HW, C)) * 2 + 0.7).astype(np.float16)
    g = (rng.standard_normal(C) * 0.3 + 1).astype(np.float16)
    b = (rng.standard_normal(C) * 0.3).astype(np.float16)
    tx1 = e.upload(np.ascontiguousarray(x[:, :, :C1]))
    tx2 = e.upload(np.ascontiguousarray(x[:, :, C1:])) if C2 else None
    tg, tb = e.upload(g), e.upload(b)
    ya, yb = e.tensor((B, HW, C)), e.tensor((B, HW, C))
    lib = sdu.load()
    args = (tx1.h, tx2.h if tx2 else None, tg.h, tb.h)
    e._check(lib.sdu_groupnorm(e.h, *args, ya.h, B, HW, C1, C2, 32, 1e-5, int(silu)))
    e._check(lib.sdu_groupnorm_noalloc(e.h, *args, yb.h, B, HW, C1, C2, 32, 1e-5, int(silu)))
    a = ya.numpy().astype(np.float32)
    bb = yb.numpy().astype(np.float32)
    xn = torch.from_numpy(x.astype(np.float32).transpose(0, 2, 1).reshape(B, C, H, W).copy())
    ref = U.group_norm(xn, torch.from_numpy(g.astype(np.float32)), torch.from_numpy(b.astype(np.float32)),
                       act_silu=silu).numpy().reshape(B, C, HW).transpose(0, 2, 1)
    return a, bb, ref


def test_groupnorm_noalloc_matches_groupnorm(op_engine):
    import sdu
    e = op_engine
    # large slabs (the chunked statistics pass that accumulates into the scratch), then a
    # smaller call on the same device: the scratch must be cleared, not reused
    for (B, H, W, C1, C2, silu, seed) in ((4, 64, 64, 640, 320, True, 1), (1, 64, 64, 320, 0, False, 2),
                                          (2, 8, 8, 1280, 0, True, 3)):
        say(f"groupnorm_noalloc B={B} {H}x{W} C1={C1} C2={C2} silu={silu}")
        a, b, ref = _case(e, B, H, W, C1, C2, silu, seed)
        assert np.isfinite(b).all()
        assert rel_err_l1(b, a) <= 1e-4 and np.abs(b - a).max() <= 2e-3
        assert rel_err_l1(b, ref) < 1e-3
    # beyond the fixed scratch (and the shape limits): a clear error, no launch
    lib = sdu.load()
    t = e.tensor((8,))
    st = lib.sdu_groupnorm_noalloc(e.h, t.h, None, t.h, t.h, t.h, 65, 1, 8, 0, 8, 1e-5, 0)
    assert st == sdu.SDU_ERR_ARG
