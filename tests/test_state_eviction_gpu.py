"""Planned-state eviction: a context keeps at most 16 planned UNet states (forward and
denoise) and each auxiliary network at most 8; planning one more evicts the least
recently used state (stream synchronised, graph destroyed, arena / workspace / staging
freed).  A shape that was evicted is planned again on its next call and must give the
same result, bit for bit, as before its eviction."""
import numpy as np
import pytest

from conftest import say

pytestmark = pytest.mark.gpu


def test_unet_state_eviction_replans_identically():
    import sdu
    rng = np.random.default_rng(21)
    eng = sdu.Engine(seed=1234)
    try:
        H = W = 16
        lat = rng.standard_normal((1, 4, H, W)).astype(np.float32)
        temb = sdu.time_proj(999)
        ctxs = {L: rng.standard_normal((1, L, 768)).astype(np.float32) for L in range(1, 18)}
        say("eviction: first forward, L=1")
        first = eng.forward(lat, temb, ctxs[1])
        # 16 more shapes: the 17th plan evicts L=1 (the least recently used)
        outs = {}
        for L in range(2, 18):
            say(f"eviction: plan L={L}")
            outs[L] = eng.forward(lat, temb, ctxs[L])
        say("eviction: L=1 again (re-planned)")
        again = eng.forward(lat, temb, ctxs[1])
        assert np.isfinite(again).all()
        np.testing.assert_array_equal(again, first)
        # that plan evicted L=2; L=17 is still planned and replays identically, and L=2
        # comes back identical too
        np.testing.assert_array_equal(eng.forward(lat, temb, ctxs[17]), outs[17])
        np.testing.assert_array_equal(eng.forward(lat, temb, ctxs[2]), outs[2])
    finally:
        eng.release()


def test_taesd_state_eviction_replans_identically():
    import sdu
    rng = np.random.default_rng(22)
    eng = sdu.Engine(flags=sdu.SDU_INIT_NO_WEIGHTS)
    try:
        eng.taesd_init(seed=77, flags=sdu.SDU_INIT_RANDOM_AFFINE)
        shapes = [(1, 8, 8 + 8 * i) for i in range(9)]  # 9 decode shapes, cap 8
        zs = [rng.standard_normal((B, 4, H, W)).astype(np.float32) for (B, H, W) in shapes]
        outs = []
        for s, z in zip(shapes, zs):
            say(f"taesd eviction: plan {s}")
            outs.append(eng.taesd_decode(z))
        say("taesd eviction: first shape again (re-planned)")
        again = eng.taesd_decode(zs[0])
        np.testing.assert_array_equal(again, outs[0])
        np.testing.assert_array_equal(eng.taesd_decode(zs[8]), outs[8])
        np.testing.assert_array_equal(eng.taesd_decode(zs[1]), outs[1])
    finally:
        eng.release()
