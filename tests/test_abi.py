"""C-ABI surface checks that need no GPU: the library loads, exports every
symbol include/sdu.h declares, and rejects a missing context without touching
the device (the reference's sentinel returns, vk_engine.cpp:801, :813, :878)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "sdu.h")


def _declared():
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|double|void\s*\*|const char\s*\*|size_t)\s+(sdu_\w+)\s*\(",
                                 txt, re.M)))


def test_header_and_binding_agree():
    import sdu
    assert _declared() == sorted(sdu.EXPORTS)


def test_library_exports_every_declared_symbol():
    import sdu
    lib = sdu.load()
    for name in _declared():
        assert hasattr(lib, name), name


def test_null_context_is_rejected():
    import sdu
    lib = sdu.load()
    assert lib.sdu_release(None) == 0
    assert lib.sdu_forward(None, None, None, None, 1, 64, 64, 77, None) == sdu.SDU_ERR_NOT_INIT
    assert lib.sdu_selftest(None, b"/nonexistent") == float(sdu.SDU_ERR_NOT_INIT)
    assert lib.sdu_synchronize(None) == sdu.SDU_ERR_NOT_INIT
    assert b"null context" in lib.sdu_last_error(None)
    assert lib.sdu_init(None, None, 0, 0) == sdu.SDU_ERR_ARG


def test_init_without_device_fails_cleanly():
    import sdu
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    lib = sdu.load()
    h = ctypes.c_void_p()
    assert lib.sdu_init(ctypes.byref(h), None, 0, 0) == sdu.SDU_ERR_DEVICE
    assert not h.value


def test_time_proj_matches_oracle():
    """sdu_time_proj (timeProj, VulkanUnetPipeline.kt:36-46) against the oracle's
    closed form; host code, no device."""
    import numpy as np
    import sdu
    from oracle import lcm
    for t in (0, 1, 259, 499, 759, 999):
        np.testing.assert_allclose(sdu.time_proj(t), lcm.time_proj(t), rtol=0, atol=1e-7)
    lib = sdu.load()
    assert lib.sdu_time_proj(-1, None) == sdu.SDU_ERR_ARG
