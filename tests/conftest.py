import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "sd-vulkan-pixel10-tensor-g5_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

REFERENCE = "/root/reference"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libsdu.so)")
    config.addinivalue_line("markers", "slow: long-running parity case")


def rel_err_l1(got, ref) -> float:
    """sum|ref-got| / sum|ref| (vk_engine.cpp:698-704; tools/run_ref.py:46)."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    return float(np.abs(ref - got).sum() / (np.abs(ref).sum() + 1e-30))


@pytest.fixture(scope="session")
def op_engine():
    """Context without UNet weights, for op-level tests."""
    import sdu
    eng = sdu.Engine(flags=sdu.SDU_INIT_NO_WEIGHTS)
    yield eng
    eng.release()


@pytest.fixture(scope="session")
def unet_engine():
    """Seeded random-init UNet (baseline rule), seed 1234."""
    import sdu
    eng = sdu.Engine(seed=1234)
    yield eng
    eng.release()


@pytest.fixture(scope="session")
def oracle_weights():
    """Oracle-side weights for seed 1234, generated independently of the library."""
    from oracle import unet_ref, weights
    return unet_ref.to_torch(weights.generate(1234))


def say(*a):
    print(*a, flush=True)
