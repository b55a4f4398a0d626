import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running check")


def _gpu_present():
    return os.path.exists("/dev/kfd")


@pytest.fixture(scope="session")
def hip():
    """The product library, initialised on device 0 (GPU tests only)."""
    import native
    L = native.bh.lib()
    if not L.bm_hip_init():
        pytest.fail("bm_hip_init failed: %s" % native.bh.last_error())
    return L


@pytest.fixture(scope="session")
def ref_lib():
    import native
    if not native.ref_available():
        pytest.skip("oracle/_ref not built (reference sources absent at build time)")
    R = native.ref()
    return R
