import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


@pytest.fixture(scope="session")
def hip():
    """A HIP context on device 0 (GPU tests only)."""
    import phonemap_amd as pm
    L = pm.lib()
    ctx = L.ss_hip_init(0)
    if not ctx:
        raise RuntimeError("ss_hip_init failed: %s" % L.ss_hip_last_error().decode())
    from tests.util import Dev
    yield Dev(L, ctx)
    L.ss_hip_free(ctx)
