import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "sabah-moe-accelerator_amd")
ORACLE = os.path.join(ROOT, "oracle")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (PKG, ORACLE, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def hip_rt_cpu():
    """The HIP runtime library loaded for its host-only entry points (no GPU,
    no sabah_rt_init).  Fails loudly if the library is missing."""
    from sabah.runtime import rt
    rt.lib()
    return rt


@pytest.fixture(scope="session")
def hip_rt():
    """The HIP runtime, initialised on device 0.  Fails loudly if the library is missing."""
    if not gpu_available():
        pytest.skip("no GPU visible")
    from sabah.runtime import rt
    rt.lib()            # raises RuntimeUnavailable if the .so is missing
    rt.init(0)
    return rt


@pytest.fixture(scope="session")
def orc():
    import oracle as O
    O.lib()
    return O
