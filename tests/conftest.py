import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libnsmlp.so")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (built on first use)."""
    from oracle import oracle as o

    if not os.path.exists(o._LIB_PATH):
        from oracle import build

        build.build()
    return o


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; fails (does not skip) when the HIP path is unusable."""
    import torch

    from next_step_ai_amd import _lib

    if not torch.cuda.is_available():
        raise RuntimeError("GPU test run without a visible GPU")
    _lib.lib()
    if not _lib.lib().nsmlp_device_supported(0):
        raise RuntimeError("device 0 is not gfx950")
    return torch.device("cuda", 0)
