import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libtbhip.so")
    config.addinivalue_line("markers", "slow: CPU test that takes more than a few seconds")


@pytest.fixture(scope="session")
def gpu():
    """Skip unless a gfx950 device is present; returns the device."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from tilebench_amd import runtime as rt

    rt.require_device()
    rt.load_library()
    return torch.device("cuda:0")
