import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: CPU test that takes more than a few seconds")


@pytest.fixture(scope="session")
def gpu():
    """The HIP library, loaded; GPU tests fail loudly when it or the device is missing."""
    import torch
    from fastforward_amd import _lib
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    lib = _lib.load()
    _lib.check_device()
    return lib
