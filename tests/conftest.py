import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libtmoe.so")


@pytest.fixture(scope="session")
def gpu():
    """The HIP device; GPU tests fail (not skip) when the library or device is missing."""
    import torch
    from tarfa_amd._lib import lib
    assert torch.cuda.is_available(), "gpu test run without a visible GPU"
    lib()
    return torch.device("cuda:0")
