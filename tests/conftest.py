import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libyapd_t3.so")


@pytest.fixture(scope="session")
def dev():
    """The GPU under test; GPU tests fail loudly if the native library is missing."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from yapd_amd import kernels
    kernels.load_library()
    return torch.device("cuda:0")
