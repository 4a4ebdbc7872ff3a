import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The CUDA (HIP) device; GPU tests fail loudly if it or the library is missing."""
    import torch

    from logo_amd import _lib

    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    _lib.lib()
    return torch.device("cuda", 0)
