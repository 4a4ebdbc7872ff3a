import json
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


@pytest.fixture(autouse=True)
def _margin_test_id(request):
    """Names the running test in the parity-margin records of tests/helpers.py."""
    from tests import helpers

    helpers.CURRENT_TEST["id"] = request.node.nodeid
    yield
    helpers.CURRENT_TEST["id"] = None


def pytest_sessionfinish(session, exitstatus):
    """With LOGO_PARITY_LOG set, append every recorded comparison (max-abs and
    mean-abs error against its bound) to that file as JSON lines."""
    path = os.environ.get("LOGO_PARITY_LOG")
    if not path:
        return
    from tests import helpers

    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "a") as f:
        for rec in helpers.MARGINS:
            f.write(json.dumps(rec) + "\n")
