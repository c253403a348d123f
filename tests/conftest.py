import os
import sys

import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The ROCm device for GPU tests; fails (never skips) when it is missing."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible ROCm device")
    from phasekv_amd import _lib
    _lib.load()   # fails loudly if the HIP library is not built
    return torch.device("cuda:0")
