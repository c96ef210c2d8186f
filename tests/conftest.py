import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); runs the HIP kernels")


@pytest.fixture
def device():
    """The GPU the HIP tests run on; fails (never skips) when none is visible,
    so a GPU run cannot pass on a silent fallback."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a visible ROCm device")
    return torch.device("cuda", 0)
