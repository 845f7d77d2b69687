"""Shared test setup: import paths, the `gpu` marker, device helpers."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "bus-fill_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs libbusfill kernels)")


@pytest.fixture(scope="session")
def dev():
    """cuda:0 for GPU tests; the HIP library must be built (no fallback)."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU")
    import busfill
    busfill.lib()
    return torch.device("cuda:0")
