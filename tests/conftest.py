import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; calls through the C ABI")


@pytest.fixture(scope="session")
def kernels():
    """One libsmoe handle on cuda:0 (GPU tests only)."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a GPU")
    import streamoe_amd

    k = streamoe_amd.Kernels(0)
    yield k
    k.close()
