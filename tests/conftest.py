import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "fast-mac-gsplat_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def gpu():
    """A GPU test must run on a GPU: fail (do not skip) when none is visible."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu-marked test run without a visible ROCm GPU")
    from torch_gsplat_bridge_fast import _lib

    _lib.load()
    return torch.device("cuda:0")
