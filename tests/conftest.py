import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def device():
    """The GPU every `gpu` test runs on. Fails (never skips) when no GPU or no library is
    present, so a GPU run cannot pass without executing the native kernels."""
    import torch

    from code_for_iclr27_amd import _lib

    assert torch.cuda.is_available(), "gpu tests need a visible GPU"
    _lib.load()
    return torch.device("cuda:0")
