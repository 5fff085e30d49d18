"""Shared pytest configuration: import paths and the ``gpu`` marker."""

import os
import sys

import pytest

try:
    # Load PyTorch's HIP runtime before any test imports matmul_module / libqmm_gfx950.so, so
    # the process holds exactly one HIP runtime (the library binds to the loaded one).
    import torch  # noqa: F401
except ImportError:
    pass

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "gfx1150-inference_amd")
for p in (REPO, PKG, os.path.join(REPO, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the C ABI")


@pytest.fixture(scope="session")
def cuda():
    """The torch CUDA/HIP device, or a skip when no GPU is visible."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")
