"""Shared pytest setup: import paths, the `gpu` marker and device fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "coverage-verified-sparse-attention_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm GPU) and libcvsa_hip.so")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; skips when no ROCm GPU is visible."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from cvsa.ops import _lib
    _lib.load()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")
