"""Test setup: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs here (no GPU): oracle pinning, host logic, C-ABI
exports.  ``-m gpu`` runs on an MI355X: the HIP kernels against the oracle.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "mlx-metal-kernels_amd")
for p in (ROOT, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a ROCm device")
    from mk import _lib

    _lib.load()  # fail loudly if the native library is missing
    return torch.device("cuda:0")
