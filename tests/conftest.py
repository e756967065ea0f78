"""Test configuration: import paths, the `gpu` marker, and shared fixtures.

`-m "not gpu"` runs everything that needs no GPU (oracle pins, host logic, the
C-ABI load/export check). `-m gpu` runs the parity tests proper, which call
libpagedkv through its C ABI on a ROCm device and compare with the oracle.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG = REPO / "llm-inference-server_amd"
for p in (str(REPO), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)

# The product reads ATTENTION at import; tests choose backends explicitly.
os.environ.setdefault("ATTENTION", "gather")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built libpagedkv.so")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(autouse=True)
def _skip_gpu_tests_without_gpu(request):
    if request.node.get_closest_marker("gpu") is not None and not gpu_available():
        pytest.skip("needs a ROCm GPU")
