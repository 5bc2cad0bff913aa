"""Shared test setup: import paths, the `gpu` marker and GPU fixtures."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG = REPO / "triton-variable-moe_amd"
for p in (str(REPO), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) GPU and libvmoe.so")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _announce(request):
    """Print the test id before it runs, so a GPU fault names its case."""
    if os.environ.get("VMOE_ANNOUNCE", "1") == "1" and request.node.get_closest_marker("gpu"):
        print(f"\n[run] {request.node.nodeid}", flush=True)
    yield
