"""Test set-up: import paths, the ``gpu`` marker and shared fixtures."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PACKAGE_PARENT = ROOT / "inference-engine-from-scratch_amd"
for path in (str(ROOT), str(PACKAGE_PARENT)):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config) -> None:
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def _gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


def pytest_collection_modifyitems(config, items) -> None:
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def device():
    import torch

    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _announce(request):
    """Print the test id before it runs so a GPU fault names its case."""
    if "gpu" in request.node.keywords:
        print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
    yield


os.environ.setdefault("PYTHONHASHSEED", "0")
