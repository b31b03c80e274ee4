"""Shared test setup: import paths, the ``gpu`` marker and tolerance helpers."""
from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT / "tiny-vllm_amd", ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def device():
    return torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before any GPU work so a fault is attributable.
    if "gpu" in request.keywords and os.environ.get("TVLLM_ANNOUNCE", "1") == "1":
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield
