"""Shared pytest configuration.

Tests marked ``gpu`` need an MI355X (HIP device) and the prebuilt
``libcdb_amd.so``; everything else runs on the CPU.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a HIP GPU and the built libcdb_amd.so")
    # The engine's host tick core is a small g++-built CPython extension that every engine test
    # imports; it is (re)built here when missing or older than its source (host code only).
    from continuous_depth_batching_amd import _build

    _build.build_tick()


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # pragma: no cover - torch import problems surface elsewhere
        return False


def pytest_collection_modifyitems(config: pytest.Config, items: list[pytest.Item]) -> None:
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="no HIP GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _name_gpu_case(request: pytest.FixtureRequest):
    """Print the case name before every GPU test so a crash log names it."""

    if "gpu" in request.keywords:
        print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
    yield
