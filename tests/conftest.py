"""Shared pytest configuration.

``gpu`` marks tests that need an MI355X (they call the HIP kernels through the
C ABI). They are never skipped silently on a machine that has a GPU: a missing
native library is a failure there.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a GPU and the built native library")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def _has_gpu() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config: pytest.Config, items: list[pytest.Item]) -> None:
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _collect_earlier_runtimes(request: pytest.FixtureRequest):
    """GPU tests set VRAM watermarks relative to torch.cuda.memory_allocated() at their
    start: collect the device buffers an earlier test's runtime still holds in reference
    cycles first, so they are not freed in the middle of the next test."""
    if "gpu" in request.keywords and _has_gpu():
        import gc

        import torch

        gc.collect()
        torch.cuda.synchronize()
    yield
