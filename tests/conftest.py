"""Shared test setup: import paths, the ``gpu`` marker, determinism, CPU thread cap.

GPU tests are marked ``gpu`` and run on the MI355X box (``pytest -m gpu``); everything
else runs on a CPU-only host. A GPU test on a host without a device fails instead of
skipping, so a broken GPU environment cannot pass silently.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for path in (ROOT, ROOT / "llm-serving_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

import torch  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X)")
    config.addinivalue_line("markers", "slow: long-running case")


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(0)
    yield


def _cap_threads() -> None:
    n = int(os.environ.get("MIATTN_TEST_THREADS", min(16, os.cpu_count() or 1)))
    torch.set_num_threads(max(1, n))


_cap_threads()


@pytest.fixture
def cuda():
    """The GPU device; fails (not skips) when the host has none."""
    assert torch.cuda.is_available(), "this test needs a HIP GPU (run it on the GPU box with -m gpu)"
    import miattn

    assert miattn.HIP_AVAILABLE, f"libmiattn.so failed to load: {miattn.LOAD_ERROR}"
    return torch.device("cuda:0")
