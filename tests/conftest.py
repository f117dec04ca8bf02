"""pytest configuration.

Markers:
- ``gpu``: needs a HIP device (MI355X). Run with ``-m gpu`` on the GPU box;
  the CPU suite is ``-m "not gpu"``. Without a visible device these tests are
  skipped; with one, a missing native library is a hard failure (there is no
  fallback path to pass on).
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a HIP (MI355X) device")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config: pytest.Config, items: list[pytest.Item]) -> None:
    if any("gpu" in item.keywords for item in items) and not _gpu_available():
        skip = pytest.mark.skip(reason="no HIP device visible")
        for item in items:
            if "gpu" in item.keywords:
                item.add_marker(skip)


@pytest.fixture(scope="session")
def cpu_threads() -> int:
    return len(os.sched_getaffinity(0))
