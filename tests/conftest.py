"""Shared pytest setup.

- puts the product package (``musa-aiter_amd/``) and the repo root (for the
  ``oracle`` test infrastructure) on ``sys.path``;
- registers the ``gpu`` marker: GPU tests need a ROCm device and the built
  HIP library and are skipped when no device is visible;
- seeds torch and numpy per test, like the reference's op_tests/conftest.py.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (os.path.join(ROOT, "musa-aiter_amd"), ROOT):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


def _gpu_available() -> bool:
    try:
        import torch

        return bool(torch.cuda.is_available())
    except Exception:  # pragma: no cover - torch import problems surface elsewhere
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _seed():
    import torch

    torch.manual_seed(42)
    np.random.seed(42)
    yield
