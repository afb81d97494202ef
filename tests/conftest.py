"""Shared test setup: repo root on sys.path, the ``gpu`` marker, device fixtures."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm MI355X device (run with -m gpu)")


@pytest.fixture(scope="session")
def device():
    """The first GPU. On a machine without one, GPU tests are skipped; where a GPU is
    present the native library must load (no fallback)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm device visible")
    from helios_amd import _capi

    _capi.lib()  # raises if the library was not built
    return torch.device("cuda", 0)
