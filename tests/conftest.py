"""Shared test setup: import paths, the ``gpu`` marker, common fixtures."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "uma-qmoe_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def hip_ext():
    """The loaded HIP extension; raises (never skips) when it is unavailable."""
    import torch

    from uma_qmoe_amd.native_backend import load_native_extension

    assert torch.cuda.is_available(), "GPU tests need a visible gfx950 device"
    _platform, ext = load_native_extension()
    return ext
