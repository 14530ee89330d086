"""Shared test setup.

* ``gpu`` marks tests that need an MI355X (run with ``-m gpu`` on the GPU box).  On
  a machine without a ROCm device they are skipped, never silently passed.
* The repository root (for ``oracle``) and ``complexity-deep_amd`` (for the product
  package ``complexity_deep``) are put on sys.path.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
for p in (REPO, REPO / "complexity-deep_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


def _has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.build()
    return o


@pytest.fixture(scope="session")
def cdx():
    """The product package with its native library loaded (GPU tests)."""
    import complexity_deep
    from complexity_deep import _native
    _native.lib()
    return complexity_deep


def pytest_report_header(config):
    return f"repo={REPO} HIP_VISIBLE_DEVICES={os.environ.get('HIP_VISIBLE_DEVICES', '')}"
