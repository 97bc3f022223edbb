"""Two tiers, as in the reference (tests/conftest.py:19-35 there): tests marked `gpu` need an
MI355X (gfx950) and the built libaneforge_hip.so; everything else runs on any CPU.

A `gpu` test is skipped only when no GPU is visible.  On a GPU box a missing library is an
error, never a silent skip or fallback."""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


def _gpu_visible() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_visible():
        return
    skip = pytest.mark.skip(reason="no GPU visible (gpu tier runs on the MI355X box)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def afx():
    """The bound HIP library (raises if it was not built)."""
    from aneforge_amd import _hip
    return _hip.load()
