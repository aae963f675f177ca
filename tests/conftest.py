"""Shared test setup: import paths, the `gpu` marker, seeded helpers.

Tests marked ``gpu`` need a HIP device and the built extension; everything else runs on
the CPU (``pytest -m "not gpu"``).  Without a GPU the gpu-marked tests are skipped when
collected anyway, so a plain ``pytest`` run on a CPU box stays green.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "tfg-flashattention_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built extension")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no HIP GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
