"""pytest configuration: the ``gpu`` marker and shared helpers.

``gpu`` tests need a visible HIP GPU and the built ``libpmdelta.so``; they
are skipped only when no GPU is visible (the reference's policy,
``pyproject.toml:45-46``), never for any other reason.
"""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built libpmdelta.so")


def _gpu_visible() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_visible():
        return
    skip = pytest.mark.skip(reason="needs a GPU (none visible)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
