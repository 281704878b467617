"""Shared pytest setup: repo root on sys.path and the ``gpu`` marker.

``-m "not gpu"`` runs everywhere (no device needed). ``-m gpu`` needs a ROCm
device and the built HIP library (``python -c "import __graft_entry__ as g;
g.build()"``).
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs a ROCm GPU and the built libpathtile_hip.so"
    )


def _gpu_available() -> bool:
    try:
        import torch

        return bool(torch.cuda.is_available())
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
