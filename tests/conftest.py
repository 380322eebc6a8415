"""Test configuration: the ``gpu`` marker and import paths.

``-m gpu`` tests need a HIP device and the built library; they are skipped (not failed)
when no GPU is visible.  Everything else runs on the CPU: the oracle against its pins,
host logic, and the C-ABI library's exports.
"""

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GPU = torch.cuda.is_available()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and libswarp_hip.so")


def pytest_collection_modifyitems(config, items):
    if GPU:
        return
    skip = pytest.mark.skip(reason="no HIP device visible")
    for item in items:
        if item.get_closest_marker("gpu") is not None:
            item.add_marker(skip)
