"""Shared pytest configuration.

CPU tests run single-threaded (CPU matmul results can depend on the thread count, as
the reference's ``tests/conftest.py:1-12`` notes). Tests marked ``gpu`` need the HIP
extension and a GPU; without a GPU they are skipped.
"""

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))

torch.set_num_threads(1)

HAS_GPU = torch.cuda.is_available()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) GPU")
    config.addinivalue_line("markers", "slow: takes more than a few seconds on the CPU")


def pytest_collection_modifyitems(config, items):
    skip = pytest.mark.skip(reason="needs a GPU")
    for item in items:
        if "gpu" in item.keywords and not HAS_GPU:
            item.add_marker(skip)
