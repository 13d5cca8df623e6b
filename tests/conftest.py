"""Shared test setup: import paths, the ``gpu`` marker, small helpers."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
for entry in (REPO / "ictc-o2-hp_amd", REPO):
    if str(entry) not in sys.path:
        sys.path.insert(0, str(entry))

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def golden_tp():
    return np.load(GOLDEN / "tp_vectors.npz")


@pytest.fixture(scope="session")
def golden_uvu():
    return np.load(GOLDEN / "uvu_vectors.npz")
