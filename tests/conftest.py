"""Shared pytest configuration.

Markers: ``gpu`` — needs a ROCm GPU and the built liblik_hip.so; everything
else runs on the CPU. The package lives in late-interaction-kernels_amd/ and
the CPU oracle in oracle/; both go on sys.path here.
"""

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "late-interaction-kernels_amd", ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _seed():
    import torch

    torch.manual_seed(0)
    np.random.seed(0)


def rel_err(actual, reference) -> float:
    """max|a - b| / max(1e-6, max|b|) — the reference's tolerance metric (tests/conftest.py:30-33)."""
    a = np.asarray(actual, dtype=np.float64)
    b = np.asarray(reference, dtype=np.float64)
    if b.size == 0:
        return 0.0
    return float(np.abs(a - b).max() / max(1e-6, np.abs(b).max()))
