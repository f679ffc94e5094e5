"""Shared pytest setup: the `gpu` marker, the GPU gate, and seeded helpers.

GPU tests call the HIP library through its C ABI (ctypes); they are skipped
when no GPU is visible and fail loudly when the library is missing.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libmxdecode.so")


def _gpu_available() -> bool:
    if not os.path.exists("/dev/kfd"):
        return False
    import torch

    return torch.cuda.is_available()


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def dev():
    """The GPU device; also loads libmxdecode.so (raises if it is not built)."""
    import torch

    from gemmagemini4hackathon2026_10_2425_amd import _lib

    _lib.load()
    torch.cuda.set_device(0)
    return torch.device("cuda", 0)


def rel_err(got, ref) -> float:
    """max |got - ref| / max |ref| (the relative error the tolerances refer to)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = max(np.abs(ref).max(), 1e-30)
    return float(np.abs(got - ref).max() / den)


@pytest.fixture
def rng():
    return np.random.default_rng(20261201)
