"""Shared pytest setup.

Markers: `gpu` = needs an MI355X (run with -m gpu on the GPU box); everything else runs on the
CPU. The CPU suite checks the oracle, the host logic and the C-ABI boundary without any GPU
call; the GPU suite compares the HIP kernels (through the C ABI) with the oracle.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "cuflash-attn_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (MI355X)")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


def pytest_collection_modifyitems(config, items):
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def lib():
    import cuflash_attn

    return cuflash_attn.load_library()


@pytest.fixture(scope="session")
def torch_gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def max_abs(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if a.size == 0:
        return 0.0
    return float(np.max(np.abs(a - b)))


def max_rel(a, b) -> float:
    """max |a - b| / max |b| (the FP32 parity measure)."""
    b = np.asarray(b, dtype=np.float64)
    denom = float(np.max(np.abs(b))) if b.size else 1.0
    return max_abs(a, b) / max(denom, 1e-30)
