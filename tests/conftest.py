"""Shared pytest setup.

Markers: ``gpu`` marks tests that need a ROCm GPU (MI355X); the CPU suite runs
with ``-m "not gpu"``.  GPU tests call the HIP kernels through the C ABI and
compare them with the CPU oracle under ``oracle/``.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

os.environ.setdefault("OMP_NUM_THREADS", "8")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X, gfx950)")


@pytest.fixture(scope="session")
def hip_backend():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from breezetoken_amd.backend import HipBackend

    backend = HipBackend("cuda")
    print(f"\n[gpu] {backend!r}", flush=True)
    yield backend
    backend.close()
