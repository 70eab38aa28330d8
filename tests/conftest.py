"""Shared pytest setup.

* ``gpu`` marks tests that launch HIP kernels (run with ``-m gpu`` on an MI355X box);
  everything else runs on the CPU.
* The drop-in modules live in ``pico-kernels_amd/`` and are imported by their reference
  names (``import gemm_int4``), exactly as the reference's tests import them.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "pico-kernels_amd"
GOLDEN = Path(__file__).resolve().parent / "golden"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) GPU and the built HIP library")


@pytest.fixture(scope="session")
def golden():
    """Reference-generated vectors (tests/golden/make_golden.py): (arrays, manifest)."""
    arrays = np.load(GOLDEN / "reference_vectors.npz", allow_pickle=False)
    meta = json.loads((GOLDEN / "reference_vectors.json").read_text())
    return arrays, meta


@pytest.fixture(scope="session")
def cuda():
    """The GPU device; GPU tests fail loudly (not skip) when the library or GPU is missing."""
    import torch

    import _pk

    _pk.lib()
    assert torch.cuda.is_available(), "gpu-marked test run without a visible ROCm GPU"
    return torch.device("cuda", 0)
