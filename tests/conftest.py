"""Shared test setup.

Markers: ``gpu`` -- needs an MI355X (run with ``-m gpu``); everything else
runs on the CPU.  GPU tests call the HIP kernels through the C ABI and fail
(never skip) when the native library is missing on a GPU box.
"""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden" / "golden.npz"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def cuda():
    """The GPU device; on a GPU run the native library must load."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    from kuillm_amd import compile as _compile
    _compile.load_library()          # raises when libkuiops.so is missing
    return torch.device("cuda:0")
