"""Shared fixtures for the ssa_amd test suite.

GPU tests are marked ``@pytest.mark.gpu``; everything else runs on the CPU
(oracle against golden vectors, host logic, C-ABI symbol exports).
"""
import glob
import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X)")


def golden_files():
    return sorted(glob.glob(os.path.join(GOLDEN, "*_s*.npz")))


def load_golden(path):
    z = np.load(path)
    meta = json.loads(str(z["meta"]))
    return z, meta


@pytest.fixture(autouse=True)
def _seed():
    import torch
    torch.manual_seed(42)
    yield


def has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def row_rel_err(got, ref):
    """Largest per-row relative error: max over rows (the last dimension) of
    max |got - ref| / max |ref| within the row."""
    g = np.asarray(got, np.float64).reshape(-1, np.shape(got)[-1])
    r = np.asarray(ref, np.float64).reshape(-1, np.shape(ref)[-1])
    scale = np.maximum(np.abs(r).max(-1), 1e-30)
    return float((np.abs(g - r).max(-1) / scale).max())
