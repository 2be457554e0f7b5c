"""Shared test setup: the `gpu` marker, repo root on sys.path, tolerance helpers."""

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def cuda():
    if not gpu_available():
        pytest.skip("no GPU visible")
    import torch
    torch.cuda.init()
    return torch.device("cuda", 0)


def row_rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """Largest per-(row, head) ||got - ref||_inf / max(||ref||_inf, 1e-6) (the parity metric)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    g = got.reshape(-1, got.shape[-1])
    r = ref.reshape(-1, ref.shape[-1])
    num = np.abs(g - r).max(axis=1)
    den = np.maximum(np.abs(r).max(axis=1), 1e-6)
    return float((num / den).max()) if num.size else 0.0


TOL = {"f32": 1e-5, "f16": 2e-3, "bf16": 2e-3, "q8_0": 2e-3}
