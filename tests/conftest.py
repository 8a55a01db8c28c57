"""Shared test setup: import paths, the `gpu` marker, tolerance helpers."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "circulantattention.jl_amd", "oracle"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


def rel_err(out, ref):
    """max |out - ref| / max |ref| (normwise relative error, max norm)."""
    out = np.asarray(out, dtype=np.complex128 if np.iscomplexobj(out) else np.float64)
    ref = np.asarray(ref, dtype=np.complex128 if np.iscomplexobj(ref) else np.float64)
    den = np.max(np.abs(ref)) if ref.size else 0.0
    num = np.max(np.abs(out - ref)) if ref.size else 0.0
    return num / den if den > 0 else num


# Tolerances stated by the task for this path (float32 against a float64
# oracle, max-norm relative): forward values 1e-5, gradients 1e-4.
TOL_FWD = 1e-5
TOL_GRAD = 1e-4


@pytest.fixture(scope="session")
def cuda():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda:0")
