"""Test configuration: import paths, the ``gpu`` marker and shared helpers."""

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "deepfold-linear_amd")
for p in (ROOT, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

# Surface kernel-side wait timeouts as exceptions in tests (synchronising check).
os.environ.setdefault("DFL_AMD_CHECK", "1")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) device and the built HIP library")


def pytest_collection_modifyitems(config, items):
    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def max_rel_err(got, want) -> float:
    """max |got - want| / max |want| (normwise, per tensor)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    scale = float(np.max(np.abs(want))) if want.size else 0.0
    err = float(np.max(np.abs(got - want))) if want.size else 0.0
    return err / scale if scale > 0 else err


def assert_close_rel(got, want, tol, name=""):
    err = max_rel_err(got, want)
    assert err <= tol, f"{name}: max rel err {err:.3e} > {tol:.1e}"
    return err
