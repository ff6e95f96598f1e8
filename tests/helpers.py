"""Comparison helpers shared by the test modules."""
from __future__ import annotations

import numpy as np
import torch

# The parity bar of this build: per tensor, max|got - ref| / max|ref| <= TOL
# against the float64 oracle (and the fp32 torch reference).
TOL = 1e-4
# The reference's own per-element tolerance (tests/test_scan.py:24).
ATOL, RTOL = 1e-4, 1e-3


def to_np(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        return t.detach().cpu().double().numpy()
    return np.asarray(t, dtype=np.float64)


def rel_err(got, ref) -> float:
    """max|got - ref| / max|ref| (max|ref| floored at 1e-30)."""
    g, r = to_np(got), to_np(ref)
    assert g.shape == r.shape, (g.shape, r.shape)
    if r.size == 0:
        return 0.0
    return float(np.abs(g - r).max() / max(np.abs(r).max(), 1e-30))


def assert_close(name: str, got, ref, tol: float = TOL) -> float:
    err = rel_err(got, ref)
    assert err <= tol, f"{name}: max rel err {err:.3e} > {tol:.1e}"
    return err
