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


# Outputs the backward reduces across channels / batch / time: with the
# atomic reduction their rounding varies from run to run. Run-to-run bar of
# those sums: max|a - b| / max|a| <= RED_TOL (fp32 sums of up to a few
# thousand terms, reordered).
REDUCED = frozenset({"dAneg", "dA", "dB", "dC", "dbias", "ddt_bias"})
RED_TOL = 2e-6


class reduction:
    """Context manager: the backward's reduction mode (_native.REDUCTION_*)."""

    def __init__(self, mode: int):
        self.mode = mode

    def __enter__(self):
        from mamba_metal_scan_amd import _native
        _native.set_reduction(self.mode)
        return self

    def __exit__(self, *exc):
        from mamba_metal_scan_amd import _native
        _native.set_reduction(_native.REDUCTION_AUTO)


def assert_same(name: str, got, ref, atomic: bool) -> float:
    """Bit-for-bit equality, except for the atomically reduced sums, which
    must agree within RED_TOL; returns the relative difference."""
    if atomic and name in REDUCED:
        return assert_close(name, got, ref, RED_TOL)
    assert torch.equal(got, ref), f"{name} differs"
    return 0.0
