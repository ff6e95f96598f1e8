"""Host-side behaviour of the scan API on the CPU (the reference's gate 1 and
its dispatch rules, tests/test_scan.py:45-96):

* selective_scan_ref is the recurrence, in float64 to 1e-10, and agrees with
  the float64 oracle in value, returned state and every gradient;
* dispatch: 'torch' runs anywhere, unknown impls raise ValueError naming
  scan_impl, 'hip'/'metal' off-device raise RuntimeError, 'auto' off-device
  returns None;
* the HIP entry validates devices first, then dtypes, then shapes, with the
  reference's exception types.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close
from mamba_metal_scan_amd import (selective_scan, selective_scan_hip, selective_scan_metal,
                                  selective_scan_ref)
from mamba_metal_scan_amd.model import scan_recurrence
from oracle import oracle

SEED = 1337


def _inputs(bt, t_len, d, n, seed=SEED, dtype=torch.float64):
    arrs = oracle.make_inputs(bt, t_len, d, n, seed, style="ref")
    return [torch.from_numpy(a).to(dtype) for a in arrs]


@pytest.mark.parametrize("shape", [(2, 40, 7, 5), (1, 1, 1, 4), (1, 33, 5, 8), (1, 64, 1, 16),
                                   (1, 97, 3, 4)])
def test_reference_matches_the_recurrence_in_float64(shape):
    x, dt, aneg, b_in, c_in = _inputs(*shape, seed=SEED + shape[1])
    a = torch.exp(-dt.unsqueeze(-1) * aneg.unsqueeze(0))
    b = dt.unsqueeze(-1) * b_in.unsqueeze(2) * x.unsqueeze(-1)
    h = scan_recurrence(a, b)
    y = selective_scan_ref(x, dt, aneg, b_in, c_in)
    assert torch.allclose(y, (h * c_in.unsqueeze(2)).sum(-1), atol=1e-10)


def test_reference_matches_the_oracle_with_gradients():
    shape = (2, 30, 6, 8)
    arrs = oracle.make_inputs(*shape, seed=5, style="bench")
    leaves = [torch.from_numpy(a).double().requires_grad_(True) for a in arrs]
    rng = np.random.default_rng(6)
    dy = rng.standard_normal((2, 30, 6))
    dh = rng.standard_normal((2, 6, 8))
    y, h = selective_scan_ref(*leaves, return_state=True)
    grads = torch.autograd.grad([y, h], leaves,
                                grad_outputs=[torch.from_numpy(dy), torch.from_numpy(dh)])
    y_ref, _, h_ref = oracle.scan_fwd(*arrs)
    g_ref = oracle.scan_bwd(*arrs, dy, dh_last=dh)
    assert_close("y", y, y_ref, tol=1e-12)
    assert_close("h_last", h, h_ref, tol=1e-12)
    for name, g, r in zip(("dx", "ddt", "dAneg", "dB", "dC"), grads, g_ref):
        assert_close(name, g, r, tol=1e-11)


def test_torch_impl_runs_on_cpu_and_returns_state():
    x, dt, aneg, b_in, c_in = _inputs(2, 12, 4, 4, dtype=torch.float32)
    y = selective_scan(x, dt, aneg, b_in, c_in, impl="torch")
    y2, h = selective_scan(x, dt, aneg, b_in, c_in, impl="torch", return_state=True)
    assert torch.equal(y, y2) and h.shape == (2, 4, 4)
    _, _, h_ref = oracle.scan_fwd(*(t.numpy() for t in (x, dt, aneg, b_in, c_in)))
    assert_close("h_last", h, h_ref)


def test_unknown_scan_impl_is_rejected():
    x, dt, aneg, b_in, c_in = _inputs(1, 4, 8, 4, dtype=torch.float32)
    with pytest.raises(ValueError, match="scan_impl"):
        selective_scan(x, dt, aneg, b_in, c_in, impl="nonsense")


@pytest.mark.parametrize("impl", ["hip", "metal"])
def test_hip_requires_device_tensors(impl):
    x, dt, aneg, b_in, c_in = _inputs(1, 8, 16, 4, dtype=torch.float32)
    with pytest.raises(RuntimeError, match="ROCm"):
        selective_scan(x, dt, aneg, b_in, c_in, impl=impl)


def test_auto_declines_off_device():
    x, dt, aneg, b_in, c_in = _inputs(1, 8, 16, 4, dtype=torch.float32)
    assert selective_scan(x, dt, aneg, b_in, c_in, impl="auto") is None


def test_direct_entry_checks_device_before_dtype_and_shape():
    x, dt, aneg, b_in, c_in = _inputs(1, 8, 16, 4, dtype=torch.float64)
    # CPU tensors of the wrong dtype and shape: the device error comes first.
    with pytest.raises(RuntimeError, match="ROCm device"):
        selective_scan_hip(x, dt, aneg[:, :3], b_in, c_in)
    with pytest.raises(RuntimeError, match="ROCm device"):
        selective_scan_metal(x, dt, aneg, b_in, c_in, 16, 64)


def test_gated_scan_checks_the_gate_then_the_device():
    """selective_scan_gated: dt_min < dt_max is checked first (ValueError),
    then the inputs' device, with selective_scan's RuntimeError."""
    from mamba_metal_scan_amd import selective_scan_gated
    x, dt, aneg, b_in, c_in = _inputs(1, 8, 16, 4, dtype=torch.float32)
    for lo, hi in ((0.1, 0.1), (0.2, 0.1)):
        with pytest.raises(ValueError, match="dt_min < dt_max"):
            selective_scan_gated(x, dt, aneg, b_in, c_in, lo, hi)
    with pytest.raises(RuntimeError, match="ROCm device"):
        selective_scan_gated(x, dt, aneg, b_in, c_in, 0.001, 0.1)
    # wrong dtype and shape as well: still the device error first
    with pytest.raises(RuntimeError, match="ROCm device"):
        selective_scan_gated(x.double(), dt, aneg[:, :3], b_in, c_in, 0.001, 0.1)


def test_out_gate_checks_device_before_dtype_and_shape():
    from mamba_metal_scan_amd import out_gate
    y = torch.zeros(1, 8, 16)
    with pytest.raises(RuntimeError, match="ROCm device"):
        out_gate(y, torch.zeros(16), y)
    with pytest.raises(RuntimeError, match="ROCm device"):
        out_gate(y.double(), torch.zeros(5), y[:, :3])
