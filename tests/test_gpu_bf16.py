"""GPU parity of the bf16-activation scan (bf16 x, dt, B, C and dy in, bf16 y,
dx, ddt, dB, dC out; fp32 Aneg, state, checkpoints and arithmetic) against the
float64 oracle run on the same bf16-rounded inputs.

Bar, per tensor (max|got - ref| / max|ref|): 4e-3 for bf16 outputs, whose
round-to-nearest-even storage alone costs up to 2^-9 = 1.95e-3 relative; 1e-4
for the fp32 outputs (h_last, checkpoints, dAneg / dA).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close
from mamba_metal_scan_amd import _native, selective_scan_gated, selective_scan_hip
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL_BF16 = 4e-3
TOL_F32 = 1e-4
LO, HI = 0.001, 0.1


def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a).to(torch.bfloat16)


def _f64(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.float64).numpy()


@pytest.mark.parametrize("bt,t_len,d,n,chunk", [(2, 64, 96, 16, 16), (1, 100, 40, 16, 7),
                                                (2, 77, 64, 8, 64), (3, 33, 70, 5, 16),
                                                (16, 512, 1536, 16, 16)])
def test_bf16_scan_matches_the_oracle(bt, t_len, d, n, chunk):
    print(f"[case] bf16 scan {bt}x{t_len}x{d}x{n} chunk {chunk}", flush=True)
    x, dt, aneg, b_in, c_in = oracle.make_inputs(bt, t_len, d, n, seed=500 + d, style="bench")
    rng = np.random.default_rng(6)
    dy = rng.standard_normal((bt, t_len, d), dtype=np.float32)
    dh = rng.standard_normal((bt, d, n), dtype=np.float32)
    acts = [_bf16(a) for a in (x, dt, b_in, c_in)]
    dyb = _bf16(dy)
    # the oracle sees exactly the bf16 values the kernels read
    ref_in = [_f64(acts[0]), _f64(acts[1]), aneg, _f64(acts[2]), _f64(acts[3])]
    y_ref, _, h_ref = oracle.scan_fwd(*ref_in)
    g_ref = oracle.scan_bwd(*ref_in, _f64(dyb), dh_last=dh)

    xl, dtl, bl, cl = (a.to(DEV).requires_grad_(True) for a in acts)
    al = torch.from_numpy(aneg).to(DEV).requires_grad_(True)
    y, h_last = selective_scan_hip(xl, dtl, al, bl, cl, chunk=chunk, return_state=True)
    assert y.dtype == torch.bfloat16 and h_last.dtype == torch.float32
    grads = torch.autograd.grad([y, h_last], [xl, dtl, al, bl, cl],
                                grad_outputs=[dyb.to(DEV), torch.from_numpy(dh).to(DEV)])
    torch.cuda.synchronize()
    assert [g.dtype for g in grads] == [torch.bfloat16] * 2 + [torch.float32] + [torch.bfloat16] * 2
    assert_close("y", y, y_ref, TOL_BF16)
    assert_close("h_last", h_last, h_ref, TOL_F32)
    for name, g, r in zip(("dx", "ddt", "dAneg", "dB", "dC"), grads, g_ref):
        assert_close(name, g, r, TOL_F32 if name == "dAneg" else TOL_BF16)


@pytest.mark.parametrize("bt,t_len,d,n,chunk", [(2, 64, 96, 16, 16), (2, 77, 64, 8, 64)])
def test_bf16_scan_with_one_state_per_lane(bt, t_len, d, n, chunk):
    """The bf16 scan's checks with one state per lane forced."""
    _native.set_variant(1)
    try:
        test_bf16_scan_matches_the_oracle(bt, t_len, d, n, chunk)
    finally:
        _native.set_variant(0)


@pytest.mark.parametrize("bt,t_len,d,n,segs,bias", [(2, 130, 70, 16, 0, False),
                                                    (16, 512, 1432, 16, 0, False),
                                                    (1, 300, 64, 16, 3, False),
                                                    (2, 130, 70, 16, 0, True),
                                                    (1, 300, 64, 16, 3, True)])
def test_bf16_gated_scan_matches_the_oracle(bt, t_len, d, n, segs, bias):
    """bf16 activations through the gate; with an fp32 dt bias, whose
    gradient (the fp32 sum of the raw dt gradient, before its rounding to
    bf16) meets the fp32 bar."""
    print(f"[case] bf16 gated scan {bt}x{t_len}x{d}x{n} segments {segs} bias {bias}", flush=True)
    rng = np.random.default_rng(d)
    x = rng.standard_normal((bt, t_len, d), dtype=np.float32)
    raw = (2.0 * rng.standard_normal((bt, t_len, d))).astype(np.float32)
    a = (np.tile(np.arange(1, n + 1, dtype=np.float32), (d, 1))
         + 0.3 * rng.standard_normal((d, n))).astype(np.float32)
    b_in = rng.standard_normal((bt, t_len, n), dtype=np.float32)
    c_in = rng.standard_normal((bt, t_len, n), dtype=np.float32)
    dy = rng.standard_normal((bt, t_len, d), dtype=np.float32)
    acts = [_bf16(v) for v in (x, raw, b_in, c_in)]
    dyb = _bf16(dy)
    dt_bias = (0.5 * rng.standard_normal(d)).astype(np.float32) if bias else None
    ref_in = [_f64(acts[0]), _f64(acts[1]), a, _f64(acts[2]), _f64(acts[3])]
    if bias:
        ref_in[1] = ref_in[1] + dt_bias.astype(np.float64)
    y_ref, _, _ = oracle.scan_gated_fwd(*ref_in, LO, HI)
    g_ref = list(oracle.scan_gated_bwd(*ref_in, LO, HI, _f64(dyb)))

    leaves = [acts[0].to(DEV), acts[1].to(DEV), torch.from_numpy(a).to(DEV), acts[2].to(DEV),
              acts[3].to(DEV)]
    leaves = [t.requires_grad_(True) for t in leaves]
    names = ["dx", "ddt_raw", "dA", "dB", "dC"]
    tb = None
    if bias:
        tb = torch.from_numpy(dt_bias).to(DEV).requires_grad_(True)
        leaves.append(tb)
        names.append("dbias")
        g_ref.append(np.asarray(g_ref[1]).sum(axis=(0, 1)))
    _native.set_time_segments(segs)
    try:
        y = selective_scan_gated(*leaves[:5], LO, HI, chunk=16, dt_bias=tb)
        grads = torch.autograd.grad(y, leaves, dyb.to(DEV))
        torch.cuda.synchronize()
    finally:
        _native.set_time_segments(0)
    assert_close("y", y, y_ref, TOL_BF16)
    for name, g, r in zip(names, grads, g_ref):
        assert_close(name, g, r, TOL_F32 if name in ("dA", "dbias") else TOL_BF16)


def test_bf16_matches_fp32_kernels_on_the_same_values():
    """The bf16 path computes what the fp32 path computes on the widened
    inputs: outputs agree to bf16 rounding of the fp32 results."""
    bt, t_len, d, n = 4, 200, 256, 16
    x, dt, aneg, b_in, c_in = oracle.make_inputs(bt, t_len, d, n, seed=77)
    acts = [_bf16(v).to(DEV) for v in (x, dt, b_in, c_in)]
    an = torch.from_numpy(aneg).to(DEV)
    y16, _, h16 = torch.ops.mamba_hip.scan_fwd(acts[0], acts[1], an, acts[2], acts[3], 16, True)
    y32, _, h32 = torch.ops.mamba_hip.scan_fwd(*(acts[0].float(), acts[1].float(), an,
                                                 acts[2].float(), acts[3].float()), 16, True)
    torch.cuda.synchronize()
    assert torch.equal(y16, y32.to(torch.bfloat16))      # same fp32 value, rounded once
    assert torch.equal(h16, h32)


def test_bf16_rejects_mixed_dtypes():
    x = torch.randn(1, 8, 16, device=DEV, dtype=torch.bfloat16)
    an = torch.ones(16, 4, device=DEV)
    bc = torch.randn(1, 8, 4, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="bf16"):
        selective_scan_hip(x, x.float(), an, bc, bc)
    with pytest.raises(RuntimeError, match="bf16"):
        selective_scan_hip(x, x, an.to(torch.bfloat16), bc, bc)
