"""GPU parity of the block's fused ops around the scan against the float64
oracle: the gated scan (dt gate and softplus(A) inside the scan kernels,
mamba_metal/model.py:197-200) and the output gate (y + D_skip) * silu(z)
(model.py:255-256).

Bar: per tensor, max|got - ref| / max|ref| <= 1e-4 against the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close, assert_same, reduction
from mamba_metal_scan_amd import (_native, out_gate, selective_scan_gated, selective_scan_hip)
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
LO, HI = 0.001, 0.1   # MambaConfig dt_min, dt_max (model.py:53-54)


def _gated_inputs(bt, t_len, d, n, seed):
    """x ~ N(0,1); dt_raw ~ N(0,2) (dt spread over the gate's range, some
    saturated); A = n+1 + 0.3 N(0,1) (the block's init, perturbed); B, C ~ N(0,1)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((bt, t_len, d), dtype=np.float32)
    raw = (2.0 * rng.standard_normal((bt, t_len, d))).astype(np.float32)
    a = (np.tile(np.arange(1, n + 1, dtype=np.float32), (d, 1))
         + 0.3 * rng.standard_normal((d, n))).astype(np.float32)
    b_in = rng.standard_normal((bt, t_len, n), dtype=np.float32)
    c_in = rng.standard_normal((bt, t_len, n), dtype=np.float32)
    return [x, raw, a, b_in, c_in]


# (B, T, D, N, chunk): T below, at and off multiples of 16; d_state not a
# multiple of 4; checkpoint strides below, at and above the backward's window
# (the last recomputes finer checkpoints, also through the gate).
GATED_CASES = [(2, 64, 96, 16, 16), (1, 100, 40, 16, 16), (2, 7, 33, 8, 16), (3, 130, 70, 5, 7),
               (2, 77, 64, 16, 64), (1, 50, 128, 32, 16), (1, 24, 64, 64, 16),
               (16, 512, 1432, 16, 16)]


@pytest.mark.parametrize("bt,t_len,d,n,chunk", GATED_CASES)
def test_gated_scan_matches_the_oracle(bt, t_len, d, n, chunk):
    print(f"[case] gated scan {bt}x{t_len}x{d}x{n} chunk {chunk}", flush=True)
    arrs = _gated_inputs(bt, t_len, d, n, seed=d + n)
    rng = np.random.default_rng(8)
    dy = rng.standard_normal((bt, t_len, d), dtype=np.float32)
    dh = rng.standard_normal((bt, d, n), dtype=np.float32)
    y_ref, _, h_ref = oracle.scan_gated_fwd(*arrs, LO, HI)
    g_ref = oracle.scan_gated_bwd(*arrs, LO, HI, dy, dh_last=dh)

    leaves = [torch.from_numpy(a).to(DEV).requires_grad_(True) for a in arrs]
    y, h_last = selective_scan_gated(*leaves, LO, HI, chunk=chunk, return_state=True)
    grads = torch.autograd.grad([y, h_last], leaves,
                                grad_outputs=[torch.from_numpy(dy).to(DEV),
                                              torch.from_numpy(dh).to(DEV)])
    torch.cuda.synchronize()
    assert_close("y", y, y_ref)
    assert_close("h_last", h_last, h_ref)
    for name, g, r in zip(("dx", "ddt_raw", "dA", "dB", "dC"), grads, g_ref):
        assert g.shape == r.shape, name
        assert_close(name, g, r)


# With the dt projection's bias inside the kernels: grids small enough to run
# in time segments (the carry passes stage the biased gate too, and every
# segment leaves its own bias partials), a stride above the backward's window
# (fine checkpoints recomputed through the biased gate), channels off the
# 32-channel blocks, and the 80M block's shape.
BIAS_CASES = [(1, 600, 64, 16, 16), (2, 333, 40, 16, 16), (2, 77, 64, 16, 64),
              (3, 130, 70, 5, 7), (16, 512, 1432, 16, 16)]


@pytest.mark.parametrize("bt,t_len,d,n,chunk", BIAS_CASES)
def test_gated_scan_with_dt_bias_matches_the_oracle(bt, t_len, d, n, chunk):
    """dt = lo + span * sigmoid(raw + bias): the oracle on raw + bias, and the
    bias gradient equal to the oracle's raw gradient summed over batch and
    time (raw + bias depends on the bias with derivative one); the bias
    gradient is also reproducible run to run (bit for bit under the
    fixed-order reduction, to rounding under atomics)."""
    print(f"[case] gated scan with dt bias {bt}x{t_len}x{d}x{n} chunk {chunk}", flush=True)
    arrs = _gated_inputs(bt, t_len, d, n, seed=3 * d + n)
    rng = np.random.default_rng(11)
    bias = (0.7 * rng.standard_normal(d)).astype(np.float32)
    dy = rng.standard_normal((bt, t_len, d), dtype=np.float32)
    ref_in = list(arrs)
    ref_in[1] = (arrs[1].astype(np.float64) + bias.astype(np.float64)).astype(np.float64)
    y_ref, _, _ = oracle.scan_gated_fwd(*ref_in, LO, HI)
    g_ref = list(oracle.scan_gated_bwd(*ref_in, LO, HI, dy))
    g_ref.append(np.asarray(g_ref[1]).sum(axis=(0, 1)))

    runs = []
    for _ in range(2):
        leaves = [torch.from_numpy(a).to(DEV).requires_grad_(True) for a in arrs]
        tb = torch.from_numpy(bias).to(DEV).requires_grad_(True)
        y = selective_scan_gated(*leaves, LO, HI, chunk=chunk, dt_bias=tb)
        grads = torch.autograd.grad(y, leaves + [tb], torch.from_numpy(dy).to(DEV))
        runs.append((y.detach(), grads))
    torch.cuda.synchronize()
    y, grads = runs[0]
    assert_close("y", y, y_ref)
    for name, g, r in zip(("dx", "ddt_raw", "dA", "dB", "dC", "dbias"), grads, g_ref):
        assert g.shape == np.asarray(r).shape, name
        assert_close(name, g, r)
    atomic = _native.bwd_reduction(bt, t_len, d, n, chunk) == _native.REDUCTION_ATOMIC
    assert_same("dbias", runs[0][1][5], runs[1][1][5], atomic)


@pytest.mark.parametrize("bt,t_len,d,n,chunk", [(1, 600, 64, 16, 16), (3, 130, 70, 5, 7),
                                                  (2, 77, 64, 16, 64)])
def test_gated_scan_with_one_state_per_lane(bt, t_len, d, n, chunk):
    """The same checks with one state per lane forced (8-wave blocks at
    d_state 16, 4-wave blocks at 5): the gate, the bias partials and, in the
    first case, the time segments' carry passes."""
    _native.set_variant(1)
    try:
        test_gated_scan_with_dt_bias_matches_the_oracle(bt, t_len, d, n, chunk)
    finally:
        _native.set_variant(0)


def test_gated_scan_rejects_a_bad_dt_bias():
    arrs = [torch.from_numpy(a).to(DEV) for a in _gated_inputs(1, 8, 32, 16, seed=1)]
    with pytest.raises(ValueError, match="dt_bias"):
        selective_scan_gated(*arrs, LO, HI, dt_bias=torch.zeros(31, device=DEV))
    with pytest.raises(ValueError, match="dt_bias"):
        selective_scan_gated(*arrs, LO, HI, dt_bias=torch.zeros(32, device=DEV,
                                                                 dtype=torch.float64))


def test_gated_scan_equals_the_scan_on_torch_gated_inputs():
    """Gate fused in the kernels == the framework's gate followed by the plain
    HIP scan, values and gradients (within fp32 rounding of dt)."""
    bt, t_len, d, n = 4, 200, 256, 16
    arrs = _gated_inputs(bt, t_len, d, n, seed=5)
    dy = torch.from_numpy(np.random.default_rng(9).standard_normal(
        (bt, t_len, d), dtype=np.float32)).to(DEV)
    l1 = [torch.from_numpy(a).to(DEV).requires_grad_(True) for a in arrs]
    y1 = selective_scan_gated(*l1, LO, HI, chunk=16)
    g1 = torch.autograd.grad(y1, l1, dy)
    l2 = [torch.from_numpy(a).to(DEV).requires_grad_(True) for a in arrs]
    dt = LO + (HI - LO) * torch.sigmoid(l2[1])
    y2 = selective_scan_hip(l2[0], dt, torch.nn.functional.softplus(l2[2]), l2[3], l2[4], chunk=16)
    g2 = torch.autograd.grad(y2, l2, dy)
    torch.cuda.synchronize()
    assert_close("y", y1, y2)
    for name, a, b in zip(("dx", "ddt_raw", "dA", "dB", "dC"), g1, g2):
        assert_close(name, a, b)


@pytest.mark.parametrize("mode", ["fixed", "atomic"])
def test_gated_scan_determinism(mode):
    """Fixed-order reduction: bit for bit run to run; atomic: y, dx, ddt_raw
    bit for bit and the reduced sums (dA, dB, dC) within RED_TOL."""
    atomic = mode == "atomic"
    arrs = _gated_inputs(8, 300, 200, 16, seed=6)
    dy = torch.from_numpy(np.random.default_rng(10).standard_normal(
        (8, 300, 200), dtype=np.float32)).to(DEV)
    runs = []
    with reduction(_native.REDUCTION_ATOMIC if atomic else _native.REDUCTION_FIXED):
        for _ in range(2):
            leaves = [torch.from_numpy(a).to(DEV).requires_grad_(True) for a in arrs]
            y = selective_scan_gated(*leaves, LO, HI, chunk=16)
            runs.append([y.detach()] + list(torch.autograd.grad(y, leaves, dy)))
    for name, a, b in zip(("y", "dx", "ddt_raw", "dA", "dB", "dC"), *runs):
        assert_same(name, a, b, atomic)


def test_gated_scan_rejects_bad_gate():
    x = torch.randn(1, 8, 16, device=DEV)
    args = (x, x.clone(), torch.randn(16, 4, device=DEV), torch.randn(1, 8, 4, device=DEV),
            torch.randn(1, 8, 4, device=DEV))
    with pytest.raises(ValueError, match="dt_min < dt_max"):
        selective_scan_gated(*args, 0.1, 0.1)
    with pytest.raises(RuntimeError, match="dt_min < dt_max"):
        torch.ops.mamba_hip.scan_gated_fwd(*args, 0.1, float("inf"), 16, False)


@pytest.mark.parametrize("bt,t_len,d", [(2, 64, 96), (1, 5, 33), (3, 100, 130), (16, 512, 1432)])
@pytest.mark.parametrize("strided", [False, True])
def test_out_gate_matches_the_oracle(bt, t_len, d, strided):
    print(f"[case] out gate {bt}x{t_len}x{d} strided={strided}", flush=True)
    rng = np.random.default_rng(d)
    y = rng.standard_normal((bt, t_len, d), dtype=np.float32)
    dsk = rng.standard_normal(d, dtype=np.float32)
    zbase = rng.standard_normal((bt, t_len, 2 * d if strided else d), dtype=np.float32)
    z = zbase[..., d:] if strided else zbase          # the z half of in_proj: rows 2d apart
    dout = rng.standard_normal((bt, t_len, d), dtype=np.float32)
    yd = torch.from_numpy(y).to(DEV).requires_grad_(True)
    dd = torch.from_numpy(dsk).to(DEV).requires_grad_(True)
    zleaf = torch.from_numpy(zbase).to(DEV).requires_grad_(True)
    zv = zleaf[..., d:] if strided else zleaf
    out = out_gate(yd, dd, zv)
    out.backward(torch.from_numpy(dout).to(DEV))
    torch.cuda.synchronize()
    o_ref = oracle.out_gate_fwd(y, dsk, z)
    gy, gd, gz = oracle.out_gate_bwd(y, dsk, z, dout)
    assert out.is_contiguous()
    assert_close("out", out, o_ref)
    assert_close("dy", yd.grad, gy)
    assert_close("dD_skip", dd.grad, gd)
    gz_got = zleaf.grad[..., d:] if strided else zleaf.grad
    assert_close("dz", gz_got, gz)
    if strided:
        assert torch.count_nonzero(zleaf.grad[..., :d]) == 0


def test_out_gate_backward_is_bitwise_deterministic():
    g = torch.Generator().manual_seed(4)
    y, z, dout = (torch.randn(8, 300, 500, generator=g).to(DEV) for _ in range(3))
    dsk = torch.randn(500, generator=g).to(DEV)
    runs = []
    for _ in range(2):
        leaves = [t.clone().requires_grad_(True) for t in (y, dsk, z)]
        out_gate(*leaves).backward(dout)
        runs.append([t.grad for t in leaves])
    for a, b in zip(*runs):
        assert torch.equal(a, b)


def test_out_gate_rejects_bad_dtypes_and_shapes():
    y = torch.zeros(2, 8, 16, device=DEV)
    d_skip = torch.zeros(16, device=DEV)
    with pytest.raises(RuntimeError, match="fp32-only"):
        out_gate(y.to(torch.bfloat16), d_skip, y)
    with pytest.raises(ValueError, match="bad shapes"):
        out_gate(y, torch.zeros(15, device=DEV), y)
    with pytest.raises(ValueError, match="bad shapes"):
        out_gate(y, d_skip, y[:, :7])


def test_gated_scan_rejects_mismatched_shapes():
    """The gated entry validates like selective_scan (ValueError on shapes)."""
    x = torch.zeros(1, 8, 16, device=DEV)
    a = torch.zeros(16, 4, device=DEV)
    bc = torch.zeros(1, 8, 4, device=DEV)
    with pytest.raises(ValueError):
        selective_scan_gated(x, x, a[:15], bc, bc, LO, HI)
    with pytest.raises(ValueError):
        selective_scan_gated(x, x, a, bc[:, :7], bc, LO, HI)


INNER_NAMES = ("dxz", "dconv_w", "dconv_b", "dW_dt", "db_dt", "dW_B", "dW_C", "dA", "dD")


@pytest.mark.parametrize("bt,t_len,d,n", [(2, 64, 96, 16), (3, 100, 256, 8), (1, 37, 64, 4),
                                          (16, 512, 1432, 16)])
def test_mamba_inner_matches_the_unfused_ops(bt, t_len, d, n):
    """The fused inner block (one projection GEMM read in place, gradients
    written in place) equals the same ops applied one by one: output and all
    nine gradients within 1e-4 (max rel per tensor; only the summation order
    of the projections' input gradient differs)."""
    import torch.nn.functional as F
    from mamba_metal_scan_amd import conv1d_silu, mamba_inner
    print(f"[case] mamba_inner {bt}x{t_len}x{d}x{n}", flush=True)
    g = torch.Generator().manual_seed(d + n)
    r = lambda *s, sc=1.0: (sc * torch.randn(*s, generator=g)).to(DEV)
    k = 4
    a_raw = (torch.log(torch.arange(1, n + 1, dtype=torch.float32)).expand(d, n)
             + 0.1 * torch.randn(d, n, generator=g)).contiguous().to(DEV)
    params = [r(bt, t_len, 2 * d), r(d, 1, k, sc=0.3), r(d, sc=0.1), r(d, d, sc=0.05),
              r(d, sc=0.5), r(n, d, sc=0.1), r(n, d, sc=0.1), a_raw, r(d)]
    dout = r(bt, t_len, d)
    p1 = [t.clone().requires_grad_(True) for t in params]
    p2 = [t.clone().requires_grad_(True) for t in params]
    out1 = mamba_inner(*p1, LO, HI, chunk=16)
    g1 = torch.autograd.grad(out1, p1, dout)
    x, z = p2[0].chunk(2, dim=-1)
    xc = conv1d_silu(x, p2[1], p2[2])
    y = selective_scan_gated(xc, F.linear(xc, p2[3], p2[4]), p2[7], F.linear(xc, p2[5]),
                             F.linear(xc, p2[6]), LO, HI, chunk=16)
    out2 = out_gate(y, p2[8], z)
    g2 = torch.autograd.grad(out2, p2, dout)
    torch.cuda.synchronize()
    assert out1.shape == (bt, t_len, d) and out1.is_contiguous()
    assert_close("out", out1, out2, 1e-5)
    for name, a1, a2 in zip(INNER_NAMES, g1, g2):
        assert a1.shape == a2.shape, name
        assert_close(name, a1, a2, 1e-4)


def test_mamba_inner_rejects_unaligned_sizes():
    from mamba_metal_scan_amd import mamba_inner
    d, n = 90, 16
    args = [torch.zeros(1, 8, 2 * d, device=DEV), torch.zeros(d, 1, 4, device=DEV),
            torch.zeros(d, device=DEV), torch.zeros(d, d, device=DEV), torch.zeros(d, device=DEV),
            torch.zeros(n, d, device=DEV), torch.zeros(n, d, device=DEV),
            torch.zeros(d, n, device=DEV), torch.zeros(d, device=DEV)]
    with pytest.raises(ValueError, match="multiples of 4"):
        mamba_inner(*args, LO, HI)
