"""GPU parity of the HIP RMSNorm (mamba_metal/model.py:85-95) with the
reference's formula differentiated in float64 on the CPU, and with the
framework's fused rms_norm in fp32 on the GPU.

Bar, per tensor (max|got - ref| / max|ref|): 1e-5 against float64 (fp32
rounding of sums over up to 8192 terms is about 1e-7 relative); the same
against the framework's fp32 result.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from helpers import assert_close
from mamba_metal_scan_amd import add_rms_norm, rms_norm, rms_norm_residual
from mamba_metal_scan_amd._native import HipScanError
from mamba_metal_scan_amd.model import MambaConfig, TinyMamba

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPS = 1e-6
TOL = 1e-5


def _inputs(rows, cols, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = scale * torch.randn(rows, cols, generator=g)
    w = 1.0 + 0.1 * torch.randn(cols, generator=g)
    dy = torch.randn(rows, cols, generator=g)
    dres = torch.randn(rows, cols, generator=g)
    return x, w, dy, dres


def _reference(x, w, dy, dres=None):
    """The reference's formula in float64: weight * (x * rsqrt(mean(x^2) + eps))."""
    xd = x.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    y = wd * (xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + EPS))
    y.backward(dy.double())
    dx = xd.grad + (dres.double() if dres is not None else 0.0)
    return y.detach(), dx, wd.grad


def _hip(x, w, dy, dres=None):
    xl = x.to(DEV).requires_grad_(True)
    wl = w.to(DEV).requires_grad_(True)
    if dres is None:
        y = rms_norm(xl, wl, EPS)
        dx, dw = torch.autograd.grad(y, [xl, wl], dy.to(DEV))
    else:
        res, y = rms_norm_residual(xl, wl, EPS)
        dx, dw = torch.autograd.grad([res, y], [xl, wl], [dres.to(DEV), dy.to(DEV)])
    torch.cuda.synchronize()
    return y.detach(), dx, dw


@pytest.mark.parametrize("rows,cols", [(8192, 640), (3, 4), (1, 2048), (37, 132), (1000, 256),
                                       (513, 1000), (4096, 128)])
@pytest.mark.parametrize("residual", [False, True])
def test_matches_float64_reference(rows, cols, residual):
    print(f"[case] rmsnorm {rows}x{cols} residual {residual}", flush=True)
    x, w, dy, dres = _inputs(rows, cols, seed=rows + cols)
    y_ref, dx_ref, dw_ref = _reference(x, w, dy, dres if residual else None)
    y, dx, dw = _hip(x, w, dy, dres if residual else None)
    assert y.shape == x.shape and dx.shape == x.shape and dw.shape == w.shape
    assert_close("y", y, y_ref, TOL)
    assert_close("dx", dx, dx_ref, TOL)
    assert_close("dweight", dw, dw_ref, TOL)


@pytest.mark.parametrize("rows,cols", [(8192, 640), (37, 132), (1, 2048)])
@pytest.mark.parametrize("use_sum", [True, False])
def test_add_then_norm_matches_float64_reference(rows, cols, use_sum):
    """add_rms_norm(x, delta) = (x + delta, its norm); both inputs get the
    sum's gradient: dy through the norm plus the sum's own gradient (absent
    when the sum is not used, as for the final norm)."""
    print(f"[case] add+rmsnorm {rows}x{cols} sum used {use_sum}", flush=True)
    x, w, dy, ds = _inputs(rows, cols, seed=7 * rows + cols)
    delta = torch.randn(rows, cols, generator=torch.Generator().manual_seed(cols))
    xd = x.double().requires_grad_(True)
    dd = delta.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    sd = xd + dd
    yd = wd * (sd * torch.rsqrt(sd.pow(2).mean(-1, keepdim=True) + EPS))
    outs, gouts = [yd], [dy.double()]
    if use_sum:
        outs.append(sd)
        gouts.append(ds.double())
    torch.autograd.backward(outs, gouts)
    xl, dl, wl = (t.to(DEV).requires_grad_(True) for t in (x, delta, w))
    s, y = add_rms_norm(xl, dl, wl, EPS)
    outs, gouts = [y], [dy.to(DEV)]
    if use_sum:
        outs.append(s)
        gouts.append(ds.to(DEV))
    gx, gd, gw = torch.autograd.grad(outs, [xl, dl, wl], gouts)
    torch.cuda.synchronize()
    assert_close("sum", s, sd.detach(), TOL)
    assert_close("y", y, yd.detach(), TOL)
    assert_close("dx", gx, xd.grad, TOL)
    assert_close("ddelta", gd, dd.grad, TOL)
    assert_close("dweight", gw, wd.grad, TOL)


def test_matches_the_framework_rms_norm():
    """The framework's fused rms_norm in fp32 on the GPU, on (B, T, C) input."""
    print("[case] rmsnorm vs framework", flush=True)
    x, w, dy, _ = _inputs(16 * 512, 640, seed=3, scale=4.0)
    x, dy = x.view(16, 512, 640), dy.view(16, 512, 640)
    xl, wl = x.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
    y_fw = F.rms_norm(xl, (640,), wl, EPS)
    dx_fw, dw_fw = torch.autograd.grad(y_fw, [xl, wl], dy.to(DEV))
    y, dx, dw = _hip(x, w, dy)
    assert y.shape == (16, 512, 640)
    assert_close("y", y, y_fw, TOL)
    assert_close("dx", dx, dx_fw, TOL)
    assert_close("dweight", dw, dw_fw, TOL)


def test_bitwise_reproducible():
    print("[case] rmsnorm determinism", flush=True)
    x, w, dy, dres = _inputs(8192, 640, seed=5)
    a = _hip(x, w, dy, dres)
    b = _hip(x, w, dy, dres)
    assert all(torch.equal(u, v) for u, v in zip(a, b))


def test_zero_rows_give_a_zero_weight_gradient():
    """Through the op: no rows, an empty y and dweight = 0."""
    w = torch.ones(640, device=DEV)
    x = torch.empty(0, 640, device=DEV)
    y, rstd = torch.ops.mamba_hip.rmsnorm_fwd(x, w, EPS)
    assert y.shape == (0, 640) and rstd.shape == (0,)
    dx, dw = torch.ops.mamba_hip.rmsnorm_bwd(x, x, w, rstd, None)
    torch.cuda.synchronize()
    assert dx.shape == (0, 640) and torch.equal(dw, torch.zeros_like(w))


def test_op_argument_errors():
    """The registered ops check on the host before any launch."""
    w = torch.ones(640, device=DEV)
    x = torch.zeros(4, 640, device=DEV)
    with pytest.raises(HipScanError, match="multiple of 4"):
        torch.ops.mamba_hip.rmsnorm_fwd(torch.zeros(4, 6, device=DEV), torch.ones(6, device=DEV),
                                        EPS)
    with pytest.raises(HipScanError, match="float32"):
        torch.ops.mamba_hip.rmsnorm_fwd(x.double(), w, EPS)
    with pytest.raises(HipScanError, match="weight"):
        torch.ops.mamba_hip.rmsnorm_fwd(x, w[:320], EPS)
    with pytest.raises(HipScanError, match="contiguous"):
        torch.ops.mamba_hip.rmsnorm_fwd(torch.zeros(640, 8, device=DEV).t(), w, EPS)
    rstd = torch.ones(4, device=DEV)
    with pytest.raises(HipScanError, match="dres"):
        torch.ops.mamba_hip.rmsnorm_bwd(x, x, w, rstd, torch.zeros(4, 320, device=DEV))
    with pytest.raises(HipScanError, match="rms_norm"):
        rms_norm(torch.zeros(4, 6, device=DEV), torch.ones(6, device=DEV), EPS)
    with pytest.raises(HipScanError, match="delta"):
        torch.ops.mamba_hip.add_rmsnorm_fwd(x, torch.zeros(4, 320, device=DEV), w, EPS)
    with pytest.raises(HipScanError, match="add_rms_norm"):
        add_rms_norm(x, torch.zeros(4, 640, device=DEV, dtype=torch.float64), w, EPS)


@pytest.mark.parametrize("fn", ["rms_norm", "rms_norm_residual", "add_rms_norm"])
def test_public_functions_check_the_weight(fn):
    """The autograd Functions (which call the ops' plain implementations) check
    the weight's length, dtype and device before any launch: a short, bf16 or
    host weight would be read past its end or through a host pointer."""
    x = torch.zeros(4, 640, device=DEV)
    call = {"rms_norm": lambda w: rms_norm(x, w, EPS),
            "rms_norm_residual": lambda w: rms_norm_residual(x, w, EPS),
            "add_rms_norm": lambda w: add_rms_norm(x, torch.zeros_like(x), w, EPS)}[fn]
    for bad, msg in ((torch.ones(320, device=DEV), "weight"),
                     (torch.ones(640, device=DEV, dtype=torch.bfloat16), "float32"),
                     (torch.ones(640), "device")):
        with pytest.raises(HipScanError, match=msg):
            call(bad)
    torch.cuda.synchronize()
    call(torch.ones(640, device=DEV))   # and a good weight still runs
    torch.cuda.synchronize()


def test_model_norms_match_the_framework_path():
    """TinyMamba's loss and every parameter gradient with the HIP norms
    against the same model with the framework's rms_norm (one block of the
    80M width, d_state 16, fp32)."""
    print("[case] rmsnorm in TinyMamba", flush=True)
    torch.manual_seed(0)
    cfg = MambaConfig(vocab_size=512, d_model=640, n_layers=2, d_state=16, scan_impl="hip")
    model = TinyMamba(cfg).to(DEV)
    idx = torch.randint(0, 512, (2, 64), device=DEV)
    grads = []
    for hip in (True, False):
        for m in model.modules():
            if hasattr(m, "uses_hip"):
                m.hip = hip
        model.zero_grad(set_to_none=True)
        _, loss = model(idx, idx)
        loss.backward()
        grads.append((loss.detach(), {n: p.grad.clone() for n, p in model.named_parameters()}))
    (l1, g1), (l2, g2) = grads
    assert_close("loss", l1, l2, 1e-5)
    for name in g1:
        assert_close(name, g1[name], g2[name], 1e-4)


def test_model_under_autocast_matches_the_per_block_path():
    """Under bf16 autocast the blocks' outputs are bf16: the folded residual
    add widens them as the per-block path's x + delta does (same loss)."""
    print("[case] rmsnorm in TinyMamba under autocast", flush=True)
    torch.manual_seed(1)
    cfg = MambaConfig(vocab_size=512, d_model=256, n_layers=2, d_state=16, scan_impl="hip")
    model = TinyMamba(cfg).to(DEV)
    idx = torch.randint(0, 512, (2, 64), device=DEV)
    losses = []
    for fused in (True, False):
        if not fused:
            model.ln_f.uses_hip = lambda x: False   # the per-block branch (framework final norm)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            _, loss = model(idx, idx)
        loss.backward()
        losses.append(float(loss.detach()))
    del model.ln_f.uses_hip
    assert abs(losses[0] - losses[1]) <= 1e-3 * abs(losses[1])
