"""Host-side argument checks of the registered ops (torch.ops.mamba_hip.*):
each mismatch with what the kernels assume raises HipScanError before any
launch -- the checkpoint buffer of another stride, fp16 or mixed dtypes,
non-contiguous operands, wrong shapes, tensors on two devices. The calls
never reach the device, so these cases are safe on the GPU; the device check
alone also runs on CPU hosts.
"""
from __future__ import annotations

import pytest
import torch

from mamba_metal_scan_amd._native import HipScanError

OPS = torch.ops.mamba_hip
BT, T, D, N = 2, 40, 64, 16


def _args(dev, dtype=torch.float32):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(BT, T, D, generator=g).to(dev, dtype)
    dt = (0.01 + 0.05 * torch.rand(BT, T, D, generator=g)).to(dev, dtype)
    aneg = torch.arange(1, N + 1, dtype=torch.float32).repeat(D, 1).to(dev)
    b_in = torch.randn(BT, T, N, generator=g).to(dev, dtype)
    c_in = torch.randn(BT, T, N, generator=g).to(dev, dtype)
    return x, dt, aneg, b_in, c_in


def test_cpu_tensors_are_rejected_before_any_call():
    x, dt, aneg, b_in, c_in = _args("cpu")
    with pytest.raises(HipScanError, match="ROCm device"):
        OPS.scan_fwd(x, dt, aneg, b_in, c_in, 16, True)
    with pytest.raises(HipScanError, match="ROCm device"):
        OPS.scan_step(torch.zeros(BT, D, N), x[:, 0], dt[:, 0], aneg, b_in[:, 0], c_in[:, 0])


@pytest.mark.gpu
def test_forward_argument_mismatches_raise():
    x, dt, aneg, b_in, c_in = _args("cuda")
    cases = [
        ("float32 or all bfloat16", (x.half(), dt.half(), aneg, b_in.half(), c_in.half())),
        ("float32 or all bfloat16", (x, dt.bfloat16(), aneg, b_in, c_in)),
        ("Aneg must be float32", (x, dt, aneg.double(), b_in, c_in)),
        ("x must be contiguous", (x.transpose(1, 2).contiguous().transpose(1, 2), dt, aneg,
                                  b_in, c_in)),
        ("dt must have shape", (x, dt[:, :-1], aneg, b_in, c_in)),
        ("B must have shape", (x, dt, aneg, b_in[..., :8], c_in)),
        ("Aneg must have shape", (x, dt, aneg[:-1], b_in, c_in)),
        ("one ROCm device", (x, dt, aneg.cpu(), b_in, c_in)),
    ]
    for match, args in cases:
        with pytest.raises(HipScanError, match=match):
            OPS.scan_fwd(*args, 16, True)
    with pytest.raises(HipScanError, match="chunk"):
        OPS.scan_fwd(x, dt, aneg, b_in, c_in, 0, True)


@pytest.mark.gpu
def test_backward_argument_mismatches_raise():
    x, dt, aneg, b_in, c_in = _args("cuda")
    _, ckpt, _ = OPS.scan_fwd(x, dt, aneg, b_in, c_in, 16, True)
    dy = torch.randn_like(x)
    # checkpoints of stride 16 passed with chunk 8: the kernel would read
    # past the buffer
    with pytest.raises(HipScanError, match="ckpt"):
        OPS.scan_bwd(x, dt, aneg, b_in, c_in, dy, None, ckpt, 8)
    with pytest.raises(HipScanError, match="dh_last"):
        OPS.scan_bwd(x, dt, aneg, b_in, c_in, dy, torch.zeros(BT, D, N - 1, device="cuda"),
                     ckpt, 16)
    with pytest.raises(HipScanError, match="dy must be contiguous"):
        OPS.scan_bwd(x, dt, aneg, b_in, c_in, dy.transpose(0, 1).contiguous().transpose(0, 1),
                     None, ckpt, 16)
    with pytest.raises(HipScanError, match="dy must have x's dtype"):
        OPS.scan_bwd(x, dt, aneg, b_in, c_in, dy.bfloat16(), None, ckpt, 16)
    with pytest.raises(HipScanError, match="ckpt"):
        OPS.scan_bwd(x, dt, aneg, b_in, c_in, dy, None, ckpt.double(), 16)


@pytest.mark.gpu
def test_step_conv_and_gate_argument_mismatches_raise():
    x, dt, aneg, b_in, c_in = _args("cuda")
    h = torch.zeros(BT, D, N, device="cuda")
    with pytest.raises(HipScanError, match="h must be contiguous"):
        OPS.scan_step(h.transpose(0, 1).contiguous().transpose(0, 1), x[:, 0], dt[:, 0], aneg,
                      b_in[:, 0], c_in[:, 0])
    with pytest.raises(HipScanError, match="B must have shape"):
        OPS.scan_step(h, x[:, 0], dt[:, 0], aneg, b_in[:, 0, :8], c_in[:, 0])
    w, cb = torch.randn(D, 4, device="cuda"), torch.zeros(D, device="cuda")
    with pytest.raises(HipScanError, match="w must be contiguous"):
        OPS.conv1d_silu_fwd(x, w.t().contiguous().t(), cb)
    with pytest.raises(HipScanError, match="float32"):
        OPS.conv1d_silu_fwd(x.bfloat16(), w, cb)
    with pytest.raises(HipScanError, match="d_skip must have shape"):
        OPS.out_gate_fwd(x, torch.zeros(D + 1, device="cuda"), x)
