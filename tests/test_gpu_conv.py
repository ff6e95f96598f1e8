"""GPU parity of the fused causal depthwise conv1d + SiLU kernels
(mamba_metal/model.py:174-175, :244) with the float64 oracle and with the
framework's own Conv1d + SiLU in fp32 (the reference's implementation).

Bar: per tensor, max|got - ref| / max|ref| <= 1e-4 against the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import assert_close
from mamba_metal_scan_amd import conv1d_silu
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(bt, t_len, d, k, seed, row_stride=None):
    g = torch.Generator().manual_seed(seed)
    rs = row_stride or d
    base = torch.randn(bt, t_len, rs, generator=g)
    w = 0.5 * torch.randn(d, 1, k, generator=g)
    bias = 0.1 * torch.randn(d, generator=g)
    dout = torch.randn(bt, t_len, d, generator=g)
    return base, w, bias, dout


@pytest.mark.parametrize("bt,t_len,d,k", [(2, 64, 96, 4), (1, 5, 33, 4), (2, 3, 70, 4),
                                          (3, 100, 130, 1), (1, 77, 64, 2), (2, 50, 65, 8),
                                          (1, 129, 200, 3), (16, 512, 1432, 4)])
@pytest.mark.parametrize("strided", [False, True])
def test_conv_matches_the_oracle(bt, t_len, d, k, strided):
    print(f"[case] conv {bt}x{t_len}x{d} K={k} strided={strided}", flush=True)
    base, w, bias, dout = _inputs(bt, t_len, d, k, seed=d + k, row_stride=2 * d if strided else d)
    x = base[..., :d]                       # rows 2d floats apart when strided
    xd = base.to(DEV)[..., :d].requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    bd = bias.to(DEV).requires_grad_(True)
    out = conv1d_silu(xd, wd, bd)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    out_ref = oracle.conv_fwd(x.numpy(), w[:, 0].numpy(), bias.numpy())
    gx, gw, gb = oracle.conv_bwd(x.numpy(), w[:, 0].numpy(), bias.numpy(), dout.numpy())
    assert out.is_contiguous()
    assert_close("out", out, out_ref)
    assert_close("dx", xd.grad, gx)
    assert_close("dw", wd.grad[:, 0], gw)
    assert_close("dbias", bd.grad, gb)


def test_conv_matches_torch_conv1d():
    """The same function as the framework's Conv1d(padding=K-1, groups=D) + SiLU."""
    bt, t_len, d, k = 4, 200, 256, 4
    base, w, bias, dout = _inputs(bt, t_len, d, k, seed=3)
    conv = torch.nn.Conv1d(d, d, k, padding=k - 1, groups=d, bias=True).to(DEV)
    with torch.no_grad():
        conv.weight.copy_(w)
        conv.bias.copy_(bias)
    x1 = base.to(DEV).requires_grad_(True)
    ref = F.silu(conv(x1.transpose(1, 2))[:, :, :t_len]).transpose(1, 2)
    ref.backward(dout.to(DEV))
    x2 = base.to(DEV).requires_grad_(True)
    w2 = conv.weight.detach().clone().requires_grad_(True)
    b2 = conv.bias.detach().clone().requires_grad_(True)
    out = conv1d_silu(x2, w2, b2)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    assert torch.allclose(out, ref, atol=1e-5, rtol=1e-4)
    assert_close("dx", x2.grad, x1.grad)
    assert_close("dw", w2.grad, conv.weight.grad)
    assert_close("dbias", b2.grad, conv.bias.grad)


def test_conv_backward_is_bitwise_deterministic():
    base, w, bias, dout = _inputs(8, 300, 500, 4, seed=9)
    grads = []
    for _ in range(2):
        xd = base.to(DEV).requires_grad_(True)
        wd = w.to(DEV).requires_grad_(True)
        bd = bias.to(DEV).requires_grad_(True)
        conv1d_silu(xd, wd, bd).backward(dout.to(DEV))
        grads.append((xd.grad, wd.grad, bd.grad))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_conv_rejects_bad_arguments():
    x = torch.randn(2, 8, 16, device=DEV)
    with pytest.raises(ValueError):
        conv1d_silu(x, torch.randn(16, 1, 9, device=DEV), torch.randn(16, device=DEV))
    with pytest.raises(RuntimeError, match="ROCm"):
        conv1d_silu(x.cpu(), torch.randn(16, 1, 4), torch.randn(16))
