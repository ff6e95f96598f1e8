"""The MambaBlock's causal depthwise conv1d + SiLU on MI355X.

The reference block runs ``F.silu(nn.Conv1d(d_inner, d_inner, K, padding=K-1,
groups=d_inner)(x^T)[:, :, :T])`` (mamba_metal/model.py:174-175, :244):
a transpose, a padded convolution through the framework's generic conv
kernels, a slice and an elementwise SiLU. ``conv1d_silu`` computes the same
function in one HIP kernel per direction, reading the (B, T, d_inner) x in
place (its rows may be strided, like the x half of the block's in_proj
output) and writing a contiguous (B, T, d_inner) result.
"""
from __future__ import annotations

import torch

from . import _native


def _hip(t: torch.Tensor) -> bool:
    return t.is_cuda and torch.version.hip is not None


class ConvSiluHIP(torch.autograd.Function):
    """conv1d_silu(x, weight, bias) forward and backward on the HIP kernels."""

    @staticmethod
    def forward(ctx, x, weight, bias):
        w = weight.reshape(weight.shape[0], -1).contiguous()
        b = bias.contiguous()
        ctx.wshape = weight.shape
        ctx.empty = x.numel() == 0
        if ctx.empty:
            ctx.save_for_backward(x, w, b)
            return x.new_zeros(x.shape)
        try:
            _native._conv_rows(x)
        except _native.HipScanError:
            x = x.contiguous()
        out = _native.dispatch("conv1d_silu_fwd")(x, w, b)
        ctx.save_for_backward(x, w, b)
        return out

    @staticmethod
    def backward(ctx, dout):
        x, w, b = ctx.saved_tensors
        if ctx.empty:
            return x.new_zeros(x.shape), w.new_zeros(ctx.wshape), torch.zeros_like(b)
        dx, dw, db = _native.dispatch("conv1d_silu_bwd")(x, w, b, dout.contiguous())
        return dx, dw.reshape(ctx.wshape), db


def conv1d_silu(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """silu(causal depthwise conv1d(x)) for x (B, T, d_inner), weight
    (d_inner, 1, K) or (d_inner, K), bias (d_inner); fp32 tensors on one ROCm
    device. Returns a contiguous (B, T, d_inner) tensor."""
    tensors = (x, weight, bias)
    if not all(_hip(t) for t in tensors):
        raise RuntimeError("conv1d_silu needs every input on the ROCm device; saw devices "
                           + ", ".join(str(t.device) for t in tensors))
    if not all(t.dtype == torch.float32 for t in tensors):
        raise RuntimeError("conv1d_silu is fp32-only; got "
                           + ", ".join(str(t.dtype) for t in tensors))
    if x.dim() != 3 or weight.shape[0] != x.shape[2] or bias.shape != (x.shape[2],):
        raise ValueError(f"bad shapes: x {tuple(x.shape)}, weight {tuple(weight.shape)}, "
                         f"bias {tuple(bias.shape)}")
    if weight.numel() // weight.shape[0] > 8:
        raise ValueError(f"conv kernel size {weight.numel() // weight.shape[0]} unsupported (1..8)")
    return ConvSiluHIP.apply(x, weight, bias)
