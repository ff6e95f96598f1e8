"""RMSNorm of the residual stream on the HIP kernels.

The reference's RMSNorm (mamba_metal/model.py:85-95) computes
``weight * x * rsqrt(mean(x^2) + eps)`` in fp32 before every block's in_proj
(model.py:225) and before the head (model.py:293). ``rms_norm`` runs it as one
HIP kernel forward and one backward pass (plus a small fixed-order sum of the
weight gradient's per-block partials). ``rms_norm_residual`` also returns the
block's residual stream: its backward then receives both gradients of x, the
normalised path's and the residual's, and adds them in the same pass, where
the framework would add them with a kernel of its own. ``add_rms_norm``
also folds in the residual add before the norm (the block's
``residual + out_proj(...)``, model.py:256).
"""
from __future__ import annotations

import torch

from . import _native
from ._native import HipScanError, dispatch, rmsnorm_supported


class RMSNormHIP(torch.autograd.Function):
    """y = weight * x * rsqrt(mean(x^2) + eps) over the last dimension; with
    `residual`, (x, y), the first an alias of x whose gradient is added into
    x's in the backward kernel."""

    @staticmethod
    def forward(ctx, x, weight, eps, residual):
        if not rmsnorm_supported(x):
            raise HipScanError(
                f"rms_norm: x must be float32 on a ROCm device with a last dimension that "
                f"is a multiple of 4 in [4, {_native.NORM_MAX_COLS}]; got {x.dtype}, "
                f"{x.device}, {tuple(x.shape)}")
        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).contiguous()
        w = weight.contiguous()
        # In eager mode dispatch() calls the op's plain implementation, which
        # skips the op's own checks: weight's device, dtype, shape and
        # alignment are checked here, before any launch (under torch.compile
        # the registered op checks them itself).
        if not torch.compiler.is_compiling():
            _native._check_norm("rms_norm", x2, w)
        y, rstd = dispatch("rmsnorm_fwd")(x2, w, float(eps))
        ctx.save_for_backward(x2, w, rstd)
        ctx.shape = shape
        ctx.residual = residual
        ctx.set_materialize_grads(False)   # an unused residual adds nothing
        y = y.view(shape)
        return (x, y) if residual else y

    @staticmethod
    def backward(ctx, *grads):
        x2, w, rstd = ctx.saved_tensors
        cols = x2.shape[1]
        g_res, g_y = grads if ctx.residual else (None, grads[0])
        dy = g_y.reshape(-1, cols).contiguous() if g_y is not None else torch.zeros_like(x2)
        dres = g_res.reshape(-1, cols).contiguous() if g_res is not None else None
        dx, dw = dispatch("rmsnorm_bwd")(dy, x2, w, rstd, dres)
        return dx.view(ctx.shape), dw, None, None


class AddRMSNormHIP(torch.autograd.Function):
    """(x + delta, rms_norm(x + delta)) in one pass: the residual stream's
    update by a block and the next norm. Both inputs receive the gradient of
    the sum, formed in the norm's backward kernel from the gradients of both
    outputs."""

    @staticmethod
    def forward(ctx, x, delta, weight, eps):
        if not rmsnorm_supported(x) or delta.shape != x.shape or delta.dtype != x.dtype:
            raise HipScanError(
                f"add_rms_norm: x and delta must be float32 on a ROCm device, of one shape "
                f"whose last dimension is a multiple of 4 in [4, {_native.NORM_MAX_COLS}]; got "
                f"{x.dtype}, {delta.dtype}, {x.device}, {tuple(x.shape)}, {tuple(delta.shape)}")
        shape = x.shape
        cols = shape[-1]
        w = weight.contiguous()
        x2 = x.reshape(-1, cols).contiguous()
        d2 = delta.reshape(-1, cols).contiguous()
        if not torch.compiler.is_compiling():   # as in RMSNormHIP.forward
            _native._check_norm("add_rms_norm", x2, w, delta=d2)
        x_out, y, rstd = dispatch("add_rmsnorm_fwd")(x2, d2, w, float(eps))
        ctx.save_for_backward(x_out, w, rstd)
        ctx.shape = shape
        ctx.set_materialize_grads(False)   # an unused x_out adds nothing
        return x_out.view(shape), y.view(shape)

    @staticmethod
    def backward(ctx, g_x, g_y):
        x_out, w, rstd = ctx.saved_tensors
        cols = x_out.shape[1]
        dy = (g_y.reshape(-1, cols).contiguous() if g_y is not None
              else torch.zeros_like(x_out))
        dres = g_x.reshape(-1, cols).contiguous() if g_x is not None else None
        dx, dw = dispatch("rmsnorm_bwd")(dy, x_out, w, rstd, dres)
        dx = dx.view(ctx.shape)
        return dx, dx, dw, None


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """The reference's RMSNorm on the HIP kernels (fp32, ROCm, last dimension
    a multiple of 4 up to 2048)."""
    return RMSNormHIP.apply(x, weight, eps, False)


def rms_norm_residual(x: torch.Tensor, weight: torch.Tensor, eps: float
                      ) -> tuple[torch.Tensor, torch.Tensor]:
    """(residual, rms_norm(x)): the residual is x itself (an alias); the
    gradients reaching both are added in the norm's backward kernel."""
    return RMSNormHIP.apply(x, weight, eps, True)


def add_rms_norm(x: torch.Tensor, delta: torch.Tensor, weight: torch.Tensor, eps: float
                 ) -> tuple[torch.Tensor, torch.Tensor]:
    """(x + delta, rms_norm(x + delta)) in one HIP pass; the gradients reaching
    both outputs are added in the norm's backward kernel, and x and delta
    both receive the sum's gradient."""
    return AddRMSNormHIP.apply(x, delta, weight, eps)
