"""Fused cross-entropy of TinyMamba's head on MI355X.

The reference computes ``F.cross_entropy(logits.reshape(-1, V),
targets.reshape(-1))`` (mamba_metal/model.py:296-297): the framework's
log_softmax writes the (rows, V) log-probabilities and keeps them for its
backward, nll_loss picks the targets' entries, and the backward passes over
the (rows, V) tensors three more times. At the 80M model's batch (8192 rows x
32768 words, 1.07 GB of logits) that is about 1.35 ms of a 35.6 ms train step.
``cross_entropy`` computes the same mean loss and gradient with one HIP kernel
per direction: the forward reads the logits once and keeps the per-row
log-sum-exp (4 bytes a row), the backward reads them once more and writes
``scale * (softmax - onehot)``. The upstream gradient and the count of rows
not ignored stay on the device (no host synchronisation).
"""
from __future__ import annotations

import torch

from . import _native


class CrossEntropyHIP(torch.autograd.Function):
    """Mean cross-entropy of logits (R, V) fp32 against targets (R) int64 on
    the HIP kernels, rows with target == ignore_index excluded."""

    @staticmethod
    def forward(ctx, logits, targets, ignore_index):
        logits = logits.contiguous()
        targets = targets.contiguous()
        lse, loss_rows = _native.dispatch("xent_fwd")(logits, targets, ignore_index)
        n_valid = (targets != ignore_index).sum()
        ctx.save_for_backward(logits, targets, lse, n_valid)
        ctx.ignore_index = ignore_index
        # 0 / 0 = NaN when every row is ignored, as the framework's mean.
        return loss_rows.sum() / n_valid

    @staticmethod
    def backward(ctx, g):
        logits, targets, lse, n_valid = ctx.saved_tensors
        scale = (g.to(torch.float32) / n_valid).reshape(1)
        dlogits = _native.dispatch("xent_bwd")(logits, targets, lse, scale, ctx.ignore_index)
        return dlogits, None, None


def cross_entropy(logits: torch.Tensor, targets: torch.Tensor,
                  ignore_index: int = -100) -> torch.Tensor:
    """``F.cross_entropy(logits, targets, ignore_index=ignore_index)`` (mean
    reduction) for fp32 logits (R, V) and int64 targets (R) on one ROCm
    device, on the fused HIP kernels."""
    if not (logits.is_cuda and targets.is_cuda and torch.version.hip is not None):
        raise RuntimeError("cross_entropy needs logits and targets on the ROCm device; got "
                           f"{logits.device}, {targets.device}")
    if logits.dtype != torch.float32:
        raise RuntimeError(f"cross_entropy is fp32-only; got {logits.dtype}")
    if logits.dim() != 2 or targets.shape != (logits.shape[0],):
        raise ValueError(f"logits must be (R, V) and targets (R,); got {tuple(logits.shape)}, "
                         f"{tuple(targets.shape)}")
    return CrossEntropyHIP.apply(logits, targets.to(torch.int64), int(ignore_index))
