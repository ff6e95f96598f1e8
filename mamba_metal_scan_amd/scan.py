"""The selective scan on MI355X: public API, autograd, and the torch reference.

    dA[t,d,n] = exp(-dt[t,d] * Aneg[d,n])
    h[t,d,n]  = dA[t,d,n] * h[t-1,d,n] + dt[t,d] * B[t,n] * x[t,d]      h[-1] = 0
    y[t,d]    = sum_n C[t,n] * h[t,d,n]

x, dt, y: (batch, T, d_inner); B, C: (batch, T, d_state); Aneg: (d_inner,
d_state), positive (e.g. softplus(A)).

API mirror of the reference's ``mamba_metal/scan.py``:

* ``selective_scan(x, dt, Aneg, B, C, impl=..., chunk=..., return_state=...)``
  dispatches like the reference (scan.py:424-447): ``impl="torch"`` runs the
  pure-torch reference anywhere; ``"hip"`` runs the gfx950 kernels and raises
  unless the tensors are on a ROCm device; ``"auto"`` runs the kernels for
  ROCm tensors and returns ``None`` otherwise, so the caller can use its own
  CPU path. ``"metal"`` is accepted as a spelling of ``"hip"`` so that code
  written against the reference keeps working.
* ``SelectiveScanHIP`` is the autograd Function (the reference's
  ``SelectiveScanMetal``, scan.py:338-411); ``selective_scan_hip`` wraps it
  (``selective_scan_metal`` is an alias).
* ``selective_scan_ref`` is the differentiable T-loop (scan.py:313-333).

Differences from the reference, by design:

* ``return_state=True`` returns h at the last step as its own tensor (never a
  view into the checkpoints) and it is differentiable: a gradient flowing into
  it reaches x, dt, Aneg, B and C. The reference returns a detached view and
  drops that gradient (scan.py:381-393).
* ``chunk`` (the checkpoint stride) defaults to ``SSM_CHUNK = 16``, the
  backward kernel's register window on gfx950; any ``chunk >= 1`` gives the
  same results.
* d_state is any value in 1..64 (the reference needs a multiple of 4).
* dB, dC and dAneg are reduced in a fixed order (bit-for-bit reproducible)
  where the grid fills the GPU, and with fp32 atomics (reproducible to
  rounding) where the backward runs in time segments; ``_native.set_reduction``
  overrides the choice and torch's deterministic mode forces the fixed order.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native

SSM_CHUNK = 16          # checkpoint stride: h is stored every SSM_CHUNK steps
_IMPLS = ("auto", "hip", "metal", "torch")


# ------------------------------------------------------- reference (pure torch)

def selective_scan_ref(x: torch.Tensor, dt: torch.Tensor, aneg: torch.Tensor,
                       b_in: torch.Tensor, c_in: torch.Tensor,
                       return_state: bool = False):
    """The recurrence as a left-to-right loop over T in plain torch ops.

    Differentiable, any device, dtype and d_state (mamba_metal/scan.py:313-333).
    This is the ``impl="torch"`` path: autograd keeps about three
    (batch, d_inner, d_state) tensors per step, so its memory grows with T.
    """
    bt, t_len, d = x.shape
    n = aneg.shape[1]
    decay_rate = aneg.unsqueeze(0)                       # (1, D, N)
    h = x.new_zeros((bt, d, n))
    ys = []
    for t in range(t_len):
        dt_t = dt[:, t, :].unsqueeze(-1)                 # (B, D, 1)
        da = torch.exp(-dt_t * decay_rate)               # (B, D, N)
        inp = dt_t * b_in[:, t, :].unsqueeze(1) * x[:, t, :].unsqueeze(-1)
        h = da * h + inp
        ys.append(torch.sum(c_in[:, t, :].unsqueeze(1) * h, dim=-1))
    y = torch.stack(ys, dim=1) if ys else x.new_zeros((bt, 0, d))
    if return_state:
        return y, h
    return y


# ------------------------------------------------------------ the HIP kernels

def _hip_device(t: torch.Tensor) -> bool:
    return t.is_cuda and torch.version.hip is not None


def _validate(x, dt, aneg, b_in, c_in, chunk) -> None:
    """Argument checks in the reference's order and exception types
    (mamba_metal/scan.py:344-365, :274-276)."""
    tensors = (x, dt, aneg, b_in, c_in)
    if not all(_hip_device(t) for t in tensors):
        raise RuntimeError("scan_impl='hip' needs every input on the ROCm device; saw devices "
                           + ", ".join(str(t.device) for t in tensors))
    if len({t.device for t in tensors}) != 1:
        raise RuntimeError("scan_impl='hip' needs every input on the same device; saw "
                           + ", ".join(str(t.device) for t in tensors))
    acts = (x, dt, b_in, c_in)
    if aneg.dtype != torch.float32 or not (all(t.dtype == torch.float32 for t in acts)
                                           or all(t.dtype == torch.bfloat16 for t in acts)):
        raise RuntimeError("scan_impl='hip' takes fp32 tensors, or bf16 x, dt, B, C with an "
                           "fp32 Aneg (fp32 state and arithmetic either way); got "
                           + ", ".join(str(t.dtype) for t in tensors))
    if x.dim() != 3 or dt.shape != x.shape or aneg.dim() != 2:
        raise ValueError(f"bad shapes: x {tuple(x.shape)}, dt {tuple(dt.shape)}, "
                         f"Aneg {tuple(aneg.shape)}")
    bt, t_len, d = x.shape
    n = aneg.shape[1]
    if aneg.shape[0] != d:
        raise ValueError(f"Aneg {tuple(aneg.shape)} does not match x's channel count {d}")
    if b_in.shape != (bt, t_len, n) or c_in.shape != (bt, t_len, n):
        raise ValueError(f"B {tuple(b_in.shape)} / C {tuple(c_in.shape)} must be "
                         f"({bt}, {t_len}, {n})")
    if not isinstance(chunk, int) or chunk < 1:
        raise ValueError(f"chunk (the checkpoint stride) must be a positive int; got {chunk!r}")
    if n > 0 and _native.preferred_chunk(n) == 0:
        raise ValueError(f"d_state {n} is not supported by the HIP scan (supported: 1..64; "
                         f"scan_impl='torch' takes any size)")


class SelectiveScanHIP(torch.autograd.Function):
    """selective_scan_hip(x, dt, Aneg, B, C) -> y (or (y, h_last)), fwd and bwd."""

    @staticmethod
    def forward(ctx, x, dt, aneg, b_in, c_in, chunk=SSM_CHUNK, return_state=False):
        _validate(x, dt, aneg, b_in, c_in, chunk)
        x, dt, aneg, b_in, c_in = (t.contiguous() for t in (x, dt, aneg, b_in, c_in))
        ctx.set_materialize_grads(False)
        ctx.chunk = chunk
        ctx.return_state = return_state
        ctx.empty = x.numel() == 0 or aneg.numel() == 0
        if ctx.empty:
            bt, t_len, d = x.shape
            y = x.new_zeros((bt, t_len, d))
            h_last = x.new_zeros((bt, d, aneg.shape[1]))
            ctx.save_for_backward(x, dt, aneg, b_in, c_in)
        else:
            need_grad = any(ctx.needs_input_grad[:5])
            y, ckpt, h_last = _native.dispatch("scan_fwd")(x, dt, aneg, b_in, c_in, chunk,
                                                           need_grad)
            ctx.save_for_backward(x, dt, aneg, b_in, c_in, ckpt)
        if return_state:
            return y, h_last
        return y

    @staticmethod
    def backward(ctx, *grads):
        dy = grads[0]
        dh_last = grads[1] if ctx.return_state and len(grads) > 1 else None
        if ctx.empty:
            x, dt, aneg, b_in, c_in = ctx.saved_tensors
            return (torch.zeros_like(x), torch.zeros_like(dt), torch.zeros_like(aneg),
                    torch.zeros_like(b_in), torch.zeros_like(c_in), None, None)
        x, dt, aneg, b_in, c_in, ckpt = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros_like(x)
        dy = dy.contiguous()
        if dh_last is not None:
            dh_last = dh_last.contiguous()
        dx, ddt, daneg, db, dc = _native.dispatch("scan_bwd")(
            x, dt, aneg, b_in, c_in, dy, dh_last, ckpt, ctx.chunk)
        return dx, ddt, daneg, db, dc, None, None


def selective_scan_hip(x: torch.Tensor, dt: torch.Tensor, aneg: torch.Tensor,
                       b_in: torch.Tensor, c_in: torch.Tensor,
                       chunk: int = SSM_CHUNK, return_state: bool = False):
    """The fused gfx950 scan (fwd + bwd kernels); inputs on one ROCm device."""
    return SelectiveScanHIP.apply(x, dt, aneg, b_in, c_in, chunk, return_state)


def selective_scan_metal(x: torch.Tensor, dt: torch.Tensor, aneg: torch.Tensor,
                         b_in: torch.Tensor, c_in: torch.Tensor,
                         chunk: int = SSM_CHUNK, dblock: Optional[int] = None,
                         return_state: bool = False):
    """Drop-in spelling of the reference's selective_scan_metal (scan.py:414-421).

    ``dblock`` (channels per Metal threadgroup there) is accepted for call
    compatibility and ignored: the gfx950 launch shape is chosen by the library.
    """
    del dblock
    return SelectiveScanHIP.apply(x, dt, aneg, b_in, c_in, chunk, return_state)


def selective_scan(x: torch.Tensor, dt: torch.Tensor, aneg: torch.Tensor,
                   b_in: torch.Tensor, c_in: torch.Tensor,
                   impl: str = "auto",
                   chunk: int = SSM_CHUNK,
                   return_state: bool = False):
    """Dispatch the scan on ``impl`` (mamba_metal/scan.py:424-447).

      'hip'    the fused kernels; raises unless the tensors are on a ROCm device
               ('metal' means the same thing).
      'torch'  selective_scan_ref, the pure-PyTorch reference, anywhere.
      'auto'   the kernels for ROCm tensors, otherwise None so the caller can
               use its own CPU path. 'auto' never silently changes the math.
    """
    if impl == "torch":
        return selective_scan_ref(x, dt, aneg, b_in, c_in, return_state=return_state)
    if impl not in _IMPLS:
        raise ValueError(f"unknown scan_impl {impl!r}; want 'auto', 'hip' or 'torch'")
    if _hip_device(x):
        return selective_scan_hip(x, dt, aneg, b_in, c_in, chunk=chunk,
                                  return_state=return_state)
    if impl in ("hip", "metal"):
        raise RuntimeError(f"scan_impl={impl!r} needs ROCm device tensors; got device "
                           f"{x.device.type!r}")
    return None


# ------------------------------------------------------------ decode step

def selective_state_step(h: torch.Tensor, x: torch.Tensor, dt: torch.Tensor,
                         aneg: torch.Tensor, b_in: torch.Tensor, c_in: torch.Tensor
                         ) -> torch.Tensor:
    """One recurrent step on the ROCm device, in place on h; returns y.

    h: (batch, d_inner, d_state); x, dt: (batch, d_inner); B, C: (batch, d_state).
    The same update as the reference's recurrent step (mamba_metal/model.py:234-241)
    in one kernel. Not differentiable (it mutates h); for inference.
    """
    tensors = (h, x, dt, aneg, b_in, c_in)
    if not all(_hip_device(t) for t in tensors):
        raise RuntimeError("selective_state_step needs every input on the ROCm device")
    if not all(t.dtype == torch.float32 for t in tensors):
        raise RuntimeError("selective_state_step is fp32-only")
    bt, d, n = h.shape
    if (x.shape != (bt, d) or dt.shape != (bt, d) or aneg.shape != (d, n)
            or b_in.shape != (bt, n) or c_in.shape != (bt, n)):
        raise ValueError(f"bad shapes: h {tuple(h.shape)}, x {tuple(x.shape)}, dt "
                         f"{tuple(dt.shape)}, Aneg {tuple(aneg.shape)}, B {tuple(b_in.shape)}, "
                         f"C {tuple(c_in.shape)}")
    if not h.is_contiguous():
        raise ValueError("selective_state_step updates h in place; h must be contiguous")
    return _native.dispatch("scan_step")(h, x.contiguous(), dt.contiguous(),
                                         aneg.contiguous(), b_in.contiguous(),
                                         c_in.contiguous())
