"""The MambaBlock's producer and consumer ops around the scan, fused on MI355X.

The reference block computes, around its selective scan
(mamba_metal/model.py:197-200 and :255-256):

    dt   = dt_min + (dt_max - dt_min) * sigmoid(dt_proj(x))     # 3 elementwise ops
    Aneg = softplus(A)
    y    = selective_scan(x, dt, Aneg, B, C)
    out  = out_proj((y + D_skip) * silu(z))                    # 3 elementwise ops

Each elementwise op is a full pass over a (batch, T, d_inner) tensor in the
forward and another one or two in the backward. Here:

* ``selective_scan_gated`` takes the raw ``dt_proj`` output and ``A``: the
  scan kernels gate dt and take softplus(A) while they stage their inputs,
  and the backward kernels return the raw inputs' gradients. dt is never
  materialised.
* ``out_gate`` computes ``(y + D_skip) * silu(z)`` in one kernel per
  direction, reading z in place from the in_proj output, with a deterministic
  reduction for D_skip's gradient.
"""
from __future__ import annotations

import torch

from . import _native
from .scan import SSM_CHUNK, _validate, _hip_device


class SelectiveScanGatedHIP(torch.autograd.Function):
    """selective_scan_gated(...) -> y (or (y, h_last)), forward and backward."""

    @staticmethod
    def forward(ctx, x, dt_raw, a_raw, b_in, c_in, dt_min, dt_max, chunk=SSM_CHUNK,
                return_state=False, dt_bias=None):
        _validate(x, dt_raw, a_raw, b_in, c_in, chunk)
        x, dt_raw, a_raw, b_in, c_in = (t.contiguous() for t in (x, dt_raw, a_raw, b_in, c_in))
        if dt_bias is not None:
            if dt_bias.shape != (x.shape[2],) or dt_bias.dtype != torch.float32:
                raise ValueError(f"dt_bias must be fp32 of shape ({x.shape[2]},); got "
                                 f"{dt_bias.dtype} {tuple(dt_bias.shape)}")
            dt_bias = dt_bias.contiguous()
        ctx.has_bias = dt_bias is not None
        ctx.set_materialize_grads(False)
        ctx.chunk = chunk
        ctx.gate = (float(dt_min), float(dt_max))
        ctx.return_state = return_state
        ctx.empty = x.numel() == 0 or a_raw.numel() == 0
        if ctx.empty:
            bt, t_len, d = x.shape
            y = x.new_zeros((bt, t_len, d))
            h_last = x.new_zeros((bt, d, a_raw.shape[1]))
            ctx.save_for_backward(x, dt_raw, a_raw, b_in, c_in, dt_bias)
        else:
            need_grad = any(ctx.needs_input_grad[:5]) or ctx.needs_input_grad[9]
            y, ckpt, h_last = _native.dispatch("scan_gated_fwd")(
                x, dt_raw, a_raw, b_in, c_in, ctx.gate[0], ctx.gate[1], chunk, need_grad, dt_bias)
            ctx.save_for_backward(x, dt_raw, a_raw, b_in, c_in, dt_bias, ckpt)
        if return_state:
            return y, h_last
        return y

    @staticmethod
    def backward(ctx, *grads):
        dy = grads[0]
        dh_last = grads[1] if ctx.return_state and len(grads) > 1 else None
        if ctx.empty:
            x, dt_raw, a_raw, b_in, c_in, dt_bias = ctx.saved_tensors
            return (torch.zeros_like(x), torch.zeros_like(dt_raw), torch.zeros_like(a_raw),
                    torch.zeros_like(b_in), torch.zeros_like(c_in), None, None, None, None,
                    torch.zeros_like(dt_bias) if ctx.has_bias else None)
        x, dt_raw, a_raw, b_in, c_in, dt_bias, ckpt = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros_like(x)
        dy = dy.contiguous()
        if dh_last is not None:
            dh_last = dh_last.contiguous()
        dx, ddt, da, db, dc, dbias = _native.dispatch("scan_gated_bwd")(
            x, dt_raw, a_raw, b_in, c_in, ctx.gate[0], ctx.gate[1], dy, dh_last, ckpt, ctx.chunk,
            dt_bias)
        return dx, ddt, da, db, dc, None, None, None, None, dbias if ctx.has_bias else None


def selective_scan_gated(x: torch.Tensor, dt_raw: torch.Tensor, a_raw: torch.Tensor,
                         b_in: torch.Tensor, c_in: torch.Tensor, dt_min: float, dt_max: float,
                         chunk: int = SSM_CHUNK, return_state: bool = False,
                         dt_bias: torch.Tensor | None = None):
    """``selective_scan(x, dt_min + (dt_max - dt_min) * sigmoid(dt_raw + dt_bias),
    softplus(a_raw), B, C)`` in the fused gfx950 kernels (the reference's
    MambaBlock._proj + _scan, mamba_metal/model.py:197-200, :213-215). dt_bias
    (optional, (d_inner,)) is the dt projection's bias, so that dt_raw may be
    the projection without it; its gradient is reduced inside the backward.
    Inputs on one ROCm device, fp32 (x, dt_raw, B, C may be bf16); needs
    dt_min < dt_max."""
    if not (float(dt_min) < float(dt_max)):
        raise ValueError(f"need dt_min < dt_max; got {dt_min}, {dt_max}")
    return SelectiveScanGatedHIP.apply(x, dt_raw, a_raw, b_in, c_in, dt_min, dt_max, chunk,
                                       return_state, dt_bias)


class OutGateHIP(torch.autograd.Function):
    """out_gate(y, d_skip, z) forward and backward on the HIP kernels."""

    @staticmethod
    def forward(ctx, y, d_skip, z):
        y = y.contiguous()
        d_skip = d_skip.contiguous()
        try:
            _native._conv_rows(z)
        except _native.HipScanError:
            z = z.contiguous()
        ctx.empty = y.numel() == 0
        ctx.save_for_backward(y, d_skip, z)
        if ctx.empty:
            return y.new_zeros(y.shape)
        return _native.dispatch("out_gate_fwd")(y, d_skip, z)

    @staticmethod
    def backward(ctx, dout):
        y, d_skip, z = ctx.saved_tensors
        if ctx.empty:
            return torch.zeros_like(y), torch.zeros_like(d_skip), torch.zeros_like(z)
        dy, dd, dz = _native.dispatch("out_gate_bwd")(y, d_skip, z, dout.contiguous())
        return dy, dd, dz


def out_gate(y: torch.Tensor, d_skip: torch.Tensor, z: torch.Tensor) -> torch.Tensor:
    """``(y + d_skip) * silu(z)`` (mamba_metal/model.py:255-256) for y, z
    (B, T, d_inner) and d_skip (d_inner), fp32 on one ROCm device; z's rows may
    be strided (the z half of the in_proj output). Returns a contiguous tensor."""
    tensors = (y, d_skip, z)
    if not all(_hip_device(t) for t in tensors):
        raise RuntimeError("out_gate needs every input on the ROCm device; saw devices "
                           + ", ".join(str(t.device) for t in tensors))
    if not all(t.dtype == torch.float32 for t in tensors):
        raise RuntimeError("out_gate is fp32-only; got " + ", ".join(str(t.dtype) for t in tensors))
    if y.dim() != 3 or z.shape != y.shape or d_skip.shape != (y.shape[2],):
        raise ValueError(f"bad shapes: y {tuple(y.shape)}, d_skip {tuple(d_skip.shape)}, "
                         f"z {tuple(z.shape)}")
    return OutGateHIP.apply(y, d_skip, z)


class MambaInnerHIP(torch.autograd.Function):
    """The inner block between in_proj and out_proj, fused (fp32):
    x, z = xz.chunk(2); xc = silu(conv(x)); [dt_raw | B | C] = xc W^T;
    y = gated scan(xc, dt_raw + b_dt, A, B, C); out = (y + D_skip) * silu(z).
    The reference computes it as separate modules (mamba_metal/model.py:
    197-200, :244-256). Fused, the three projections are one GEMM (no bias:
    the dt projection's bias is added by the scan kernels as they gate dt)
    whose output rows the scan reads in place; in the backward the scan writes
    its dt_raw, B and C gradients into one projection gradient and reduces the
    bias gradient itself, the projections' input gradient is accumulated onto
    the scan's dx by the GEMM, and the conv and output gate write dx and dz
    straight into the two halves of xz's gradient (no concatenation, no
    separate gradient sums)."""

    @staticmethod
    def forward(ctx, xz, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_raw, d_skip, dt_min, dt_max,
                chunk):
        bt, t_len, d2 = xz.shape
        d, n = d2 // 2, a_raw.shape[1]
        x, z = xz[..., :d], xz[..., d:]
        w2 = conv_w.reshape(d, -1).contiguous()
        cb = conv_b.contiguous()
        xc = _native.dispatch("conv1d_silu_fwd")(x, w2, cb)
        w_proj = torch.cat([w_dt, w_b, w_c], 0)
        bias = b_dt.contiguous()
        proj = torch.mm(xc.view(-1, d), w_proj.t()).view(bt, t_len, d + 2 * n)
        need_grad = any(ctx.needs_input_grad)
        y, ckpt, _ = _native.dispatch("scan_gated_fwd")(
            xc, proj[..., :d], a_raw, proj[..., d:d + n], proj[..., d + n:], float(dt_min),
            float(dt_max), chunk, need_grad, bias)
        out = _native.dispatch("out_gate_fwd")(y, d_skip, z)
        ctx.gate = (float(dt_min), float(dt_max))
        ctx.chunk = chunk
        ctx.conv_shape = conv_w.shape
        if need_grad:
            ctx.save_for_backward(xz, w2, cb, w_proj, bias, a_raw, d_skip, xc, proj, y, ckpt)
        return out

    @staticmethod
    def backward(ctx, dout):
        xz, w2, cb, w_proj, bias, a_raw, d_skip, xc, proj, y, ckpt = ctx.saved_tensors
        bt, t_len, d2 = xz.shape
        d, n = d2 // 2, a_raw.shape[1]
        dxz = torch.empty_like(xz)
        dy, dd = _native.dispatch("out_gate_bwd_into")(y, d_skip, xz[..., d:],
                                                       dout.contiguous(), dxz[..., d:])
        dproj = torch.empty_like(proj)
        dxc, da, db_dt = _native.dispatch("scan_gated_bwd_into")(
            xc, proj[..., :d], a_raw, proj[..., d:d + n], proj[..., d + n:], ctx.gate[0],
            ctx.gate[1], dy, None, ckpt, ctx.chunk, dproj, bias)
        dp2 = dproj.view(-1, d + 2 * n)
        dxc.view(-1, d).addmm_(dp2, w_proj)            # + the projections' input gradient
        dw = dp2.t().mm(xc.view(-1, d))
        dcw, dcb = _native.dispatch("conv1d_silu_bwd_into")(xz[..., :d], w2, cb, dxc,
                                                            dxz[..., :d])
        return (dxz, dcw.reshape(ctx.conv_shape), dcb, dw[:d], db_dt, dw[d:d + n],
                dw[d + n:], da, dd, None, None, None)


def mamba_inner(xz: torch.Tensor, conv_w: torch.Tensor, conv_b: torch.Tensor,
                w_dt: torch.Tensor, b_dt: torch.Tensor, w_b: torch.Tensor, w_c: torch.Tensor,
                a_raw: torch.Tensor, d_skip: torch.Tensor, dt_min: float, dt_max: float,
                chunk: int = SSM_CHUNK) -> torch.Tensor:
    """The fused inner block (see MambaInnerHIP): xz (B, T, 2 d_inner), conv
    weight (d_inner, 1, K) / bias (d_inner), dt_proj weight (d_inner, d_inner)
    and bias (d_inner), B_proj / C_proj weights (d_state, d_inner), A
    (d_inner, d_state), D_skip (d_inner); fp32 on one ROCm device, d_inner and
    d_state multiples of 4. Returns (B, T, d_inner), contiguous."""
    tensors = (xz, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_raw, d_skip)
    if not all(_hip_device(t) for t in tensors):
        raise RuntimeError("mamba_inner needs every input on the ROCm device")
    if not all(t.dtype == torch.float32 for t in tensors):
        raise RuntimeError("mamba_inner is fp32-only")
    if not (float(dt_min) < float(dt_max)):
        raise ValueError(f"need dt_min < dt_max; got {dt_min}, {dt_max}")
    if xz.dim() != 3 or xz.shape[2] % 2 or not xz.is_contiguous():
        raise ValueError(f"xz must be a contiguous (B, T, 2 d_inner) tensor; got {tuple(xz.shape)}")
    d, n = xz.shape[2] // 2, a_raw.shape[1]
    if (a_raw.shape != (d, n) or w_dt.shape != (d, d) or b_dt.shape != (d,)
            or w_b.shape != (n, d) or w_c.shape != (n, d) or d_skip.shape != (d,)
            or conv_w.shape[0] != d or conv_b.shape != (d,)):
        raise ValueError("mamba_inner: parameter shapes do not match d_inner "
                         f"{d}, d_state {n}")
    if d % 4 or n % 4:
        raise ValueError(f"mamba_inner needs d_inner and d_state multiples of 4; got {d}, {n}")
    return MambaInnerHIP.apply(xz, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_raw, d_skip, dt_min,
                               dt_max, chunk)
