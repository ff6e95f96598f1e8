"""TinyMamba: the small Mamba language model that drives the scan.

Same architecture, parameter names and shapes as the reference's
``mamba_metal/model.py`` (so state dicts load across the two), rebuilt in
plain torch; the selective scan is the only custom kernel:

* ``MambaConfig`` (model.py:37-55): ``scan_impl`` in {"auto", "hip", "torch"}
  ("metal" = "hip"). "auto" uses the gfx950 scan for ROCm tensors and the
  associative ``parallel_scan`` on CPU.
* ``MambaBlock`` (model.py:161-256): RMSNorm -> in_proj -> (x, z); causal
  depthwise conv + SiLU; dt = dt_min + (dt_max-dt_min)*sigmoid(dt_proj(x));
  Aneg = softplus(A); the scan; + D_skip (a per-channel bias); * silu(z);
  out_proj; residual. On a ROCm device the conv + SiLU is the fused
  ``conv1d_silu`` kernel, the dt gate and softplus(A) run inside the scan
  kernels (``selective_scan_gated``) and ``(y + D_skip) * silu(z)`` is the
  fused ``out_gate`` kernel. In fp32 without a cache, everything between
  in_proj and out_proj is one autograd Function (``mamba_inner``): the dt, B
  and C projections become one GEMM whose output the scan reads in place,
  and the backward writes its gradients in place (no concatenations or
  separate gradient sums).
* ``TinyMamba`` (model.py:259-302): embedding, blocks, final RMSNorm, head tied
  to the embedding, cross entropy.
* Recurrent cache: a prefill stores each block's conv tail and final state;
  a one-token call then advances the state. On a ROCm device without
  autograd that step is the fused ``selective_state_step`` kernel; with
  autograd enabled it is the differentiable torch update.
* d_inner is solved so that a Mamba block costs what a transformer block of
  the same d_model / d_ff costs (model.py:58-82).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from ._native import rmsnorm_supported
from .conv import conv1d_silu
from .fused import mamba_inner, out_gate, selective_scan_gated
from .norm import add_rms_norm, rms_norm, rms_norm_residual
from .scan import SSM_CHUNK, _hip_device, selective_scan, selective_state_step
from .xent import cross_entropy


@dataclass
class MambaConfig:
    vocab_size: int
    d_model: int = 384
    n_layers: int = 10
    d_ff: int = 1536          # only used to size d_inner to a transformer's budget
    max_seq_len: int = 512
    d_state: int = 16
    d_conv: int = 4
    d_inner: Optional[int] = None   # None: solve for the transformer budget
    scan_chunk: int = 0       # time-slice length of the CPU parallel_scan (0 = whole)
    scan_impl: str = "auto"   # 'auto' | 'hip' | 'torch' ('metal' = 'hip')
    dt_min: float = 0.001
    dt_max: float = 0.1
    norm_eps: float = 1e-6
    ckpt_chunk: int = SSM_CHUNK   # checkpoint stride of the HIP scan


def transformer_block_params(d_model: int, d_ff: int) -> int:
    """Parameters of one pre-norm transformer block: attention, MLP, two norms."""
    attention = 4 * d_model * d_model
    mlp = 2 * d_model * d_ff
    norms = 2 * d_model
    return attention + mlp + norms


def mamba_block_params(d_model: int, d_inner: int, d_state: int, d_conv: int) -> int:
    """Parameters of one MambaBlock, term by term as the block builds them."""
    in_proj = d_model * 2 * d_inner
    conv = d_inner * d_conv + d_inner
    dt_proj = d_inner * d_inner + d_inner
    a_b_c = 3 * d_inner * d_state
    d_skip = d_inner
    out_proj = d_inner * d_model
    norm = d_model
    return in_proj + conv + dt_proj + a_b_c + d_skip + out_proj + norm


def d_inner_for_budget(target: int, d_model: int, d_state: int, d_conv: int) -> int:
    """Largest multiple of 8 whose MambaBlock costs at most `target` parameters.

    mamba_block_params is d_inner^2 + c*d_inner + d_model with
    c = 3*d_model + d_conv + 3 + 3*d_state; solve the quadratic, round down.
    """
    c = 3 * d_model + d_conv + 3 + 3 * d_state
    root = (math.sqrt(c * c + 4 * (target - d_model)) - c) / 2.0
    return max(8, int(root // 8) * 8)


class RMSNorm(nn.Module):
    """weight * x * rsqrt(mean(x^2) + eps) over the last dim, in fp32
    (mamba_metal/model.py:85-95); same parameter name and function as the
    reference's. With `hip` set (the model's scan_impl is not 'torch') fp32
    rows on a ROCm device go through the HIP RMSNorm kernels (norm.py), else
    through the framework's fused rms_norm."""

    def __init__(self, d: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.eps = eps
        self.hip = False

    def uses_hip(self, x) -> bool:
        return self.hip and rmsnorm_supported(x)

    def forward(self, x):
        if self.uses_hip(x):
            return rms_norm(x, self.weight, self.eps)
        xf = x.float()
        return F.rms_norm(xf, (xf.shape[-1],), self.weight, self.eps).to(x.dtype)


# ------------------------------------------------------------ CPU-side scans

def scan_recurrence(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """h_t = a_t * h_{t-1} + b_t along dim 1, one step at a time."""
    h = torch.zeros_like(b[:, 0])
    hs = []
    for t in range(a.shape[1]):
        h = a[:, t] * h + b[:, t]
        hs.append(h)
    return torch.stack(hs, dim=1)


def _scan_core(a: torch.Tensor, b: torch.Tensor):
    """Inclusive associative scan of (a, b) pairs along dim 1 (Hillis-Steele).

    Returns (P, H): P[t] = prod_{j<=t} a_j, H[t] = h_t from a zero state.
    The length is padded to a power of two with the identity pair (1, 0).
    """
    t_len = a.shape[1]
    size = 1 << max(0, (t_len - 1).bit_length())
    if size != t_len:
        pad = [0, 0] * (a.dim() - 2) + [0, size - t_len]
        a = F.pad(a, pad, value=1.0)
        b = F.pad(b, pad, value=0.0)
    shift = 1
    while shift < size:
        # (a_early, b_early) then (a_late, b_late) = (a_early*a_late, a_late*b_early + b_late)
        a_late, b_late = a[:, shift:], b[:, shift:]
        a_new = torch.cat([a[:, :shift], a[:, :-shift] * a_late], dim=1)
        b_new = torch.cat([b[:, :shift], a_late * b[:, :-shift] + b_late], dim=1)
        a, b = a_new, b_new
        shift *= 2
    return a[:, :t_len], b[:, :t_len]


def parallel_scan(a: torch.Tensor, b: torch.Tensor, chunk: int = 0) -> torch.Tensor:
    """h_t = a_t * h_{t-1} + b_t for all t (time is dim 1).

    chunk > 0 scans time slices of that length and folds the carried state in
    with the slice's running product (h += P * carry), bounding the memory of
    the intermediates without changing the result.
    """
    if not chunk or a.shape[1] <= chunk:
        return _scan_core(a, b)[1]
    out = []
    carry = None
    for s in range(0, a.shape[1], chunk):
        prod, h = _scan_core(a[:, s:s + chunk], b[:, s:s + chunk])
        if carry is not None:
            h = h + prod * carry.unsqueeze(1)
        carry = h[:, -1]
        out.append(h)
    return torch.cat(out, dim=1)


# ------------------------------------------------------------------ the block

class MambaBlock(nn.Module):
    """Gated causal depthwise conv + diagonal selective SSM, with a residual."""

    def __init__(self, cfg: MambaConfig, d_inner: int):
        super().__init__()
        d_model, d_state, d_conv = cfg.d_model, cfg.d_state, cfg.d_conv
        self.d_inner = d_inner
        self.scan_chunk = cfg.scan_chunk
        self.scan_impl = cfg.scan_impl
        self.ckpt_chunk = cfg.ckpt_chunk
        self.dt_min, self.dt_max = cfg.dt_min, cfg.dt_max
        self.norm = RMSNorm(d_model, cfg.norm_eps)
        self.norm.hip = cfg.scan_impl != "torch"
        self.in_proj = nn.Linear(d_model, 2 * d_inner, bias=False)
        # Left-padded by d_conv-1 and cut to T outputs: causal.
        self.conv = nn.Conv1d(d_inner, d_inner, kernel_size=d_conv, padding=d_conv - 1,
                              groups=d_inner, bias=True)
        self.dt_proj = nn.Linear(d_inner, d_inner, bias=True)
        self.A = nn.Parameter(torch.arange(1, d_state + 1, dtype=torch.float32)
                              .repeat(d_inner, 1))
        self.B_proj = nn.Linear(d_inner, d_state, bias=False)
        self.C_proj = nn.Linear(d_inner, d_state, bias=False)
        self.D_skip = nn.Parameter(torch.ones(d_inner))
        self.out_proj = nn.Linear(d_inner, d_model, bias=False)

    def _proj(self, x):
        """(dt, B, C, Aneg) from the post-conv, post-SiLU activations x."""
        gate = torch.sigmoid(self.dt_proj(x))
        dt = self.dt_min + (self.dt_max - self.dt_min) * gate
        return dt, self.B_proj(x), self.C_proj(x), F.softplus(self.A)

    def _fused(self, t) -> bool:
        """True where the block runs its fused HIP ops: fp32 ROCm tensors and a
        scan_impl other than 'torch'."""
        return self.scan_impl != "torch" and _hip_device(t) and t.dtype == torch.float32

    def _fused_scan(self, t) -> bool:
        """The gated HIP scan also takes bf16 activations (fp32 state), e.g.
        under autocast."""
        return (self.scan_impl != "torch" and _hip_device(t)
                and t.dtype in (torch.float32, torch.bfloat16))

    def _scan(self, x, return_state=False):
        """y_t = sum_n C_tn h_tn over the selective recurrence (+ final state).

        On a ROCm device the dt gate and softplus(A) of _proj run inside the
        scan kernels (selective_scan_gated): the same function as _proj followed
        by selective_scan (mamba_metal/model.py:197-200, :213-215)."""
        if self._fused_scan(x):
            return selective_scan_gated(x, self.dt_proj(x), self.A, self.B_proj(x),
                                        self.C_proj(x), self.dt_min, self.dt_max,
                                        chunk=self.ckpt_chunk, return_state=return_state)
        dt, b_t, c_t, aneg = self._proj(x)
        r = selective_scan(x, dt, aneg, b_t, c_t, impl=self.scan_impl,
                           chunk=self.ckpt_chunk, return_state=return_state)
        if r is not None:
            return r
        a = torch.exp(-dt.unsqueeze(-1) * aneg)
        b = dt.unsqueeze(-1) * b_t.unsqueeze(2) * x.unsqueeze(-1)
        h = parallel_scan(a, b, chunk=self.scan_chunk)
        y = (h * c_t.unsqueeze(2)).sum(-1)
        return (y, h[:, -1]) if return_state else y

    def _step(self, x, cache):
        """One token (x: (B, 1, d_inner) pre-conv) against the cached window/state."""
        k = self.conv.kernel_size[0]
        window = torch.cat([cache["conv"], x.transpose(1, 2)], dim=2)   # (B, d_inner, K)
        cache["conv"] = window[:, :, 1:]
        xc = F.silu(self.conv(window)[:, :, k - 1:k]).transpose(1, 2)   # (B, 1, d_inner)
        dt, b_t, c_t, aneg = self._proj(xc)
        h = cache["h"]
        use_kernel = (self.scan_impl != "torch" and _hip_device(h)
                      and not torch.is_grad_enabled() and h.dtype == torch.float32)
        if use_kernel:
            # The cache owns its state tensor: it is advanced in place.
            h = h.contiguous()
            y = selective_state_step(h, xc[:, 0], dt[:, 0], aneg, b_t[:, 0], c_t[:, 0])
            cache["h"] = h
            return y.unsqueeze(1)
        da = torch.exp(-dt[:, 0].unsqueeze(-1) * aneg)                   # (B, D, N)
        inp = dt[:, 0].unsqueeze(-1) * b_t[:, 0].unsqueeze(1) * xc[:, 0].unsqueeze(-1)
        h = h * da + inp
        cache["h"] = h
        return (h * c_t[:, 0].unsqueeze(1)).sum(-1).unsqueeze(1)        # (B, 1, D)

    def _conv_silu(self, x):
        """silu(causal depthwise conv) of the (B, T, d_inner) x half of in_proj.

        On a ROCm device (scan_impl other than 'torch') this is the fused HIP
        kernel, reading x in place; elsewhere the framework's Conv1d on the
        transposed view, as the reference does (model.py:244)."""
        if self._fused(x):
            return conv1d_silu(x, self.conv.weight, self.conv.bias)
        xt = x.transpose(1, 2)                                           # (B, d_inner, T)
        return F.silu(self.conv(xt)[:, :, :xt.shape[2]]).transpose(1, 2)

    def _inner(self, xz) -> bool:
        """Whether the fused inner block (conv, projections, scan and output
        gate in one autograd Function) applies: the HIP path in fp32, with
        d_inner and d_state multiples of 4 and a conv of at most 8 taps."""
        return (self._fused(xz) and self.d_inner % 4 == 0 and self.A.shape[1] % 4 == 0
                and self.conv.kernel_size[0] <= 8)

    def forward(self, x, cache=None):
        if self.norm.uses_hip(x):
            # x itself, and its norm; the backward adds x's two gradients in
            # the norm's kernel.
            residual, h = rms_norm_residual(x, self.norm.weight, self.norm.eps)
        else:
            residual, h = x, self.norm(x)
        return residual + self.mix(h, cache)

    def mix(self, h, cache=None):
        """The block after its norm, without the residual add: in_proj, conv,
        scan, gate, out_proj of the normalised h (model.py:226-256)."""
        xz = self.in_proj(h)
        if cache is None and self._inner(xz):
            out = mamba_inner(xz, self.conv.weight, self.conv.bias, self.dt_proj.weight,
                              self.dt_proj.bias, self.B_proj.weight, self.C_proj.weight, self.A,
                              self.D_skip, self.dt_min, self.dt_max, chunk=self.ckpt_chunk)
            return self.out_proj(out)
        x, z = xz.chunk(2, dim=-1)
        k = self.conv.kernel_size[0]
        if cache is not None and cache.get("h") is not None and x.shape[1] == 1:
            y = self._step(x, cache)
        else:
            xt = x.transpose(1, 2)                                       # (B, d_inner, T)
            x = self._conv_silu(x)
            if cache is not None:
                tail = xt[:, :, -(k - 1):]
                if tail.shape[2] < k - 1:
                    tail = F.pad(tail, (k - 1 - tail.shape[2], 0))
                cache["conv"] = tail
            y, h_last = self._scan(x, return_state=True)
            if cache is not None:
                cache["h"] = h_last
        if self._fused(y):
            return self.out_proj(out_gate(y, self.D_skip, z))
        y = y + self.D_skip
        return self.out_proj(y * F.silu(z))


def _plain_block(b: nn.Module) -> bool:
    """Whether calling b.mix() in place of b(x) skips nothing: b is a
    MambaBlock itself (not a wrapper or a subclass) and neither it nor the
    module-global registries hold forward or backward hooks."""
    g = nn.modules.module
    return (type(b) is MambaBlock and not b._forward_hooks and not b._forward_pre_hooks
            and not b._backward_hooks and not b._backward_pre_hooks
            and not g._global_forward_hooks and not g._global_forward_pre_hooks
            and not g._global_backward_hooks and not g._global_backward_pre_hooks)


class TinyMamba(nn.Module):
    """A Mamba language model sized to a transformer's parameter budget."""

    def __init__(self, cfg: MambaConfig):
        super().__init__()
        self.cfg = cfg
        d_inner = cfg.d_inner
        if d_inner is None:
            budget = transformer_block_params(cfg.d_model, cfg.d_ff)
            d_inner = d_inner_for_budget(budget, cfg.d_model, cfg.d_state, cfg.d_conv)
        self.d_inner = d_inner
        self.tok = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.blocks = nn.ModuleList(MambaBlock(cfg, d_inner) for _ in range(cfg.n_layers))
        self.ln_f = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.ln_f.hip = cfg.scan_impl != "torch"
        self.head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False)
        self.head.weight = self.tok.weight          # tied
        self.apply(self._init)

    @staticmethod
    def _init(m):
        if isinstance(m, nn.Linear):
            nn.init.normal_(m.weight, mean=0.0, std=0.02)
            if m.bias is not None:
                nn.init.zeros_(m.bias)
        elif isinstance(m, nn.Embedding):
            nn.init.normal_(m.weight, mean=0.0, std=0.02)

    def forward(self, idx, targets=None, cache=None):
        if cache is not None and "blocks" not in cache:
            cache["blocks"] = [{} for _ in self.blocks]
        x = self.tok(idx)
        caches = cache["blocks"] if cache is not None else [None] * len(self.blocks)
        if self.ln_f.uses_hip(x) and all(_plain_block(b) and b.norm.uses_hip(x)
                                         for b in self.blocks):
            # The HIP norms: each block's residual add goes into the next norm's
            # kernel (x + delta and its norm in one pass). This calls each
            # block's mix() rather than the block itself, so it is taken only
            # for unwrapped MambaBlocks without hooks (any other block is
            # called as block(x, cache) in the loop below).
            delta = None
            for block, bc in zip(self.blocks, caches):
                if delta is None:
                    x, h = rms_norm_residual(x, block.norm.weight, block.norm.eps)
                else:
                    x, h = add_rms_norm(x, delta, block.norm.weight, block.norm.eps)
                # (under autocast out_proj yields bf16: widened exactly, as x + delta would)
                delta = block.mix(h, bc).to(x.dtype)
            h = (add_rms_norm(x, delta, self.ln_f.weight, self.ln_f.eps)[1] if delta is not None
                 else self.ln_f(x))
        else:
            for block, bc in zip(self.blocks, caches):
                x = block(x, bc)
            h = self.ln_f(x)
        logits = self.head(h)
        loss = None
        if targets is not None:
            flat, tflat = logits.reshape(-1, logits.size(-1)), targets.reshape(-1)
            if (self.cfg.scan_impl != "torch" and _hip_device(flat)
                    and flat.dtype == torch.float32):
                # The fused HIP cross-entropy: the same mean loss and gradient
                # without the (rows, vocab) log-probabilities in memory.
                loss = cross_entropy(flat, tflat, ignore_index=-100)
            else:
                loss = F.cross_entropy(flat, tflat, ignore_index=-100)
        return logits, loss

    def count_params(self) -> int:
        """Unique parameters (the tied head counts once)."""
        return sum(p.numel() for p in self.parameters())
