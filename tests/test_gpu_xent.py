"""GPU parity of the fused cross-entropy of the TinyMamba head
(F.cross_entropy over the tied head's logits, mamba_metal/model.py:296-297)
with the framework's cross-entropy in float64 on the CPU and in fp32 on the
GPU (the reference's own implementation).

Bar: loss and logits gradient, max|got - ref| / max|ref| <= 1e-5 against the
float64 reference (fp32 rounding of a 32768-term sum is about 1e-7 relative).
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from mamba_metal_scan_amd import cross_entropy
from mamba_metal_scan_amd._native import HipScanError

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(rows, vocab, seed, scale=3.0, ignore_frac=0.1):
    g = torch.Generator().manual_seed(seed)
    logits = scale * torch.randn(rows, vocab, generator=g)
    targets = torch.randint(0, vocab, (rows,), generator=g)
    ignored = torch.rand(rows, generator=g) < ignore_frac
    targets[ignored] = -100
    return logits, targets


def _rel(got, ref):
    got, ref = got.detach().double().cpu(), ref.detach().double().cpu()
    return float((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


def _reference(logits, targets, upstream):
    x = logits.double().requires_grad_(True)
    loss = F.cross_entropy(x, targets, ignore_index=-100)
    (loss * upstream).backward()
    return loss.detach(), x.grad


def _hip(logits, targets, upstream, storage=None):
    x = (storage if storage is not None else logits.to(DEV)).requires_grad_(True)
    loss = cross_entropy(x, targets.to(DEV), ignore_index=-100)
    (loss * upstream).backward()
    torch.cuda.synchronize()
    return loss.detach(), x.grad


@pytest.mark.parametrize("rows,vocab,upstream", [(64, 32768, 1.0), (37, 1001, 2.5), (8, 4, 1.0),
                                                 (130, 50257, 0.25), (1, 32768, -1.5)])
def test_matches_float64_framework(rows, vocab, upstream):
    print(f"[case] xent {rows}x{vocab} upstream {upstream}", flush=True)
    logits, targets = _case(rows, vocab, seed=rows + vocab)
    l_ref, g_ref = _reference(logits, targets, upstream)
    l_hip, g_hip = _hip(logits, targets, upstream)
    assert _rel(l_hip, l_ref) <= 1e-5, (float(l_hip), float(l_ref))
    assert _rel(g_hip, g_ref) <= 1e-5
    # and the framework's fp32 path on the GPU, the reference's own
    l32, g32 = _hip_framework(logits, targets, upstream)
    assert _rel(l_hip, l32) <= 1e-5 and _rel(g_hip, g32) <= 1e-5


def _hip_framework(logits, targets, upstream):
    x = logits.to(DEV).requires_grad_(True)
    loss = F.cross_entropy(x, targets.to(DEV), ignore_index=-100)
    (loss * upstream).backward()
    return loss.detach(), x.grad


def test_single_word_vocabulary():
    """V = 1: the loss is exactly 0 in float64 and the gradient 0; here both
    are within fp32 rounding of the one logit (absolute 1e-5)."""
    print("[case] xent vocab 1", flush=True)
    logits, targets = _case(3, 1, seed=2, ignore_frac=0.0)
    l_hip, g_hip = _hip(logits, targets, 1.0)
    assert abs(float(l_hip)) <= 1e-5 and float(g_hip.abs().max()) <= 1e-5


def test_large_logits_are_stable():
    """Logits up to +-90: exp overflows fp32 without the running maximum."""
    print("[case] xent large logits", flush=True)
    logits, targets = _case(16, 4096, seed=3, scale=30.0)
    l_ref, g_ref = _reference(logits, targets, 1.0)
    l_hip, g_hip = _hip(logits, targets, 1.0)
    assert torch.isfinite(l_hip) and torch.isfinite(g_hip).all()
    assert _rel(l_hip, l_ref) <= 1e-5 and _rel(g_hip, g_ref) <= 1e-5


def test_every_row_ignored_gives_nan_loss_and_zero_grad():
    """As the framework's mean reduction: 0 / 0 loss, zero gradient."""
    print("[case] xent all ignored", flush=True)
    logits, targets = _case(5, 300, seed=4, ignore_frac=1.0)
    l_hip, g_hip = _hip(logits, targets, 1.0)
    l_ref, g_ref = _reference(logits, targets, 1.0)
    assert torch.isnan(l_hip) and torch.isnan(l_ref)
    assert (g_hip == 0).all() and (g_ref == 0).all()


def test_misaligned_rows_take_the_scalar_path():
    """A contiguous (R, V) view 4 bytes into its storage: no 16-byte loads."""
    print("[case] xent misaligned", flush=True)
    rows, vocab = 9, 2048
    logits, targets = _case(rows, vocab, seed=5)
    buf = torch.empty(rows * vocab + 1, device=DEV)
    view = buf[1:].view(rows, vocab)
    view.copy_(logits.to(DEV))
    l_ref, g_ref = _reference(logits, targets, 1.0)
    l_hip, g_hip = _hip(logits, targets, 1.0, storage=view)
    assert _rel(l_hip, l_ref) <= 1e-5 and _rel(g_hip, g_ref) <= 1e-5


@pytest.mark.parametrize("rows,vocab,lo,hi,storage_offset",
                         [(8, 32768, 32000, 32768, 0),   # 16-value groups all -inf (vec4)
                          (6, 5000, 4000, 5000, 0),      # float4 tail groups all -inf
                          (5, 301, 40, 301, 0),          # scalar threads of -inf only
                          (5, 2048, 0, 1500, 1),         # leading mask, scalar (misaligned)
                          (4, 4096, 0, 3000, 0)])        # leading mask, vec4
def test_minus_inf_masked_columns(rows, vocab, lo, hi, storage_offset):
    """Vocabulary padding masked with -inf: the loss and gradient stay finite
    and match the framework's (the masked columns get gradient 0). Targets lie
    outside the mask."""
    print(f"[case] xent -inf columns {rows}x{vocab} [{lo}, {hi}) off {storage_offset}",
          flush=True)
    logits, _ = _case(rows, vocab, seed=vocab + lo)
    logits[:, lo:hi] = float("-inf")
    free = torch.cat([torch.arange(0, lo), torch.arange(hi, vocab)])
    g = torch.Generator().manual_seed(7)
    targets = free[torch.randint(0, free.numel(), (rows,), generator=g)]
    l_ref, g_ref = _reference(logits, targets, 1.0)
    assert torch.isfinite(l_ref) and torch.isfinite(g_ref).all()
    storage = None
    if storage_offset:
        buf = torch.empty(rows * vocab + storage_offset, device=DEV)
        storage = buf[storage_offset:].view(rows, vocab)
        storage.copy_(logits.to(DEV))
    l_hip, g_hip = _hip(logits, targets, 1.0, storage=storage)
    assert torch.isfinite(l_hip) and torch.isfinite(g_hip).all()
    assert _rel(l_hip, l_ref) <= 1e-5 and _rel(g_hip, g_ref) <= 1e-5
    assert (g_hip[:, lo:hi] == 0).all()


def test_bitwise_reproducible():
    print("[case] xent determinism", flush=True)
    logits, targets = _case(256, 32768, seed=6)
    a = _hip(logits, targets, 1.0)
    b = _hip(logits, targets, 1.0)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_op_argument_errors():
    """The registered ops check on the host before any launch."""
    logits = torch.zeros(4, 8, device=DEV)
    targets = torch.zeros(4, dtype=torch.int64, device=DEV)
    with pytest.raises(HipScanError, match="float32"):
        torch.ops.mamba_hip.xent_fwd(logits.half(), targets, -100)
    with pytest.raises(HipScanError, match="int64"):
        torch.ops.mamba_hip.xent_fwd(logits, targets.int(), -100)
    with pytest.raises(HipScanError, match="targets"):
        torch.ops.mamba_hip.xent_fwd(logits, targets[:3], -100)
    with pytest.raises(HipScanError, match="contiguous"):
        torch.ops.mamba_hip.xent_fwd(logits.t(), targets.repeat(2), -100)
    lse = torch.zeros(4, device=DEV)
    with pytest.raises(HipScanError, match="scale"):
        torch.ops.mamba_hip.xent_bwd(logits, targets, lse, torch.ones(2, device=DEV), -100)
