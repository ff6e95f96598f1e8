"""Memory bounds of the HIP scan, the property the reference exists for
(its torch scan's autograd tape OOM'd at 47.7 GB for an 18M-class train step
that its fused kernels run in 4.14 GB: mamba_metal/scan.py:6-11, gated by
tests/test_scan.py:259-290):

* between forward and backward the scan holds y and the checkpoints, one
  (D, N) state per `chunk` steps: O(T / chunk), never a (B, T, D, N) tape;
* the backward's transient memory is its gradients plus the workspace the
  library asks for (the reduction partials, and at strides above 16 the
  stride-16 checkpoints it recomputes);
* the reference's gate itself: the 18M-class TinyMamba train step
  (d_model 384, 10 layers, d_state 8, batch 16 x seq 512, AdamW) under 16 GB.

Byte counts are torch's caching-allocator statistics (memory_allocated and
max_memory_allocated), which count every tensor the scan allocates.
"""
from __future__ import annotations

import pytest
import torch

from mamba_metal_scan_amd import MambaConfig, TinyMamba, _native, selective_scan_hip

pytestmark = pytest.mark.gpu
DEV = "cuda"
BT, T, D, N = 16, 512, 1536, 16
MIB = 1 << 20
TAPE = BT * T * D * N * 4          # one (B, T, D, N) fp32 tensor: 805 MB


def _inputs():
    g = torch.Generator().manual_seed(31)
    x = torch.randn(BT, T, D, generator=g)
    dt = torch.nn.functional.softplus(torch.randn(BT, T, D, generator=g) - 4.0)
    aneg = torch.arange(1, N + 1, dtype=torch.float32).repeat(D, 1)
    b_in = torch.randn(BT, T, N, generator=g)
    c_in = torch.randn(BT, T, N, generator=g)
    dy = torch.randn(BT, T, D, generator=g)
    leaves = [t.to(DEV).requires_grad_(True) for t in (x, dt, aneg, b_in, c_in)]
    return leaves, dy.to(DEV)


@pytest.mark.parametrize("chunk", [16, 64, 128])
def test_forward_holds_y_and_checkpoints_only(chunk):
    print(f"[case] scan memory {BT}x{T}x{D}x{N} chunk {chunk}", flush=True)
    leaves, dy = _inputs()
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    y = selective_scan_hip(*leaves, chunk=chunk)
    torch.cuda.synchronize()
    held = torch.cuda.memory_allocated() - before
    ckpt = BT * ((T + chunk - 1) // chunk) * D * N * 4
    expect = y.numel() * 4 + ckpt
    print(f"[memory] chunk {chunk}: held {held / MIB:.1f} MiB = y {y.numel() * 4 / MIB:.1f} + "
          f"checkpoints {ckpt / MIB:.1f} (a (B,T,D,N) tape: {TAPE / MIB:.0f} MiB)", flush=True)
    assert expect <= held <= expect + 2 * MIB
    assert held < TAPE / 5

    # Backward: peak over what was held is the gradients plus the workspace.
    ws = _native.library().mhs_scan_bwd_workspace_bytes(BT, T, D, N, chunk)
    grads_bytes = sum(t.numel() * 4 for t in leaves)
    torch.cuda.reset_peak_memory_stats()
    start = torch.cuda.memory_allocated()
    grads = torch.autograd.grad(y, leaves, dy)
    torch.cuda.synchronize()
    transient = torch.cuda.max_memory_allocated() - start
    print(f"[memory] chunk {chunk}: backward transient {transient / MIB:.1f} MiB = grads "
          f"{grads_bytes / MIB:.1f} + workspace {ws / MIB:.1f}", flush=True)
    assert transient <= grads_bytes + ws + 4 * MIB
    del grads, y


def test_checkpoint_memory_scales_as_one_over_the_stride():
    """Held memory minus y at strides 16, 64, 128: exactly the checkpoint
    buffers, in the ratio 8 : 2 : 1."""
    leaves, _ = _inputs()
    held = {}
    for chunk in (16, 64, 128):
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        y = selective_scan_hip(*leaves, chunk=chunk)
        torch.cuda.synchronize()
        held[chunk] = torch.cuda.memory_allocated() - before - y.numel() * 4
        del y
    assert held[16] == 8 * held[128] and held[64] == 2 * held[128]
    assert held[128] == BT * (T // 128) * D * N * 4


def test_18m_class_train_step_fits_in_16gb():
    """The reference's memory gate (tests/test_scan.py:259-290): TinyMamba
    d_model 384, 10 layers, d_ff 1536, d_state 8, d_conv 4, batch 16 x seq
    512, one full train step (forward, backward, AdamW) after a warm-up step;
    peak allocated HBM under 16 GB."""
    print("[case] 18M-class train step memory", flush=True)
    torch.manual_seed(1337)
    cfg = MambaConfig(vocab_size=32768, d_model=384, n_layers=10, d_ff=1536,
                      max_seq_len=512, d_state=8, d_conv=4, scan_impl="hip")
    model = TinyMamba(cfg).to(DEV)
    opt = torch.optim.AdamW(model.parameters(), lr=3e-4)
    g = torch.Generator().manual_seed(1337)
    idx = torch.randint(0, 32768, (16, 513), generator=g).to(DEV)

    def step():
        _, loss = model(idx[:, :-1], idx[:, 1:])
        opt.zero_grad(set_to_none=True)
        loss.backward()
        opt.step()
        return loss

    step()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    loss = step()
    torch.cuda.synchronize()
    gb = torch.cuda.max_memory_allocated() / 2**30
    print(f"[gate] 18M-class step: peak HBM {gb:.2f} GiB (target < 16), "
          f"{model.count_params():,} params, loss {loss.item():.4f}", flush=True)
    assert torch.isfinite(loss)
    assert gb < 16.0
    del model, opt
    torch.cuda.empty_cache()
