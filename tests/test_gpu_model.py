"""GPU parity beyond the bare scan: the decode-step kernel against the
oracle, TinyMamba end to end with scan_impl 'hip' vs 'torch' (the
reference's tests/test_scan.py:177-202), and the recurrent cache on the device
(prefill through the HIP scan, then the fused step kernel)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close
from mamba_metal_scan_amd import selective_state_step
from mamba_metal_scan_amd.model import MambaConfig, TinyMamba
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
SEED = 1337
VOCAB = 200


@pytest.mark.parametrize("bt,d,n", [(3, 96, 16), (2, 130, 8), (1, 64, 5), (2, 40, 64),
                                    (32, 4096, 16)])
def test_decode_step_matches_the_oracle(bt, d, n):
    print(f"[case] decode step {bt}x{d}x{n}", flush=True)
    rng = np.random.default_rng(bt * 1000 + n)
    h = rng.standard_normal((bt, d, n)).astype(np.float32)
    x = rng.standard_normal((bt, d)).astype(np.float32)
    dt = np.log1p(np.exp(rng.standard_normal((bt, d)) - 4.0)).astype(np.float32)
    aneg = np.tile(np.arange(1, n + 1, dtype=np.float32), (d, 1))
    b_in = rng.standard_normal((bt, n)).astype(np.float32)
    c_in = rng.standard_normal((bt, n)).astype(np.float32)
    h_ref, y_ref = oracle.scan_step(h, x, dt, aneg, b_in, c_in)
    hd = torch.from_numpy(h).to(DEV)
    y = selective_state_step(hd, *(torch.from_numpy(a).to(DEV) for a in (x, dt, aneg, b_in, c_in)))
    torch.cuda.synchronize()
    assert_close("y", y, y_ref)
    assert_close("h", hd, h_ref)


def _cfg(**over):
    kw = dict(vocab_size=VOCAB, d_model=64, n_layers=2, d_ff=128, max_seq_len=64, d_state=16,
              d_conv=4, scan_chunk=0)
    kw.update(over)
    return MambaConfig(**kw)


def test_end_to_end_torch_vs_hip():
    """Same weights, same batch: loss and every parameter gradient agree."""
    torch.manual_seed(SEED)
    m_hip = TinyMamba(_cfg(scan_impl="hip")).to(DEV)
    m_ref = TinyMamba(_cfg(scan_impl="torch")).to(DEV)
    m_ref.load_state_dict(m_hip.state_dict())
    x = torch.randint(0, VOCAB, (4, 48), generator=torch.Generator().manual_seed(SEED)).to(DEV)
    _, l_hip = m_hip(x, x)
    _, l_ref = m_ref(x, x)
    l_hip.backward()
    l_ref.backward()
    assert torch.allclose(l_hip, l_ref, atol=1e-5, rtol=1e-5), (l_hip.item(), l_ref.item())
    for (name, p1), p2 in zip(m_hip.named_parameters(), m_ref.parameters()):
        assert_close(name, p1.grad, p2.grad, tol=2e-4)


def test_block_hooks_run_and_keep_the_loss():
    """A forward hook on a block makes TinyMamba call block(x) for every block
    (the folded-norm path calls block.mix() and would skip the hook): the hook
    runs once per block and the loss equals the folded path's."""
    torch.manual_seed(SEED)
    model = TinyMamba(_cfg(scan_impl="hip")).to(DEV)
    x = torch.randint(0, VOCAB, (4, 48), generator=torch.Generator().manual_seed(SEED)).to(DEV)
    with torch.no_grad():
        _, l_folded = model(x, x)
        seen = []
        h = model.blocks[1].register_forward_hook(lambda m, i, o: seen.append(o.shape))
        _, l_hooked = model(x, x)
        h.remove()
    assert seen == [torch.Size((4, 48, 64))]
    assert torch.allclose(l_folded, l_hooked, atol=1e-5, rtol=1e-5)


def test_recurrent_cache_on_device_matches_full_recomputation():
    torch.manual_seed(SEED)
    model = TinyMamba(_cfg(scan_impl="hip")).to(DEV).eval()
    full = torch.randint(0, VOCAB, (4, 26), generator=torch.Generator().manual_seed(3)).to(DEV)
    ctx, rest = full[:, :20], full[:, 20:]
    with torch.no_grad():
        cache: dict = {}
        model(ctx, cache=cache)
        for t in range(rest.shape[1]):
            step_logits, _ = model(rest[:, t:t + 1], cache=cache)
            full_logits, _ = model(torch.cat([ctx, rest[:, :t + 1]], dim=1))
            delta = (step_logits[:, -1] - full_logits[:, -1]).abs().max().item()
            assert delta < 1e-4, f"step {t}: cache diverges by {delta:.2e}"


def test_decode_step_replays_from_a_hip_graph():
    """The step kernel captured in a HIP graph: every replay (with eager work
    and synchronisation between replays) matches the eager result."""
    bt, d, n, steps = 4, 256, 16, 8
    g = torch.Generator().manual_seed(11)
    xs = torch.randn(steps, bt, d, generator=g).to(DEV)
    dts = torch.nn.functional.softplus(torch.randn(steps, bt, d, generator=g) - 4.0).to(DEV)
    aneg = torch.arange(1, n + 1, dtype=torch.float32).repeat(d, 1).to(DEV)
    bs = torch.randn(steps, bt, n, generator=g).to(DEV)
    cs = torch.randn(steps, bt, n, generator=g).to(DEV)
    h0 = torch.randn(bt, d, n, generator=g).to(DEV)

    def run(h, ys):
        for i in range(steps):
            ys[i] = selective_state_step(h, xs[i], dts[i], aneg, bs[i], cs[i])

    h_ref, y_ref = h0.clone(), torch.empty(steps, bt, d, device=DEV)
    run(h_ref, y_ref)
    h, ys = h0.clone(), torch.empty(steps, bt, d, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run(h, ys)                      # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(h, ys)
    for rep in range(3):
        h.copy_(h0)
        ys.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ys, y_ref), f"replay {rep}: y differs"
        assert torch.equal(h, h_ref), f"replay {rep}: h differs"


def test_prefill_then_decode_matches_rerunning_the_context():
    """32 x 2048 x 4096 x 16: prefill with return_state, then 256 decode steps
    with the step kernel; each decoded y equals the full-context scan's."""
    from mamba_metal_scan_amd import selective_scan_hip
    bt, t_pre, d, n, steps = 32, 2048, 4096, 16, 256
    print(f"[case] prefill {bt}x{t_pre}x{d}x{n} + {steps} decode steps", flush=True)
    g = torch.Generator().manual_seed(21)
    t_all = t_pre + steps
    x = torch.randn(bt, t_all, d, generator=g).to(DEV)
    dt = torch.nn.functional.softplus(torch.randn(bt, t_all, d, generator=g) - 4.0).to(DEV)
    aneg = torch.arange(1, n + 1, dtype=torch.float32).repeat(d, 1).to(DEV)
    b_in = torch.randn(bt, t_all, n, generator=g).to(DEV)
    c_in = torch.randn(bt, t_all, n, generator=g).to(DEV)
    with torch.no_grad():
        y_full = selective_scan_hip(x, dt, aneg, b_in, c_in)
        _, h = selective_scan_hip(x[:, :t_pre], dt[:, :t_pre], aneg, b_in[:, :t_pre],
                                  c_in[:, :t_pre], return_state=True)
        h = h.contiguous()
        ys = []
        for i in range(t_pre, t_all):
            ys.append(selective_state_step(h, x[:, i].contiguous(), dt[:, i].contiguous(), aneg,
                                           b_in[:, i].contiguous(), c_in[:, i].contiguous()))
        torch.cuda.synchronize()
    assert_close("decoded y", torch.stack(ys, dim=1), y_full[:, t_pre:])


def test_80m_train_step_hip_matches_torch():
    """The 80M TinyMamba (vocab 32768, d_model 640, 12 layers, d_state 16) at
    batch 16 x seq 512: loss and every parameter gradient with scan_impl 'hip'
    match scan_impl 'torch' within 1e-4 (max rel per tensor)."""
    print("[case] 80M train step hip vs torch", flush=True)
    cfg = dict(vocab_size=32768, d_model=640, n_layers=12, d_ff=2560, max_seq_len=512,
               d_state=16, d_conv=4)
    torch.manual_seed(SEED)
    m_hip = TinyMamba(MambaConfig(scan_impl="hip", **cfg)).to(DEV)
    m_ref = TinyMamba(MambaConfig(scan_impl="torch", **cfg)).to(DEV)
    m_ref.load_state_dict(m_hip.state_dict())
    assert m_hip.count_params() == 79_525_728
    idx = torch.randint(0, 32768, (16, 513), generator=torch.Generator().manual_seed(SEED)).to(DEV)
    x, y = idx[:, :-1], idx[:, 1:]
    _, l_hip = m_hip(x, y)
    l_hip.backward()
    _, l_ref = m_ref(x, y)
    l_ref.backward()
    torch.cuda.synchronize()
    assert abs(l_hip.item() - l_ref.item()) <= 1e-4 * abs(l_ref.item())
    for (name, p1), p2 in zip(m_hip.named_parameters(), m_ref.parameters()):
        assert_close(name, p1.grad, p2.grad)
