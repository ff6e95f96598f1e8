"""The registered custom ops (mamba_hip::*) under torch.library.opcheck, and
the scan and the fused inner block under torch.compile against eager mode.

opcheck runs each op through its schema and mutation checks, its fake
(meta) implementation against the real one (shapes, strides, dtypes), and
AOT dispatch: what torch.compile relies on. The compiled runs use the
aot_eager backend, which traces the autograd Functions and the registered
ops with their fake implementations but generates no code of its own.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from helpers import assert_close, assert_same, reduction
from mamba_metal_scan_amd import _native, mamba_inner, selective_scan_gated, selective_scan_hip

pytestmark = pytest.mark.gpu
DEV = "cuda"
OPS = torch.ops.mamba_hip


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _scan_args(bt=2, t_len=40, d=48, n=16, seed=0):
    g = _gen(seed)
    x = torch.randn(bt, t_len, d, generator=g)
    dt = F.softplus(torch.randn(bt, t_len, d, generator=g) - 4.0)
    aneg = torch.arange(1, n + 1, dtype=torch.float32).repeat(d, 1)
    b_in = torch.randn(bt, t_len, n, generator=g)
    c_in = torch.randn(bt, t_len, n, generator=g)
    dy = torch.randn(bt, t_len, d, generator=g)
    return [v.to(DEV) for v in (x, dt, aneg, b_in, c_in, dy)]


def test_opcheck_scan_ops():
    print("[case] opcheck scan_fwd / scan_bwd / scan_step", flush=True)
    x, dt, aneg, b_in, c_in, dy = _scan_args()
    torch.library.opcheck(OPS.scan_fwd, (x, dt, aneg, b_in, c_in, 16, True))
    torch.library.opcheck(OPS.scan_fwd, (x, dt, aneg, b_in, c_in, 7, False))
    _, ckpt, h_last = OPS.scan_fwd(x, dt, aneg, b_in, c_in, 16, True)
    torch.library.opcheck(OPS.scan_bwd, (x, dt, aneg, b_in, c_in, dy, None, ckpt, 16))
    torch.library.opcheck(OPS.scan_bwd, (x, dt, aneg, b_in, c_in, dy, h_last, ckpt, 16))
    h = h_last.clone()
    torch.library.opcheck(OPS.scan_step, (h, x[:, 0].contiguous(), dt[:, 0].contiguous(), aneg,
                                          b_in[:, 0].contiguous(), c_in[:, 0].contiguous()))


def test_opcheck_gated_scan_ops():
    print("[case] opcheck gated scan ops", flush=True)
    bt, t_len, d, n = 2, 40, 48, 16
    x, _, _, _, _, dy = _scan_args(bt, t_len, d, n, seed=1)
    g = _gen(2)
    proj = torch.randn(bt, t_len, d + 2 * n, generator=g).to(DEV)   # rows [dt_raw | B | C]
    a_raw = (torch.arange(1, n + 1, dtype=torch.float32).repeat(d, 1)
             + 0.1 * torch.randn(d, n, generator=g)).to(DEV)
    bias = torch.randn(d, generator=g).to(DEV)
    raw, b_in, c_in = proj[..., :d], proj[..., d:d + n], proj[..., d + n:]
    for dt_bias in (None, bias):
        torch.library.opcheck(OPS.scan_gated_fwd,
                              (x, raw, a_raw, b_in, c_in, 0.001, 0.1, 16, True, dt_bias))
    _, ckpt, _ = OPS.scan_gated_fwd(x, raw, a_raw, b_in, c_in, 0.001, 0.1, 16, True, bias)
    torch.library.opcheck(OPS.scan_gated_bwd,
                          (x, raw, a_raw, b_in, c_in, 0.001, 0.1, dy, None, ckpt, 16, bias))
    dproj = torch.empty_like(proj)
    torch.library.opcheck(OPS.scan_gated_bwd_into, (x, raw, a_raw, b_in, c_in, 0.001, 0.1, dy,
                                                    None, ckpt, 16, dproj, bias))


def test_opcheck_conv_and_gate_ops():
    print("[case] opcheck conv and output gate ops", flush=True)
    bt, t_len, d, k = 2, 40, 48, 4
    g = _gen(3)
    xz = torch.randn(bt, t_len, 2 * d, generator=g).to(DEV)
    x, z = xz[..., :d], xz[..., d:]
    w = (0.3 * torch.randn(d, k, generator=g)).to(DEV)
    cb = (0.1 * torch.randn(d, generator=g)).to(DEV)
    dout = torch.randn(bt, t_len, d, generator=g).to(DEV)
    y = torch.randn(bt, t_len, d, generator=g).to(DEV)
    d_skip = torch.randn(d, generator=g).to(DEV)
    dxz = torch.empty_like(xz)
    torch.library.opcheck(OPS.conv1d_silu_fwd, (x, w, cb))
    torch.library.opcheck(OPS.conv1d_silu_bwd, (x, w, cb, dout))
    torch.library.opcheck(OPS.conv1d_silu_bwd_into, (x, w, cb, dout, dxz[..., :d]))
    torch.library.opcheck(OPS.out_gate_fwd, (y, d_skip, z))
    torch.library.opcheck(OPS.out_gate_bwd, (y, d_skip, z, dout))
    torch.library.opcheck(OPS.out_gate_bwd_into, (y, d_skip, z, dout, dxz[..., d:]))


def test_opcheck_cross_entropy_ops():
    print("[case] opcheck cross-entropy ops", flush=True)
    g = _gen(4)
    logits = torch.randn(6, 1000, generator=g).to(DEV)
    targets = torch.tensor([3, -100, 999, 0, 512, 7]).to(DEV)
    torch.library.opcheck(OPS.xent_fwd, (logits, targets, -100))
    lse, _ = OPS.xent_fwd(logits, targets, -100)
    scale = torch.full((1,), 0.2, device=DEV)
    torch.library.opcheck(OPS.xent_bwd, (logits, targets, lse, scale, -100))


def test_opcheck_rmsnorm_ops():
    print("[case] opcheck RMSNorm ops", flush=True)
    g = _gen(5)
    x = torch.randn(37, 132, generator=g).to(DEV)
    w = torch.randn(132, generator=g).to(DEV)
    torch.library.opcheck(OPS.rmsnorm_fwd, (x, w, 1e-6))
    _, rstd = OPS.rmsnorm_fwd(x, w, 1e-6)
    dy = torch.randn(37, 132, generator=g).to(DEV)
    dres = torch.randn(37, 132, generator=g).to(DEV)
    torch.library.opcheck(OPS.rmsnorm_bwd, (dy, x, w, rstd, dres))
    torch.library.opcheck(OPS.rmsnorm_bwd, (dy, x, w, rstd, None))
    torch.library.opcheck(OPS.add_rmsnorm_fwd, (x, dres, w, 1e-6))


def test_compiled_scan_matches_eager():
    """torch.compile (aot_eager) of a function around the scan: the traced
    graph calls the registered ops; values and all gradients match eager."""
    print("[case] torch.compile scan", flush=True)
    x, dt, aneg, b_in, c_in, dy = _scan_args(2, 100, 64, 16, seed=4)

    def f(x, dt, aneg, b_in, c_in):
        y, h = selective_scan_hip(torch.tanh(x), dt, aneg, b_in, c_in, chunk=16,
                                  return_state=True)
        return y * 2.0, h.sum()

    results = []
    for fn in (f, torch.compile(f, backend="aot_eager", fullgraph=True)):
        leaves = [v.clone().requires_grad_(True) for v in (x, dt, aneg, b_in, c_in)]
        y, hs = fn(*leaves)
        grads = torch.autograd.grad([y, hs], leaves, [dy, torch.ones_like(hs)])
        results.append((y.detach(), hs.detach(), grads))
    torch.cuda.synchronize()
    (y1, h1, g1), (y2, h2, g2) = results
    assert_close("y", y1, y2, 1e-6)
    assert_close("h", h1, h2, 1e-6)
    for name, a, b in zip(("dx", "ddt", "dAneg", "dB", "dC"), g1, g2):
        assert_close(name, a, b, 1e-6)


def test_compiled_gated_scan_and_inner_block_match_eager():
    print("[case] torch.compile gated scan and inner block", flush=True)
    bt, t_len, d, n = 2, 64, 64, 16
    g = _gen(5)
    params = [torch.randn(bt, t_len, 2 * d, generator=g), 0.3 * torch.randn(d, 1, 4, generator=g),
              0.1 * torch.randn(d, generator=g), 0.05 * torch.randn(d, d, generator=g),
              0.5 * torch.randn(d, generator=g), 0.1 * torch.randn(n, d, generator=g),
              0.1 * torch.randn(n, d, generator=g),
              torch.log(torch.arange(1, n + 1, dtype=torch.float32)).expand(d, n).contiguous(),
              torch.randn(d, generator=g)]
    params = [p.to(DEV) for p in params]
    dout = torch.randn(bt, t_len, d, generator=g).to(DEV)

    def inner(*p):
        return mamba_inner(*p, 0.001, 0.1, chunk=16)

    def gated(xz, w_dt, b_dt, a_raw):
        x = xz[..., :d].contiguous()
        return selective_scan_gated(x, x @ w_dt.t(), a_raw, x[..., :n], x[..., n:2 * n],
                                    0.001, 0.1, chunk=16, dt_bias=b_dt)

    for fn, idx in ((inner, list(range(9))), (gated, [0, 3, 4, 7])):
        outs = []
        for f in (fn, torch.compile(fn, backend="aot_eager", fullgraph=True)):
            leaves = [params[i].clone().requires_grad_(True) for i in idx]
            out = f(*leaves)
            outs.append((out.detach(), torch.autograd.grad(out, leaves, dout)))
        torch.cuda.synchronize()
        (o1, g1), (o2, g2) = outs
        assert_close("out", o1, o2, 1e-6)
        for a, b in zip(g1, g2):
            assert_close("grad", a, b, 1e-5)


def test_compiled_tinymamba_train_step_matches_eager():
    """A small TinyMamba loss and every parameter gradient under torch.compile
    (aot_eager, one graph) against eager: the block's HIP path (conv, fused
    inner block, output projection) traces without breaks."""
    from mamba_metal_scan_amd import MambaConfig, TinyMamba
    print("[case] torch.compile TinyMamba", flush=True)
    torch.manual_seed(0)
    cfg = MambaConfig(vocab_size=256, d_model=64, n_layers=2, d_ff=256, max_seq_len=64,
                      d_state=16, scan_impl="hip")
    model = TinyMamba(cfg).to(DEV)
    idx = torch.randint(0, 256, (2, 33), generator=_gen(6)).to(DEV)
    x, y = idx[:, :-1], idx[:, 1:]
    results = []
    for fn in (model, torch.compile(model, backend="aot_eager", fullgraph=True)):
        model.zero_grad(set_to_none=True)
        _, loss = fn(x, y)
        loss.backward()
        results.append((loss.detach(), [p.grad.clone() for p in model.parameters()]))
    torch.cuda.synchronize()
    (l1, g1), (l2, g2) = results
    assert_close("loss", l1, l2, 1e-6)
    for (name, _), a, b in zip(model.named_parameters(), g1, g2):
        assert_close(name, a, b, 1e-5)


def _capture(fn):
    """fn() warmed up on a side stream, then captured in a HIP graph; returns
    (graph, the captured outputs)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = fn()
    return graph, outs


@pytest.mark.parametrize("mode", ["fixed", "atomic"])
@pytest.mark.parametrize("shape", [(4, 256, 512, 16), (1, 1024, 128, 16)])
def test_scan_fwd_bwd_replays_from_a_hip_graph(shape, mode):
    """Forward + backward launches captured once and replayed three times,
    with other eager scans and synchronizations between the replays: every
    replay equals the eager result bit for bit (with the atomic reduction:
    the atomically reduced sums within RED_TOL; their zero-fill is a kernel,
    captured with the rest). The second shape is small enough to run in time
    segments (forward workspace, carry kernels)."""
    bt, t_len, d, n = shape
    atomic = mode == "atomic"
    print(f"[case] HIP graph scan fwd+bwd {shape} {mode}", flush=True)
    x, dt, aneg, b_in, c_in, dy = _scan_args(bt, t_len, d, n, seed=7)

    def step(x=x):
        y, ckpt, h_last = OPS.scan_fwd(x, dt, aneg, b_in, c_in, 16, True)
        return (y, h_last) + tuple(OPS.scan_bwd(x, dt, aneg, b_in, c_in, dy, None, ckpt, 16))

    with reduction(_native.REDUCTION_ATOMIC if atomic else _native.REDUCTION_FIXED):
        ref = [t.clone() for t in step()]
        graph, outs = _capture(step)
        for rep in range(3):
            other = step(x * (0.5 + rep))     # eager work on other inputs between replays
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            for name, a, b in zip(("y", "h_last", "dx", "ddt", "dAneg", "dB", "dC"), outs, ref):
                assert_same(name, a, b, atomic)
            del other


def test_inner_block_fwd_bwd_replays_from_a_hip_graph():
    """The fused inner block's forward and autograd backward (conv, GEMMs,
    gated scan with its bias, output gate) captured and replayed."""
    print("[case] HIP graph mamba_inner fwd+bwd", flush=True)
    bt, t_len, d, n = 4, 128, 256, 16
    g = _gen(8)
    params = [torch.randn(bt, t_len, 2 * d, generator=g), 0.3 * torch.randn(d, 1, 4, generator=g),
              0.1 * torch.randn(d, generator=g), 0.05 * torch.randn(d, d, generator=g),
              0.5 * torch.randn(d, generator=g), 0.1 * torch.randn(n, d, generator=g),
              0.1 * torch.randn(n, d, generator=g),
              torch.log(torch.arange(1, n + 1, dtype=torch.float32)).expand(d, n).contiguous(),
              torch.randn(d, generator=g)]
    dout = torch.randn(bt, t_len, d, generator=g).to(DEV)

    def step(leaves):
        out = mamba_inner(*leaves, 0.001, 0.1, chunk=16)
        return (out,) + tuple(torch.autograd.grad(out, leaves, dout))

    # The eager runs use their own leaf tensors: the captured leaves' autograd
    # nodes then belong to the capture's streams only. Fixed-order reduction:
    # the atomically reduced dB, dC feed the weight GEMMs, so with atomics
    # nearly every output would carry their rounding.
    eager = [p.to(DEV).requires_grad_(True) for p in params]
    leaves = [p.to(DEV).requires_grad_(True) for p in params]
    with reduction(_native.REDUCTION_FIXED):
        ref = [t.detach().clone() for t in step(eager)]
        graph, outs = _capture(lambda: step(leaves))
        for rep in range(3):
            step(eager)                       # eager work between replays
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(zip(outs, ref)):
                assert torch.equal(a, b), f"replay {rep}: output {i} differs"
