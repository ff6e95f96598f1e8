"""Parity of the gfx950 scan kernels with the float64 oracle and the fp32 torch
reference (the reference's gates, tests/test_scan.py:86-230, on a ROCm GPU).

Bar: per tensor, max|got - ref| / max|ref| <= 1e-4 against the float64 oracle
(oracle/scan_oracle.c); the reference-style allclose(atol=1e-4, rtol=1e-3)
against selective_scan_ref in fp32 on the same device.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import ATOL, RED_TOL, RTOL, TOL, assert_close, assert_same, reduction, rel_err, to_np
from mamba_metal_scan_amd import _native, selective_scan, selective_scan_hip, selective_scan_ref
from oracle import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda"

# (B, T, D, N): the reference's kernel shapes (tests/test_scan.py:86-95), the
# CPU-runnable configuration (2x128x64x16) and edge shapes of the training
# configuration (T not a multiple of the window, D not a multiple of 64,
# T = 1, batch 1, d_state 8).
REF_SHAPES = [(2, 64, 32, 16), (1, 100, 17, 16), (4, 63, 128, 16), (1, 1, 16, 16),
              (2, 130, 40, 8), (3, 512, 856, 16)]
EDGE_SHAPES = [(2, 128, 64, 16), (2, 1000, 64, 16), (2, 96, 1000, 16), (1, 1, 1536, 16),
               (1, 512, 1536, 16), (4, 512, 256, 8), (2, 33, 70, 4), (2, 40, 64, 12),
               (1, 20, 64, 5), (2, 48, 96, 32), (1, 24, 128, 64), (2, 37, 96, 40),
               (1, 50, 33, 1)]
# Grids of two to three blocks per CU (of 256 CUs), as at the training shape:
# d_inner 1500 and 3000 end in a partial channel block, T 50 in a partial
# sub-chunk.
GROUPED_SHAPES = [(16, 96, 1500, 16), (12, 64, 2048, 16), (6, 50, 3000, 16)]


def _to_dev(arrs):
    return [torch.from_numpy(a).to(DEV) for a in arrs]


def _bench_inputs(bt, t_len, d, n, seed):
    """The benchmark's seeded inputs (torch generator on the CPU, then moved):
    x, B, C, dy ~ N(0,1), dt = softplus(N(-4,1)), Aneg[d,n] = n+1."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(bt, t_len, d, generator=g)
    dt = torch.nn.functional.softplus(torch.randn(bt, t_len, d, generator=g) - 4.0)
    aneg = torch.arange(1, n + 1, dtype=torch.float32).repeat(d, 1)
    b_in = torch.randn(bt, t_len, n, generator=g)
    c_in = torch.randn(bt, t_len, n, generator=g)
    dy = torch.randn(bt, t_len, d, generator=g)
    return [t.to(DEV) for t in (x, dt, aneg, b_in, c_in, dy)]


def _run_hip(inp, dy, chunk=None, dh_last=None):
    """HIP forward + backward via autograd: (y, h_last, grads)."""
    leaves = [t.clone().requires_grad_(True) for t in inp]
    kw = {} if chunk is None else {"chunk": chunk}
    y, h_last = selective_scan_hip(*leaves, return_state=True, **kw)
    outs, gouts = [y], [dy]
    if dh_last is not None:
        outs.append(h_last)
        gouts.append(dh_last)
    grads = torch.autograd.grad(outs, leaves, grad_outputs=gouts)
    torch.cuda.synchronize()
    return y.detach(), h_last.detach(), grads


@pytest.mark.parametrize("shape", REF_SHAPES + EDGE_SHAPES + GROUPED_SHAPES)
def test_forward_and_gradients_match_the_oracle(shape):
    bt, t_len, d, n = shape
    print(f"[case] oracle parity {shape}", flush=True)
    arrs = oracle.make_inputs(bt, t_len, d, n, seed=1000 + d, style="bench")
    rng = np.random.default_rng(7)
    dy = rng.standard_normal((bt, t_len, d), dtype=np.float32)
    y_ref, _, h_ref = oracle.scan_fwd(*arrs)
    grads_ref = oracle.scan_bwd(*arrs, dy)

    y, h_last, grads = _run_hip(_to_dev(arrs), torch.from_numpy(dy).to(DEV))
    assert y.shape == (bt, t_len, d) and y.dtype == torch.float32
    assert_close("y", y, y_ref)
    assert_close("h_last", h_last, h_ref)
    for name, g, r in zip(("dx", "ddt", "dAneg", "dB", "dC"), grads, grads_ref):
        assert g.shape == r.shape, name
        assert_close(name, g, r)


@pytest.mark.parametrize("shape", REF_SHAPES)
def test_matches_torch_reference_in_fp32(shape):
    """The reference's own gate: kernel vs selective_scan_ref on the device."""
    bt, t_len, d, n = shape
    print(f"[case] torch-ref parity {shape}", flush=True)
    arrs = oracle.make_inputs(bt, t_len, d, n, seed=1337 + d, style="ref")
    inp = _to_dev(arrs)
    dy = torch.from_numpy(np.random.default_rng(3).standard_normal(
        (bt, t_len, d), dtype=np.float32)).to(DEV)
    y, _, g_hip = _run_hip(inp, dy)
    leaves = [t.clone().requires_grad_(True) for t in inp]
    ref = selective_scan_ref(*leaves)
    g_ref = torch.autograd.grad(ref, leaves, grad_outputs=dy)
    assert torch.allclose(y, ref, atol=ATOL, rtol=RTOL), rel_err(y, ref)
    assert_close("y", y, ref)
    for name, g, r in zip(("dx", "ddt", "dAneg", "dB", "dC"), g_hip, g_ref):
        assert torch.allclose(g, r, atol=ATOL, rtol=RTOL), \
            f"{name}: max delta {(g - r).abs().max().item():.3e} scale {r.abs().max().item():.3e}"
        assert_close(name, g, r)


def test_state_gradient_flows():
    """dh_last (gradient of the returned state) reaches every input."""
    bt, t_len, d, n = 2, 77, 96, 16
    print("[case] dh_last", flush=True)
    arrs = oracle.make_inputs(bt, t_len, d, n, seed=5, style="bench")
    rng = np.random.default_rng(11)
    dy = rng.standard_normal((bt, t_len, d), dtype=np.float32)
    dh = rng.standard_normal((bt, d, n), dtype=np.float32)
    grads_ref = oracle.scan_bwd(*arrs, dy, dh)
    _, _, grads = _run_hip(_to_dev(arrs), torch.from_numpy(dy).to(DEV),
                           dh_last=torch.from_numpy(dh).to(DEV))
    for name, g, r in zip(("dx", "ddt", "dAneg", "dB", "dC"), grads, grads_ref):
        assert_close(name, g, r)


@pytest.mark.parametrize("chunk", [1, 7, 16, 64, 511, 512])
def test_checkpoint_stride_is_not_a_result(chunk):
    """Strides 1, 7, 64, 511, 512 (tests/test_scan.py:213-221) -- fwd and bwd."""
    bt, t_len, d, n = 2, 512, 96, 16
    print(f"[case] chunk {chunk}", flush=True)
    arrs = oracle.make_inputs(bt, t_len, d, n, seed=1337 + 5, style="ref")
    dy = np.random.default_rng(9).standard_normal((bt, t_len, d), dtype=np.float32)
    y_ref, ck_ref, h_ref = oracle.scan_fwd(*arrs, chunk=chunk)
    grads_ref = oracle.scan_bwd(*arrs, dy)
    inp = _to_dev(arrs)
    y, h_last, grads = _run_hip(inp, torch.from_numpy(dy).to(DEV), chunk=chunk)
    assert_close("y", y, y_ref)
    assert_close("h_last", h_last, h_ref)
    for name, g, r in zip(("dx", "ddt", "dAneg", "dB", "dC"), grads, grads_ref):
        assert_close(name, g, r)
    # The checkpoints themselves: h at the end of every chunk.
    _, ckpt, _ = torch.ops.mamba_hip.scan_fwd(*inp, chunk, True)
    assert ckpt.shape == ck_ref.shape
    assert_close("ckpt", ckpt, ck_ref)


def test_returned_state_is_the_recurrence_state():
    arrs = oracle.make_inputs(1, 100, 16, 16, seed=1337 + 7, style="ref")
    inp = _to_dev(arrs)
    _, state = selective_scan_hip(*inp, return_state=True)
    _, ref_state = selective_scan_ref(*inp, return_state=True)
    assert state.shape == ref_state.shape
    assert torch.allclose(state, ref_state, atol=ATOL, rtol=RTOL)


def test_training_shape_fwd_bwd_matches_the_oracle():
    """Batch 16 x T 512 x d_inner 1536 x d_state 16 against the float64 oracle."""
    bt, t_len, d, n = 16, 512, 1536, 16
    print("[case] 16x512x1536x16", flush=True)
    arrs = oracle.make_inputs(bt, t_len, d, n, seed=2024, style="bench")
    dy = np.random.default_rng(1).standard_normal((bt, t_len, d), dtype=np.float32)
    y_ref, _, h_ref = oracle.scan_fwd(*arrs)
    grads_ref = oracle.scan_bwd(*arrs, dy)
    y, h_last, grads = _run_hip(_to_dev(arrs), torch.from_numpy(dy).to(DEV))
    errs = {"y": assert_close("y", y, y_ref), "h_last": assert_close("h_last", h_last, h_ref)}
    for name, g, r in zip(("dx", "ddt", "dAneg", "dB", "dC"), grads, grads_ref):
        errs[name] = assert_close(name, g, r)
    print("[errors vs fp64]", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)


def test_training_shape_matches_the_torch_reference_in_fp32():
    """16x512x1536x16: the HIP scan against selective_scan(impl="torch") in
    fp32 on the same device and the same seeded inputs, y and all five
    gradients within max relative error 1e-4 (max|hip - torch| / max|torch|)."""
    bt, t_len, d, n = 16, 512, 1536, 16
    print("[case] torch-ref parity 16x512x1536x16", flush=True)
    inp = _bench_inputs(bt, t_len, d, n, seed=31)
    dy = inp.pop()
    y, _, g_hip = _run_hip(inp, dy)
    leaves = [t.clone().requires_grad_(True) for t in inp]
    ref = selective_scan(*leaves, impl="torch")
    g_ref = torch.autograd.grad(ref, leaves, grad_outputs=dy)
    torch.cuda.synchronize()
    errs = {"y": assert_close("y", y, ref)}
    for name, g, r in zip(("dx", "ddt", "dAneg", "dB", "dC"), g_hip, g_ref):
        errs[name] = assert_close(name, g, r)
    print("[errors vs torch fp32]", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)


@pytest.mark.parametrize("chunk", [1, 7, 64, 511, 512])
def test_training_shape_stride_sweep(chunk):
    """16x512x1536x16 at checkpoint strides 1, 7, 64, 511, 512 against
    stride 16 (fixed-order reduction): y, the state and every gradient agree
    to fp32 rounding (the backward recomputes the same states from the
    checkpoints, whatever their stride)."""
    bt, t_len, d, n = 16, 512, 1536, 16
    print(f"[case] 16x512x1536x16 chunk {chunk} vs 16", flush=True)
    x, dt, aneg, b_in, c_in, dy = _bench_inputs(bt, t_len, d, n, seed=7)

    def run(k):
        y, ckpt, h_last = torch.ops.mamba_hip.scan_fwd(x, dt, aneg, b_in, c_in, k, True)
        assert ckpt.shape == (bt, (t_len + k - 1) // k, d, n)
        grads = torch.ops.mamba_hip.scan_bwd(x, dt, aneg, b_in, c_in, dy, None, ckpt, k)
        return (y, h_last) + tuple(grads)

    with reduction(_native.REDUCTION_FIXED):
        base, other = run(16), run(chunk)
    torch.cuda.synchronize()
    for name, a, b in zip(("y", "h_last", "dx", "ddt", "dAneg", "dB", "dC"), other, base):
        assert_close(name, a, b, 1e-6)


@pytest.mark.parametrize("mode", ["fixed", "atomic"])
def test_backward_determinism(mode):
    """Fixed-order reduction: every gradient bit for bit equal run to run.
    Atomic reduction: dx and ddt still bit for bit; dB, dC, dAneg within
    RED_TOL (their rounding depends on the order the atomics land in)."""
    atomic = mode == "atomic"
    arrs = oracle.make_inputs(4, 200, 300, 16, seed=77, style="bench")
    inp = _to_dev(arrs)
    dy = torch.randn(4, 200, 300, device=DEV, generator=torch.Generator(DEV).manual_seed(0))
    with reduction(_native.REDUCTION_ATOMIC if atomic else _native.REDUCTION_FIXED):
        g1 = _run_hip(inp, dy)[2]
        g2 = _run_hip(inp, dy)[2]
    for name, a, b in zip(("dx", "ddt", "dAneg", "dB", "dC"), g1, g2):
        assert_same(name, a, b, atomic)


def test_atomic_and_fixed_order_reductions_agree_at_the_training_shape():
    """16x512x1536x16: the atomic backward against the fixed-order one (dx,
    ddt bit for bit; the reduced sums within RED_TOL), and the atomic path's
    run-to-run spread over five backward calls, printed."""
    bt, t_len, d, n = 16, 512, 1536, 16
    print("[case] reductions at 16x512x1536x16", flush=True)
    x, dt, aneg, b_in, c_in, dy = _bench_inputs(bt, t_len, d, n, seed=2024)
    _, ckpt, _ = torch.ops.mamba_hip.scan_fwd(x, dt, aneg, b_in, c_in, 16, True)
    bwd = lambda: torch.ops.mamba_hip.scan_bwd(x, dt, aneg, b_in, c_in, dy, None, ckpt, 16)
    with reduction(_native.REDUCTION_FIXED):
        fixed = bwd()
    with reduction(_native.REDUCTION_ATOMIC):
        runs = [bwd() for _ in range(5)]
    torch.cuda.synchronize()
    names = ("dx", "ddt", "dAneg", "dB", "dC")
    for name, a, b in zip(names, runs[0], fixed):
        assert_same(name, a, b, atomic=True)
    spread = {name: max(rel_err(r[i], runs[0][i]) for r in runs[1:])
              for i, name in enumerate(names)}
    print("[atomic run-to-run max rel diff]", {k: f"{v:.1e}" for k, v in spread.items()},
          flush=True)
    assert spread["dx"] == 0.0 and spread["ddt"] == 0.0
    assert max(spread.values()) <= RED_TOL


@pytest.mark.parametrize("npl,n", [(2, 16), (4, 16), (2, 7), (4, 7), (4, 24), (2, 32),
                                   (1, 16), (1, 13), (1, 8), (1, 3)])
def test_every_state_split_agrees(npl, n):
    """Forcing 1, 2 or 4 states per lane (other block shapes, other padding
    of d_state; one state per lane runs 8-wave blocks at d_state 9..16 and
    4-wave blocks up to 8) gives the same results."""
    bt, t_len, d = 2, 100, 130
    print(f"[case] npl {npl} d_state {n}", flush=True)
    arrs = oracle.make_inputs(bt, t_len, d, n, seed=31, style="bench")
    dy = np.random.default_rng(2).standard_normal((bt, t_len, d), dtype=np.float32)
    y_ref, _, _ = oracle.scan_fwd(*arrs)
    grads_ref = oracle.scan_bwd(*arrs, dy)
    try:
        _native.set_variant(npl)
        y, _, grads = _run_hip(_to_dev(arrs), torch.from_numpy(dy).to(DEV))
    finally:
        _native.set_variant(0)
    assert_close("y", y, y_ref)
    for name, g, r in zip(("dx", "ddt", "dAneg", "dB", "dC"), grads, grads_ref):
        assert_close(name, g, r)


def test_gradients_match_finite_differences():
    """Central differences of the kernel's own forward (tests/test_scan.py:133-161)."""
    bt, t_len, d, n = 1, 24, 12, 8
    arrs = oracle.make_inputs(bt, t_len, d, n, seed=1337 + 11, style="ref")
    inp = _to_dev(arrs)
    dy = torch.from_numpy(np.random.default_rng(4).standard_normal(
        (bt, t_len, d), dtype=np.float32)).to(DEV)
    _, _, grads = _run_hip(inp, dy)

    def f(i, j, v):
        p = [t.clone() for t in inp]
        p[i].view(-1)[j] = v
        return (selective_scan_hip(*p).double() * dy.double()).sum().item()

    rng = np.random.default_rng(1337)
    worst = 0.0
    for i, t in enumerate(inp):
        flat = t.reshape(-1)
        for j in rng.permutation(flat.numel())[:6].tolist():
            v = flat[j].item()
            h = 1e-2 * max(1.0, abs(v))
            num = (f(i, j, v + h) - f(i, j, v - h)) / (2 * h)
            ana = grads[i].reshape(-1)[j].item()
            worst = max(worst, abs(num - ana) / max(1.0, abs(num), abs(ana)))
    assert worst < 0.05, f"finite-difference mismatch {worst:.3f}"


def test_dispatch_on_device():
    arrs = oracle.make_inputs(1, 8, 16, 4, seed=1, style="ref")
    inp = _to_dev(arrs)
    y = selective_scan(*inp, impl="auto")
    assert y is not None and y.is_cuda
    y2 = selective_scan(*inp, impl="metal")
    assert torch.equal(y, y2)
    with pytest.raises(RuntimeError, match="fp32"):
        selective_scan(*[t.double() for t in inp], impl="hip")
    with pytest.raises(RuntimeError, match="ROCm device"):
        selective_scan(inp[0], inp[1], inp[2].cpu(), inp[3], inp[4], impl="hip")


def test_empty_sequence():
    x = torch.zeros(2, 0, 8, device=DEV)
    aneg = torch.ones(8, 4, device=DEV)
    b = torch.zeros(2, 0, 4, device=DEV)
    y, h = selective_scan_hip(x, x, aneg, b, b, return_state=True)
    assert y.shape == (2, 0, 8) and h.shape == (2, 8, 4)
    assert torch.count_nonzero(h) == 0


# (B, T, D, N, chunk, segments): the chunk-parallel-over-time backward, forced
# on small shapes (the automatic choice uses it only for grids under two
# blocks per CU): segment counts above the chunk count, uneven last segments,
# chunk strides off the 16-step window, the fine-checkpoint recompute path and
# the state gradient entering the last segment.
# Stride 32 is swept inside the backward kernel, from the caller's
# checkpoints, also in segments that start inside a caller chunk; other
# strides above 16 first recompute stride-16 checkpoints, in segments that
# start on the caller's checkpoints (lcm(16, chunk) steps).
SEGMENT_CASES = [(2, 100, 64, 16, 16, 2), (1, 300, 96, 16, 16, 3), (2, 257, 40, 8, 7, 5),
                 (1, 64, 64, 16, 16, 8), (3, 200, 130, 5, 64, 3), (1, 20, 32, 16, 16, 4),
                 (2, 513, 64, 32, 16, 8), (1, 1000, 64, 16, 48, 4), (2, 777, 96, 16, 20, 6),
                 (1, 2048, 64, 16, 64, 0)]


def _run_hip_split(inp, dy, chunk, fwd_segs, bwd_segs):
    """_run_hip with the forced time-segment count set separately for the
    forward and the backward launch (the count is process-wide)."""
    leaves = [t.clone().requires_grad_(True) for t in inp]
    try:
        _native.set_time_segments(fwd_segs)
        y, h_last = selective_scan_hip(*leaves, return_state=True, chunk=chunk)
        _native.set_time_segments(bwd_segs)
        grads = torch.autograd.grad([y], leaves, grad_outputs=[dy])
        torch.cuda.synchronize()
    finally:
        _native.set_time_segments(0)
    return y.detach(), h_last.detach(), grads


@pytest.mark.parametrize("segs", [1, 3, 5])
def test_strides_32_48_64_equal_stride_16_bit_for_bit(segs):
    """The backward at strides 32 (swept), 48 and 64 (stride-16 checkpoints
    recomputed) keeps the stride-16 time segments; with 3 or 5 of them over
    1000 steps (63 chunks of 16) some segments start inside a caller chunk,
    and the last caller chunk is partial. With the forward unsegmented (every checkpoint a sequential
    state) every gradient equals stride 16's bit for bit (fixed order).
    A segmented forward starts each segment from its combined carry, and
    stride 16 then checkpoints states that derive from it where a sweep
    rebuilds them from the caller's checkpoint before the segment: equal to
    fp32 rounding, not bit for bit (the oracle tests cover that case)."""
    bt, t_len, d, n = 2, 1000, 96, 16
    arrs = oracle.make_inputs(bt, t_len, d, n, seed=4242, style="bench")
    dy = torch.from_numpy(np.random.default_rng(43).standard_normal((bt, t_len, d),
                                                                     dtype=np.float32)).to(DEV)
    with reduction(_native.REDUCTION_FIXED):
        base = _run_hip_split(_to_dev(arrs), dy, 16, 1, segs)
        for chunk in (32, 48, 64):
            print(f"[case] stride {chunk} vs 16, {segs} backward segments", flush=True)
            other = _run_hip_split(_to_dev(arrs), dy, chunk, 1, segs)
            assert torch.equal(base[0], other[0]) and torch.equal(base[1], other[1])
            for name, a, b in zip(("dx", "ddt", "dAneg", "dB", "dC"), base[2], other[2]):
                assert torch.equal(a, b), f"chunk {chunk}, {segs} segments: {name}"


@pytest.mark.parametrize("mode", ["auto", "fixed"])
@pytest.mark.parametrize("bt,t_len,d,n,chunk,segs", SEGMENT_CASES)
def test_time_segments_match_the_oracle(bt, t_len, d, n, chunk, segs, mode):
    """Split backwards reduce with atomics under the automatic choice; the
    fixed order is forced as well."""
    print(f"[case] time segments {segs}: {bt}x{t_len}x{d}x{n} chunk {chunk} {mode}", flush=True)
    arrs = oracle.make_inputs(bt, t_len, d, n, seed=77 + d, style="bench")
    rng = np.random.default_rng(78)
    dy = rng.standard_normal((bt, t_len, d), dtype=np.float32)
    dh = rng.standard_normal((bt, d, n), dtype=np.float32)
    y_ref, _, h_ref = oracle.scan_fwd(*arrs)
    g_ref = oracle.scan_bwd(*arrs, dy, dh_last=dh)
    _native.set_time_segments(segs)
    try:
        with reduction(_native.REDUCTION_FIXED if mode == "fixed" else _native.REDUCTION_AUTO):
            y, h_last, grads = _run_hip(_to_dev(arrs), torch.from_numpy(dy).to(DEV), chunk=chunk,
                                        dh_last=torch.from_numpy(dh).to(DEV))
            _, ckpt, _ = torch.ops.mamba_hip.scan_fwd(*_to_dev(arrs), chunk, True)
            torch.cuda.synchronize()
    finally:
        _native.set_time_segments(0)
    assert_close("y", y, y_ref)
    assert_close("h_last", h_last, h_ref)
    assert_close("ckpt", ckpt, oracle.scan_fwd(*arrs, chunk=chunk)[1])
    for name, g, r in zip(("dx", "ddt", "dAneg", "dB", "dC"), grads, g_ref):
        assert_close(name, g, r)


# One state per lane (d_state <= 16) under forced time segments: the carry
# passes, the segmented gradient pass and both reductions with 8-wave blocks
# (d_state 9..16) and 4-wave blocks (d_state <= 8).
NPL1_SEGMENT_CASES = [(2, 100, 64, 16, 16, 2), (1, 300, 96, 8, 16, 3), (2, 257, 40, 13, 7, 5),
                      (1, 1000, 64, 16, 48, 4), (3, 200, 130, 5, 64, 1)]


@pytest.mark.parametrize("mode", ["auto", "fixed"])
@pytest.mark.parametrize("bt,t_len,d,n,chunk,segs", NPL1_SEGMENT_CASES)
def test_one_state_per_lane_matches_the_oracle(bt, t_len, d, n, chunk, segs, mode):
    print(f"[case] one state per lane, {segs} segments: {bt}x{t_len}x{d}x{n} chunk {chunk} "
          f"{mode}", flush=True)
    arrs = oracle.make_inputs(bt, t_len, d, n, seed=177 + d, style="bench")
    rng = np.random.default_rng(79)
    dy = rng.standard_normal((bt, t_len, d), dtype=np.float32)
    dh = rng.standard_normal((bt, d, n), dtype=np.float32)
    y_ref, _, h_ref = oracle.scan_fwd(*arrs)
    g_ref = oracle.scan_bwd(*arrs, dy, dh_last=dh)
    _native.set_variant(1)
    _native.set_time_segments(segs)
    try:
        with reduction(_native.REDUCTION_FIXED if mode == "fixed" else _native.REDUCTION_ATOMIC):
            y, h_last, grads = _run_hip(_to_dev(arrs), torch.from_numpy(dy).to(DEV), chunk=chunk,
                                        dh_last=torch.from_numpy(dh).to(DEV))
            _, ckpt, _ = torch.ops.mamba_hip.scan_fwd(*_to_dev(arrs), chunk, True)
            torch.cuda.synchronize()
    finally:
        _native.set_time_segments(0)
        _native.set_variant(0)
    assert_close("y", y, y_ref)
    assert_close("h_last", h_last, h_ref)
    assert_close("ckpt", ckpt, oracle.scan_fwd(*arrs, chunk=chunk)[1])
    for name, g, r in zip(("dx", "ddt", "dAneg", "dB", "dC"), grads, g_ref):
        assert_close(name, g, r)


def test_time_segments_auto_split_at_the_long_sequence_shape():
    """4 x 16384 x 2048 x 16 (256 blocks): the automatic split (2 forward
    segments, 3 backward segments with the atomic reduction) against the
    single-segment passes (fixed-order reduction) on the same inputs."""
    bt, t_len, d, n = 4, 16384, 2048, 16
    print(f"[case] auto time segments {bt}x{t_len}x{d}x{n}", flush=True)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(bt, t_len, d, generator=g).to(DEV)
    dt = torch.nn.functional.softplus(torch.randn(bt, t_len, d, generator=g) - 4.0).to(DEV)
    aneg = torch.arange(1, n + 1, dtype=torch.float32).repeat(d, 1).to(DEV)
    b_in = torch.randn(bt, t_len, n, generator=g).to(DEV)
    c_in = torch.randn(bt, t_len, n, generator=g).to(DEV)
    dy = torch.randn(bt, t_len, d, generator=g).to(DEV)
    fwd_auto = torch.ops.mamba_hip.scan_fwd(x, dt, aneg, b_in, c_in, 16, True)
    auto = torch.ops.mamba_hip.scan_bwd(x, dt, aneg, b_in, c_in, dy, None, fwd_auto[1], 16)
    _native.set_time_segments(1)
    try:
        fwd_one = torch.ops.mamba_hip.scan_fwd(x, dt, aneg, b_in, c_in, 16, True)
        one = torch.ops.mamba_hip.scan_bwd(x, dt, aneg, b_in, c_in, dy, None, fwd_one[1], 16)
    finally:
        _native.set_time_segments(0)
    torch.cuda.synchronize()
    for name, a_, b_ in zip(("y", "ckpt", "h_last"), fwd_auto, fwd_one):
        assert_close(name, a_, b_)
    for name, a_, b_ in zip(("dx", "ddt", "dAneg", "dB", "dC"), auto, one):
        assert_close(name, a_, b_)
