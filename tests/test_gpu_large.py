"""The HIP scan at the long-sequence size 4 x 16384 x 2048 x 16, where the
float64 oracle cannot run on the whole problem:

* channels are independent in y, dx and ddt, and dAneg[d] only needs channel
  d: the oracle runs on a few channel slices of the full-length problem;
* dB and dC are sums over all channels: for one batch row the oracle runs on
  all 2048 channels (in channel slices on host threads, their dB, dC added);
* dC = sum_d dy * h, with every state h taken from the forward's own
  checkpoints at stride 1 (8.6 GB on the device);
* dB is linear in dy;
* the checkpoint stride is not a result: strides 16, 32, 64 and 128 (the
  last three recompute fine checkpoints inside the backward) give
  bit-identical outputs with the fixed-order reduction.

And the prefill of the inference configuration, 32 x 2048 x 4096 x 16 with
the final state, against the oracle on channel slices.
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from helpers import assert_close, reduction
from mamba_metal_scan_amd import _native
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
BT, T, D, N = 4, 16384, 2048, 16
CHANNELS = [0, 1027, 2047]


@pytest.fixture(scope="module")
def problem():
    print(f"[case] long sequence {BT}x{T}x{D}x{N}", flush=True)
    g = torch.Generator().manual_seed(2024)
    x = torch.randn(BT, T, D, generator=g)
    dt = torch.nn.functional.softplus(torch.randn(BT, T, D, generator=g) - 4.0)
    aneg = torch.arange(1, N + 1, dtype=torch.float32).repeat(D, 1)
    b_in = torch.randn(BT, T, N, generator=g)
    c_in = torch.randn(BT, T, N, generator=g)
    dy = torch.randn(BT, T, D, generator=g)
    return [t.to(DEV) for t in (x, dt, aneg, b_in, c_in, dy)]


def _fwd_bwd(p, chunk, dy=None):
    x, dt, aneg, b_in, c_in, dy0 = p
    y, ckpt, h_last = torch.ops.mamba_hip.scan_fwd(x, dt, aneg, b_in, c_in, chunk, True)
    grads = torch.ops.mamba_hip.scan_bwd(x, dt, aneg, b_in, c_in, dy0 if dy is None else dy,
                                         None, ckpt, chunk)
    torch.cuda.synchronize()
    return y, h_last, grads


def test_channel_slices_match_the_oracle(problem):
    x, dt, aneg, b_in, c_in, dy = problem
    y, h_last, (dx, ddt, daneg, _, _) = _fwd_bwd(problem, 16)
    sel = torch.tensor(CHANNELS, device=DEV)
    xs, dts = (t.index_select(2, sel).cpu().numpy() for t in (x, dt))
    an = aneg.index_select(0, sel).cpu().numpy()
    bs, cs = b_in.cpu().numpy(), c_in.cpu().numpy()
    dys = dy.index_select(2, sel).cpu().numpy()
    y_ref, _, h_ref = oracle.scan_fwd(xs, dts, an, bs, cs)
    g_ref = oracle.scan_bwd(xs, dts, an, bs, cs, dys)
    assert_close("y", y.index_select(2, sel), y_ref)
    assert_close("h_last", h_last.index_select(1, sel), h_ref)
    assert_close("dx", dx.index_select(2, sel), g_ref[0])
    assert_close("ddt", ddt.index_select(2, sel), g_ref[1])
    assert_close("dAneg", daneg.index_select(0, sel), g_ref[2])


def test_dc_is_dy_times_every_state(problem):
    x, dt, aneg, b_in, c_in, dy = problem
    _, _, (_, _, _, _, dc) = _fwd_bwd(problem, 16)
    ref = torch.zeros(BT, T, N, device=DEV, dtype=torch.float64)
    for b in range(BT):
        _, h_all, _ = torch.ops.mamba_hip.scan_fwd(x[b:b + 1], dt[b:b + 1], aneg, b_in[b:b + 1],
                                                   c_in[b:b + 1], 1, True)   # (1, T, D, N)
        ref[b] = torch.bmm(dy[b].unsqueeze(1), h_all[0]).squeeze(1).double()
        del h_all
    assert_close("dC", dc, ref)


def test_db_is_linear_in_dy(problem):
    dy = problem[5]
    dy2 = torch.randn(dy.shape, device=DEV, generator=torch.Generator(DEV).manual_seed(5))
    db1 = _fwd_bwd(problem, 16, dy)[2][3]
    db2 = _fwd_bwd(problem, 16, dy2)[2][3]
    db12 = _fwd_bwd(problem, 16, dy + 0.5 * dy2)[2][3]
    assert_close("dB", db12, db1 + 0.5 * db2)


def test_checkpoint_stride_is_not_a_result(problem):
    """Bit for bit across strides, although the forward runs in two time
    segments here: over its 2048-step carry units the state carried in from
    before a unit decays below fp32 rounding, so the second segment's
    combined start state equals the sequential one exactly (with short units
    they agree to rounding only)."""
    with reduction(_native.REDUCTION_FIXED):
        base = _fwd_bwd(problem, 16)
        for chunk in (32, 64, 128):
            print(f"[case] long sequence chunk {chunk} vs 16", flush=True)
            other = _fwd_bwd(problem, chunk)
            assert torch.equal(base[0], other[0]) and torch.equal(base[1], other[1])
            for name, a, b in zip(("dx", "ddt", "dAneg", "dB", "dC"), base[2], other[2]):
                assert torch.equal(a, b), f"chunk {chunk}: {name}"


def _oracle_bwd_all_channels(xs, dts, an, bs, cs, dys, parts=8):
    """The float64 oracle's gradients over every channel, run on `parts`
    channel slices in host threads (the C oracle releases the GIL); dB and dC,
    sums over the channels, are the sums of the slices'."""
    bounds = np.linspace(0, xs.shape[2], parts + 1).astype(int)

    def one(i):
        sl = slice(bounds[i], bounds[i + 1])
        return oracle.scan_bwd(xs[:, :, sl], dts[:, :, sl], an[sl], bs, cs, dys[:, :, sl])

    with ThreadPoolExecutor(parts) as pool:
        res = list(pool.map(one, range(parts)))
    dx = np.concatenate([r[0] for r in res], axis=2)
    ddt = np.concatenate([r[1] for r in res], axis=2)
    daneg = np.concatenate([r[2] for r in res], axis=0)
    return dx, ddt, daneg, sum(r[3] for r in res), sum(r[4] for r in res)


def test_db_dc_of_one_batch_row_match_the_oracle(problem):
    """Batch row 0 on its own (1 x 16384 x 2048 x 16, the automatic time
    segments and the atomic reduction): all five gradients against the
    float64 oracle over every channel."""
    x, dt, aneg, b_in, c_in, dy = problem
    row = [t[:1].contiguous() for t in (x, dt)] + [aneg] + \
        [t[:1].contiguous() for t in (b_in, c_in, dy)]
    print("[case] long sequence batch row 0, all channels, vs oracle", flush=True)
    y, ckpt, _ = torch.ops.mamba_hip.scan_fwd(*row[:5], 16, True)
    grads = torch.ops.mamba_hip.scan_bwd(*row[:5], row[5], None, ckpt, 16)
    torch.cuda.synchronize()
    ref = _oracle_bwd_all_channels(*(t.cpu().numpy() for t in row))
    for name, g, r in zip(("dx", "ddt", "dAneg", "dB", "dC"), grads, ref):
        assert_close(name, g, r)


INF_BT, INF_T, INF_D = 32, 2048, 4096
INF_CHANNELS = [0, 2049, 4095]


def test_prefill_channel_slices_match_the_oracle():
    """Prefill 32 x 2048 x 4096 x 16 (forward with the final state, as the
    inference workload runs it): y and h_last on channel slices of the
    full-length problem against the float64 oracle."""
    print(f"[case] prefill {INF_BT}x{INF_T}x{INF_D}x{N}", flush=True)
    g = torch.Generator().manual_seed(77)
    x = torch.randn(INF_BT, INF_T, INF_D, generator=g)
    dt = torch.nn.functional.softplus(torch.randn(INF_BT, INF_T, INF_D, generator=g) - 4.0)
    aneg = torch.arange(1, N + 1, dtype=torch.float32).repeat(INF_D, 1)
    b_in = torch.randn(INF_BT, INF_T, N, generator=g)
    c_in = torch.randn(INF_BT, INF_T, N, generator=g)
    dev = [t.to(DEV) for t in (x, dt, aneg, b_in, c_in)]
    y, _, h_last = torch.ops.mamba_hip.scan_fwd(*dev, INF_T, False)
    torch.cuda.synchronize()
    sel = torch.tensor(INF_CHANNELS)
    y_ref, _, h_ref = oracle.scan_fwd(x.index_select(2, sel).numpy(),
                                      dt.index_select(2, sel).numpy(),
                                      aneg.index_select(0, sel).numpy(), b_in.numpy(),
                                      c_in.numpy())
    sel_d = sel.to(DEV)
    assert_close("y", y.index_select(2, sel_d), y_ref)
    assert_close("h_last", h_last.index_select(1, sel_d), h_ref)
