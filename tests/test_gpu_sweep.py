"""Seeded random sweep of the scan kernels against the float64 oracle.

Each case draws a shape (batch 1-4, T 1-300, d_inner 1-200, d_state 1-64),
a checkpoint stride 1-300, and whether the final state is returned with a
gradient, then runs either the plain scan (selective_scan(impl="hip")) or the
gated scan with the dt projection's bias (selective_scan_gated with dt_bias)
forward and backward. Both go through the public autograd path: plan
choice, time segments, fine-checkpoint recompute and the channel and step
tails all vary from case to case. Sizes stay small enough for the oracle.

Bar: per tensor, max|got - ref| / max|ref| <= 1e-4.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close
from mamba_metal_scan_amd import selective_scan, selective_scan_gated
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
LO, HI = 0.001, 0.1
NCASES = 40


def _case(i):
    rng = np.random.default_rng(9000 + i)
    bt = int(rng.integers(1, 5))
    t_len = int(rng.choice([int(rng.integers(1, 40)), int(rng.integers(40, 301))]))
    d = int(rng.integers(1, 201))
    n = int(rng.choice([int(rng.integers(1, 17)), 16, int(rng.integers(17, 65))]))
    chunk = int(rng.choice([16, int(rng.integers(1, 301))]))
    with_state = bool(rng.integers(0, 2))
    gated = bool(rng.integers(0, 2))
    return bt, t_len, d, n, chunk, with_state, gated


@pytest.mark.parametrize("i", range(NCASES))
def test_random_case_matches_the_oracle(i):
    bt, t_len, d, n, chunk, with_state, gated = _case(i)
    print(f"[case] sweep {i}: {bt}x{t_len}x{d}x{n} chunk {chunk} state {with_state} "
          f"gated {gated}", flush=True)
    rng = np.random.default_rng(500 + i)
    dy = rng.standard_normal((bt, t_len, d), dtype=np.float32)
    dh = rng.standard_normal((bt, d, n), dtype=np.float32) if with_state else None
    if gated:
        x = rng.standard_normal((bt, t_len, d), dtype=np.float32)
        raw = (2.0 * rng.standard_normal((bt, t_len, d))).astype(np.float32)
        a = (np.tile(np.arange(1, n + 1, dtype=np.float32), (d, 1))
             + 0.3 * rng.standard_normal((d, n))).astype(np.float32)
        b_in = rng.standard_normal((bt, t_len, n), dtype=np.float32)
        c_in = rng.standard_normal((bt, t_len, n), dtype=np.float32)
        bias = (0.5 * rng.standard_normal(d)).astype(np.float32)
        arrs = [x, raw, a, b_in, c_in]
        ref_in = [x, raw.astype(np.float64) + bias.astype(np.float64), a, b_in, c_in]
        y_ref, _, h_ref = oracle.scan_gated_fwd(*ref_in, LO, HI)
        g_ref = list(oracle.scan_gated_bwd(*ref_in, LO, HI, dy, dh_last=dh))
        g_ref.append(np.asarray(g_ref[1]).sum(axis=(0, 1)))
        names = ("dx", "ddt_raw", "dA", "dB", "dC", "dbias")
    else:
        arrs = oracle.make_inputs(bt, t_len, d, n, seed=700 + i, style="bench")
        y_ref, _, h_ref = oracle.scan_fwd(*arrs)
        g_ref = list(oracle.scan_bwd(*arrs, dy, dh))
        names = ("dx", "ddt", "dAneg", "dB", "dC")

    leaves = [torch.from_numpy(v).to(DEV).requires_grad_(True) for v in arrs]
    if gated:
        leaves.append(torch.from_numpy(bias).to(DEV).requires_grad_(True))
        y, h_last = selective_scan_gated(*leaves[:5], LO, HI, chunk=chunk, return_state=True,
                                         dt_bias=leaves[5])
    else:
        y, h_last = selective_scan(*leaves, impl="hip", chunk=chunk, return_state=True)
    outs, gouts = [y], [torch.from_numpy(dy).to(DEV)]
    if with_state:
        outs.append(h_last)
        gouts.append(torch.from_numpy(dh).to(DEV))
    grads = torch.autograd.grad(outs, leaves, gouts)
    torch.cuda.synchronize()
    assert_close("y", y, y_ref)
    assert_close("h_last", h_last, h_ref)
    for name, g, r in zip(names, grads, g_ref):
        assert g.shape == np.asarray(r).shape, name
        assert_close(name, g, r)
