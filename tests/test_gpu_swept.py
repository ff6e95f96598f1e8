"""GPU parity of the backward at checkpoint strides 32, 48 and 64 against
the float64 oracle, through the public autograd path, with the final-state
gradient: stride 32 (or a sequence of 17..32 steps at a longer stride) by the
in-kernel sweep (the states between the caller's checkpoints rebuilt inside
the backward kernel), 48 and 64 by the recompute pass of stride-16
checkpoints.

Cases cover every plan the sweep is instantiated for (two states per lane;
four, d_state above 32; one, d_state 8), the gated kernels with the dt
projection's bias, bf16 activations, a d_state and d_inner off the tile
sizes, sequences shorter than one caller chunk or ending in a partial one,
and forced time segments (which then start inside a caller chunk) under
both reductions.

Bar, per tensor (max|got - ref| / max|ref|): 1e-4 for fp32 outputs; 4e-3
for bf16 outputs, whose round-to-nearest-even storage alone costs up to
2^-9 relative.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close, reduction
from mamba_metal_scan_amd import _native, selective_scan, selective_scan_gated
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
LO, HI = 0.001, 0.1
TOL_F32, TOL_BF16 = 1e-4, 4e-3
AUTO, FIXED, ATOMIC = _native.REDUCTION_AUTO, _native.REDUCTION_FIXED, _native.REDUCTION_ATOMIC

# (batch, T, d_inner, d_state, chunk, gated, bf16, forced segments, reduction)
CASES = [
    (2, 200, 96, 16, 32, False, False, 0, AUTO),
    (2, 173, 70, 16, 48, True, False, 0, AUTO),      # T off 16, gated with dt bias
    (1, 300, 64, 40, 64, False, False, 0, AUTO),     # four states per lane
    (3, 150, 33, 8, 64, True, False, 0, AUTO),       # one state per lane, d_inner off 32
    (2, 100, 96, 5, 48, False, False, 3, FIXED),     # odd d_state, segments inside chunks
    (1, 64, 32, 16, 64, True, False, 0, AUTO),       # one caller chunk, T == chunk
    (2, 40, 32, 16, 32, False, False, 0, AUTO),      # last caller chunk of 8 steps
    (1, 32, 32, 16, 64, False, False, 0, AUTO),      # T == 32 < chunk: stride 32 swept
    (2, 130, 70, 16, 64, False, True, 0, AUTO),      # bf16
    (1, 300, 64, 16, 48, True, True, 3, AUTO),       # bf16, gated, segments (atomics)
    (1, 777, 96, 16, 64, False, False, 5, ATOMIC),
    (2, 257, 64, 16, 32, True, False, 4, FIXED),
]


def _bf16_round(a: np.ndarray) -> np.ndarray:
    """a rounded to bf16 (nearest even) and widened back to float64."""
    return torch.from_numpy(a).to(torch.bfloat16).to(torch.float64).numpy()


@pytest.mark.parametrize("bt,t_len,d,n,chunk,gated,bf16,segs,mode", CASES)
def test_swept_backward_matches_the_oracle(bt, t_len, d, n, chunk, gated, bf16, segs, mode):
    print(f"[case] swept {bt}x{t_len}x{d}x{n} chunk {chunk} gated {gated} bf16 {bf16} "
          f"segments {segs} reduction {mode}", flush=True)
    # The swept kernel runs at an effective stride of 32: no fine
    # checkpoints in the workspace; a longer one that is not swept
    # recomputes stride-16 checkpoints into it.
    ws = _native.library().mhs_scan_bwd_workspace_bytes
    if min(chunk, t_len) == 32:
        assert ws(bt, t_len, d, n, chunk) == ws(bt, t_len, d, n, 16)
    else:
        assert ws(bt, t_len, d, n, chunk) > ws(bt, t_len, d, n, 16)
    rng = np.random.default_rng(31 * t_len + d + n)
    dy = rng.standard_normal((bt, t_len, d), dtype=np.float32)
    dh = rng.standard_normal((bt, d, n), dtype=np.float32)
    if gated:
        x = rng.standard_normal((bt, t_len, d), dtype=np.float32)
        raw = (2.0 * rng.standard_normal((bt, t_len, d))).astype(np.float32)
        a = (np.tile(np.arange(1, n + 1, dtype=np.float32), (d, 1))
             + 0.3 * rng.standard_normal((d, n))).astype(np.float32)
        b_in = rng.standard_normal((bt, t_len, n), dtype=np.float32)
        c_in = rng.standard_normal((bt, t_len, n), dtype=np.float32)
        bias = (0.5 * rng.standard_normal(d)).astype(np.float32)
        acts, params = [x, raw, b_in, c_in], [a]
    else:
        x, dt, aneg, b_in, c_in = oracle.make_inputs(bt, t_len, d, n, seed=t_len + d,
                                                     style="bench")
        acts, params = [x, dt, b_in, c_in], [aneg]
    # The oracle sees exactly the values the kernels read.
    ref_acts = [_bf16_round(v) if bf16 else v.astype(np.float64) for v in acts]
    dy_ref = _bf16_round(dy) if bf16 else dy
    ref_in = [ref_acts[0], ref_acts[1], params[0], ref_acts[2], ref_acts[3]]
    if gated:
        ref_in[1] = ref_in[1] + bias.astype(np.float64)
        y_ref, _, h_ref = oracle.scan_gated_fwd(*ref_in, LO, HI)
        g_ref = list(oracle.scan_gated_bwd(*ref_in, LO, HI, dy_ref, dh_last=dh))
        g_ref.append(np.asarray(g_ref[1]).sum(axis=(0, 1)))
        names = ["dx", "ddt_raw", "dA", "dB", "dC", "dbias"]
    else:
        y_ref, _, h_ref = oracle.scan_fwd(*ref_in)
        g_ref = list(oracle.scan_bwd(*ref_in, dy_ref, dh_last=dh))
        names = ["dx", "ddt", "dAneg", "dB", "dC"]

    dt_act = torch.bfloat16 if bf16 else torch.float32
    dev_acts = [torch.from_numpy(v).to(DEV).to(dt_act) for v in acts]
    leaves = [dev_acts[0], dev_acts[1], torch.from_numpy(params[0]).to(DEV), dev_acts[2],
              dev_acts[3]]
    if gated:
        leaves.append(torch.from_numpy(bias).to(DEV))
    leaves = [t.requires_grad_(True) for t in leaves]
    _native.set_time_segments(segs)
    try:
        with reduction(mode):
            if gated:
                y, h_last = selective_scan_gated(*leaves[:5], LO, HI, chunk=chunk,
                                                 return_state=True, dt_bias=leaves[5])
            else:
                y, h_last = selective_scan(*leaves, impl="hip", chunk=chunk, return_state=True)
            grads = torch.autograd.grad(
                [y, h_last], leaves,
                [torch.from_numpy(dy).to(DEV).to(dt_act), torch.from_numpy(dh).to(DEV)])
            torch.cuda.synchronize()
    finally:
        _native.set_time_segments(0)
    assert y.dtype == dt_act and h_last.dtype == torch.float32
    tol_act = TOL_BF16 if bf16 else TOL_F32
    assert_close("y", y, y_ref, tol_act)
    assert_close("h_last", h_last, h_ref, TOL_F32)
    for name, g, r in zip(names, grads, g_ref):
        assert g.shape == np.asarray(r).shape, name
        fp32_out = name in ("dAneg", "dA", "dbias")
        assert_close(name, g, r, TOL_F32 if fp32_out else tol_act)
