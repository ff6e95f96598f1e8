"""The committed golden vectors (tests/golden/scan_golden.npz, written by
tests/golden/make_golden.py) against the float64 oracle on the CPU, and
against the HIP kernels on the GPU (through the autograd path, chunk stride
and returned-state gradient included)."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import assert_close
from oracle import oracle

GOLDEN = Path(__file__).resolve().parent / "golden" / "scan_golden.npz"
OUTS = ("y", "ckpt", "h_last", "dx", "ddt", "daneg", "dB", "dC")


def _cases():
    with np.load(GOLDEN, allow_pickle=False) as z:
        data = {k: z[k] for k in z.files}
    names = sorted({k.split("/")[0] for k in data})
    return {n: {k.split("/")[1]: v for k, v in data.items() if k.startswith(n + "/")}
            for n in names}


CASES = _cases()


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_reproduces_the_golden_vectors(name):
    c = CASES[name]
    ins = [c[k] for k in ("x", "dt", "aneg", "B", "C")]
    y, ckpt, h_last = oracle.scan_fwd(*ins, chunk=int(c["chunk"]))
    grads = oracle.scan_bwd(*ins, c["dy"], dh_last=c["dh_last"])
    for k, v in zip(OUTS, (y, ckpt, h_last) + tuple(grads)):
        np.testing.assert_allclose(v, c[k], rtol=1e-12, atol=1e-14, err_msg=f"{name}/{k}")


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_hip_matches_the_golden_vectors(name):
    from mamba_metal_scan_amd import selective_scan_hip
    c = CASES[name]
    chunk = int(c["chunk"])
    print(f"[case] golden {name} shape {c['x'].shape} d_state {c['aneg'].shape[1]} "
          f"chunk {chunk}", flush=True)
    leaves = [torch.from_numpy(c[k]).cuda().requires_grad_(True)
              for k in ("x", "dt", "aneg", "B", "C")]
    y, h_last = selective_scan_hip(*leaves, chunk=chunk, return_state=True)
    grads = torch.autograd.grad([y, h_last], leaves,
                                grad_outputs=[torch.from_numpy(c["dy"]).cuda(),
                                              torch.from_numpy(c["dh_last"]).cuda()])
    _, ckpt, _ = torch.ops.mamba_hip.scan_fwd(*(t.detach() for t in leaves), chunk, True)
    torch.cuda.synchronize()
    got = dict(zip(OUTS, (y, ckpt, h_last) + tuple(grads)))
    for k in OUTS:
        assert_close(f"{name}/{k}", got[k], c[k])
