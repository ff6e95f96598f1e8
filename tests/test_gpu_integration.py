"""INTEGRATION.md section 2 -- the ctypes binding a maintainer would add to
the reference (its SelectiveScanMetal with the two Metal launches replaced by
mhs_scan_fwd_f32 and mhs_scan_bwd_f32) -- executed exactly as the document
shows it, against the float64 oracle (the reference's kernel gate,
tests/test_scan.py:98-130, and its stride cases, :213-221).
"""
from __future__ import annotations

import os
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import assert_close
from mamba_metal_scan_amd import _native
from oracle import oracle

DOC = Path(__file__).resolve().parents[1] / "INTEGRATION.md"


def binding_namespace() -> dict:
    """Run the document's section-2 code block, unchanged, with the library
    path in MHS_LIB (the block's own way to find it); returns its globals."""
    section = DOC.read_text().split("## 2.", 1)[1].split("\n## 3.", 1)[0]
    code = section.split("```python\n", 1)[1].split("```", 1)[0]
    os.environ["MHS_LIB"] = str(_native.LIB_PATH)
    ns: dict = {"__name__": "integration_binding"}
    exec(compile(code, f"{DOC.name}#2", "exec"), ns)
    return ns


def test_binding_block_loads_the_library():
    """CPU hosts too: the block runs, binds the two entry points and defines
    the Function (no GPU call is made)."""
    ns = binding_namespace()
    assert issubclass(ns["SelectiveScanROCm"], torch.autograd.Function)
    assert ns["_hip"].mhs_scan_bwd_workspace_bytes(2, 128, 64, 16, 64) > 0


@pytest.mark.gpu
@pytest.mark.parametrize("shape,chunk", [((2, 128, 64, 16), 64), ((2, 64, 32, 16), 1),
                                         ((4, 63, 128, 16), 7), ((3, 512, 856, 16), 512),
                                         ((1, 100, 17, 16), 64)])
def test_binding_matches_the_oracle(shape, chunk):
    bt, t_len, d, n = shape
    print(f"[case] INTEGRATION binding {shape} chunk {chunk}", flush=True)
    fn = binding_namespace()["SelectiveScanROCm"]
    arrs = oracle.make_inputs(bt, t_len, d, n, seed=900 + d, style="ref")
    dy = np.random.default_rng(3).standard_normal((bt, t_len, d), dtype=np.float32)
    leaves = [torch.from_numpy(a).cuda().requires_grad_(True) for a in arrs]
    y = fn.apply(*leaves, chunk)
    grads = torch.autograd.grad(y, leaves, torch.from_numpy(dy).cuda())
    torch.cuda.synchronize()
    y_ref, _, _ = oracle.scan_fwd(*arrs)
    g_ref = oracle.scan_bwd(*arrs, dy)
    assert_close("y", y, y_ref)
    for name, g, r in zip(("dx", "ddt", "dAneg", "dB", "dC"), grads, g_ref):
        assert_close(name, g, r)
