"""The allocation-free forward, mhs_scan_fwd_noalloc_f32, through the C ABI.

It is mhs_scan_fwd_ws_f32 with the time segments' carries in the library's
static device scratch instead of a caller workspace. Both run the same
kernels, so their outputs must agree bit for bit (and therefore within the
1e-4 bar). Two calls in a row, the second on a smaller problem, check that
the scratch's leftover contents from the first call do not matter. The shapes
are small grids, which run in time segments and so use the scratch.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from helpers import assert_close
from mamba_metal_scan_amd import _native
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
MHS_EINVAL = 1

# (batch, T, d_inner, d_state, chunk): 48 and 16 blocks of 32 channels, far
# below two per compute unit, so both run in time segments.
CASES = [(1, 4096, 1536, 16, 16), (1, 1000, 512, 16, 64)]


def _inputs(bt, t_len, d, n, seed):
    arrs = oracle.make_inputs(bt, t_len, d, n, seed=seed, style="bench")
    return [torch.from_numpy(a).to(DEV) for a in arrs]


def _outputs(bt, t_len, d, n, chunk):
    ck = torch.full((bt, (t_len + chunk - 1) // chunk, d, n), float("nan"), device=DEV)
    return (torch.full((bt, t_len, d), float("nan"), device=DEV), ck,
            torch.full((bt, d, n), float("nan"), device=DEV))


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def test_noalloc_forward_matches_the_workspace_forward():
    lib = _native.library()
    for i, (bt, t_len, d, n, chunk) in enumerate(CASES):
        print(f"[case] noalloc forward {bt}x{t_len}x{d}x{n} chunk {chunk}", flush=True)
        need = lib.mhs_scan_fwd_workspace_bytes(bt, t_len, d, n)
        assert 0 < need <= _native.NOALLOC_SCRATCH_BYTES, need   # the scratch is used
        inp = _inputs(bt, t_len, d, n, seed=40 + i)
        ws = torch.empty(need, dtype=torch.uint8, device=DEV)
        ref = _outputs(bt, t_len, d, n, chunk)
        rc = lib.mhs_scan_fwd_ws_f32(*map(_p, inp), *map(_p, ref), _p(ws), need,
                                     bt, t_len, d, n, chunk, _stream())
        assert rc == 0, lib.mhs_last_error().decode()
        got = _outputs(bt, t_len, d, n, chunk)
        rc = lib.mhs_scan_fwd_noalloc_f32(*map(_p, inp), *map(_p, got),
                                          bt, t_len, d, n, chunk, _stream())
        assert rc == 0, lib.mhs_last_error().decode()
        torch.cuda.synchronize()
        for name, g, r in zip(("y", "ckpt", "h_last"), got, ref):
            assert not torch.isnan(g).any(), name
            assert_close(name, g, r)
            assert torch.equal(g, r), name
        # The workspace forward itself against the float64 oracle, on the
        # second (smaller) case.
        if i == 1:
            arrs = [t.cpu().numpy() for t in inp]
            y_ref, ck_ref, h_ref = oracle.scan_fwd(*arrs, chunk=chunk)
            for name, g, r in zip(("y", "ckpt", "h_last"), got, (y_ref, ck_ref, h_ref)):
                assert_close(name, g, r)


def test_noalloc_forward_rejects_shapes_beyond_its_scratch():
    """A forced split whose carries exceed the static scratch fails on the
    host, before any launch, with a message naming the way out."""
    lib = _native.library()
    bt, t_len, d, n = 16, 256, 16384, 16     # 8 segments, 7 carried: 7 x 16 x 16384 x 17 x 4 B > 16 MiB
    x = torch.zeros(16, device=DEV)
    try:
        _native.set_time_segments(8)
        need = lib.mhs_scan_fwd_workspace_bytes(bt, t_len, d, n)
        assert need > _native.NOALLOC_SCRATCH_BYTES
        rc = lib.mhs_scan_fwd_noalloc_f32(*([_p(x)] * 8), bt, t_len, d, n, 16, _stream())
    finally:
        _native.set_time_segments(0)
    assert rc == MHS_EINVAL
    assert "mhs_scan_fwd_ws_f32" in lib.mhs_last_error().decode()
