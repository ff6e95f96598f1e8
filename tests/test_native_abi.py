"""The C-ABI library on the CPU: it loads, exports every symbol the header
declares, and rejects bad arguments with MHS_EINVAL and a message before any
HIP call is made (no GPU needed; no kernel is launched here).
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from mamba_metal_scan_amd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "mamba_hip_scan.h"
MHS_OK, MHS_EINVAL = 0, 1

# Fake device addresses: the calls below fail validation before any use. So
# that a regression in validation can never turn them into kernel launches on
# bogus pointers, the module runs only on hosts without a GPU.
pytestmark = pytest.mark.skipif(torch.cuda.is_available(),
                                reason="argument checks with fake device addresses: CPU hosts only")
A16 = ctypes.c_void_p(0x7F0000001000)     # 16-byte (and 256-byte) aligned
MIS = ctypes.c_void_p(0x7F0000001004)     # misaligned


def _declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(mhs_\w+)\s*\(", text)))


def _err(lib) -> str:
    return lib.mhs_last_error().decode()


def test_header_and_binding_agree():
    assert _declared_symbols() == sorted(_native.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = _native.library()
    for name in _declared_symbols():
        assert hasattr(lib, name), name
    assert lib.mhs_version() >> 16 == 0 and (lib.mhs_version() >> 8) & 0xFF >= 1


def test_chunk_arithmetic():
    lib = _native.library()
    assert lib.mhs_num_chunks(512, 16) == 32
    assert lib.mhs_num_chunks(512, 64) == 8
    assert lib.mhs_num_chunks(100, 7) == 15
    assert lib.mhs_num_chunks(1, 512) == 1
    assert lib.mhs_num_chunks(0, 16) == 0
    for n in (1, 5, 8, 16, 17, 32, 40, 64):
        assert lib.mhs_preferred_chunk(n) == 16
    assert lib.mhs_preferred_chunk(0) == 0
    assert lib.mhs_preferred_chunk(65) == 0


def test_workspace_size_formula():
    """Fixed-order reduction: dB/dC block partials (48 blocks of 32 channels)
    + dAneg batch partials + the gated dt-bias batch partials. Atomic
    reduction: only the fp32 dB/dC sums a bf16 backward rounds from. Either
    way + fine checkpoints when the stride exceeds the 16-step window and is
    not swept in the kernel (stride 32 is)."""
    lib = _native.library()
    nblk, s, a = 48, 16 * 512 * 16, 16 * 1536 * 16
    try:
        _native.set_reduction(_native.REDUCTION_FIXED)
        assert lib.mhs_deterministic() == 1
        base = 2 * nblk * s * 4 + a * 4 + 16 * 1536 * 4
        assert lib.mhs_scan_bwd_workspace_bytes(16, 512, 1536, 16, 16) == base
        assert lib.mhs_scan_bwd_workspace_bytes(16, 512, 1536, 16, 32) == base
        assert lib.mhs_scan_bwd_workspace_bytes(16, 512, 1536, 16, 64) == base + 32 * a * 4
        assert lib.mhs_scan_bwd_workspace_bytes(16, 512, 1536, 16, 128) == base + 32 * a * 4
        assert lib.mhs_scan_bwd_workspace_bytes(16, 512, 1536, 16, 40) == base + 32 * a * 4
        assert lib.mhs_scan_bwd_workspace_bytes(16, 512, 1536, 0, 16) == 0
        _native.set_reduction(_native.REDUCTION_ATOMIC)
        assert lib.mhs_deterministic() == 0
        assert lib.mhs_scan_bwd_workspace_bytes(16, 512, 1536, 16, 16) == 2 * s * 4
        assert lib.mhs_scan_bwd_workspace_bytes(16, 512, 1536, 16, 32) == 2 * s * 4
        assert lib.mhs_scan_bwd_workspace_bytes(16, 512, 1536, 16, 64) == 2 * s * 4 + 32 * a * 4
        assert lib.mhs_scan_bwd_workspace_bytes(16, 512, 1536, 16, 128) == 2 * s * 4 + 32 * a * 4
    finally:
        _native.set_reduction(_native.REDUCTION_AUTO)
    # automatic: per shape, so not bit for bit at every shape
    assert lib.mhs_deterministic() == 0
    with pytest.raises(_native.HipScanError, match="reduction mode"):
        _native.set_reduction(3)


def test_automatic_reduction_follows_the_time_segments():
    """Automatic: the fixed order where the backward runs in one time segment
    (16x512x1536x16: 768 blocks, three per CU), atomics where it runs in
    several (4x16384x2048x16: 256 blocks); forced modes hold at every shape,
    and the workspace follows the mode the shape gets."""
    lib = _native.library()
    one, several = (16, 512, 1536, 16, 16), (4, 16384, 2048, 16, 16)
    assert _native.bwd_reduction(*one) == _native.REDUCTION_FIXED
    assert _native.bwd_reduction(*several) == _native.REDUCTION_ATOMIC
    auto_ws = lib.mhs_scan_bwd_workspace_bytes(*several)
    try:
        for mode in (_native.REDUCTION_FIXED, _native.REDUCTION_ATOMIC):
            _native.set_reduction(mode)
            assert _native.bwd_reduction(*one) == mode
            assert _native.bwd_reduction(*several) == mode
            if mode == _native.REDUCTION_ATOMIC:
                assert lib.mhs_scan_bwd_workspace_bytes(*several) == auto_ws
            else:
                assert lib.mhs_scan_bwd_workspace_bytes(*several) > auto_ws
        # a forced split turns the automatic choice to atomics
        _native.set_reduction(_native.REDUCTION_AUTO)
        _native.set_time_segments(2)
        assert _native.bwd_reduction(*one) == _native.REDUCTION_ATOMIC
    finally:
        _native.set_time_segments(0)
        _native.set_reduction(_native.REDUCTION_AUTO)
    with pytest.raises(_native.HipScanError, match="d_state"):
        _native.bwd_reduction(16, 512, 1536, 0, 16)


def test_set_variant_rejects_unknown_splits():
    lib = _native.library()
    with pytest.raises(_native.HipScanError, match="states per lane"):
        _native.set_variant(3)
    assert lib.mhs_set_variant(8) == MHS_EINVAL
    assert lib.mhs_set_variant(0) == MHS_OK
    # With two states per lane, d_state above 32 has no plan; with one, d_state
    # above 16.
    try:
        _native.set_variant(2)
        assert lib.mhs_preferred_chunk(40) == 0
        _native.set_variant(1)
        assert lib.mhs_preferred_chunk(16) == 16
        assert lib.mhs_preferred_chunk(17) == 0
    finally:
        _native.set_variant(0)
    assert lib.mhs_preferred_chunk(40) == 16


def _fwd(lib, ptrs, sizes):
    return lib.mhs_scan_fwd_f32(*ptrs, *sizes, None)


def test_forward_argument_errors():
    lib = _native.library()
    good = [A16] * 8
    assert _fwd(lib, [None] + good[1:], (2, 8, 32, 16, 16)) == MHS_EINVAL
    assert "null" in _err(lib)
    assert _fwd(lib, [MIS] + good[1:], (2, 8, 32, 16, 16)) == MHS_EINVAL
    assert "16-byte aligned" in _err(lib)
    assert _fwd(lib, good, (2, 8, 32, 65, 16)) == MHS_EINVAL
    assert "d_state" in _err(lib)
    assert _fwd(lib, good, (0, 8, 32, 16, 16)) == MHS_EINVAL
    assert "positive" in _err(lib)
    assert _fwd(lib, good, (2, 8, 32, 16, 0)) == MHS_EINVAL
    assert "chunk" in _err(lib)
    assert _fwd(lib, good, (70000, 8, 32, 16, 16)) == MHS_EINVAL
    assert "batch" in _err(lib)
    assert _fwd(lib, good, (1, 8, 1 << 25, 16, 16)) == MHS_EINVAL
    assert "too large" in _err(lib)


def test_backward_argument_errors():
    lib = _native.library()
    sizes = (2, 8, 32, 16, 16)
    ptrs = [A16] * 13
    need = lib.mhs_scan_bwd_workspace_bytes(*sizes)
    assert need > 0
    rc = lib.mhs_scan_bwd_f32(*ptrs, A16, need - 4, *sizes, None)
    assert rc == MHS_EINVAL and "workspace too small" in _err(lib)
    rc = lib.mhs_scan_bwd_f32(*ptrs, MIS, need, *sizes, None)
    assert rc == MHS_EINVAL and "256-byte" in _err(lib)
    bad = list(ptrs)
    bad[7] = None       # ckpt
    rc = lib.mhs_scan_bwd_f32(*bad, A16, need, *sizes, None)
    assert rc == MHS_EINVAL and "null" in _err(lib)


def test_step_argument_errors():
    lib = _native.library()
    rc = lib.mhs_scan_step_f32(*([A16] * 6), None, 2, 32, 16, None)
    assert rc == MHS_EINVAL and "null" in _err(lib)
    rc = lib.mhs_scan_step_f32(*([A16] * 6), MIS, 2, 32, 16, None)
    assert rc == MHS_EINVAL and "aligned" in _err(lib)


def test_gated_scan_argument_errors():
    lib = _native.library()
    sizes = (2, 8, 32, 16, 16)
    outs = [A16] * 3 + [None, 0]          # y, ckpt, h_last; no workspace
    rc = lib.mhs_scan_gated_fwd_f32(*([A16] * 5), 0.1, 0.1, None, *outs, *sizes, 0, 0, None)
    assert rc == MHS_EINVAL and "dt_min < dt_max" in _err(lib)
    rc = lib.mhs_scan_gated_fwd_f32(*([A16] * 5), 0.001, float("nan"), None, *outs, *sizes, 0, 0, None)
    assert rc == MHS_EINVAL and "dt_min < dt_max" in _err(lib)
    rc = lib.mhs_scan_gated_fwd_f32(*([A16] * 5), 0.001, 0.1, None, *outs, 2, 8, 32, 65, 16, 0, 0, None)
    assert rc == MHS_EINVAL and "d_state" in _err(lib)
    # row strides below d_inner (dt) or d_state (B, C) are rejected
    rc = lib.mhs_scan_gated_fwd_f32(*([A16] * 5), 0.001, 0.1, None, *outs, *sizes, 31, 0, None)
    assert rc == MHS_EINVAL and "row strides" in _err(lib)
    rc = lib.mhs_scan_gated_fwd_f32(*([A16] * 5), 0.001, 0.1, None, *outs, *sizes, 64, 15, None)
    assert rc == MHS_EINVAL and "row strides" in _err(lib)
    need = lib.mhs_scan_bwd_workspace_bytes(*sizes)
    rc = lib.mhs_scan_gated_bwd_f32(*([A16] * 5), 0.001, 0.1, None, *([A16] * 8), None, A16, need - 4,
                                    *sizes, 0, 0, 0, 0, None)
    assert rc == MHS_EINVAL and "workspace too small" in _err(lib)
    rc = lib.mhs_scan_gated_bwd_f32(*([A16] * 5), 1.0, 0.5, None, *([A16] * 8), None, A16, need, *sizes,
                                    0, 0, 0, 0, None)
    assert rc == MHS_EINVAL and "dt_min < dt_max" in _err(lib)
    rc = lib.mhs_scan_gated_bwd_f32(*([A16] * 5), 0.001, 0.1, None, *([A16] * 8), None, A16, need, *sizes,
                                    0, 0, 0, 15, None)
    assert rc == MHS_EINVAL and "row strides" in _err(lib)


def test_out_gate_argument_errors():
    lib = _native.library()
    assert lib.mhs_out_gate_bwd_workspace_bytes(16, 512, 1432) == 8 * 16 * 1432 * 4
    rc = lib.mhs_out_gate_fwd_f32(A16, A16, A16, 31, A16, 2, 8, 32, None)
    assert rc == MHS_EINVAL and "row stride" in _err(lib)
    rc = lib.mhs_out_gate_fwd_f32(A16, None, A16, 64, A16, 2, 8, 32, None)
    assert rc == MHS_EINVAL and "null" in _err(lib)
    need = lib.mhs_out_gate_bwd_workspace_bytes(2, 8, 32)
    rc = lib.mhs_out_gate_bwd_f32(A16, A16, A16, 64, A16, A16, A16, 0, A16, A16, need - 4, 2, 8,
                                  32, None)
    assert rc == MHS_EINVAL and "workspace too small" in _err(lib)
    rc = lib.mhs_out_gate_bwd_f32(A16, A16, A16, 64, A16, A16, A16, 31, A16, A16, need, 2, 8, 32,
                                  None)
    assert rc == MHS_EINVAL and "dz row stride" in _err(lib)


def test_time_segments_knob_and_workspace():
    """Automatic split: one segment at 16x512x1536x16 (768 blocks), three at
    4x16384x2048x16 (256 blocks: 3 blocks per CU); forced splits add the
    per-segment dAneg and dt-bias partials and the carries of the carry
    units (L: units x batch x D x N, sum dt: units x batch x D). At
    4x16384x2048x16 each segment of 342 chunks splits into 2 carry units of
    171, so that the carry pass has 4 blocks per CU: 6 units over the 1024
    chunks."""
    lib = _native.library()
    with pytest.raises(_native.HipScanError, match="time segments"):
        _native.set_time_segments(9)
    assert lib.mhs_set_time_segments(-1) == MHS_EINVAL

    def ru(v):
        return (v + 255) // 256 * 256

    def expect(bt, t, d, n, segs, units, atomic):
        nblk = 1 if atomic else (d + 31) // 32
        s_ = bt * t * n
        a = bt * d * n
        base = 2 * ru(nblk * s_ * 4)
        if not atomic:
            base += ru(segs * a * 4) + ru(segs * bt * d * 4)
        if segs > 1:
            base += ru(units * a * 4) + ru(units * bt * d * 4)
        return base

    for mode, atomic in ((_native.REDUCTION_FIXED, False), (_native.REDUCTION_ATOMIC, True)):
        try:
            _native.set_reduction(mode)
            ws = lib.mhs_scan_bwd_workspace_bytes
            assert ws(16, 512, 1536, 16, 16) == expect(16, 512, 1536, 16, 1, 1, atomic)
            assert ws(4, 16384, 2048, 16, 16) == expect(4, 16384, 2048, 16, 3, 6, atomic)
            # 768 blocks: the carry pass (1536 blocks) needs no finer units
            _native.set_time_segments(3)
            assert ws(16, 512, 1536, 16, 16) == expect(16, 512, 1536, 16, 3, 3, atomic)
            # 5 chunks at most: 5 segments of one chunk, units of at least 2
            # chunks do not fit
            _native.set_time_segments(8)
            assert ws(1, 80, 64, 16, 16) == expect(1, 80, 64, 16, 5, 5, atomic)
        finally:
            _native.set_time_segments(0)
            _native.set_reduction(_native.REDUCTION_AUTO)


def test_forward_workspace():
    """The forward needs no workspace where the grid fills the GPU; below two
    blocks per CU it holds the carried states and dt sums of the carry units
    before the last segment."""
    lib = _native.library()
    assert lib.mhs_scan_fwd_workspace_bytes(16, 512, 1536, 16) == 0
    # 4 x 16384 x 2048 x 16: 256 blocks -> 2 segments (the forward plans for
    # two blocks per CU) of 512 sub-chunks, 4 carry units each (4 blocks per
    # CU in the carry pass): the 4 units of the first segment carried
    ru = lambda v: (v + 255) // 256 * 256
    assert lib.mhs_scan_fwd_workspace_bytes(4, 16384, 2048, 16) == \
        ru(4 * 4 * 2048 * 16 * 4) + ru(4 * 4 * 2048 * 4)
    sizes = (4, 16384, 2048, 16, 16)
    need = lib.mhs_scan_fwd_workspace_bytes(*sizes[:4])
    rc = lib.mhs_scan_fwd_ws_f32(*([A16] * 8), A16, need - 4, *sizes, None)
    assert rc == MHS_EINVAL and "workspace too small" in _err(lib)
    rc = lib.mhs_scan_fwd_ws_f32(*([A16] * 8), MIS, need, *sizes, None)
    assert rc == MHS_EINVAL and "256-byte" in _err(lib)


def test_conv_argument_errors():
    lib = _native.library()
    need = lib.mhs_conv1d_silu_bwd_workspace_bytes(2, 8, 32, 4)
    assert need > 0
    rc = lib.mhs_conv1d_silu_fwd_f32(A16, 31, A16, A16, A16, 2, 8, 32, 4, None)
    assert rc == MHS_EINVAL and "row stride" in _err(lib)
    rc = lib.mhs_conv1d_silu_bwd_f32(A16, 64, A16, A16, A16, A16, 0, A16, A16, A16, need - 4,
                                     2, 8, 32, 4, None)
    assert rc == MHS_EINVAL and "workspace too small" in _err(lib)
    rc = lib.mhs_conv1d_silu_bwd_f32(A16, 64, A16, A16, A16, A16, 31, A16, A16, A16, need,
                                     2, 8, 32, 4, None)
    assert rc == MHS_EINVAL and "dx row stride" in _err(lib)


def test_segment_split_follows_the_compute_unit_count():
    """The automatic split plans for the device's compute units: 256 blocks
    (4 x 16384 x 2048 x 16) get two forward segments at 256 CUs, one at 128
    (two blocks per CU already) and eight (the maximum) at 1024; the carry
    units and the forward's workspace follow (1024 CUs: 7 carried segments x
    2 units; 256 CUs: 1 x 4). Without a device the count is MI355X's 256."""
    lib = _native.library()
    assert lib.mhs_cu_count() == 256
    ru = lambda v: (v + 255) // 256 * 256
    fwd_ws = lambda units: ru(units * 4 * 2048 * 16 * 4) + ru(units * 4 * 2048 * 4)
    shape = (4, 16384, 2048, 16)
    try:
        _native.set_cu_count(128)
        assert lib.mhs_cu_count() == 128
        assert lib.mhs_scan_fwd_workspace_bytes(*shape) == 0
        _native.set_cu_count(1024)
        assert lib.mhs_scan_fwd_workspace_bytes(*shape) == fwd_ws(14)
        _native.set_cu_count(256)
        assert lib.mhs_scan_fwd_workspace_bytes(*shape) == fwd_ws(4)
        with pytest.raises(_native.HipScanError, match="compute-unit count"):
            _native.set_cu_count(-1)
    finally:
        _native.set_cu_count(0)
    assert lib.mhs_cu_count() == 256


def test_xent_argument_errors():
    lib = _native.library()
    assert lib.mhs_xent_fwd_f32(A16, A16, A16, A16, 0, 16, -100, None) == MHS_OK   # no rows
    rc = lib.mhs_xent_fwd_f32(A16, A16, A16, A16, 4, 0, -100, None)
    assert rc == MHS_EINVAL and "vocab" in _err(lib)
    rc = lib.mhs_xent_fwd_f32(A16, None, A16, A16, 4, 16, -100, None)
    assert rc == MHS_EINVAL and "null" in _err(lib)
    rc = lib.mhs_xent_fwd_f32(A16, A16, A16, A16, 1 << 31, 16, -100, None)
    assert rc == MHS_EINVAL and "rows" in _err(lib)
    rc = lib.mhs_xent_bwd_f32(A16, A16, A16, None, A16, 4, 16, -100, None)
    assert rc == MHS_EINVAL and "null" in _err(lib)
    rc = lib.mhs_xent_bwd_f32(A16, A16, A16, A16, A16, 4, 16, -100, None)
    assert rc == MHS_EINVAL and "alias" in _err(lib)


def test_rmsnorm_argument_errors():
    """Host-side checks of the RMSNorm entry points (no launch reaches a
    device: every call here fails or has no rows)."""
    lib = _native.library()
    a, b = A16.value, A16.value + 1024     # distinct, 16-byte aligned stand-ins
    assert lib.mhs_rmsnorm_fwd_f32(None, None, None, None, 0, 640, 1e-6, None) == MHS_OK
    rc = lib.mhs_rmsnorm_fwd_f32(a, a, b, a, 4, 6, 1e-6, None)
    assert rc == MHS_EINVAL and "multiple of 4" in _err(lib)
    rc = lib.mhs_rmsnorm_fwd_f32(a, a, b, a, 4, 4096, 1e-6, None)
    assert rc == MHS_EINVAL and "2048" in _err(lib)
    rc = lib.mhs_rmsnorm_fwd_f32(a, None, b, a, 4, 640, 1e-6, None)
    assert rc == MHS_EINVAL and "null" in _err(lib)
    rc = lib.mhs_rmsnorm_fwd_f32(a + 4, a, b, a, 4, 640, 1e-6, None)
    assert rc == MHS_EINVAL and "aligned" in _err(lib)
    rc = lib.mhs_rmsnorm_fwd_f32(a, a, b, a, 4, 640, float("nan"), None)
    assert rc == MHS_EINVAL and "eps" in _err(lib)
    rc = lib.mhs_rmsnorm_fwd_f32(a, a, a, b, 4, 640, 1e-6, None)
    assert rc == MHS_EINVAL and "alias" in _err(lib)
    c, d = b + 1024, b + 2048
    rc = lib.mhs_add_rmsnorm_fwd_f32(a, None, a, b, c, d, 4, 640, 1e-6, None)
    assert rc == MHS_EINVAL and "null" in _err(lib)
    rc = lib.mhs_add_rmsnorm_fwd_f32(a, b, a, a, c, d, 4, 640, 1e-6, None)
    assert rc == MHS_EINVAL and "x_out may not alias" in _err(lib)
    rc = lib.mhs_add_rmsnorm_fwd_f32(a, b, a, c, b, d, 4, 640, 1e-6, None)
    assert rc == MHS_EINVAL and "y may not alias delta" in _err(lib)
    assert lib.mhs_add_rmsnorm_fwd_f32(None, None, None, None, None, None, 0, 640, 1e-6,
                                       None) == MHS_OK
    ws = lib.mhs_rmsnorm_bwd_workspace_bytes(8192, 640)
    assert ws == 512 * 640 * 4 and lib.mhs_rmsnorm_bwd_workspace_bytes(5, 8) == 256
    rc = lib.mhs_rmsnorm_bwd_f32(a, a, a, a, None, b, a, b, 16, 8192, 640, None)
    assert rc == MHS_EINVAL and "workspace" in _err(lib)
    rc = lib.mhs_rmsnorm_bwd_f32(a, a, a, a, None, a, a, b, ws, 8192, 640, None)
    assert rc == MHS_EINVAL and "alias" in _err(lib)
    rc = lib.mhs_rmsnorm_bwd_f32(a, a, a, a, a + 8, b, a, b, ws, 8192, 640, None)
    assert rc == MHS_EINVAL and "aligned" in _err(lib)
    rc = lib.mhs_rmsnorm_bwd_f32(a, a, a, None, None, b, a, b, ws, 8192, 640, None)
    assert rc == MHS_EINVAL and "null" in _err(lib)
