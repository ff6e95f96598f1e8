"""ctypes binding of the gfx950 scan library and the torch custom ops over it.

The shared library (``libmamba_hip_scan.so``, built in place by ``build.py``)
exports the C ABI of ``include/mamba_hip_scan.h``. It links only the HIP
runtime and is loaded after ``torch``: the dynamic loader then resolves its
``libamdhip64.so.7`` to the copy torch already mapped, so the kernels run in
torch's HIP context and on torch's streams.

The ops registered here are the product path. There is no CPU or torch
fallback behind them: if the library is absent they raise.
"""
from __future__ import annotations

import contextlib
import ctypes
import functools
import threading
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().with_name("libmamba_hip_scan.so")

# Every symbol the C header declares (checked by the CPU test suite).
EXPORTED_SYMBOLS = (
    "mhs_version", "mhs_last_error", "mhs_num_chunks", "mhs_preferred_chunk",
    "mhs_set_variant", "mhs_scan_fwd_f32", "mhs_scan_bwd_workspace_bytes",
    "mhs_scan_bwd_f32", "mhs_scan_step_f32", "mhs_conv1d_silu_fwd_f32",
    "mhs_conv1d_silu_bwd_workspace_bytes", "mhs_conv1d_silu_bwd_f32",
    "mhs_scan_gated_fwd_f32", "mhs_scan_gated_bwd_f32", "mhs_out_gate_fwd_f32",
    "mhs_out_gate_bwd_workspace_bytes", "mhs_out_gate_bwd_f32", "mhs_set_time_segments",
    "mhs_scan_fwd_workspace_bytes", "mhs_scan_fwd_ws_f32", "mhs_scan_fwd_bf16",
    "mhs_scan_bwd_bf16", "mhs_scan_gated_fwd_bf16", "mhs_scan_gated_bwd_bf16",
    "mhs_set_cu_count", "mhs_cu_count", "mhs_scan_fwd_noalloc_f32", "mhs_set_reduction",
    "mhs_deterministic",
    "mhs_scan_bwd_reduction", "mhs_xent_fwd_f32", "mhs_xent_bwd_f32",
    "mhs_rmsnorm_fwd_f32", "mhs_rmsnorm_bwd_workspace_bytes", "mhs_rmsnorm_bwd_f32",
    "mhs_add_rmsnorm_fwd_f32",
)

# Size of the static device scratch of mhs_scan_fwd_noalloc_f32 (the header's
# MHS_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 16 << 20

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F32 = ctypes.c_float


class HipScanError(RuntimeError):
    """A call into the HIP scan library failed."""


def library() -> ctypes.CDLL:
    """Load (once) and return the HIP scan library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise HipScanError(
                    f"the HIP scan library is not built ({LIB_PATH} is missing); "
                    "run `python -m mamba_metal_scan_amd.build` or __graft_entry__.build()")
            lib = ctypes.CDLL(str(LIB_PATH))
            lib.mhs_version.restype = ctypes.c_int
            lib.mhs_version.argtypes = []
            lib.mhs_last_error.restype = ctypes.c_char_p
            lib.mhs_last_error.argtypes = []
            lib.mhs_num_chunks.restype = _I64
            lib.mhs_num_chunks.argtypes = [_I64, _I64]
            lib.mhs_preferred_chunk.restype = _I64
            lib.mhs_preferred_chunk.argtypes = [_I64]
            lib.mhs_set_variant.restype = ctypes.c_int
            lib.mhs_set_variant.argtypes = [ctypes.c_int]
            lib.mhs_set_time_segments.restype = ctypes.c_int
            lib.mhs_set_time_segments.argtypes = [ctypes.c_int]
            lib.mhs_set_cu_count.restype = ctypes.c_int
            lib.mhs_set_cu_count.argtypes = [ctypes.c_int]
            lib.mhs_cu_count.restype = ctypes.c_int
            lib.mhs_cu_count.argtypes = []
            lib.mhs_set_reduction.restype = ctypes.c_int
            lib.mhs_set_reduction.argtypes = [ctypes.c_int]
            lib.mhs_deterministic.restype = ctypes.c_int
            lib.mhs_deterministic.argtypes = []
            lib.mhs_scan_bwd_reduction.restype = ctypes.c_int
            lib.mhs_scan_bwd_reduction.argtypes = [_I64] * 5
            lib.mhs_scan_fwd_f32.restype = ctypes.c_int
            lib.mhs_scan_fwd_f32.argtypes = [_P] * 8 + [_I64] * 5 + [_P]
            lib.mhs_scan_fwd_noalloc_f32.restype = ctypes.c_int
            lib.mhs_scan_fwd_noalloc_f32.argtypes = [_P] * 8 + [_I64] * 5 + [_P]
            lib.mhs_scan_fwd_workspace_bytes.restype = ctypes.c_size_t
            lib.mhs_scan_fwd_workspace_bytes.argtypes = [_I64] * 4
            lib.mhs_scan_fwd_ws_f32.restype = ctypes.c_int
            lib.mhs_scan_fwd_ws_f32.argtypes = [_P] * 9 + [ctypes.c_size_t] + [_I64] * 5 + [_P]
            lib.mhs_scan_bwd_workspace_bytes.restype = ctypes.c_size_t
            lib.mhs_scan_bwd_workspace_bytes.argtypes = [_I64] * 5
            lib.mhs_scan_bwd_f32.restype = ctypes.c_int
            lib.mhs_scan_bwd_f32.argtypes = [_P] * 14 + [ctypes.c_size_t] + [_I64] * 5 + [_P]
            lib.mhs_scan_step_f32.restype = ctypes.c_int
            lib.mhs_scan_step_f32.argtypes = [_P] * 7 + [_I64] * 3 + [_P]
            lib.mhs_conv1d_silu_fwd_f32.restype = ctypes.c_int
            lib.mhs_conv1d_silu_fwd_f32.argtypes = [_P, _I64, _P, _P, _P] + [_I64] * 4 + [_P]
            lib.mhs_conv1d_silu_bwd_workspace_bytes.restype = ctypes.c_size_t
            lib.mhs_conv1d_silu_bwd_workspace_bytes.argtypes = [_I64] * 4
            lib.mhs_conv1d_silu_bwd_f32.restype = ctypes.c_int
            lib.mhs_conv1d_silu_bwd_f32.argtypes = ([_P, _I64] + [_P] * 4 + [_I64] + [_P] * 3
                                                    + [ctypes.c_size_t] + [_I64] * 4 + [_P])
            lib.mhs_scan_gated_fwd_f32.restype = ctypes.c_int
            lib.mhs_scan_gated_fwd_f32.argtypes = ([_P] * 5 + [_F32] * 2 + [_P] * 5
                                                   + [ctypes.c_size_t] + [_I64] * 7 + [_P])
            lib.mhs_scan_gated_bwd_f32.restype = ctypes.c_int
            lib.mhs_scan_gated_bwd_f32.argtypes = ([_P] * 5 + [_F32] * 2 + [_P] * 11
                                                   + [ctypes.c_size_t] + [_I64] * 9 + [_P])
            lib.mhs_out_gate_fwd_f32.restype = ctypes.c_int
            lib.mhs_out_gate_fwd_f32.argtypes = [_P] * 3 + [_I64, _P] + [_I64] * 3 + [_P]
            lib.mhs_out_gate_bwd_workspace_bytes.restype = ctypes.c_size_t
            lib.mhs_out_gate_bwd_workspace_bytes.argtypes = [_I64] * 3
            lib.mhs_out_gate_bwd_f32.restype = ctypes.c_int
            lib.mhs_out_gate_bwd_f32.argtypes = ([_P] * 3 + [_I64] + [_P] * 3 + [_I64] + [_P] * 2
                                                 + [ctypes.c_size_t] + [_I64] * 3 + [_P])
            for name in ("mhs_scan_fwd_bf16", "mhs_scan_bwd_bf16"):
                getattr(lib, name).restype = ctypes.c_int
            lib.mhs_scan_fwd_bf16.argtypes = lib.mhs_scan_fwd_ws_f32.argtypes
            lib.mhs_scan_bwd_bf16.argtypes = lib.mhs_scan_bwd_f32.argtypes
            lib.mhs_scan_gated_fwd_bf16.restype = ctypes.c_int
            lib.mhs_scan_gated_fwd_bf16.argtypes = lib.mhs_scan_gated_fwd_f32.argtypes
            lib.mhs_scan_gated_bwd_bf16.restype = ctypes.c_int
            lib.mhs_scan_gated_bwd_bf16.argtypes = lib.mhs_scan_gated_bwd_f32.argtypes
            lib.mhs_xent_fwd_f32.restype = ctypes.c_int
            lib.mhs_xent_fwd_f32.argtypes = [_P] * 4 + [_I64] * 3 + [_P]
            lib.mhs_xent_bwd_f32.restype = ctypes.c_int
            lib.mhs_xent_bwd_f32.argtypes = [_P] * 5 + [_I64] * 3 + [_P]
            lib.mhs_rmsnorm_fwd_f32.restype = ctypes.c_int
            lib.mhs_rmsnorm_fwd_f32.argtypes = [_P] * 4 + [_I64] * 2 + [ctypes.c_float, _P]
            lib.mhs_add_rmsnorm_fwd_f32.restype = ctypes.c_int
            lib.mhs_add_rmsnorm_fwd_f32.argtypes = [_P] * 6 + [_I64] * 2 + [ctypes.c_float, _P]
            lib.mhs_rmsnorm_bwd_workspace_bytes.restype = ctypes.c_size_t
            lib.mhs_rmsnorm_bwd_workspace_bytes.argtypes = [_I64] * 2
            lib.mhs_rmsnorm_bwd_f32.restype = ctypes.c_int
            lib.mhs_rmsnorm_bwd_f32.argtypes = [_P] * 8 + [ctypes.c_size_t] + [_I64] * 2 + [_P]
            _lib = lib
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = library().mhs_last_error().decode(errors="replace")
        raise HipScanError(f"{what} failed (code {rc}): {msg}")


def _ptr(t: Optional[torch.Tensor]):
    # plain ints: the c_void_p argtypes convert them (None is NULL)
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(dev: torch.device) -> int:
    """The device's current stream (hipStream_t as an int)."""
    if _raw_stream is not None:
        return _raw_stream(dev.index if dev.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(dev).cuda_stream


def _on(dev: torch.device):
    """torch.cuda.device(dev), or no context switch when dev is already current."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(dev)


def num_chunks(seqlen: int, chunk: int) -> int:
    return (seqlen + chunk - 1) // chunk


@torch.compiler.assume_constant_result
def preferred_chunk(d_state: int) -> int:
    """Largest checkpoint stride the backward kernel walks without recomputing
    (0: d_state unsupported). A constant for a given d_state and variant
    setting, so torch.compile evaluates it once while tracing instead of
    tracing the library call."""
    return int(library().mhs_preferred_chunk(d_state))


def set_variant(states_per_lane: int) -> None:
    """Force 1, 2 or 4 states per lane (0 = automatic), process-wide."""
    _check(library().mhs_set_variant(int(states_per_lane)), "mhs_set_variant")


def set_time_segments(segments: int) -> None:
    """Force the backward's number of time segments (1..8; 0 = automatic), process-wide."""
    _check(library().mhs_set_time_segments(int(segments)), "mhs_set_time_segments")


REDUCTION_AUTO, REDUCTION_FIXED, REDUCTION_ATOMIC = 0, 1, 2
_reduction = REDUCTION_AUTO      # the mode last set through set_reduction
_reduction_lock = threading.Lock()


def set_reduction(mode: int) -> None:
    """How the backward reduces dB, dC, dAneg (and the gated dt-bias gradient),
    process-wide: REDUCTION_FIXED (fixed-order partials, bit-for-bit
    reproducible), REDUCTION_ATOMIC (fp32 atomics into the zeroed gradients)
    or REDUCTION_AUTO (the library's choice per shape: the fixed order where
    the backward's grid fills the GPU, atomics where it runs in time segments;
    each measured the faster there on MI355X; bwd_reduction() tells which a
    shape gets). While torch's deterministic algorithms are enabled
    (torch.use_deterministic_algorithms) the backward ops use the fixed order
    whatever this says."""
    global _reduction
    with _reduction_lock:
        _check(library().mhs_set_reduction(int(mode)), "mhs_set_reduction")
        _reduction = int(mode)


def bwd_reduction(batch: int, seqlen: int, d_inner: int, d_state: int, chunk: int) -> int:
    """The reduction (REDUCTION_FIXED or REDUCTION_ATOMIC) a backward of this
    shape uses under the process-wide mode (not counting torch's
    deterministic mode, which forces the fixed order)."""
    mode = library().mhs_scan_bwd_reduction(batch, seqlen, d_inner, d_state, chunk)
    if mode == 0:
        raise HipScanError(f"mhs_scan_bwd_reduction: {library().mhs_last_error().decode()}")
    return mode


@contextlib.contextmanager
def _bwd_reduction():
    """Around one backward call (workspace query and launch): the fixed-order
    reduction while torch's deterministic algorithms are enabled, else the
    process-wide mode. Every backward holds the lock from its workspace query
    to its launch, so that a deterministic call in another thread cannot
    switch the library's mode in between (the workspace would then be sized
    for the other reduction)."""
    with _reduction_lock:
        if not torch.are_deterministic_algorithms_enabled():
            yield
            return
        lib = library()
        lib.mhs_set_reduction(REDUCTION_FIXED)
        try:
            yield
        finally:
            lib.mhs_set_reduction(_reduction)


def set_cu_count(cus: int) -> None:
    """Force the compute-unit count the automatic time-segment split plans for
    (0 = query the current device), process-wide."""
    _check(library().mhs_set_cu_count(int(cus)), "mhs_set_cu_count")


# ------------------------------------------------------- host-side checks
#
# The registered ops are public (torch.ops.mamba_hip.*), so each checks what
# its kernels assume before anything is launched: one ROCm device, the dtypes
# the kernels read, shapes, dense layouts (or the row strides the kernel
# takes), and the checkpoint buffer's shape for the stride. A mismatch raises
# HipScanError; nothing reaches the device.

_ACT = (torch.float32, torch.bfloat16)


def _need(ok: bool, what: str, msg: str) -> None:
    if not ok:
        raise HipScanError(f"{what}: {msg}")


def _on_one_device(what: str, *ts: Optional[torch.Tensor]) -> None:
    ts = [t for t in ts if t is not None]
    dev = ts[0].device
    _need(dev.type == "cuda" and all(t.device == dev for t in ts), what,
          "every tensor must be on one ROCm device; got " + ", ".join(str(t.device) for t in ts))


def _dense(what: str, **ts: Optional[torch.Tensor]) -> None:
    for name, t in ts.items():
        if t is not None and not t.is_contiguous():
            raise HipScanError(f"{what}: {name} must be contiguous; got strides {t.stride()} "
                               f"for shape {tuple(t.shape)}")


def _fp32(what: str, **ts: Optional[torch.Tensor]) -> None:
    for name, t in ts.items():
        if t is not None and t.dtype != torch.float32:
            raise HipScanError(f"{what}: {name} must be float32; got {t.dtype}")


def _shaped(what: str, name: str, t: Optional[torch.Tensor], shape) -> None:
    if t is not None and tuple(t.shape) != tuple(shape):
        raise HipScanError(f"{what}: {name} must have shape {tuple(shape)}; got "
                           f"{tuple(t.shape)}")


def _check_scan(what: str, x, dt, aneg, b_in, c_in, chunk: int, dense_dt_bc: bool = True) -> None:
    """Common checks of the scan ops: x (B,T,D); dt (B,T,D); Aneg / A (D,N)
    fp32; B, C (B,T,N); x, dt, B, C all fp32 or all bf16; x (and unless the
    op takes row strides, dt, B, C) contiguous; chunk >= 1."""
    _on_one_device(what, x, dt, aneg, b_in, c_in)
    _need(x.dim() == 3 and aneg.dim() == 2, what,
          f"x must be (B,T,D) and Aneg (D,N); got {tuple(x.shape)}, {tuple(aneg.shape)}")
    bt, t_len, d = x.shape
    n = aneg.shape[1]
    _shaped(what, "dt", dt, (bt, t_len, d))
    _shaped(what, "Aneg", aneg, (d, n))
    _shaped(what, "B", b_in, (bt, t_len, n))
    _shaped(what, "C", c_in, (bt, t_len, n))
    _need(x.dtype in _ACT and all(t.dtype == x.dtype for t in (dt, b_in, c_in)), what,
          "x, dt, B, C must all be float32 or all bfloat16; got "
          + ", ".join(str(t.dtype) for t in (x, dt, b_in, c_in)))
    _fp32(what, Aneg=aneg)
    _dense(what, x=x, Aneg=aneg)
    if dense_dt_bc:
        _dense(what, dt=dt, B=b_in, C=c_in)
    _need(isinstance(chunk, int) and chunk >= 1, what, f"chunk must be an int >= 1; got {chunk!r}")


def _check_bwd(what: str, x, aneg, dy, dh_last, ckpt, chunk: int) -> None:
    """The backward's extra operands: dy like x; dh_last None or (B,D,N)
    fp32; ckpt the forward's (B, ceil(T/chunk), D, N) fp32 checkpoints."""
    bt, t_len, d = x.shape
    n = aneg.shape[1]
    _on_one_device(what, x, dy, dh_last, ckpt)
    _shaped(what, "dy", dy, (bt, t_len, d))
    _need(dy.dtype == x.dtype, what, f"dy must have x's dtype {x.dtype}; got {dy.dtype}")
    _shaped(what, "dh_last", dh_last, (bt, d, n))
    _shaped(what, f"ckpt (chunk {chunk})", ckpt, (bt, num_chunks(t_len, chunk), d, n))
    _fp32(what, dh_last=dh_last, ckpt=ckpt)
    _dense(what, dy=dy, dh_last=dh_last, ckpt=ckpt)


# --------------------------------------------------------------- custom ops

def _fwd_outputs(x: torch.Tensor, n: int, chunk: int, with_ckpt: bool):
    """y (x's dtype), checkpoints and final state (fp32, the state's type)."""
    bt, t_len, d = x.shape
    f32 = dict(dtype=torch.float32, device=x.device)
    ckpt = (torch.empty((bt, num_chunks(t_len, chunk), d, n), **f32) if with_ckpt
            else torch.empty((0,), **f32))
    return torch.empty_like(x), ckpt, torch.empty((bt, d, n), **f32)


def _fwd_workspace(x: torch.Tensor, n: int):
    """(workspace tensor or None, bytes) for a forward on (B,T,D) x with d_state n."""
    bt, t_len, d = x.shape
    nbytes = int(library().mhs_scan_fwd_workspace_bytes(bt, t_len, d, n))
    if nbytes == 0:
        return None, 0
    return torch.empty(nbytes, dtype=torch.uint8, device=x.device), nbytes


def _bwd_workspace(x: torch.Tensor, n: int, chunk: int):
    """(workspace tensor, bytes) for a backward on (B,T,D) x with d_state n
    and checkpoint stride chunk, under the current reduction mode."""
    bt, t_len, d = x.shape
    nbytes = int(library().mhs_scan_bwd_workspace_bytes(bt, t_len, d, n, chunk))
    if nbytes == 0:
        raise HipScanError(f"no backward workspace size for shape {(bt, t_len, d, n)} "
                           f"chunk {chunk}")
    return torch.empty(nbytes, dtype=torch.uint8, device=x.device), nbytes


_IMPLS: dict = {}


def _register(name: str, impl, mutates_args, check):
    """Register impl, preceded by the host-side argument checks `check` (same
    arguments), as the custom op mamba_hip::<name> (for torch.compile and
    torch.ops callers); keep the plain impl for dispatch()."""
    _IMPLS[name] = impl

    @functools.wraps(impl)
    def checked(*args, **kwargs):
        check(*args, **kwargs)
        return impl(*args, **kwargs)

    return torch.library.custom_op(f"mamba_hip::{name}", checked, mutates_args=mutates_args)


def dispatch(name: str):
    """The op the autograd Functions call: the registered torch.ops.mamba_hip
    op while torch.compile traces, else its plain implementation (the same
    code without the dispatcher's per-call overhead and without the op's
    argument checks, which the Functions' own validation and .contiguous()
    calls already cover; together these are as long as the kernels' GPU time
    at the training shape, and the GPU would wait for them)."""
    if torch.compiler.is_compiling():
        return getattr(torch.ops.mamba_hip, name)
    return _IMPLS[name]


def _scan_fwd_impl(x: torch.Tensor, dt: torch.Tensor, aneg: torch.Tensor, b_in: torch.Tensor,
             c_in: torch.Tensor, chunk: int, with_ckpt: bool
             ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """y (B,T,D), ckpt (B,ceil(T/chunk),D,N) or an empty tensor, h_last (B,D,N)."""
    bt, t_len, d = x.shape
    n = aneg.shape[1]
    y, ckpt, h_last = _fwd_outputs(x, n, chunk, with_ckpt)
    ws, ws_bytes = _fwd_workspace(x, n)
    lib = library()
    fn = lib.mhs_scan_fwd_bf16 if x.dtype == torch.bfloat16 else lib.mhs_scan_fwd_ws_f32
    with _on(x.device):
        rc = fn(_ptr(x), _ptr(dt), _ptr(aneg), _ptr(b_in), _ptr(c_in), _ptr(y),
                _ptr(ckpt) if with_ckpt else None, _ptr(h_last), _ptr(ws), ws_bytes,
                bt, t_len, d, n, chunk, _stream(x.device))
    _check(rc, "scan forward")
    return y, ckpt, h_last


scan_fwd = _register(
    "scan_fwd", _scan_fwd_impl, (),
    lambda x, dt, aneg, b_in, c_in, chunk, with_ckpt:
        _check_scan("scan_fwd", x, dt, aneg, b_in, c_in, chunk))


@scan_fwd.register_fake
def _scan_fwd_fake(x, dt, aneg, b_in, c_in, chunk, with_ckpt):
    return _fwd_outputs(x, aneg.shape[1], chunk, with_ckpt)


def _scan_bwd_impl(x: torch.Tensor, dt: torch.Tensor, aneg: torch.Tensor, b_in: torch.Tensor,
             c_in: torch.Tensor, dy: torch.Tensor, dh_last: Optional[torch.Tensor],
             ckpt: torch.Tensor, chunk: int
             ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dx, ddt, dAneg, dB, dC) for the forward that produced `ckpt`."""
    bt, t_len, d = x.shape
    n = aneg.shape[1]
    lib = library()
    dx = torch.empty_like(x)
    ddt = torch.empty_like(dt)
    daneg = torch.empty_like(aneg)
    db = torch.empty_like(b_in)
    dc = torch.empty_like(c_in)
    fn = lib.mhs_scan_bwd_bf16 if x.dtype == torch.bfloat16 else lib.mhs_scan_bwd_f32
    with _bwd_reduction(), _on(x.device):
        ws, ws_bytes = _bwd_workspace(x, n, chunk)
        rc = fn(_ptr(x), _ptr(dt), _ptr(aneg), _ptr(b_in), _ptr(c_in), _ptr(dy),
                _ptr(dh_last), _ptr(ckpt), _ptr(dx), _ptr(ddt), _ptr(daneg), _ptr(db), _ptr(dc),
                _ptr(ws), ws_bytes, bt, t_len, d, n, chunk, _stream(x.device))
    _check(rc, "scan backward")
    return dx, ddt, daneg, db, dc


def _check_scan_bwd(x, dt, aneg, b_in, c_in, dy, dh_last, ckpt, chunk):
    _check_scan("scan_bwd", x, dt, aneg, b_in, c_in, chunk)
    _check_bwd("scan_bwd", x, aneg, dy, dh_last, ckpt, chunk)


scan_bwd = _register("scan_bwd", _scan_bwd_impl, (), _check_scan_bwd)


@scan_bwd.register_fake
def _scan_bwd_fake(x, dt, aneg, b_in, c_in, dy, dh_last, ckpt, chunk):
    return (torch.empty_like(x), torch.empty_like(dt), torch.empty_like(aneg),
            torch.empty_like(b_in), torch.empty_like(c_in))


def _scan_step_impl(h: torch.Tensor, x: torch.Tensor, dt: torch.Tensor, aneg: torch.Tensor,
              b_in: torch.Tensor, c_in: torch.Tensor) -> torch.Tensor:
    """One decode step in place on h (B,D,N); returns y (B,D)."""
    bt, d, n = h.shape
    y = x.new_empty((bt, d))
    with _on(h.device):
        rc = library().mhs_scan_step_f32(
            _ptr(h), _ptr(x), _ptr(dt), _ptr(aneg), _ptr(b_in), _ptr(c_in), _ptr(y),
            bt, d, n, _stream(h.device))
    _check(rc, "mhs_scan_step_f32")
    return y


def _check_scan_step(h, x, dt, aneg, b_in, c_in):
    what = "scan_step"
    _on_one_device(what, h, x, dt, aneg, b_in, c_in)
    _need(h.dim() == 3, what, f"h must be (B,D,N); got {tuple(h.shape)}")
    bt, d, n = h.shape
    for name, t, shape in (("x", x, (bt, d)), ("dt", dt, (bt, d)), ("Aneg", aneg, (d, n)),
                           ("B", b_in, (bt, n)), ("C", c_in, (bt, n))):
        _shaped(what, name, t, shape)
    _fp32(what, h=h, x=x, dt=dt, Aneg=aneg, B=b_in, C=c_in)
    _dense(what, h=h, x=x, dt=dt, Aneg=aneg, B=b_in, C=c_in)


scan_step = _register("scan_step", _scan_step_impl, ("h",), _check_scan_step)


@scan_step.register_fake
def _scan_step_fake(h, x, dt, aneg, b_in, c_in):
    return x.new_empty((h.shape[0], h.shape[1]))


def _rows(x: torch.Tensor) -> int:
    """Row stride (elements) of a (B,T,D) tensor whose rows are dense and whose
    batch rows follow each other (a contiguous tensor, or a column slice of a
    wider one); raises for other layouts."""
    bt, t_len, d = x.shape
    if x.stride(2) != 1 or x.stride(1) < d or (bt > 1 and x.stride(0) != t_len * x.stride(1)):
        raise HipScanError(f"unsupported strides {x.stride()} for shape {tuple(x.shape)}: "
                           "need dense rows, batch rows back to back")
    return x.stride(1)


_conv_rows = _rows


def _check_conv(what: str, x, w, bias, dout=None, dx=None) -> None:
    """conv1d + SiLU: fp32 x (B,T,D) with dense rows (row stride allowed), w
    (D,K) and bias (D,) contiguous, dout (B,T,D) contiguous, dx (B,T,D) with
    dense rows."""
    _on_one_device(what, x, w, bias, dout, dx)
    _need(x.dim() == 3 and w.dim() == 2, what,
          f"x must be (B,T,D) and w (D,K); got {tuple(x.shape)}, {tuple(w.shape)}")
    _shaped(what, "w", w, (x.shape[2], w.shape[1]))
    _shaped(what, "bias", bias, (x.shape[2],))
    _shaped(what, "dout", dout, x.shape)
    _shaped(what, "dx", dx, x.shape)
    _fp32(what, x=x, w=w, bias=bias, dout=dout, dx=dx)
    _dense(what, w=w, bias=bias, dout=dout)
    _rows(x)
    if dx is not None:
        _rows(dx)


def _check_gate(what: str, y, d_skip, z, dout=None, dz=None) -> None:
    """Output gate: fp32 y (B,T,D) and dout contiguous, d_skip (D,)
    contiguous, z and dz (B,T,D) with dense rows."""
    _on_one_device(what, y, d_skip, z, dout, dz)
    _need(y.dim() == 3, what, f"y must be (B,T,D); got {tuple(y.shape)}")
    _shaped(what, "d_skip", d_skip, (y.shape[2],))
    _shaped(what, "z", z, y.shape)
    _shaped(what, "dout", dout, y.shape)
    _shaped(what, "dz", dz, y.shape)
    _fp32(what, y=y, d_skip=d_skip, z=z, dout=dout, dz=dz)
    _dense(what, y=y, d_skip=d_skip, dout=dout)
    _rows(z)
    if dz is not None:
        _rows(dz)


def _bc_rows(b_in: torch.Tensor, c_in: torch.Tensor) -> int:
    """The common row stride of B and C (both contiguous, or both column
    slices of one wider tensor)."""
    ld = _rows(b_in)
    if _rows(c_in) != ld:
        raise HipScanError(f"B and C need one row stride; got {b_in.stride()} and {c_in.stride()}")
    return ld


def _conv1d_silu_fwd_impl(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """silu(causal depthwise conv1d) of (B,T,D) x (rows may be strided), w (D,K): (B,T,D)."""
    bt, t_len, d = x.shape
    out = x.new_empty((bt, t_len, d))
    with _on(x.device):
        rc = library().mhs_conv1d_silu_fwd_f32(
            _ptr(x), _conv_rows(x), _ptr(w), _ptr(bias), _ptr(out), bt, t_len, d, w.shape[1],
            _stream(x.device))
    _check(rc, "mhs_conv1d_silu_fwd_f32")
    return out


conv1d_silu_fwd = _register("conv1d_silu_fwd", _conv1d_silu_fwd_impl, (),
                            lambda x, w, bias: _check_conv("conv1d_silu_fwd", x, w, bias))


@conv1d_silu_fwd.register_fake
def _conv1d_silu_fwd_fake(x, w, bias):
    return x.new_empty(x.shape)


def _conv1d_silu_bwd_impl(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor, dout: torch.Tensor
                    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dx (B,T,D) contiguous, dw (D,K), dbias (D))."""
    bt, t_len, d = x.shape
    k = w.shape[1]
    lib = library()
    dx = x.new_empty((bt, t_len, d))
    dw = torch.empty_like(w)
    dbias = torch.empty_like(bias)
    ws_bytes = int(lib.mhs_conv1d_silu_bwd_workspace_bytes(bt, t_len, d, k))
    if ws_bytes == 0:
        raise HipScanError(f"no conv workspace size for shape {(bt, t_len, d)} kernel {k}")
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    with _on(x.device):
        rc = lib.mhs_conv1d_silu_bwd_f32(
            _ptr(x), _rows(x), _ptr(w), _ptr(bias), _ptr(dout), _ptr(dx), 0, _ptr(dw),
            _ptr(dbias), _ptr(ws), ws_bytes, bt, t_len, d, k, _stream(x.device))
    _check(rc, "mhs_conv1d_silu_bwd_f32")
    return dx, dw, dbias


conv1d_silu_bwd = _register(
    "conv1d_silu_bwd", _conv1d_silu_bwd_impl, (),
    lambda x, w, bias, dout: _check_conv("conv1d_silu_bwd", x, w, bias, dout))


@conv1d_silu_bwd.register_fake
def _conv1d_silu_bwd_fake(x, w, bias, dout):
    return x.new_empty(x.shape), torch.empty_like(w), torch.empty_like(bias)


def _conv1d_silu_bwd_into_impl(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor,
                               dout: torch.Tensor, dx: torch.Tensor
                               ) -> tuple[torch.Tensor, torch.Tensor]:
    """conv1d_silu_bwd writing dx into the given (B,T,D) tensor, which may be
    a column slice of a wider one (the x half of the in_proj output's
    gradient); returns (dw, dbias)."""
    bt, t_len, d = x.shape
    k = w.shape[1]
    lib = library()
    dw = torch.empty_like(w)
    dbias = torch.empty_like(bias)
    ws_bytes = int(lib.mhs_conv1d_silu_bwd_workspace_bytes(bt, t_len, d, k))
    if ws_bytes == 0:
        raise HipScanError(f"no conv workspace size for shape {(bt, t_len, d)} kernel {k}")
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    with _on(x.device):
        rc = lib.mhs_conv1d_silu_bwd_f32(
            _ptr(x), _rows(x), _ptr(w), _ptr(bias), _ptr(dout), _ptr(dx), _rows(dx), _ptr(dw),
            _ptr(dbias), _ptr(ws), ws_bytes, bt, t_len, d, k, _stream(x.device))
    _check(rc, "mhs_conv1d_silu_bwd_f32")
    return dw, dbias


conv1d_silu_bwd_into = _register(
    "conv1d_silu_bwd_into", _conv1d_silu_bwd_into_impl, ("dx",),
    lambda x, w, bias, dout, dx: _check_conv("conv1d_silu_bwd_into", x, w, bias, dout, dx))


@conv1d_silu_bwd_into.register_fake
def _conv1d_silu_bwd_into_fake(x, w, bias, dout, dx):
    return torch.empty_like(w), torch.empty_like(bias)


def _dt_bias(dt_bias: Optional[torch.Tensor], x: torch.Tensor) -> None:
    """The dt projection's bias: None, or fp32 (d_inner,) contiguous on x's device."""
    d = x.shape[2]
    if dt_bias is not None and (dt_bias.dtype != torch.float32 or dt_bias.shape != (d,)
                                or not dt_bias.is_contiguous() or dt_bias.device != x.device):
        raise HipScanError(f"dt_bias must be a contiguous fp32 ({d},) tensor on {x.device}; got "
                           f"{dt_bias.dtype} {tuple(dt_bias.shape)} on {dt_bias.device}")


def _scan_gated_fwd_impl(x: torch.Tensor, dt_raw: torch.Tensor, a_raw: torch.Tensor,
                   b_in: torch.Tensor, c_in: torch.Tensor, dt_min: float, dt_max: float,
                   chunk: int, with_ckpt: bool, dt_bias: Optional[torch.Tensor] = None
                   ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """scan_fwd with dt = dt_min + (dt_max - dt_min) * sigmoid(dt_raw + dt_bias)
    and Aneg = softplus(a_raw) formed inside the kernels (dt_bias: the dt
    projection's bias, or None). dt_raw, B and C may be column slices of a
    wider tensor (dense rows; B and C with one row stride)."""
    bt, t_len, d = x.shape
    n = a_raw.shape[1]
    _dt_bias(dt_bias, x)
    ld_dt, ld_bc = _rows(dt_raw), _bc_rows(b_in, c_in)
    y, ckpt, h_last = _fwd_outputs(x, n, chunk, with_ckpt)
    ws, ws_bytes = _fwd_workspace(x, n)
    lib = library()
    fn = lib.mhs_scan_gated_fwd_bf16 if x.dtype == torch.bfloat16 else lib.mhs_scan_gated_fwd_f32
    with _on(x.device):
        rc = fn(_ptr(x), _ptr(dt_raw), _ptr(a_raw), _ptr(b_in), _ptr(c_in), dt_min, dt_max,
                _ptr(dt_bias), _ptr(y), _ptr(ckpt) if with_ckpt else None, _ptr(h_last),
                _ptr(ws), ws_bytes, bt, t_len, d, n, chunk, ld_dt, ld_bc, _stream(x.device))
    _check(rc, "gated scan forward")
    return y, ckpt, h_last


scan_gated_fwd = _register(
    "scan_gated_fwd", _scan_gated_fwd_impl, (),
    lambda x, dt_raw, a_raw, b_in, c_in, dt_min, dt_max, chunk, with_ckpt, dt_bias=None:
        _check_scan("scan_gated_fwd", x, dt_raw, a_raw, b_in, c_in, chunk, dense_dt_bc=False))


@scan_gated_fwd.register_fake
def _scan_gated_fwd_fake(x, dt_raw, a_raw, b_in, c_in, dt_min, dt_max, chunk, with_ckpt,
                         dt_bias=None):
    return _scan_fwd_fake(x, dt_raw, a_raw, b_in, c_in, chunk, with_ckpt)


def _scan_gated_bwd_impl(x: torch.Tensor, dt_raw: torch.Tensor, a_raw: torch.Tensor,
                   b_in: torch.Tensor, c_in: torch.Tensor, dt_min: float, dt_max: float,
                   dy: torch.Tensor, dh_last: Optional[torch.Tensor], ckpt: torch.Tensor,
                   chunk: int, dt_bias: Optional[torch.Tensor] = None
                   ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                              torch.Tensor]:
    """(dx, d dt_raw, d a_raw, dB, dC, d dt_bias) for the gated forward that
    produced `ckpt` (same dt_bias); the gradients are contiguous (inputs as
    scan_gated_fwd). d dt_bias, the sum of d dt_raw over batch and time, is
    fp32 (d_inner,) also when dt_bias is None."""
    bt, t_len, d = x.shape
    n = a_raw.shape[1]
    _dt_bias(dt_bias, x)
    ld_dt, ld_bc = _rows(dt_raw), _bc_rows(b_in, c_in)
    lib = library()
    dx = torch.empty_like(x)
    ddt = x.new_empty((bt, t_len, d))
    da = torch.empty_like(a_raw)
    db = x.new_empty((bt, t_len, n))
    dc = x.new_empty((bt, t_len, n))
    dbias = a_raw.new_empty((d,))
    fn = lib.mhs_scan_gated_bwd_bf16 if x.dtype == torch.bfloat16 else lib.mhs_scan_gated_bwd_f32
    with _bwd_reduction(), _on(x.device):
        ws, ws_bytes = _bwd_workspace(x, n, chunk)
        rc = fn(_ptr(x), _ptr(dt_raw), _ptr(a_raw), _ptr(b_in), _ptr(c_in), dt_min, dt_max,
                _ptr(dt_bias), _ptr(dy), _ptr(dh_last), _ptr(ckpt), _ptr(dx), _ptr(ddt),
                _ptr(da), _ptr(db), _ptr(dc), _ptr(dbias), _ptr(ws), ws_bytes, bt, t_len, d, n,
                chunk, ld_dt, ld_bc, 0, 0, _stream(x.device))
    _check(rc, "gated scan backward")
    return dx, ddt, da, db, dc, dbias


def _check_scan_gated_bwd(x, dt_raw, a_raw, b_in, c_in, dt_min, dt_max, dy, dh_last, ckpt,
                          chunk, dt_bias=None):
    _check_scan("scan_gated_bwd", x, dt_raw, a_raw, b_in, c_in, chunk, dense_dt_bc=False)
    _check_bwd("scan_gated_bwd", x, a_raw, dy, dh_last, ckpt, chunk)


scan_gated_bwd = _register("scan_gated_bwd", _scan_gated_bwd_impl, (), _check_scan_gated_bwd)


def _scan_gated_bwd_into_impl(x: torch.Tensor, dt_raw: torch.Tensor, a_raw: torch.Tensor,
                              b_in: torch.Tensor, c_in: torch.Tensor, dt_min: float,
                              dt_max: float, dy: torch.Tensor, dh_last: Optional[torch.Tensor],
                              ckpt: torch.Tensor, chunk: int, dproj: torch.Tensor,
                              dt_bias: Optional[torch.Tensor] = None
                              ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """scan_gated_bwd writing d dt_raw, dB and dC into the column slices
    [0, D), [D, D+N), [D+N, D+2N) of dproj (B, T, D+2N, contiguous): the
    gradient of one projection whose output rows are [dt_raw | B | C].
    Returns (dx, d a_raw, d dt_bias)."""
    bt, t_len, d = x.shape
    n = a_raw.shape[1]
    _dt_bias(dt_bias, x)
    if dproj.shape != (bt, t_len, d + 2 * n) or not dproj.is_contiguous():
        raise HipScanError(f"dproj must be a contiguous {(bt, t_len, d + 2 * n)} tensor; got "
                           f"{tuple(dproj.shape)} strides {dproj.stride()}")
    ld_dt, ld_bc = _rows(dt_raw), _bc_rows(b_in, c_in)
    lib = library()
    dx = torch.empty_like(x)
    da = torch.empty_like(a_raw)
    dbias = a_raw.new_empty((d,))
    fn = lib.mhs_scan_gated_bwd_bf16 if x.dtype == torch.bfloat16 else lib.mhs_scan_gated_bwd_f32
    es = dproj.element_size()
    base = dproj.data_ptr()
    w = d + 2 * n
    with _bwd_reduction(), _on(x.device):
        ws, ws_bytes = _bwd_workspace(x, n, chunk)
        rc = fn(_ptr(x), _ptr(dt_raw), _ptr(a_raw), _ptr(b_in), _ptr(c_in), dt_min, dt_max,
                _ptr(dt_bias), _ptr(dy), _ptr(dh_last), _ptr(ckpt), _ptr(dx), base, _ptr(da),
                base + d * es, base + (d + n) * es, _ptr(dbias), _ptr(ws), ws_bytes, bt, t_len,
                d, n, chunk, ld_dt, ld_bc, w, w, _stream(x.device))
    _check(rc, "gated scan backward")
    return dx, da, dbias


def _check_scan_gated_bwd_into(x, dt_raw, a_raw, b_in, c_in, dt_min, dt_max, dy, dh_last, ckpt,
                               chunk, dproj, dt_bias=None):
    what = "scan_gated_bwd_into"
    _check_scan(what, x, dt_raw, a_raw, b_in, c_in, chunk, dense_dt_bc=False)
    _check_bwd(what, x, a_raw, dy, dh_last, ckpt, chunk)
    _on_one_device(what, x, dproj)
    _need(dproj.dtype == x.dtype, what, f"dproj must have x's dtype {x.dtype}; got {dproj.dtype}")


scan_gated_bwd_into = _register("scan_gated_bwd_into", _scan_gated_bwd_into_impl, ("dproj",),
                                _check_scan_gated_bwd_into)


@scan_gated_bwd_into.register_fake
def _scan_gated_bwd_into_fake(x, dt_raw, a_raw, b_in, c_in, dt_min, dt_max, dy, dh_last, ckpt,
                              chunk, dproj, dt_bias=None):
    return torch.empty_like(x), torch.empty_like(a_raw), a_raw.new_empty((x.shape[2],))


@scan_gated_bwd.register_fake
def _scan_gated_bwd_fake(x, dt_raw, a_raw, b_in, c_in, dt_min, dt_max, dy, dh_last, ckpt, chunk,
                         dt_bias=None):
    bt, t_len, d = x.shape
    n = a_raw.shape[1]
    return (torch.empty_like(x), x.new_empty((bt, t_len, d)), torch.empty_like(a_raw),
            x.new_empty((bt, t_len, n)), x.new_empty((bt, t_len, n)), a_raw.new_empty((d,)))


def _out_gate_fwd_impl(y: torch.Tensor, d_skip: torch.Tensor, z: torch.Tensor) -> torch.Tensor:
    """(y + d_skip) * silu(z) for (B,T,D) y and z (z rows may be strided)."""
    bt, t_len, d = y.shape
    out = y.new_empty((bt, t_len, d))
    with _on(y.device):
        rc = library().mhs_out_gate_fwd_f32(
            _ptr(y), _ptr(d_skip), _ptr(z), _conv_rows(z), _ptr(out), bt, t_len, d,
            _stream(y.device))
    _check(rc, "mhs_out_gate_fwd_f32")
    return out


out_gate_fwd = _register("out_gate_fwd", _out_gate_fwd_impl, (),
                         lambda y, d_skip, z: _check_gate("out_gate_fwd", y, d_skip, z))


@out_gate_fwd.register_fake
def _out_gate_fwd_fake(y, d_skip, z):
    return y.new_empty(y.shape)


def _out_gate_bwd_impl(y: torch.Tensor, d_skip: torch.Tensor, z: torch.Tensor, dout: torch.Tensor
                 ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dy, dd_skip, dz), dy and dz (B,T,D) contiguous."""
    bt, t_len, d = y.shape
    lib = library()
    dy = y.new_empty((bt, t_len, d))
    dz = y.new_empty((bt, t_len, d))
    dd = torch.empty_like(d_skip)
    ws_bytes = int(lib.mhs_out_gate_bwd_workspace_bytes(bt, t_len, d))
    if ws_bytes == 0:
        raise HipScanError(f"no output-gate workspace size for shape {(bt, t_len, d)}")
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=y.device)
    with _on(y.device):
        rc = lib.mhs_out_gate_bwd_f32(
            _ptr(y), _ptr(d_skip), _ptr(z), _rows(z), _ptr(dout), _ptr(dy), _ptr(dz), 0,
            _ptr(dd), _ptr(ws), ws_bytes, bt, t_len, d, _stream(y.device))
    _check(rc, "mhs_out_gate_bwd_f32")
    return dy, dd, dz


out_gate_bwd = _register(
    "out_gate_bwd", _out_gate_bwd_impl, (),
    lambda y, d_skip, z, dout: _check_gate("out_gate_bwd", y, d_skip, z, dout))


@out_gate_bwd.register_fake
def _out_gate_bwd_fake(y, d_skip, z, dout):
    return y.new_empty(y.shape), torch.empty_like(d_skip), y.new_empty(y.shape)


def _out_gate_bwd_into_impl(y: torch.Tensor, d_skip: torch.Tensor, z: torch.Tensor,
                            dout: torch.Tensor, dz: torch.Tensor
                            ) -> tuple[torch.Tensor, torch.Tensor]:
    """out_gate_bwd writing dz into the given (B,T,D) tensor, which may be a
    column slice of a wider one (the z half of the in_proj output's
    gradient); returns (dy, dd_skip)."""
    bt, t_len, d = y.shape
    lib = library()
    dy = y.new_empty((bt, t_len, d))
    dd = torch.empty_like(d_skip)
    ws_bytes = int(lib.mhs_out_gate_bwd_workspace_bytes(bt, t_len, d))
    if ws_bytes == 0:
        raise HipScanError(f"no output-gate workspace size for shape {(bt, t_len, d)}")
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=y.device)
    with _on(y.device):
        rc = lib.mhs_out_gate_bwd_f32(
            _ptr(y), _ptr(d_skip), _ptr(z), _rows(z), _ptr(dout), _ptr(dy), _ptr(dz), _rows(dz),
            _ptr(dd), _ptr(ws), ws_bytes, bt, t_len, d, _stream(y.device))
    _check(rc, "mhs_out_gate_bwd_f32")
    return dy, dd


out_gate_bwd_into = _register(
    "out_gate_bwd_into", _out_gate_bwd_into_impl, ("dz",),
    lambda y, d_skip, z, dout, dz: _check_gate("out_gate_bwd_into", y, d_skip, z, dout, dz))


@out_gate_bwd_into.register_fake
def _out_gate_bwd_into_fake(y, d_skip, z, dout, dz):
    return y.new_empty(y.shape), torch.empty_like(d_skip)


# ----------------------------------------------------------- cross-entropy

def _check_xent(what: str, logits, targets, lse=None, scale=None) -> None:
    """logits (R, V) fp32 contiguous, targets (R) int64 contiguous, lse (R)
    and scale (1) fp32, all on one ROCm device."""
    _on_one_device(what, logits, targets, lse, scale)
    _need(logits.dim() == 2 and targets.shape == (logits.shape[0],), what,
          f"logits must be (R, V) and targets (R,); got {tuple(logits.shape)}, "
          f"{tuple(targets.shape)}")
    _need(logits.shape[1] >= 1, what, "the vocabulary must not be empty")
    _need(targets.dtype == torch.int64, what, f"targets must be int64; got {targets.dtype}")
    _fp32(what, logits=logits, lse=lse, scale=scale)
    _shaped(what, "lse", lse, (logits.shape[0],))
    _shaped(what, "scale", scale, (1,))
    _dense(what, logits=logits, targets=targets, lse=lse)


def _xent_fwd_impl(logits: torch.Tensor, targets: torch.Tensor, ignore_index: int
                   ) -> tuple[torch.Tensor, torch.Tensor]:
    """(lse (R), loss_rows (R)) for logits (R, V) and targets (R)."""
    rows, vocab = logits.shape
    lse = logits.new_empty((rows,))
    loss_rows = logits.new_empty((rows,))
    with _on(logits.device):
        rc = library().mhs_xent_fwd_f32(_ptr(logits), _ptr(targets), _ptr(lse), _ptr(loss_rows),
                                        rows, vocab, ignore_index, _stream(logits.device))
    _check(rc, "mhs_xent_fwd_f32")
    return lse, loss_rows


xent_fwd = _register("xent_fwd", _xent_fwd_impl, (),
                     lambda logits, targets, ignore_index: _check_xent("xent_fwd", logits, targets))


@xent_fwd.register_fake
def _xent_fwd_fake(logits, targets, ignore_index):
    return logits.new_empty((logits.shape[0],)), logits.new_empty((logits.shape[0],))


def _xent_bwd_impl(logits: torch.Tensor, targets: torch.Tensor, lse: torch.Tensor,
                   scale: torch.Tensor, ignore_index: int) -> torch.Tensor:
    """dlogits (R, V), scale (1) = the loss's upstream gradient / rows not ignored."""
    rows, vocab = logits.shape
    dlogits = torch.empty_like(logits)
    with _on(logits.device):
        rc = library().mhs_xent_bwd_f32(_ptr(logits), _ptr(targets), _ptr(lse), _ptr(scale),
                                        _ptr(dlogits), rows, vocab, ignore_index,
                                        _stream(logits.device))
    _check(rc, "mhs_xent_bwd_f32")
    return dlogits


xent_bwd = _register(
    "xent_bwd", _xent_bwd_impl, (),
    lambda logits, targets, lse, scale, ignore_index:
    _check_xent("xent_bwd", logits, targets, lse, scale))


@xent_bwd.register_fake
def _xent_bwd_fake(logits, targets, lse, scale, ignore_index):
    return torch.empty_like(logits)


# ------------------------------------------------------------------ RMSNorm

NORM_MAX_COLS = 2048   # the kernels' limit: rows of at most 2048 features


def rmsnorm_supported(x: torch.Tensor) -> bool:
    """Whether the HIP RMSNorm takes rows of x's last dimension: fp32 on a ROCm
    device, a multiple of 4 features up to NORM_MAX_COLS, at least one row."""
    c = x.shape[-1] if x.dim() >= 1 else 0
    return (x.dtype == torch.float32 and x.is_cuda and torch.version.hip is not None
            and c % 4 == 0 and 4 <= c <= NORM_MAX_COLS and x.numel() > 0)


def _check_norm(what: str, x, weight, rstd=None, dy=None, dres=None, delta=None) -> None:
    """x (R, C) fp32 contiguous with C a multiple of 4 in [4, 2048]; weight
    (C) fp32; rstd (R) fp32; dy, dres, delta (R, C) fp32; all on one ROCm
    device and 16-byte aligned."""
    _on_one_device(what, x, weight, rstd, dy, dres, delta)
    _need(x.dim() == 2, what, f"x must be (rows, cols); got {tuple(x.shape)}")
    rows, cols = x.shape
    _need(cols % 4 == 0 and 4 <= cols <= NORM_MAX_COLS, what,
          f"cols must be a multiple of 4 in [4, {NORM_MAX_COLS}]; got {cols}")
    _fp32(what, x=x, weight=weight, rstd=rstd, dy=dy, dres=dres, delta=delta)
    _shaped(what, "weight", weight, (cols,))
    _shaped(what, "rstd", rstd, (rows,))
    _shaped(what, "dy", dy, (rows, cols))
    _shaped(what, "dres", dres, (rows, cols))
    _shaped(what, "delta", delta, (rows, cols))
    _dense(what, x=x, weight=weight, rstd=rstd, dy=dy, dres=dres, delta=delta)
    for name, t in (("x", x), ("weight", weight), ("rstd", rstd), ("dy", dy), ("dres", dres),
                    ("delta", delta)):
        _need(t is None or t.data_ptr() % 16 == 0, what, f"{name} must be 16-byte aligned")


def _rmsnorm_fwd_impl(x: torch.Tensor, weight: torch.Tensor, eps: float
                      ) -> tuple[torch.Tensor, torch.Tensor]:
    """(y (R, C), rstd (R)) for x (R, C): y = x * rstd * weight."""
    rows, cols = x.shape
    y = torch.empty_like(x)
    rstd = x.new_empty((rows,))
    with _on(x.device):
        rc = library().mhs_rmsnorm_fwd_f32(_ptr(x), _ptr(weight), _ptr(y), _ptr(rstd), rows, cols,
                                           eps, _stream(x.device))
    _check(rc, "mhs_rmsnorm_fwd_f32")
    return y, rstd


rmsnorm_fwd = _register("rmsnorm_fwd", _rmsnorm_fwd_impl, (),
                        lambda x, weight, eps: _check_norm("rmsnorm_fwd", x, weight))


@rmsnorm_fwd.register_fake
def _rmsnorm_fwd_fake(x, weight, eps):
    return torch.empty_like(x), x.new_empty((x.shape[0],))


def _add_rmsnorm_fwd_impl(x: torch.Tensor, delta: torch.Tensor, weight: torch.Tensor, eps: float
                          ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(x_out = x + delta, y = rms_norm(x_out), rstd) for x, delta (R, C)."""
    rows, cols = x.shape
    x_out = torch.empty_like(x)
    y = torch.empty_like(x)
    rstd = x.new_empty((rows,))
    with _on(x.device):
        rc = library().mhs_add_rmsnorm_fwd_f32(_ptr(x), _ptr(delta), _ptr(weight), _ptr(x_out),
                                               _ptr(y), _ptr(rstd), rows, cols, eps,
                                               _stream(x.device))
    _check(rc, "mhs_add_rmsnorm_fwd_f32")
    return x_out, y, rstd


add_rmsnorm_fwd = _register(
    "add_rmsnorm_fwd", _add_rmsnorm_fwd_impl, (),
    lambda x, delta, weight, eps: _check_norm("add_rmsnorm_fwd", x, weight, delta=delta))


@add_rmsnorm_fwd.register_fake
def _add_rmsnorm_fwd_fake(x, delta, weight, eps):
    return torch.empty_like(x), torch.empty_like(x), x.new_empty((x.shape[0],))


def _rmsnorm_bwd_impl(dy: torch.Tensor, x: torch.Tensor, weight: torch.Tensor,
                      rstd: torch.Tensor, dres: Optional[torch.Tensor]
                      ) -> tuple[torch.Tensor, torch.Tensor]:
    """(dx (R, C), dweight (C)); dres, the residual stream's other gradient,
    is added into dx when given."""
    rows, cols = x.shape
    dx = torch.empty_like(x)
    dweight = torch.empty_like(weight)
    lib = library()
    nbytes = int(lib.mhs_rmsnorm_bwd_workspace_bytes(rows, cols))
    ws = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=x.device)
    with _on(x.device):
        rc = lib.mhs_rmsnorm_bwd_f32(_ptr(dy), _ptr(x), _ptr(weight), _ptr(rstd), _ptr(dres),
                                     _ptr(dx), _ptr(dweight), _ptr(ws), nbytes, rows, cols,
                                     _stream(x.device))
    _check(rc, "mhs_rmsnorm_bwd_f32")
    return dx, dweight


rmsnorm_bwd = _register(
    "rmsnorm_bwd", _rmsnorm_bwd_impl, (),
    lambda dy, x, weight, rstd, dres: _check_norm("rmsnorm_bwd", x, weight, rstd, dy, dres))


@rmsnorm_bwd.register_fake
def _rmsnorm_bwd_fake(dy, x, weight, rstd, dres):
    return torch.empty_like(x), torch.empty_like(weight)
