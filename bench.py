#!/usr/bin/env python3
"""Benchmark of the MI355X selective scan (one JSON line on stdout).

Default workload: the fused selective scan, forward + backward, at the Mamba
training shape batch 16 x T 512 x d_inner 1536 x d_state 16, fp32. One step is
one forward + backward of the scan over one batch of synthetic inputs already
resident in HBM (x, B, C, dy ~ N(0,1); dt = softplus(N(-4,1)); Aneg[d,n] = n+1),
through the public autograd path (selective_scan_hip + backward).

Reported:
  value          whole-job tokens/s (batch*T per step / step time)
  ms_per_step    ms per fwd+bwd step (wall clock, synchronized)
  roofline       the dominant kernel launch (the backward: bwd kernel + its
                 reduction; the fixed order at this shape), timed live with HIP events around
                 it in every 4th timed step, on the launch stream: algorithmic
                 bytes / average duration vs 8 TB/s
  clock_settle   untimed steps run before the warmup until the GPU clock
                 is steady (about 40 ms of load from idle)
  cpu_baseline   selective_scan(impl="torch") fwd+bwd on the host CPU, same
                 inputs, all threads of the process's CPU share; the
                 long-sequence and prefill keys carry their own, each on the
                 whole workload, one rep in a child process under a
                 wall-clock limit (timeouts and out-of-memory are recorded),
                 with a bounded sample of the same sizes beside it

  train_80m      the 80M TinyMamba train step (fwd + bwd + AdamW) with the HIP
                 scan at batch 16 x seq 512: tokens/s and peak HBM

Other workloads (--workload): "train" (the 80M train step alone; --size 18M
for the reference bench's smaller size, --ref to add the torch scan at its
small size), "longt" (4 x 16384 x 2048 x 16 fwd+bwd, checkpoint-stride
sweep), "infer" (prefill 32 x 2048 x 4096 x 16 + 256 recurrent decode steps).

Only one GPU is used: --gpus N > 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = ("fwd+bwd scan ms & % HBM roofline (16x512x1536x16 fp32); 80M train tok/s")
HBM_PEAK_GBS = 8000.0
COPY_BYTES = 50_331_648      # calibration copy for the --pmc traffic figures


def scan_bytes(bt: int, t_len: int, d: int, n: int) -> dict:
    """Algorithmic (compulsory fp32) bytes: fwd reads x, dt, B, C, Aneg and writes
    y; bwd reads x, dt, dy, B, C, Aneg and writes dx, ddt, dB, dC, dAneg."""
    e, s, a = bt * t_len * d, bt * t_len * n, d * n
    return {"fwd": 4 * (3 * e + 2 * s + a), "bwd": 4 * (5 * e + 4 * s + 2 * a),
            "fwd_bwd": 4 * (8 * e + 6 * s + 3 * a)}


CPU_THREAD_CAP = 16   # the host CPU share of one GPU on the benchmark machines


def affinity_cpus() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_threads() -> int:
    """Threads for the CPU baseline: the process's CPU affinity, at most the
    host share of one GPU (CPU_THREAD_CAP; the affinity mask of a one-GPU job
    can name every core of the host while its fair share is 16)."""
    return max(1, min(affinity_cpus(), CPU_THREAD_CAP))


def keep_heap() -> str:
    """glibc: serve the CPU path's blocks from one heap (one arena, no mmap)
    and never trim it, so that later reps reuse the pages the first one
    faulted in instead of mapping and faulting fresh ones (mallopt
    M_ARENA_MAX 1, M_MMAP_MAX 0, M_TRIM_THRESHOLD off). Measured: the reps
    that hit millions of minor page faults took 4.6-5.5 s against 0.61 s for
    those that did not. Returns what was set."""
    import ctypes
    try:
        libc = ctypes.CDLL("libc.so.6")
        m_trim_threshold, m_mmap_max, m_arena_max = -1, -4, -8
        ok = (libc.mallopt(m_arena_max, 1) and libc.mallopt(m_mmap_max, 0)
              and libc.mallopt(m_trim_threshold, -1))
        return "glibc mallopt: one arena, no mmap, no trim" if ok else "glibc mallopt refused"
    except OSError:
        return "default allocator"


def make_inputs(bt, t_len, d, n, seed=2024):
    """Seeded synthetic scan inputs drawn on the CPU (torch generator)."""
    import torch
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(bt, t_len, d, generator=g)
    dt = torch.nn.functional.softplus(torch.randn(bt, t_len, d, generator=g) - 4.0)
    aneg = torch.arange(1, n + 1, dtype=torch.float32).repeat(d, 1)
    b_in = torch.randn(bt, t_len, n, generator=g)
    c_in = torch.randn(bt, t_len, n, generator=g)
    dy = torch.randn(bt, t_len, d, generator=g)
    return x, dt, aneg, b_in, c_in, dy


SETTLE_MS = 100.0
EVENT_EVERY = 4   # timed steps per step with per-launch HIP events
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000
USE_TORCH_EVENTS = False   # --torch-events: torch.cuda.Event instead of TimingEvent


class TimingEvent:
    """A HIP event for GPU timing only, recorded on torch's current stream and
    created with hipEventDisableSystemFence: recording it skips the
    system-scope cache writeback and invalidate that a default event (torch's
    torch.cuda.Event) performs, which costs the GPU several us per marker and
    slows the work right after it. Its timestamps are read after a device
    synchronize. The runtime is the one torch loaded (same soname)."""
    _hip = None

    @classmethod
    def _lib(cls):
        import ctypes
        if cls._hip is None:
            lib = ctypes.CDLL("libamdhip64.so.7")
            lib.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
            lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                ctypes.c_void_p]
            lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
            cls._hip = lib
        return cls._hip

    def __init__(self):
        import ctypes
        self.ev = ctypes.c_void_p()
        rc = self._lib().hipEventCreateWithFlags(ctypes.byref(self.ev),
                                                 HIP_EVENT_DISABLE_SYSTEM_FENCE)
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")

    def record(self):
        import ctypes
        import torch
        rc = self._lib().hipEventRecord(self.ev,
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_time(self, end: "TimingEvent") -> float:
        """Milliseconds from this event to `end`."""
        import ctypes
        ms = ctypes.c_float()
        rc = self._lib().hipEventElapsedTime(ctypes.byref(ms), self.ev, end.ev)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def __del__(self):
        if getattr(self, "ev", None) and TimingEvent._hip is not None:
            TimingEvent._hip.hipEventDestroy(self.ev)


def timing_event():
    """A GPU timing event on torch's current stream (TimingEvent, or
    torch.cuda.Event with --torch-events)."""
    import torch
    return torch.cuda.Event(enable_timing=True) if USE_TORCH_EVENTS else TimingEvent()


def event_kind() -> str:
    return ("torch.cuda.Event (default HIP event)" if USE_TORCH_EVENTS
            else "HIP event with hipEventDisableSystemFence")


def settle_clocks(fn, ms: float = SETTLE_MS) -> int:
    """Run fn() back to back, untimed, until ms of wall time have passed, so
    that what is timed next runs at the GPU's sustained clock. From idle,
    MI355X takes about 40 ms of continuous load to get there: a 16x512x1536x16
    scan fwd+bwd step takes 230 us at first and 187 us from then on. Returns
    the number of calls (after a first one, which also pays one-time costs
    such as loading the kernels and is not counted)."""
    import torch
    fn()
    torch.cuda.synchronize()
    t0, calls = time.perf_counter(), 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(4):
            fn()
        calls += 4
        torch.cuda.synchronize()
    return calls


def copy_bandwidth(nbytes: int = 256 << 20) -> dict:
    """A device-to-device copy of nbytes (read + write: 2 nbytes of traffic),
    timed with HIP events after a clock settle: the practical HBM rate next to
    the 8 TB/s spec. The copy is large enough that its kernel, not the host's
    per-call cost, sets the pace."""
    import torch
    src = torch.empty(nbytes // 4, device="cuda")
    dst = torch.empty_like(src)
    settle_clocks(lambda: dst.copy_(src), ms=30.0)
    ms = time_events(lambda: dst.copy_(src), 50)
    del src, dst
    return {"bytes": 2 * nbytes, "avg_ms": ms, "GBs": 2 * nbytes / (ms * 1e-3) / 1e9}


def time_events(fn, reps: int) -> float:
    """Average GPU duration (ms) of fn() over reps, HIP events on the current
    stream: one marker between consecutive calls ends one interval and starts
    the next."""
    import torch
    ev = [timing_event() for _ in range(reps + 1)]
    ev[0].record()
    for i in range(reps):
        fn()
        ev[i + 1].record()
    torch.cuda.synchronize()
    return sum(ev[i].elapsed_time(ev[i + 1]) for i in range(reps)) / reps


def cpu_baseline_scan(bt, t_len, d, n, reps: int = 3, warmup: int = 2, grad: bool = True,
                      what: str = "the full workload") -> dict:
    """selective_scan(impl='torch') on the host CPU: fwd+bwd (grad) or the
    forward under no_grad, on a (bt, t_len, d, n) workload; `warmup` untimed
    reps, then `reps` timed ones (value: their median). Every rep's time and
    minor page faults are reported. `what` says how the shape relates to the
    benchmarked workload."""
    import resource
    import statistics
    import torch
    from mamba_metal_scan_amd import selective_scan
    threads = cpu_threads()
    torch.set_num_threads(threads)
    heap = keep_heap()
    x, dt, aneg, b_in, c_in, dy = make_inputs(bt, t_len, d, n)
    kind = "fwd+bwd" if grad else "fwd (no_grad)"

    def one():
        leaves = [t.clone().requires_grad_(grad) for t in (x, dt, aneg, b_in, c_in)]
        f0 = resource.getrusage(resource.RUSAGE_SELF).ru_minflt
        t0 = time.perf_counter()
        if grad:
            y = selective_scan(*leaves, impl="torch")
            y.backward(dy)
        else:
            with torch.no_grad():
                selective_scan(*leaves, impl="torch")
        el = time.perf_counter() - t0
        return el, resource.getrusage(resource.RUSAGE_SELF).ru_minflt - f0

    try:
        warm = [one() for _ in range(warmup)]
        timed = [one() for _ in range(reps)]
    except (RuntimeError, MemoryError) as exc:   # e.g. out of host memory
        return {"value": None, "unit": "tokens/s", "cores": threads, "kind": "port",
                "sample": f"selective_scan(impl='torch') {kind} {bt}x{t_len}x{d}x{n}: "
                          f"failed ({type(exc).__name__})"}
    times = [t for t, _ in timed]
    el = statistics.median(times)
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": bt * t_len / el, "unit": "tokens/s", "cores": threads, "kind": "port",
            "ms_per_step": el * 1e3, "min_ms": min(times) * 1e3, "cpu": cpu_model,
            "affinity_cpus": affinity_cpus(), "thread_cap": CPU_THREAD_CAP, "heap": heap,
            "rep_ms": [round(t * 1e3, 1) for t in times],
            "warmup_ms": [round(t * 1e3, 1) for t, _ in warm],
            "rep_minor_faults": [f for _, f in timed],
            "warmup_minor_faults": [f for _, f in warm],
            "sample": f"selective_scan(impl='torch') {kind} on {bt}x{t_len}x{d}x{n} ({what}), "
                      f"{warmup} warm-up + median of {reps} reps, torch CPU threads={threads}"}


# Wall-clock limits of the CPU baselines that run in a child process. The
# limits stay under three minutes, so that a run is never silent for longer.
CPU_CHILD_LIMIT_S = {"longt": 150, "infer": 120}


# The bounded samples run first in the same child: (batch, steps, d_inner,
# d_state) sequences of the workload's other sizes, short enough for seconds.
CPU_CHILD_SAMPLE = {"longt": (4, 1024, 2048, 16), "infer": (32, 256, 4096, 16)}


def cpu_baseline_child(workload: str) -> dict:
    """The CPU baseline of a whole workload, one rep, in a fresh child
    process under a wall-clock limit: "longt" (4 x 16384 x 2048 x 16
    fwd+bwd; the torch path keeps a tape of about 26 GB) or "infer" (the
    32 x 2048 x 4096 x 16 prefill under no_grad). The child first times a
    bounded sample of the same shape ("sample"), then the whole workload. A
    child that runs out of time or host memory is recorded as such (value
    None, "result" the reason, the sample kept), not retried."""
    import subprocess
    limit = CPU_CHILD_LIMIT_S[workload]
    bt, t_len, d, n = {"longt": LONGT, "infer": INFER}[workload]
    kind = "fwd+bwd" if workload == "longt" else "fwd (no_grad)"
    what = (f"selective_scan(impl='torch') {kind} on {bt}x{t_len}x{d}x{n} (the full workload), "
            f"one rep in a child process, wall-clock limit {limit} s")
    cmd = [sys.executable, str(ROOT / "bench.py"), "--cpu-baseline-only", workload]
    print(f"cpu baseline {workload}: started, limit {limit} s", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    failed = None
    try:
        res = subprocess.run(cmd, stdout=subprocess.PIPE, text=True, timeout=limit)
        stdout, rc = res.stdout, res.returncode
    except subprocess.TimeoutExpired as exc:
        stdout = exc.stdout.decode() if isinstance(exc.stdout, bytes) else (exc.stdout or "")
        rc, failed = None, f"timeout after {limit} s"
    wall = time.perf_counter() - t0
    lines = []
    for ln in stdout.splitlines():   # a line cut short by the kill is dropped
        try:
            lines.append(json.loads(ln))
        except ValueError:
            pass
    if rc:
        sig = -rc if rc < 0 else None
        failed = (f"killed by signal {sig}" + (" (out of host memory)" if sig == 9 else "")
                  if sig else f"exit status {rc}")
    print(f"cpu baseline {workload}: ended after {wall:.1f} s"
          + (f" ({failed})" if failed else ""), file=sys.stderr, flush=True)
    sample = lines[0] if lines else None
    if failed or len(lines) < 2:
        return {"value": None, "unit": "tokens/s", "cores": cpu_threads(), "kind": "port",
                "result": failed or "no result", "sample": what, "bounded_sample": sample}
    out = lines[1]
    out["sample"] = what + (f"; {out['result']}" if out.get("result") else "")
    out["child_wall_s"] = round(wall, 1)
    out["bounded_sample"] = sample
    return out


def cpu_baseline_only(workload: str) -> int:
    """The child of cpu_baseline_child (touches no GPU): one JSON line for
    the bounded sample, then one for the whole workload."""
    grad = workload == "longt"
    full = LONGT if grad else INFER
    sb, st, sd, sn = CPU_CHILD_SAMPLE[workload]
    r = cpu_baseline_scan(sb, st, sd, sn, reps=1, warmup=0, grad=grad,
                          what=f"a {st}-step sequence of the workload's other sizes")
    print(json.dumps(r), flush=True)
    print(f"cpu baseline {workload}: sample done ({r.get('ms_per_step', 0) / 1e3:.1f} s), "
          f"whole workload next", file=sys.stderr, flush=True)
    r = cpu_baseline_scan(*full, reps=1, warmup=0, grad=grad)
    if r.get("value") is None:
        r["result"] = r["sample"].rsplit(": ", 1)[-1]
    print(json.dumps(r), flush=True)
    return 0


def run_launches(args) -> None:
    """Profiling driver: the scan's forward and backward launches (no timing,
    no CPU work) and a calibration copy of a known byte count, for
    `rocprofv3 --kernel-trace --stats` and `rocprofv3 --pmc ...` passes."""
    import torch
    from mamba_metal_scan_amd import _native   # registers the mamba_hip ops
    _native.library()
    bt, t_len, d, n = args.batch, args.seqlen, args.d_inner, args.d_state
    dev = torch.device("cuda", 0)
    x, dt, aneg, b_in, c_in, dy = (t.to(dev) for t in make_inputs(bt, t_len, d, n))
    for i in range(args.launches):
        if args.forward_only:
            # the inference forward: y and the final state, no checkpoints
            torch.ops.mamba_hip.scan_fwd(x, dt, aneg, b_in, c_in, args.chunk, False)
            continue
        _, ckpt, _ = torch.ops.mamba_hip.scan_fwd(x, dt, aneg, b_in, c_in, args.chunk, True)
        torch.ops.mamba_hip.scan_bwd(x, dt, aneg, b_in, c_in, dy, None, ckpt, args.chunk)
    src = torch.empty(COPY_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(args.launches):
        dst.copy_(src)
    torch.cuda.synchronize()
    ops = "scan_fwd without checkpoints" if args.forward_only else "scan_fwd, scan_bwd"
    print(f"launches done: {args.launches} x ({ops}) at {bt}x{t_len}x{d}x{n} "
          f"chunk {args.chunk}, {args.launches} x copy of {COPY_BYTES} B", flush=True)


def _short_kernel(name: str) -> str:
    for key, short in (("fwd_kernel", "fwd_kernel"), ("bwd_reduce", "bwd_reduce_kernel"),
                       ("bwd_kernel", "bwd_kernel"), ("copyBuffer", "copy")):
        if key in name:
            return short
    return name[:40]


PROFILE_RUN_NOTE = ("All commands run from /tmp with `TMPDIR=/tmp`, `bench.py` standing for the "
                    "path of the repository's bench.py; OUT is the output folder.")
ISSUE_COUNTERS = ("GRBM_GUI_ACTIVE SQ_WAVES SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_VALU2 SQ_INSTS_VALU "
                  "SQ_INSTS_VALU_TRANS_F32 SQ_WAVE_CYCLES SQ_LDS_BANK_CONFLICT")
N_XCD, N_CU = 8, 256   # MI355X: GRBM_GUI_ACTIVE is summed over its 8 XCDs


def issue_counter_lines(mean: dict) -> list:
    """Markdown for the third pmc pass: per scan kernel, its GPU-clock cycles
    and the shares of them the CUs spent issuing VALU instructions, with two
    VALU instructions issued together (a transcendental beside another), with
    resident waves, and stalled on LDS bank conflicts. SQ_* cycle counters
    are in quad-cycles summed over the SIMDs of each CU."""
    out = ["", "## Issue counters", "",
           f"Kernel cycles = GRBM_GUI_ACTIVE / {N_XCD} (the counter is summed over the XCDs). "
           f"VALU busy = SQ_ACTIVE_INST_VALU / ({N_CU} CUs x cycles); dual issue = "
           "SQ_ACTIVE_INST_VALU2 / SQ_ACTIVE_INST_VALU; resident waves per CU = "
           "4 x SQ_WAVE_CYCLES / (CUs x cycles); LDS conflict = SQ_LDS_BANK_CONFLICT / "
           "(CUs x cycles); VALU instructions and v_exp_f32 per wave.", "",
           "| kernel | cycles | VALU busy | dual issue | waves / CU | LDS conflict "
           "| VALU / wave | exp / wave |", "|---|---|---|---|---|---|---|---|"]
    for kern in ("fwd_kernel", "bwd_kernel"):
        g = lambda c: mean.get((kern, c), 0.0)
        cyc = g("GRBM_GUI_ACTIVE") / N_XCD
        waves = max(g("SQ_WAVES"), 1.0)
        out.append(f"| {kern} | {cyc:.0f} | {g('SQ_ACTIVE_INST_VALU') / (N_CU * cyc):.2f} | "
                   f"{g('SQ_ACTIVE_INST_VALU2') / max(g('SQ_ACTIVE_INST_VALU'), 1):.2f} | "
                   f"{4 * g('SQ_WAVE_CYCLES') / (N_CU * cyc):.1f} | "
                   f"{g('SQ_LDS_BANK_CONFLICT') / (N_CU * cyc):.3f} | "
                   f"{g('SQ_INSTS_VALU') / waves:.0f} | {g('SQ_INSTS_VALU_TRANS_F32') / waves:.0f} |")
    return out


COUNTERS_NAME = "scan_{shape}_counters.json"
N_SIMD = 4 * N_CU


def shape_tag(bt, t_len, d, n) -> str:
    return f"{bt}x{t_len}x{d}x{n}"


def reduction_name(bt, t_len, d, n, chunk):
    """'fixed' or 'atomic': the reduction the backward uses at this shape."""
    from mamba_metal_scan_amd import _native
    mode = _native.bwd_reduction(bt, t_len, d, n, chunk)
    return "atomic" if mode == _native.REDUCTION_ATOMIC else "fixed"


def load_counters(bt, t_len, d, n, chunk):
    """The committed counter summary of this workload (None if there is none,
    or it was taken at another checkpoint stride or reduction)."""
    from mamba_metal_scan_amd import _native
    path = ROOT / "profiles" / COUNTERS_NAME.format(shape=shape_tag(bt, t_len, d, n))
    try:
        c = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    red = reduction_name(bt, t_len, d, n, chunk)
    if c.get("chunk") != chunk or c.get("reduction") != red:
        return None
    return c


def valu_block(c):
    """VALU issue of the scan kernels from the committed counters: the lane
    operations per second of SQ_INSTS_VALU (wave instructions x 64 lanes)
    over the kernel-trace duration, against 1024 SIMDs x 16 lanes per clock
    (non-packed fp32; the clock is GRBM_GUI_ACTIVE over the duration), and the
    share of cycles the VALUs were busy (SQ_ACTIVE_INST_VALU)."""
    if not c:
        return None
    out = {"bound": "valu", "unit": "G lane-op/s",
           "source": f"profiles/{COUNTERS_NAME.format(shape=c['shape'])}"}
    for name in ("bwd_kernel", "fwd_kernel"):
        k = c["kernels"].get(name)
        if not k or "valu_insts" not in k:
            return None
        sec = k["duration_us"] * 1e-6
        clk = k["cycles"] / sec
        achieved = k["valu_insts"] * 64 / sec
        peak = N_SIMD * 16 * clk
        entry = {"achieved": achieved / 1e9, "peak": peak / 1e9, "frac": achieved / peak,
                 "busy": k["valu_busy"], "clock_GHz": clk / 1e9,
                 "valu_insts_per_wave": k["valu_insts"] / k["waves"],
                 "duration_us": k["duration_us"]}
        if name == "bwd_kernel":
            out.update({"kernel": name, **entry})
        else:
            out["fwd_kernel"] = entry
    return out


def _read_pmc(root: str) -> dict:
    """Mean counter value per (kernel, counter) over every counter-collection
    CSV under root."""
    import csv
    import glob
    vals: dict = {}
    for f in glob.glob(os.path.join(root, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            k = (_short_kernel(r["Kernel_Name"]), r["Counter_Name"])
            vals.setdefault(k, []).append(float(r["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in vals.items()}


def traced_step_us(out_dir: str):
    """us per autograd step that bench.py printed under the kernel tracer
    (OUT/kt.log, the traced command's output), or None."""
    log = os.path.join(out_dir, "kt.log")
    if not os.path.exists(log):
        return None
    for line in open(log):
        if line.startswith("{"):
            try:
                return 1e3 * float(json.loads(line)["ms_per_step"])
            except (ValueError, KeyError):
                return None
    return None


def trace_spans(trace: str, n_steps: int):
    """From a rocprofv3 kernel trace (run_kernel_trace.csv) of `bench.py
    --steps n_steps --no-extra --no-train`: the timed steps' per-kernel
    durations (us) and their launch spans (`spans`, None where the trace
    does not have that shape). The timed steps are the last n_steps
    (forward, backward, reduction) dispatch triples."""
    import csv
    durs: dict = {}
    spans = None
    if os.path.exists(trace):
        rows = sorted(csv.DictReader(open(trace)), key=lambda r: int(r["Start_Timestamp"]))
        # The timed steps' launches as the bench's events bracket them: the
        # backward launch from bwd_kernel's start to bwd_reduce_kernel's end,
        # and the idle gaps before each forward and each backward (markers).
        scan = [(_short_kernel(r["Kernel_Name"]), int(r["Start_Timestamp"]),
                 int(r["End_Timestamp"])) for r in rows
                if _short_kernel(r["Kernel_Name"]) in ("fwd_kernel", "bwd_kernel",
                                                       "bwd_reduce_kernel")]
        end = len(scan)
        steps = [scan[i:i + 3] for i in range(end - 3 * n_steps, end, 3)] if end > 0 else []
        if steps and all([k[0] for k in st] == ["fwd_kernel", "bwd_kernel", "bwd_reduce_kernel"]
                         for st in steps):
            n = len(steps)
            for st in steps:
                for name, t0, t1 in st:
                    durs.setdefault(name, []).append((t1 - t0) / 1e3)
            spans = {"steps": n,
                     "fwd_us": sum(st[0][2] - st[0][1] for st in steps) / n / 1e3,
                     "bwd_launch_us": sum(st[2][2] - st[1][1] for st in steps) / n / 1e3,
                     "gap_before_bwd_us": sum(st[1][1] - st[0][2] for st in steps) / n / 1e3,
                     "gap_before_fwd_us": sum(b[0][1] - a[2][2] for a, b in zip(steps, steps[1:]))
                     / max(n - 1, 1) / 1e3,
                     "steps_with_gaps": sum(1 for st in steps if st[1][1] - st[0][2] > 1000)}
    return durs, spans


def pmc_summary(args) -> None:
    """Per-launch HBM traffic from two rocprofv3 --pmc passes (FETCH_SIZE, then
    WRITE_SIZE, KiB per dispatch), each scaled by what the counter reads for
    the calibration copy of COPY_BYTES; VALU issue counters from a third pass;
    kernel durations from a --kernel-trace --stats run (kt/). Writes
    profiles/scan_<shape>_counters.json (what bench.py reports from) and
    profiles/scan_<shape>.md, and prints the markdown."""
    import csv
    from mamba_metal_scan_amd import _native
    mean = _read_pmc(args.pmc_summary)
    fetch_factor = COPY_BYTES / (mean[("copy", "FETCH_SIZE")] * 1024)
    write_factor = COPY_BYTES / (mean[("copy", "WRITE_SIZE")] * 1024)
    shape = (args.batch, args.seqlen, args.d_inner, args.d_state)
    tag = shape_tag(*shape)
    nbytes = scan_bytes(*shape)
    durs, spans = trace_spans(os.path.join(args.pmc_summary, "kt", "run_kernel_trace.csv"),
                              args.steps)
    kernels = {}
    for kern in ("fwd_kernel", "bwd_kernel", "bwd_reduce_kernel"):
        if (kern, "FETCH_SIZE") not in mean:
            continue
        rd = mean[(kern, "FETCH_SIZE")] * 1024 * fetch_factor
        wr = mean[(kern, "WRITE_SIZE")] * 1024 * write_factor
        k = {"read_bytes": rd, "write_bytes": wr, "hbm_bytes": rd + wr}
        last = durs.get(kern, [])[-args.steps:]
        if last:
            k["duration_us"] = sum(last) / len(last)
        if (kern, "SQ_INSTS_VALU") in mean:
            cyc = mean[(kern, "GRBM_GUI_ACTIVE")] / N_XCD
            k.update({"cycles": cyc, "valu_insts": mean[(kern, "SQ_INSTS_VALU")],
                      "waves": mean[(kern, "SQ_WAVES")],
                      "valu_busy": mean[(kern, "SQ_ACTIVE_INST_VALU")] / (N_CU * cyc),
                      "valu_dual_issue": mean[(kern, "SQ_ACTIVE_INST_VALU2")]
                      / max(mean[(kern, "SQ_ACTIVE_INST_VALU")], 1.0),
                      "exp_insts": mean[(kern, "SQ_INSTS_VALU_TRANS_F32")],
                      "lds_bank_conflict": mean[(kern, "SQ_LDS_BANK_CONFLICT")] / (N_CU * cyc)})
        kernels[kern] = k
    bwd_total = sum(kernels[k]["hbm_bytes"] for k in ("bwd_kernel", "bwd_reduce_kernel")
                    if k in kernels)
    extra = " ".join(f"--{k.replace('_', '-')} {getattr(args, k)}"
                     for k, dflt in (("batch", 16), ("seqlen", 512), ("d_inner", 1536),
                                     ("d_state", 16), ("chunk", 16)) if getattr(args, k) != dflt)
    out = {
        "shape": tag, "chunk": args.chunk,
        "reduction": reduction_name(*shape, args.chunk),
        "workload": f"selective_scan {tag} chunk {args.chunk}",
        "bwd_launch": {"hbm_bytes": bwd_total, "algorithmic_bytes": nbytes["bwd"],
                       "kernels": "bwd_kernel + bwd_reduce_kernel"},
        "fwd_launch": {"hbm_bytes": kernels["fwd_kernel"]["hbm_bytes"],
                       "algorithmic_bytes": nbytes["fwd"]},
        "kernels": kernels,
        "trace_launch": spans,
        "calibration": {"copy_bytes": COPY_BYTES, "fetch_factor": fetch_factor,
                        "write_factor": write_factor},
        "commands": {
            "kernel_trace": "rocprofv3 --kernel-trace --stats -d OUT/kt -o run --output-format csv "
                            f"-- python3 bench.py --steps {args.steps} --warmup {args.warmup} "
                            f"--no-cpu-baseline --no-train --no-extra {extra}".strip() + " > OUT/kt.log",
            "fetch": f"rocprofv3 --pmc FETCH_SIZE -d OUT/fetch -o run --output-format csv -- "
                     f"python3 bench.py --launches 5 {extra}".strip(),
            "write": f"rocprofv3 --pmc WRITE_SIZE -d OUT/write -o run --output-format csv -- "
                     f"python3 bench.py --launches 5 {extra}".strip(),
            "valu": f"rocprofv3 --pmc {ISSUE_COUNTERS} -d OUT/valu -o run --output-format csv "
                    f"-- python3 bench.py --launches 5 {extra}".strip(),
            "summary": f"python3 bench.py --pmc-summary OUT {extra}".strip()},
    }
    path = ROOT / "profiles" / COUNTERS_NAME.format(shape=tag)
    path.write_text(json.dumps(out, indent=1) + "\n")
    lines = [f"# Scan kernels at {tag}, chunk {args.chunk} (fp32, {out['reduction']}-order "
             "reduction): kernel time, HBM traffic, VALU issue", "",
             PROFILE_RUN_NOTE, "",
             "    " + out["commands"]["kernel_trace"], "    " + out["commands"]["fetch"],
             "    " + out["commands"]["write"], "    " + out["commands"]["valu"],
             "    " + out["commands"]["summary"], ""]
    stats = os.path.join(args.pmc_summary, "kt", "run_kernel_stats.csv")
    if os.path.exists(stats):
        lines += ["## Kernel trace", "",
                  f"| kernel | calls | avg us | min us | max us | avg us, last {args.steps} |",
                  "|---|---|---|---|---|---|"]
        for r in csv.DictReader(open(stats)):
            last = durs.get(_short_kernel(r["Name"]), [])[-args.steps:]
            tail = f"{sum(last) / len(last):.1f}" if len(last) == args.steps else ""
            lines.append(f"| `{r['Name'][:60]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} "
                         f"| {float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | {tail} |")
        lines += ["", "The backward launch (the `scan_bwd` op) is `bwd_kernel` + "
                  "`bwd_reduce_kernel`. The calls include bench.py's untimed clock-settle "
                  "steps, which begin at the idle clock; the last column averages the "
                  "timed steps' launches only.", ""]
        if spans:
            kernel_us = spans["fwd_us"] + spans["bwd_launch_us"]
            host_us = traced_step_us(args.pmc_summary)
            if host_us is not None and host_us > kernel_us + 10:
                why = (f"the traced run's host loop took {host_us:.1f} us per autograd step "
                       f"against {kernel_us:.1f} us of kernel time, so the GPU waited for the "
                       "host's launches (the tracer's interception slows the host; untraced, "
                       "bench.py's step takes about the kernel time)")
            else:
                why = ("bench.py times one step in four with events, and each marker holds "
                       "the queue for a few us; bench.py's event-timed launches include one "
                       "such marker each, and so read a few us above these spans")
            lines += [f"Over the {spans['steps']} timed steps the backward launch spans "
                      f"{spans['bwd_launch_us']:.1f} us from `bwd_kernel`'s start to "
                      f"`bwd_reduce_kernel`'s end, the forward {spans['fwd_us']:.1f} us; the "
                      f"GPU idles {spans['gap_before_bwd_us']:.1f} us before a backward and "
                      f"{spans['gap_before_fwd_us']:.1f} us before a forward on average "
                      f"(a gap over 1 us before the backward at {spans['steps_with_gaps']} of "
                      f"{spans['steps']} steps): {why}.", ""]
    lines += ["## HBM traffic per launch", "",
              f"Calibration: a {COPY_BYTES} B device copy reads FETCH_SIZE x{fetch_factor:.3f} and "
              f"WRITE_SIZE x{write_factor:.3f} of its true bytes; the figures below are scaled by "
              f"those factors (KiB counters x 1024 x factor).", "",
              "| kernel | read MB | write MB | HBM MB | algorithmic MB |", "|---|---|---|---|---|"]
    for kern, r in kernels.items():
        alg = {"fwd_kernel": nbytes["fwd"], "bwd_kernel": nbytes["bwd"]}.get(kern)
        lines.append(f"| {kern} | {r['read_bytes'] / 1e6:.1f} | {r['write_bytes'] / 1e6:.1f} | "
                     f"{r['hbm_bytes'] / 1e6:.1f} | {'' if alg is None else f'{alg / 1e6:.1f}'} |")
    if ("bwd_kernel", "SQ_ACTIVE_INST_VALU") in mean:
        lines += issue_counter_lines(mean)
    md = ROOT / "profiles" / f"scan_{tag}.md"
    md.write_text("\n".join(lines) + "\n")
    print("\n".join(lines))
    print(f"\nwrote {path.relative_to(ROOT)} and {md.relative_to(ROOT)}")


TRAIN_GROUPS = (  # (label, substrings of the kernel name), first match wins
    ("fp32 GEMMs (rocBLAS / hipBLASLt)", ("Cijk_", "gemm", "Gemm")),
    ("HIP scan (fwd, bwd, reduce)", ("mhs::fwd_kernel", "mhs::bwd_kernel", "mhs::bwd_reduce")),
    ("HIP conv1d + SiLU", ("mhs::conv",)),
    ("HIP output gate", ("mhs::out_gate",)),
    ("cross-entropy (HIP, or the framework's softmax)", ("mhs::xent", "SoftMax", "nll_loss")),
    ("AdamW (fused)", ("FusedOpti",)),
    ("RMSNorm (HIP, or the framework's rms_norm)", ("mhs::rmsnorm", "layer_norm", "rms_norm",
                                                    "RmsNorm")),
)


def kernel_label(name: str) -> str:
    """A scan kernel's role from its template arguments (the demangled name):
    fwd_kernel<NPL, G, MINW, KALIGNED, GATED, PASS, ES> and
    bwd_kernel<NPL, G, MINW, GATED, CARRY, ES, ATOM, SWEEP>."""
    import re
    m = re.search(r"(fwd_kernel|bwd_kernel)<([^>]*)>", name)
    if m:
        a = [v.strip() for v in m.group(2).split(",")]
        if m.group(1) == "fwd_kernel":
            return {"0": "forward", "1": "forward carry pass", "2": "backward checkpoint recompute"}[a[5]]
        if a[4] == "true":
            return "backward carry pass"
        red = "atomics" if len(a) > 6 and a[6] == "true" else "fixed order"
        sweep = " swept" if len(a) > 7 and a[7] != "0" else ""
        return f"backward{sweep} ({red})"
    for key, short in (("bwd_reduce", "backward reduction"), ("zero_grads", "zero fill"),
                       ("copyBuffer", "copy")):
        if key in name:
            return short
    return name[:40]


def kernel_counters(args) -> None:
    """Per-kernel counters of one scan workload (args' shape and --chunk),
    every kernel labelled by its role: kernel-trace durations (OUT/kt, a
    `--launches` run), HBM traffic from FETCH_SIZE and WRITE_SIZE passes
    (copy-calibrated) and the VALU issue counters. Writes
    profiles/scan_<shape>_chunk<K>_kernels.md and prints it."""
    import csv
    import glob
    root = args.kernel_counters
    vals: dict = {}
    for f in glob.glob(os.path.join(root, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            vals.setdefault((kernel_label(r["Kernel_Name"]), r["Counter_Name"]),
                            []).append(float(r["Counter_Value"]))
    mean = {k: sum(v) / len(v) for k, v in vals.items()}
    # A counter summed over a launch's dispatches of one kernel role (the
    # forward's carry pass and main pass are separate roles; a role
    # dispatched once per launch is the common case).
    per_launch = {k: sum(v) / args.launches for k, v in vals.items()}
    fetch_factor = COPY_BYTES / (mean[("copy", "FETCH_SIZE")] * 1024)
    write_factor = COPY_BYTES / (mean[("copy", "WRITE_SIZE")] * 1024)
    durs: dict = {}
    trace = os.path.join(root, "kt", "run_kernel_trace.csv")
    for r in csv.DictReader(open(trace)):
        durs.setdefault(kernel_label(r["Kernel_Name"]), []).append(
            (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    shape = (args.batch, args.seqlen, args.d_inner, args.d_state)
    tag = shape_tag(*shape)
    nbytes = scan_bytes(*shape)
    extra = (f"--batch {args.batch} --seqlen {args.seqlen} --d-inner {args.d_inner} "
             f"--d-state {args.d_state} --chunk {args.chunk}"
             + (f" --reduction {args.reduction}" if args.reduction != "auto" else "")
             + (" --forward-only" if args.forward_only else ""))
    # One --pmc pass per sub-folder, with the counters its CSV holds.
    cmds = [f"rocprofv3 --kernel-trace --stats -d OUT/kt -o run --output-format csv -- "
            f"python3 bench.py --launches {args.launches} {extra}"]
    for sub in sorted(os.listdir(root)):
        f = glob.glob(os.path.join(root, sub, "*counter_collection.csv"))
        if not f:
            continue
        names = list(dict.fromkeys(r["Counter_Name"] for r in csv.DictReader(open(f[0]))))
        cmds.append(f"rocprofv3 --pmc {' '.join(names)} -d OUT/{sub} -o run --output-format csv "
                    f"-- python3 bench.py --launches {args.launches} {extra}")
    cmds.append(f"python3 bench.py --kernel-counters OUT --launches {args.launches} {extra}")
    what = ("the forward without checkpoints" if args.forward_only
            else f"{reduction_name(*shape, args.chunk)} reduction")
    lines = [f"# Scan kernels at {tag}, chunk {args.chunk} (fp32, {what}): per-kernel time, "
             "HBM traffic, VALU issue", "", PROFILE_RUN_NOTE, ""] + ["    " + c for c in cmds] + [
        "", f"{args.launches} launches of the forward"
        + (" without checkpoints (y and the final state)" if args.forward_only
           else " and the backward") + ". Durations: kernel-trace "
        "average over all dispatches (the first launch included). HBM traffic per launch: the "
        f"counters summed over a launch's dispatches of the kernel, scaled by what a "
        f"{COPY_BYTES} B device copy reads (FETCH_SIZE x{fetch_factor:.3f}, WRITE_SIZE "
        f"x{write_factor:.3f}). Issue counters as in `scan_16x512x1536x16.md`: cycles = "
        f"GRBM_GUI_ACTIVE / {N_XCD} per dispatch, VALU busy = SQ_ACTIVE_INST_VALU / ({N_CU} "
        "CUs x cycles), waves / CU = 4 x SQ_WAVE_CYCLES / (CUs x cycles), VALU / wave = "
        "SQ_INSTS_VALU / SQ_WAVES.", "",
        "| kernel | dispatches per launch | avg us | read MB | write MB | HBM MB | achieved GB/s "
        "| cycles | VALU busy | waves / CU | VALU / wave | LDS conflict |",
        "|---|---|---|---|---|---|---|---|---|---|---|---|"]
    order = ["forward carry pass", "forward", "backward checkpoint recompute", "zero fill",
             "backward carry pass"]
    labels = sorted({k for k, _ in vals} - {"copy"},
                    key=lambda k: (order.index(k) if k in order else len(order), k))
    tot = {"fwd": 0.0, "bwd": 0.0, "fwd_us": 0.0, "bwd_us": 0.0}
    for lab in labels:
        g = lambda c: mean.get((lab, c), 0.0)
        d = durs.get(lab, [])
        disp = len(d) / args.launches if d else 0
        avg = sum(d) / len(d) if d else 0.0
        rd = per_launch.get((lab, "FETCH_SIZE"), 0.0) * 1024 * fetch_factor
        wr = per_launch.get((lab, "WRITE_SIZE"), 0.0) * 1024 * write_factor
        side = "fwd" if lab.startswith("forward") else "bwd"
        tot[side] += rd + wr
        tot[side + "_us"] += avg * disp
        row = f"| {lab} | {disp:g} | {avg:.1f} | {rd / 1e6:.1f} | {wr / 1e6:.1f} | " \
              f"{(rd + wr) / 1e6:.1f} | {(rd + wr) / (avg * disp * 1e-6) / 1e9 if avg else 0:.0f} | "
        if (lab, "SQ_INSTS_VALU") in mean:
            cyc = g("GRBM_GUI_ACTIVE") / N_XCD
            row += (f"{cyc:.0f} | {g('SQ_ACTIVE_INST_VALU') / (N_CU * cyc):.2f} | "
                    f"{4 * g('SQ_WAVE_CYCLES') / (N_CU * cyc):.1f} | "
                    f"{g('SQ_INSTS_VALU') / max(g('SQ_WAVES'), 1.0):.0f} | "
                    f"{g('SQ_LDS_BANK_CONFLICT') / (N_CU * cyc):.3f} |")
        else:
            row += " |  |  |  |  |"
        lines.append(row)
    lines += ["", "| launch | kernel time us | HBM MB | algorithmic MB | HBM / algorithmic "
              "| algorithmic GB/s over kernel time |", "|---|---|---|---|---|---|"]
    for side, name in (("fwd", "forward"), ("bwd", "backward")):
        alg = nbytes[side]
        us = tot[side + "_us"]
        if not us:
            continue
        lines.append(f"| {name} | {us:.1f} | {tot[side] / 1e6:.1f} | {alg / 1e6:.1f} | "
                     f"{tot[side] / alg:.2f} | {alg / (us * 1e-6) / 1e9 if us else 0:.0f} |")
    known = {"FETCH_SIZE", "WRITE_SIZE"} | set(ISSUE_COUNTERS.split())
    other = sorted({c for _, c in vals} - known)
    if other:
        lines += ["", "Other counters, summed over a launch's dispatches of the kernel (the "
                  "`_sum` counters are summed over the hardware instances):", "",
                  "| kernel | " + " | ".join(other) + " |",
                  "|---|" + "---|" * len(other)]
        for lab in labels:
            lines.append(f"| {lab} | " + " | ".join(
                f"{per_launch[(lab, c)]:.4g}" if (lab, c) in per_launch else ""
                for c in other) + " |")
    red = "" if args.reduction == "auto" else f"_{args.reduction}"
    fo = "_forward" if args.forward_only else ""
    md = ROOT / "profiles" / f"scan_{tag}_chunk{args.chunk}{red}{fo}_kernels.md"
    md.write_text("\n".join(lines) + "\n")
    print("\n".join(lines))
    print(f"\nwrote {md.relative_to(ROOT)}")


def trace_summary(args) -> None:
    """Per-step kernel time of the train step from a rocprofv3 --kernel-trace
    --stats run under args.trace_summary (kt/run_kernel_stats.csv), grouped
    by kind; the run covered args.warmup + args.steps steps. For the longt
    and infer workloads, the per-kernel table of such a run. Writes the
    markdown under profiles/ and prints it."""
    import csv
    stats = os.path.join(args.trace_summary, "kt", "run_kernel_stats.csv")
    rows = list(csv.DictReader(open(stats)))
    if args.workload in ("longt", "infer"):
        workload_trace_summary(args, rows)
        return
    n = args.warmup + args.steps
    per = lambda r: float(r["TotalDurationNs"]) / n / 1e3   # us per step
    groups: dict = {}
    for r in rows:
        label = next((g for g, keys in TRAIN_GROUPS if any(k in r["Name"] for k in keys)),
                     "other framework ops")
        groups[label] = groups.get(label, 0.0) + per(r)
    total = sum(groups.values())
    lines = ["# 80M TinyMamba train step (batch 16 x seq 512, fp32): kernel time per step", "",
             PROFILE_RUN_NOTE, "",
             "    rocprofv3 --kernel-trace --stats -d OUT/kt -o run --output-format csv -- \\",
             f"        python3 bench.py --workload train --steps {args.steps} --warmup {args.warmup}",
             f"    python3 bench.py --trace-summary OUT --steps {args.steps} --warmup {args.warmup}",
             "", f"Kernel time summed over the {n} traced steps (warmup included) / {n}. "
             "Under tracing each dispatch reads a few us longer than in a plain run.", "",
             "| kind | ms / step | share |", "|---|---|---|"]
    for label, us in sorted(groups.items(), key=lambda kv: -kv[1]):
        lines.append(f"| {label} | {us / 1e3:.2f} | {us / total:.1%} |")
    lines += [f"| total | {total / 1e3:.2f} | |", "", "Largest kernels:", "",
              "| kernel | calls / step | us / step |", "|---|---|---|"]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"]))[:16]:
        lines.append(f"| `{r['Name'][:72]}` | {int(r['Calls']) / n:g} | {per(r):.0f} |")
    md = ROOT / "profiles" / "train_80m_16x512.md"
    md.write_text("\n".join(lines) + "\n")
    print("\n".join(lines))
    print(f"\nwrote {md.relative_to(ROOT)}")


def workload_trace_summary(args, rows) -> None:
    """Markdown of a kernel-trace run of --workload longt (at the strides of
    args.strides) or --workload infer: every kernel with its calls and
    durations."""
    if args.workload == "longt":
        title = f"Long-sequence scan 4x16384x2048x16 fwd+bwd, stride {args.strides}"
        run = f"python3 bench.py --workload longt --strides {args.strides} --no-cpu-baseline"
        md = ROOT / "profiles" / f"longt_4x16384x2048x16_stride{args.strides.replace(',', '_')}.md"
    else:
        title = "Prefill 32x2048x4096x16 (forward + final state) and 256 decode steps"
        run = "python3 bench.py --workload infer --no-cpu-baseline"
        md = ROOT / "profiles" / "infer_32x2048x4096x16.md"
    lines = [f"# {title}: kernel time", "",
             PROFILE_RUN_NOTE, "",
             "    rocprofv3 --kernel-trace --stats -d OUT/kt -o run --output-format csv -- \\",
             f"        {run}",
             f"    python3 bench.py --trace-summary OUT --workload {args.workload}"
             + (f" --strides {args.strides}" if args.workload == "longt" else ""), "",
             "The calls include bench.py's untimed clock-settle calls and the warm-up "
             "before each timing.", "",
             "| kernel | calls | avg us | min us | max us |", "|---|---|---|---|---|"]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        lines.append(f"| `{r['Name'][:72]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} "
                     f"| {float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} |")
    md.write_text("\n".join(lines) + "\n")
    print("\n".join(lines))
    print(f"\nwrote {md.relative_to(ROOT)}")


# The reference bench's model sizes (bench/bench.py:37-40), named for the
# transformer budget each Mamba is matched to; "60M" counts 79.5M parameters
# with its 32768 x 640 embedding (the headline "80M" train step). "ref" is the
# small size the reference also runs with the torch scan (--ref).
TRAIN_SIZES = {
    "18M": dict(d_model=384, n_layers=10, d_ff=1536, batch=16, seq=512),
    "60M": dict(d_model=640, n_layers=12, d_ff=2560, batch=16, seq=512),
    "ref": dict(d_model=128, n_layers=2, d_ff=512, batch=4, seq=128),
}


def bench_train(steps: int = 10, warmup: int = 3, size: str = "60M",
                scan_impl: str = "hip") -> dict:
    """A TinyMamba train step (fwd + bwd + AdamW lr 3e-4) of one of the
    reference bench's sizes: vocab 32768, d_state 16, d_conv 4, random init,
    tokens uniform in [0, 32768). Peak HBM is torch's allocator peak over the
    timed steps (the reference's gate: under 16 GB at 18M, where its torch
    scan needed 47.7 GB)."""
    import torch
    from mamba_metal_scan_amd import MambaConfig, TinyMamba
    from mamba_metal_scan_amd.gemm_tuning import TABLE, use_tuned_gemms
    tuned = use_tuned_gemms()
    torch.manual_seed(1337)
    dev = torch.device("cuda", 0)
    sz = TRAIN_SIZES[size]
    bt, seq = sz["batch"], sz["seq"]
    cfg = MambaConfig(vocab_size=32768, d_model=sz["d_model"], n_layers=sz["n_layers"],
                      d_ff=sz["d_ff"], max_seq_len=seq, d_state=16, d_conv=4,
                      scan_impl=scan_impl)
    model = TinyMamba(cfg).to(dev)
    # The reference's optimizer (AdamW, lr 3e-4, bench/bench.py:90); torch's
    # fused implementation of the same update runs it in one pass per step.
    opt = torch.optim.AdamW(model.parameters(), lr=3e-4, fused=True)
    idx = torch.randint(0, 32768, (bt, seq + 1),
                        generator=torch.Generator().manual_seed(1337)).to(dev)
    x, y = idx[:, :-1], idx[:, 1:]

    def step():
        _, loss = model(x, y)
        opt.zero_grad(set_to_none=True)
        loss.backward()
        opt.step()
        return loss

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    out = {"tokens_per_s": bt * seq * steps / el, "ms_per_step": el * 1e3 / steps,
           "steps": steps, "warmup": warmup, "loss": float(loss.item()),
           "params": model.count_params(), "d_inner": model.d_inner,
           "peak_hbm_GB": torch.cuda.max_memory_allocated(dev) / 1e9,
           "config": f"TinyMamba {size} class ({model.count_params() / 1e6:.1f}M parameters: "
                     f"vocab 32768, d_model {sz['d_model']}, {sz['n_layers']} layers, d_state "
                     f"16), batch {bt} x seq {seq}, fp32, AdamW (fused), scan_impl={scan_impl}",
           "gemm_solutions": TABLE.name if tuned else "library default"}
    del model, opt
    torch.cuda.empty_cache()
    return out


LONGT = (4, 16384, 2048, 16)


def longt_measure(strides) -> list:
    """The long-sequence scan 4 x 16384 x 2048 x 16 fwd+bwd at each checkpoint
    stride: HIP-event times of the forward and backward launches (5 each,
    after a clock settle), algorithmic GB/s, checkpoint bytes."""
    import torch
    from mamba_metal_scan_amd import _native
    _native.library()
    bt, t_len, d, n = LONGT
    dev = torch.device("cuda", 0)
    x, dt, aneg, b_in, c_in, dy = (t.to(dev) for t in make_inputs(bt, t_len, d, n))
    nbytes = scan_bytes(bt, t_len, d, n)
    rows = []
    for chunk in strides:
        fwd = lambda: torch.ops.mamba_hip.scan_fwd(x, dt, aneg, b_in, c_in, chunk, True)
        _, ckpt, _ = fwd()
        bwd = lambda: torch.ops.mamba_hip.scan_bwd(x, dt, aneg, b_in, c_in, dy, None, ckpt, chunk)
        bwd()
        settle_clocks(lambda: (fwd(), bwd()))
        f_ms, b_ms = time_events(fwd, 5), time_events(bwd, 5)
        rows.append({"chunk": chunk, "fwd_ms": f_ms, "bwd_ms": b_ms, "fwd_bwd_ms": f_ms + b_ms,
                     "fwd_bwd_GBs": nbytes["fwd_bwd"] / ((f_ms + b_ms) * 1e-3) / 1e9,
                     "ckpt_bytes": ckpt.numel() * 4,
                     "reduction": reduction_name(bt, t_len, d, n, chunk)})
        print(f"longt chunk {chunk}: fwd {f_ms:.3f} ms bwd {b_ms:.3f} ms", file=sys.stderr,
              flush=True)
        del ckpt
    del x, dt, aneg, b_in, c_in, dy
    torch.cuda.empty_cache()
    return rows


def bench_longt(args) -> dict:
    """Long-sequence scan 4 x 16384 x 2048 x 16 fwd+bwd, checkpoint strides 16/32/64/128."""
    bt, t_len, d, n = LONGT
    rows = longt_measure([int(v) for v in args.strides.split(",")])
    best = min(rows, key=lambda r: r["fwd_bwd_ms"])
    nbytes = scan_bytes(bt, t_len, d, n)
    # The CPU path on the whole workload, one rep under a wall-clock limit
    # (value None with the reason when it runs out of time or memory), and on
    # a bounded sample beside it: a 1024-step sequence of the same sizes.
    cpu = cpu_baseline_child("longt") if not args.no_cpu_baseline else None
    return {"metric": "long-sequence scan fwd+bwd GB/s (4x16384x2048x16 fp32)",
            "value": best["fwd_bwd_GBs"], "unit": "GB/s", "n_gpus": 1,
            "ms_per_step": best["fwd_bwd_ms"], "higher_is_better": True, "dtype": "f32",
            "data": "synthetic", "algorithmic_bytes": nbytes["fwd_bwd"],
            "config": {"workload": "selective_scan fwd+bwd 4x16384x2048x16, stride sweep"},
            "strides": rows, "gpu_tokens_per_s": bt * t_len / (best["fwd_bwd_ms"] * 1e-3),
            "cpu_baseline": cpu}


INFER = (32, 2048, 4096, 16)


def infer_measure() -> dict:
    """Prefill 32 x 2048 x 4096 x 16 (forward + final state; HIP events, 5
    launches after a clock settle), then 256 recurrent decode steps, eager
    and replayed from one HIP graph."""
    import torch
    from mamba_metal_scan_amd import _native, selective_state_step
    _native.library()
    bt, t_len, d, n = INFER
    dev = torch.device("cuda", 0)
    x, dt, aneg, b_in, c_in, _ = (t.to(dev) for t in make_inputs(bt, t_len, d, n))
    prefill = lambda: torch.ops.mamba_hip.scan_fwd(x, dt, aneg, b_in, c_in, t_len, False)
    prefill()
    settle_clocks(prefill)
    p_ms = time_events(prefill, 5)
    p_bytes = 4 * (3 * bt * t_len * d + 2 * bt * t_len * n + d * n) + 4 * bt * d * n
    _, _, h = prefill()
    g = torch.Generator().manual_seed(7)
    steps = 256
    xs = torch.randn(steps, bt, d, generator=g).to(dev)
    dts = torch.nn.functional.softplus(torch.randn(steps, bt, d, generator=g) - 4.0).to(dev)
    bs = torch.randn(steps, bt, n, generator=g).to(dev)
    cs = torch.randn(steps, bt, n, generator=g).to(dev)

    def decode():
        for i in range(steps):
            selective_state_step(h, xs[i], dts[i], aneg, bs[i], cs[i])

    decode()
    torch.cuda.synchronize()
    start, stop = timing_event(), timing_event()
    start.record()
    decode()
    stop.record()
    torch.cuda.synchronize()
    eager_us = start.elapsed_time(stop) * 1e3 / steps
    # The same 256 steps captured once in a HIP graph and replayed: no host
    # launch cost per step.
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        decode()
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        decode()
    graph.replay()
    torch.cuda.synchronize()
    start.record()
    for _ in range(3):
        graph.replay()
    stop.record()
    torch.cuda.synchronize()
    graph_us = start.elapsed_time(stop) * 1e3 / (3 * steps)
    s_bytes = 4 * (2 * bt * d * n + 3 * bt * d + 2 * bt * n + d * n)
    del graph, x, dt, aneg, b_in, c_in, h, xs, dts, bs, cs
    torch.cuda.empty_cache()
    return {"prefill_ms": p_ms, "prefill_GBs": p_bytes / (p_ms * 1e-3) / 1e9,
            "prefill_algorithmic_bytes": p_bytes,
            "prefill_tokens_per_s": bt * t_len / (p_ms * 1e-3),
            "decode_us_per_step": graph_us, "decode_GBs": s_bytes / (graph_us * 1e-6) / 1e9,
            "decode_us_per_step_eager": eager_us, "decode_algorithmic_bytes": s_bytes}


def bench_infer(args) -> dict:
    """Prefill 32 x 2048 x 4096 x 16 (forward + final state), then 256 decode steps."""
    bt, t_len, d, n = INFER
    m = infer_measure()
    cpu = cpu_baseline_child("infer") if not args.no_cpu_baseline else None
    return {"metric": "prefill GB/s and decode us/step (32x2048x4096x16 fp32)",
            "value": m["prefill_GBs"], "unit": "GB/s", "n_gpus": 1,
            "ms_per_step": m["prefill_ms"], "higher_is_better": True, "dtype": "f32",
            "data": "synthetic", "config": {"workload": "prefill 32x2048x4096x16 + 256 decode steps"},
            **m, "cpu_baseline": cpu}


def bench_scan(args) -> dict:
    import torch
    from mamba_metal_scan_amd import _native, selective_scan_hip
    bt, t_len, d, n = args.batch, args.seqlen, args.d_inner, args.d_state
    chunk = args.chunk
    dev = torch.device("cuda", 0)
    x, dt, aneg, b_in, c_in, dy = (t.to(dev) for t in make_inputs(bt, t_len, d, n))
    leaves = [t.clone().requires_grad_(True) for t in (x, dt, aneg, b_in, c_in)]

    # Every EVENT_EVERY-th timed step also records HIP events around its
    # forward launch and its backward launch, on the stream the kernels run
    # on (torch's current stream, which the autograd backward also uses): the
    # per-launch averages come from the timed steps themselves. Each event is
    # a marker packet that costs the GPU time (in a kernel trace about 5 us
    # each for torch's default events, 4 us without the system fence,
    # TimingEvent); on every step they would add that to the step time.
    # Three events per instrumented step: before the forward, between the
    # forward and the backward (one marker serves both intervals), after the
    # backward. The instrumented steps are the last of every EVENT_EVERY: the
    # timed region starts from a synchronized, idle GPU, and its first step's
    # forward would include the host's launch latency.
    marked = [i for i in range(args.steps) if i % EVENT_EVERY == EVENT_EVERY - 1] or \
        [args.steps - 1]
    events = [[timing_event() for _ in range(3)] for _ in marked]
    event_of = dict(zip(marked, events))

    def step(ev=None):
        for t in leaves:
            t.grad = None
        if ev is not None:
            ev[0].record()
        y = selective_scan_hip(*leaves, chunk=chunk)
        if ev is not None:
            ev[1].record()
        y.backward(dy)
        if ev is not None:
            ev[2].record()

    settled = settle_clocks(step)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(event_of.get(i))
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed * 1e3 / args.steps
    fwd_ms = sum(e[0].elapsed_time(e[1]) for e in events) / len(events)
    bwd_each = [e[1].elapsed_time(e[2]) for e in events]
    bwd_ms = sum(bwd_each) / len(events)
    nbytes = scan_bytes(bt, t_len, d, n)
    bwd_gbs = nbytes["bwd"] / (bwd_ms * 1e-3) / 1e9
    fwd_gbs = nbytes["fwd"] / (fwd_ms * 1e-3) / 1e9
    pair_gbs = nbytes["fwd_bwd"] / ((fwd_ms + bwd_ms) * 1e-3) / 1e9
    # HBM traffic and VALU counters of this workload's kernels, from the
    # committed rocprofv3 summary (written by --pmc-summary; the counters
    # cannot be read from inside a timed run).
    counters = load_counters(bt, t_len, d, n, chunk)
    traffic = counters["bwd_launch"]["hbm_bytes"] if counters else None
    out = {
        "metric": METRIC,
        "value": bt * t_len / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (x,B,C,dy~N(0,1); dt=softplus(N(-4,1)); Aneg[d,n]=n+1)",
        "config": {"workload": f"selective_scan fwd+bwd {bt}x{t_len}x{d}x{n}",
                   "batch": bt, "seqlen": t_len, "d_inner": d, "d_state": n, "chunk": chunk,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": bwd_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": bwd_gbs / HBM_PEAK_GBS, "traffic": traffic,
                     "traffic_source": (f"profiles/{COUNTERS_NAME.format(shape=shape_tag(bt, t_len, d, n))}"
                                        " (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, copy-calibrated)"
                                        if counters else None),
                     "kernel": "scan backward launch (bwd_kernel + bwd_reduce_kernel)",
                     "avg_ms": bwd_ms, "algorithmic_bytes": nbytes["bwd"],
                     "timed_launches": len(events), "events": event_kind(),
                     "launch_ms_min": min(bwd_each),
                     "launch_ms_median": sorted(bwd_each)[len(bwd_each) // 2]},
        "valu": valu_block(counters),
        "scan_fwd": {"avg_ms": fwd_ms, "achieved_GBs": fwd_gbs,
                     "algorithmic_bytes": nbytes["fwd"]},
        "scan_fwd_bwd": {"avg_ms": fwd_ms + bwd_ms, "achieved_GBs": pair_gbs,
                         "frac": pair_gbs / HBM_PEAK_GBS,
                         "algorithmic_bytes": nbytes["fwd_bwd"]},
        "library_version": hex(_native.library().mhs_version()),
        "clock_settle": {"ms": SETTLE_MS, "steps": settled,
                         "note": "untimed steps before the warmup, until the GPU clock is steady"},
        "hbm_copy": copy_bandwidth(),
    }
    if not args.no_extra:
        # The same shape at the reference's default checkpoint stride (64),
        # and the backward with fp32 atomics instead of the fixed-order
        # reduction.
        out["scan_fwd_bwd_chunk64"] = pair_events(x, dt, aneg, b_in, c_in, dy, 64)
        _native.set_reduction(_native.REDUCTION_ATOMIC)
        try:
            out["scan_bwd_atomic"] = {k: v for k, v in pair_events(
                x, dt, aneg, b_in, c_in, dy, chunk).items() if k.startswith("bwd")}
        finally:
            _native.set_reduction(_native.REDUCTION_AUTO)
    del x, dt, aneg, b_in, c_in, dy, leaves
    torch.cuda.empty_cache()
    if not args.no_extra:
        out["longt_4x16384x2048x16"] = {
            "strides": longt_measure([16, 32, 64, 128]),
            "algorithmic_bytes": scan_bytes(*LONGT)["fwd_bwd"]}
        out["infer_32x2048x4096x16"] = infer_measure()
    if not args.no_train:
        out["train_80m"] = bench_train()
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_scan(bt, t_len, d, n)
        if not args.no_extra:
            # The other configurations' CPU paths, each on its whole workload.
            out["longt_4x16384x2048x16"]["cpu_baseline"] = cpu_baseline_child("longt")
            out["infer_32x2048x4096x16"]["cpu_baseline_prefill"] = cpu_baseline_child("infer")
    return out


def pair_events(x, dt, aneg, b_in, c_in, dy, chunk: int, reps: int = 20) -> dict:
    """The scan's forward and backward launches (the registered ops) at one
    checkpoint stride: HIP-event averages over `reps` each, after a short
    clock settle."""
    import torch
    ops = torch.ops.mamba_hip
    fwd = lambda: ops.scan_fwd(x, dt, aneg, b_in, c_in, chunk, True)
    _, ckpt, _ = fwd()
    bwd = lambda: ops.scan_bwd(x, dt, aneg, b_in, c_in, dy, None, ckpt, chunk)
    settle_clocks(lambda: (fwd(), bwd()), ms=30.0)
    f_ms, b_ms = time_events(fwd, reps), time_events(bwd, reps)
    nbytes = scan_bytes(*x.shape, aneg.shape[1])
    return {"chunk": chunk, "fwd_ms": f_ms, "bwd_ms": b_ms, "fwd_bwd_ms": f_ms + b_ms,
            "bwd_GBs": nbytes["bwd"] / (b_ms * 1e-3) / 1e9,
            "fwd_bwd_GBs": nbytes["fwd_bwd"] / ((f_ms + b_ms) * 1e-3) / 1e9,
            "ckpt_bytes": ckpt.numel() * 4}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="scan", choices=["scan", "train", "longt", "infer"])
    ap.add_argument("--no-train", action="store_true", help="skip the 80M train-step figure")
    ap.add_argument("--size", default="60M", choices=["18M", "60M"],
                    help="--workload train: the reference bench's model size (60M: the 79.5M-"
                         "parameter headline step)")
    ap.add_argument("--ref", action="store_true",
                    help="--workload train: also the torch scan at the reference bench's "
                         "small size")
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--seqlen", type=int, default=512)
    ap.add_argument("--d-inner", dest="d_inner", type=int, default=1536)
    ap.add_argument("--d-state", dest="d_state", type=int, default=16)
    ap.add_argument("--chunk", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--torch-events", action="store_true",
                    help="time with torch.cuda.Event (default HIP events, with the system-scope "
                         "fence) instead of HIP events created with hipEventDisableSystemFence")
    ap.add_argument("--no-extra", action="store_true",
                    help="only the headline workload (no chunk-64, atomic, long-sequence and "
                         "inference figures)")
    ap.add_argument("--reduction", default="auto", choices=["auto", "fixed", "atomic"],
                    help="the backward's reduction of dB, dC, dAneg (default: the library's)")
    ap.add_argument("--launches", type=int, default=0,
                    help="profiling driver: only N scan_fwd/scan_bwd launches + N copies")
    ap.add_argument("--forward-only", action="store_true",
                    help="with --launches / --kernel-counters: the forward alone, without "
                         "checkpoints (the prefill's launch; pass --chunk = --seqlen)")
    ap.add_argument("--pmc-summary", default=None, metavar="DIR",
                    help="summarise rocprofv3 FETCH_SIZE / WRITE_SIZE passes under DIR")
    ap.add_argument("--strides", default="16,32,64,128",
                    help="checkpoint strides of --workload longt (comma-separated)")
    ap.add_argument("--kernel-counters", default=None, metavar="DIR",
                    help="summarise per-kernel rocprofv3 passes of --launches runs under DIR "
                         "(any shape; every scan kernel labelled by its role)")
    ap.add_argument("--trace-summary", default=None, metavar="DIR",
                    help="summarise a kernel-trace run of --workload train under DIR")
    ap.add_argument("--cpu-baseline-only", default=None, choices=["longt", "infer"],
                    help="internal: the CPU baseline of a workload alone, one JSON line "
                         "(the child process of the default line's long-sequence and "
                         "prefill baselines; touches no GPU)")
    args = ap.parse_args()
    if args.cpu_baseline_only:
        return cpu_baseline_only(args.cpu_baseline_only)
    global USE_TORCH_EVENTS
    USE_TORCH_EVENTS = args.torch_events

    from mamba_metal_scan_amd import _native
    _native.set_reduction({"auto": _native.REDUCTION_AUTO, "fixed": _native.REDUCTION_FIXED,
                           "atomic": _native.REDUCTION_ATOMIC}[args.reduction])
    if args.pmc_summary:
        pmc_summary(args)
        return 0
    if args.trace_summary:
        trace_summary(args)
        return 0
    if args.kernel_counters:
        kernel_counters(args)
        return 0

    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs on a single MI355X and has no "
              f"multi-GPU path (asked for --gpus {args.gpus}).", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU (torch.cuda.is_available() is False)", file=sys.stderr)
        return 1
    if args.launches:
        run_launches(args)
        return 0
    if args.workload == "train":
        t = bench_train(steps=args.steps, warmup=args.warmup, size=args.size)
        name = "80M" if args.size == "60M" else args.size
        out = {"metric": f"{name} TinyMamba fp32 train step tok/s (batch 16 x seq 512)",
               "value": t["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1,
               "steps": args.steps, "warmup": args.warmup, "ms_per_step": t["ms_per_step"],
               "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
               "data": "synthetic tokens U[0, 32768)", "config": {"workload": t["config"]},
               f"train_{name.lower()}": t}
        if args.ref:
            # The torch scan (a Python loop over time) at the reference's
            # small size, with the HIP scan at the same size beside it.
            out["ref_torch"] = bench_train(steps=args.steps, warmup=1, size="ref",
                                           scan_impl="torch")
            out["ref_hip"] = bench_train(steps=args.steps, warmup=1, size="ref")
    else:
        out = {"scan": bench_scan, "longt": bench_longt, "infer": bench_infer}[args.workload](args)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
