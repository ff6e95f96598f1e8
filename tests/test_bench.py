"""bench.py's contract on the CPU: the one-GPU rule, the failure without a GPU,
and the algorithmic byte counts its roofline figures divide by."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def _run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True,
                          text=True, timeout=300)


def test_more_than_one_gpu_exits_with_a_message():
    r = _run("--gpus", "2")
    assert r.returncode != 0
    assert "single MI355X" in r.stderr and "--gpus 2" in r.stderr
    assert r.stdout.strip() == ""            # no JSON line


def test_without_a_gpu_it_fails_cleanly():
    if torch.cuda.is_available():
        return
    r = _run("--steps", "1", "--warmup", "0")
    assert r.returncode == 1 and "needs a ROCm GPU" in r.stderr


def test_algorithmic_bytes():
    """fwd = 4(3E + 2S + A), bwd = 4(5E + 4S + 2A) with E = B T D, S = B T N,
    A = D N: 406,093,824 B for the fwd+bwd pair at 16x512x1536x16 (50.76 us at
    8 TB/s), and 378.8 MB per layer at the 80M model's d_inner of 1432."""
    b = bench.scan_bytes(16, 512, 1536, 16)
    assert b["fwd_bwd"] == 406_093_824 == b["fwd"] + b["bwd"]
    assert b["fwd"] == 4 * (3 * 12_582_912 + 2 * 131_072 + 24_576)
    assert abs(b["fwd_bwd"] / 8e12 * 1e6 - 50.76) < 0.01
    assert round(bench.scan_bytes(16, 512, 1432, 16)["fwd_bwd"] / 1e6, 1) == 378.8


def test_cpu_baseline_child_records_a_timeout(monkeypatch):
    """The long-sequence and prefill CPU baselines run in a child process
    under a wall-clock limit; one that runs out of time is recorded with the
    reason and no value (here: a 3 s limit on the prefill)."""
    monkeypatch.setitem(bench.CPU_CHILD_LIMIT_S, "infer", 3)
    r = bench.cpu_baseline_child("infer")
    assert r["value"] is None and r["result"] == "timeout after 3 s"
    assert "32x2048x4096x16 (the full workload)" in r["sample"] and r["kind"] == "port"


def test_kernel_labels_name_each_pass():
    """The per-kernel counter summary labels every scan kernel by the role its
    template arguments give it."""
    f = "void mhs::fwd_kernel<2, 4, 3, true, false, {}, 4>(mhs::FwdArgs)"
    b = "void mhs::bwd_kernel<2, 4, 3, false, {}, 4, {}, {}>(mhs::BwdArgs)"
    assert bench.kernel_label(f.format(0)) == "forward"
    assert bench.kernel_label(f.format(1)) == "forward carry pass"
    assert bench.kernel_label(f.format(2)) == "backward checkpoint recompute"
    assert bench.kernel_label(b.format("true", "false", 0)) == "backward carry pass"
    assert bench.kernel_label(b.format("false", "false", 0)) == "backward (fixed order)"
    assert bench.kernel_label(b.format("false", "true", 0)) == "backward (atomics)"
    assert bench.kernel_label(b.format("false", "true", 4)) == "backward swept (atomics)"
    assert bench.kernel_label("void mhs::bwd_reduce_kernel<4>(float const*)") == \
        "backward reduction"
    assert bench.kernel_label("void mhs::zero_grads_kernel<0>(float*)") == "zero fill"
    assert bench.kernel_label("__amd_rocclr_copyBuffer") == "copy"


def test_trace_spans_of_the_timed_steps(tmp_path):
    """bench.py's kernel-trace summary: the timed steps' launch spans are
    those of the last (forward, backward, reduction) dispatch triples (a
    synthetic trace: 2 warm-up steps, then 3 timed steps of fwd 50 us, bwd
    100 + reduce 12 us with 1 us between them and a 4 us marker gap before
    each backward)."""
    names = {"fwd": "void mhs::fwd_kernel<2, 4, 3, true, false, 0, 4>(mhs::FwdArgs)",
             "bwd": "void mhs::bwd_kernel<2, 4, 3, false, false, 4, false, 0>(mhs::BwdArgs)",
             "red": "void mhs::bwd_reduce_kernel<4>(float const*, float const*)"}
    rows, t = [], 0

    def launch(kind, us, gap=1.0):
        nonlocal t
        t += int(gap * 1000)
        rows.append((names[kind], t, t + int(us * 1000)))
        t += int(us * 1000)
    for _ in range(2):                 # warm-up steps (not counted)
        launch("fwd", 60); launch("bwd", 130); launch("red", 15)
    for _ in range(3):                 # timed steps
        launch("fwd", 50, gap=2); launch("bwd", 100, gap=4); launch("red", 12)
    path = tmp_path / "run_kernel_trace.csv"
    with open(path, "w") as f:
        f.write("Kernel_Name,Start_Timestamp,End_Timestamp\n")
        for name, t0, t1 in rows:
            f.write(f'"{name}",{t0},{t1}\n')
    durs, spans = bench.trace_spans(str(path), 3)
    assert spans["steps"] == 3 and spans["fwd_us"] == 50 and spans["bwd_launch_us"] == 113
    assert spans["gap_before_bwd_us"] == 4 and spans["gap_before_fwd_us"] == 2
    assert spans["steps_with_gaps"] == 3
    assert durs["bwd_kernel"] == [100.0] * 3 and durs["fwd_kernel"] == [50.0] * 3
    assert bench.trace_spans(str(path), 6)[1] is None   # not 6 timed steps
