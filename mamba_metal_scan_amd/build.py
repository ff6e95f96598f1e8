"""Build recipe for the gfx950 shared library (hipcc, in-tree, no torch link).

The library is a plain C-ABI `.so` (include/mamba_hip_scan.h) that links only
the HIP runtime; Python reaches it through ctypes (`_native.py`). It is built
in place next to this file so that it travels with the source tree.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libmamba_hip_scan.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

# The host code and small kernels, and the scan kernels' instantiations in
# five units (forward / backward x fp32 / bf16, and the fp32 backward with
# atomics) compiled in parallel.
SOURCES = ["mhs_capi.hip", "mhs_kern_fwd_f32.hip", "mhs_kern_fwd_bf16.hip",
           "mhs_kern_bwd_f32.hip", "mhs_kern_bwd_bf16.hip", "mhs_kern_bwd_atom.hip",
           "mhs_kern_bwd_atom_bf16.hip"]
HEADERS = ["mhs_common.hpp", "mhs_fwd.hpp", "mhs_bwd.hpp", "mhs_step.hpp", "mhs_conv.hpp",
           "mhs_gate.hpp", "mhs_instances.hpp", "mhs_xent.hpp", "mhs_norm.hpp"]


def hipcc() -> str:
    cand = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(cand).exists():
        raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")
    return cand


def compile_flags() -> list[str]:
    return [
        "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC",
        # Packed FP32 (v_pk_*_f32) is kept out of the generated code.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", str(REPO_DIR / "include"), "-I", str(CSRC),
        "-Wall", "-Wno-unused-result",
    ]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln and ln.strip()]
    if verbose and msgs:
        print("\n".join(msgs), file=sys.stderr)


def build_library(verbose: bool = False, out: Path | None = None) -> Path:
    """Compile csrc/*.hip into the in-tree shared library; returns its path.

    Each source compiles to an object in a temporary folder, in parallel;
    hipcc then links them into the library."""
    out = Path(out) if out is not None else LIB_PATH
    tmp = out.with_suffix(".so.tmp")
    with tempfile.TemporaryDirectory(prefix="mhs_build_") as objdir:
        objs = [str(Path(objdir) / (Path(src).stem + ".o")) for src in SOURCES]
        cmds = [[hipcc(), *compile_flags(), "-c", "-o", obj, str(CSRC / src)]
                for src, obj in zip(SOURCES, objs)]
        with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as pool:
            for f in [pool.submit(_run, c, verbose) for c in cmds]:
                f.result()
        _run([hipcc(), *compile_flags(), "-shared", "-o", str(tmp), *objs], verbose)
    os.replace(tmp, out)
    return out


def emit_assembly(out_dir: Path) -> Path:
    """Device assembly of the library (for register / instruction audits)."""
    out_dir.mkdir(parents=True, exist_ok=True)
    asm = out_dir / "mhs_capi-gfx950.s"
    cmd = [hipcc(), *compile_flags(), "--cuda-device-only", "-S", "-o", str(asm),
           str(CSRC / "mhs_capi.hip")]
    subprocess.run(cmd, check=True, capture_output=True)
    return asm


if __name__ == "__main__":
    print(build_library(verbose=True))
