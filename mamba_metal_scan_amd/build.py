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
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libmamba_hip_scan.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

SOURCES = ["mhs_capi.hip"]
HEADERS = ["mhs_common.hpp", "mhs_fwd.hpp", "mhs_bwd.hpp", "mhs_step.hpp", "mhs_conv.hpp",
           "mhs_gate.hpp"]


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


def build_library(verbose: bool = False, out: Path | None = None) -> Path:
    """Compile csrc/*.hip into the in-tree shared library; returns its path."""
    out = Path(out) if out is not None else LIB_PATH
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), *compile_flags(), "-shared", "-o", str(tmp),
           *[str(CSRC / s) for s in SOURCES]]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln and ln.strip()]
    if verbose and msgs:
        print("\n".join(msgs), file=sys.stderr)
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
