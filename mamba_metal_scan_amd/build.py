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


def _vgprs(operand: str) -> set[int]:
    import re
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", operand.strip())
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", operand.strip())
    return {int(m.group(1))} if m else set()


def dpp_hazards(asm: str) -> list[str]:
    """DPP reads of a VGPR that a VALU instruction wrote less than 2 wait
    states before, in the inline-asm blocks of gfx950 assembly (between the
    compiler's ;;#ASMSTART and ;;#ASMEND): the hardware then reads the old
    value. The compiler pads its own DPP instructions; the kernels'
    inline-asm ones (v_fmac_f32_dpp of the quad broadcasts, the bank-masked
    adds) rely on their DPP source coming from an LDS load or on their own
    s_nop, which this checks on the code that ships. Such a DPP instruction
    within 2 wait states after a label is reported too (the predecessors
    are not followed)."""
    import re
    found: list[str] = []
    func, hist = "?", []          # (opcode, VGPRs written, wait states)
    in_asm = False
    for ln, raw in enumerate(asm.splitlines(), 1):
        if ";;#ASMSTART" in raw or ";;#ASMEND" in raw:
            in_asm = ";;#ASMSTART" in raw
            continue
        s = raw.split(";")[0].strip()
        if re.match(r"^[_A-Za-z.][\w.$]*:$", s):
            if s.startswith(".LBB"):
                hist.append(("label", set(), 0))
            else:
                func, hist = s[:-1], []
            continue
        if not s or s.startswith("."):
            continue
        op = s.split()[0]
        ops = [o.strip() for o in s[len(op):].split(",")]
        if in_asm and op.startswith("v_") and ("_dpp" in op or "quad_perm" in s or "row_" in s):
            src0 = _vgprs(ops[1].split()[0]) if len(ops) > 1 and ops[1] else set()
            ws = 0
            for hop, hdst, hw in reversed(hist):
                if ws >= 2:
                    break
                if hop == "label":
                    found.append(f"line {ln} ({func}): DPP after a label: {s}")
                    break
                if hop.startswith("v_") and hdst & src0:
                    found.append(f"line {ln} ({func}): DPP source written {ws} wait "
                                 f"states before: {s}")
                    break
                ws += hw
        dst = _vgprs(ops[0].split()[0]) if op.startswith("v_") and ops and ops[0] else set()
        m = re.match(r"s_nop\s+(\d+)", s)
        hist = (hist + [(op, dst, int(m.group(1)) + 1 if m else 1)])[-8:]
    return found


def build_library(verbose: bool = False, out: Path | None = None) -> Path:
    """Compile csrc/*.hip into the in-tree shared library; returns its path.

    Each source compiles to an object in a temporary folder, in parallel,
    keeping its device assembly (-save-temps: the object is assembled from
    it), which is checked for DPP wait-state hazards (dpp_hazards); hipcc
    then links the objects into the library."""
    out = Path(out) if out is not None else LIB_PATH
    tmp = out.with_suffix(".so.tmp")
    with tempfile.TemporaryDirectory(prefix="mhs_build_") as objdir:
        objs = [str(Path(objdir) / (Path(src).stem + ".o")) for src in SOURCES]
        cmds = [[hipcc(), *compile_flags(), "-save-temps=obj", "-c", "-o", obj, str(CSRC / src)]
                for src, obj in zip(SOURCES, objs)]
        with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as pool:
            for f in [pool.submit(_run, c, verbose) for c in cmds]:
                f.result()
        for src in SOURCES:
            asm = Path(objdir) / f"{Path(src).stem}-hip-amdgcn-amd-amdhsa-{ARCH}.s"
            if not asm.exists():
                raise RuntimeError(f"device assembly of {src} not found ({asm.name})")
            bad = dpp_hazards(asm.read_text())
            if bad:
                raise RuntimeError(f"{src}: {len(bad)} DPP wait-state hazard(s):\n"
                                   + "\n".join(bad[:10]))
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


# ----------------------------------------------------- register / LDS audit
#
# The compiler's resource remarks (-Rpass-analysis=kernel-resource-usage) for
# every kernel of the library, and the dynamic LDS each scan kernel is
# launched with. The LDS sizes mirror the constexpr helpers of the kernel
# headers (fwd_lds_floats in mhs_fwd.hpp, bwd_lds_floats and
# bwd_sweep_lds_floats in mhs_bwd.hpp) with the header constants below, which
# tests/test_build.py reads back from the headers.
K_CH, K_STEPS, K_BC_PAD, K_SWEEP_MAX = 32, 16, 4, 2
K_CM_ROW = 20                    # kCmRow: a row of the backward's padded channel-major tiles
K_BC_GROUP2 = 4 * 16 + 16        # kBCGroup2: a state group of the row broadcast tile
K_BC_GROUPQ = 4 * 16 + 8         # kBCGroupQ: a state group of the quad broadcast tile
LDS_PER_CU = 160 * 1024          # gfx950
VGPRS_PER_SIMD_LANE = 512        # wave64 VGPR file per SIMD lane (gfx950, no AGPR split used)


def _bc_tile_floats(nq: int, npl: int) -> int:
    return nq * (K_STEPS * npl + K_BC_PAD)


def scan_lds_bytes(kind: str, g: int, npl: int) -> int:
    """Dynamic LDS per block of the scan kernels of plan (NPL, G): "fwd" (a
    forward launch that writes checkpoints), "fwd_nock" (one that does not:
    the prefill, the carry pass), "bwd" (the gradient kernels), "bwd_carry"
    (the adjoint-carry pass) or "bwd_sweep" (the swept backward, checkpoint
    stride 32)."""
    if kind in ("fwd", "fwd_nock"):
        # two states per lane: the broadcast tile (fwd_bc_floats)
        bc = 2 * g * K_BC_GROUP2 if npl == 2 else 2 * _bc_tile_floats(2 * g, npl)
        buf = 2 * K_CH * K_STEPS + bc + g * K_CH * K_STEPS
        # the staged checkpoint tiles
        ck = 2 * K_CH * (2 * g * npl + 2) if npl == 2 and kind == "fwd" else 0
        return 4 * (2 * buf + ck)
    rl = kind != "bwd_carry" and npl == 2   # swapped state pairs (bwd_relabel)
    rp = kind == "bwd" and npl == 2         # row-partial channel sums (bwd_row_partial)
    np_ = 2 * g * npl
    # B and C: the quad broadcast tile (rl) or the per-group tiles
    bc = 2 * g * K_BC_GROUPQ if rl else 2 * _bc_tile_floats(2 * g, npl)
    # dt, dy, x, dt*x: padded channel-major tiles, swizzled in the carry pass
    buf = 4 * K_CH * (K_STEPS if kind == "bwd_carry" else K_CM_ROW) + bc
    sums = 4 * (K_STEPS * (16 if np_ <= 16 else 48) + 4) if rp else 2 * K_STEPS * np_
    floats = 2 * buf + g * 64 * K_STEPS + sums
    if kind == "bwd_sweep":
        floats += K_SWEEP_MAX * 64 * g * npl
    return 4 * floats


def resource_usage(verbose: bool = False) -> dict:
    """{demangled kernel name: {remark: value}} from a device-only compile of
    every source with the compiler's kernel-resource-usage remarks."""
    import re
    with tempfile.TemporaryDirectory(prefix="mhs_ru_") as objdir:
        cmds = [[hipcc(), *compile_flags(), "--cuda-device-only", "-c", "-o",
                 str(Path(objdir) / (Path(src).stem + ".o")), str(CSRC / src),
                 "-Rpass-analysis=kernel-resource-usage"] for src in SOURCES]
        with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as pool:
            res = list(pool.map(lambda c: subprocess.run(c, capture_output=True, text=True),
                                cmds))
    rows: dict = {}
    cur = None
    for r in res:
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed ({r.returncode}):\n{r.stderr}")
        for ln in r.stderr.splitlines():
            m = re.search(r"remark: Function Name: (\S+)", ln)
            if m:
                cur = rows.setdefault(m.group(1), {})
                continue
            m = re.search(r"remark:\s+([^:]+): (\S+) \[-Rpass-analysis", ln)
            if m and cur is not None:
                cur[m.group(1).strip()] = m.group(2)
    names = list(rows)
    dem = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True,
                         check=True).stdout.splitlines()
    return {d.replace("mhs::", ""): rows[n] for n, d in zip(names, dem)}


# The kernels of the benchmarked workloads (d_state 16: NPL 2, G 4; the
# one-state-per-lane plan NPL 1, G 8 beside them), with what each one is.
AUDIT = [
    ("fwd_kernel<2, 4, 3, true, false, 0, 4>", "forward, checkpoint stride a multiple of 16",
     "fwd", 4, 2),
    ("fwd_kernel<2, 4, 3, true, false, 1, 4>", "forward carry pass (time segments)", "fwd_nock",
     4, 2),
    ("fwd_kernel<2, 4, 3, true, true, 0, 4>", "gated forward (TinyMamba block)", "fwd", 4, 2),
    ("bwd_kernel<2, 4, 3, false, false, 4, false, 0>", "backward, fixed-order partials",
     "bwd", 4, 2),
    ("bwd_kernel<2, 4, 3, false, false, 4, true, 0>", "backward, fp32 atomics", "bwd", 4, 2),
    ("bwd_kernel<2, 4, 3, false, false, 4, false, 2>", "backward, swept stride 32",
     "bwd_sweep", 4, 2),
    ("bwd_kernel<2, 4, 3, false, false, 4, true, 2>", "backward, swept stride, atomics",
     "bwd_sweep", 4, 2),
    ("bwd_kernel<2, 4, 3, false, true, 4, false, 0>", "backward carry pass (time segments)",
     "bwd_carry", 4, 2),
    ("bwd_kernel<2, 4, 3, true, false, 4, false, 0>", "gated backward (TinyMamba block)",
     "bwd", 4, 2),
    ("fwd_kernel<1, 8, 4, true, false, 0, 4>", "forward, one state per lane", "fwd", 8, 1),
    ("bwd_kernel<1, 8, 4, false, false, 4, false, 0>", "backward, one state per lane",
     "bwd", 8, 1),
    ("bwd_reduce_kernel<4>", "dB / dC / dAneg partial sums", None, 4, 0),
    ("zero_grads_kernel<0>", "zero fill before the atomics", None, 4, 0),
    ("step_kernel_vec<1, 4>", "decode step, d_state 16", None, 4, 0),
]


def resource_table(usage: dict) -> list:
    """Markdown rows of the audited kernels: registers, scratch, spills,
    dynamic LDS, and the waves per SIMD each of them allows."""
    out = ["| kernel | what | VGPRs | AGPRs | SGPRs | scratch B/lane | VGPR / SGPR spills "
           "| waves/SIMD (registers) | LDS B/block | waves/SIMD (LDS) |",
           "|---|---|---|---|---|---|---|---|---|---|"]
    for prefix, what, kind, waves_per_block, npl in AUDIT:
        hits = [k for k in usage if k.startswith("void " + prefix + "(")]
        if not hits:
            raise KeyError(f"no kernel {prefix} in the library's resource remarks")
        r = usage[hits[0]]
        lds = scan_lds_bytes(kind, waves_per_block, npl) if kind else 0
        lds_waves = (f"{(LDS_PER_CU // lds) * waves_per_block // 4}" if lds else "-")
        out.append(f"| `{prefix}` | {what} | {r['VGPRs']} | {r['AGPRs']} | {r['TotalSGPRs']} | "
                   f"{r['ScratchSize [bytes/lane]']} | {r['VGPRs Spill']} / {r['SGPRs Spill']} | "
                   f"{r['Occupancy [waves/SIMD]']} | {lds or '-'} | {lds_waves} |")
    return out


def write_resource_profile(path: Path) -> Path:
    """profiles/kernel_resources_gfx950.md: the register and LDS audit."""
    usage = resource_usage()
    lines = ["# Scan kernels on gfx950: registers, scratch, LDS and the occupancy they allow",
             "", "Made by", "",
             "    python3 -m mamba_metal_scan_amd.build --resource-usage "
             "profiles/kernel_resources_gfx950.md", "",
             "from the compiler's `-Rpass-analysis=kernel-resource-usage` remarks of a "
             "device-only build of the library's sources (the flags of `build.py`). "
             "`waves/SIMD (registers)` is the compiler's occupancy from VGPRs, SGPRs and the "
             "launch bounds; `LDS B/block` is the dynamic LDS the host launches each scan "
             "kernel with (a forward that writes checkpoints; one that does not, as the "
             f"prefill, leaves out the {scan_lds_bytes('fwd', 4, 2) - scan_lds_bytes('fwd_nock', 4, 2)} "
             "B of checkpoint tiles at d_state 16), and `waves/SIMD (LDS)` what "
             f"{LDS_PER_CU // 1024} KiB of LDS per CU "
             "allows for that block size (blocks per CU x waves per block / 4 SIMDs). A kernel "
             "runs at the smaller of the two, or fewer when its grid is smaller than the GPU: "
             "at 16x512x1536x16 the forward and backward grids are 768 blocks of 4 waves, 3 per "
             "SIMD (the resident waves the issue counters measure are in "
             "`scan_16x512x1536x16.md`).", ""]
    lines += resource_table(usage)
    path.write_text("\n".join(lines) + "\n")
    return path


if __name__ == "__main__":
    if len(sys.argv) == 3 and sys.argv[1] == "--resource-usage":
        print(write_resource_profile(Path(sys.argv[2])))
    else:
        print(build_library(verbose=True))
