"""The build recipe's register/LDS audit on the CPU: the LDS sizes it
reports mirror the kernel headers' constexpr helpers, with the headers'
constants."""
from __future__ import annotations

import re
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
from mamba_metal_scan_amd import build  # noqa: E402

CSRC = ROOT / "mamba_metal_scan_amd" / "csrc"


def _constant(header: str, name: str) -> int:
    m = re.search(rf"constexpr int {name} = (\d+);", (CSRC / header).read_text())
    assert m, f"{name} not found in {header}"
    return int(m.group(1))


def test_audit_constants_match_the_headers():
    assert build.K_CH == _constant("mhs_fwd.hpp", "kCH")
    assert build.K_STEPS == _constant("mhs_common.hpp", "kSteps")
    assert build.K_BC_PAD == _constant("mhs_common.hpp", "kBCPad")
    assert build.K_SWEEP_MAX == _constant("mhs_bwd.hpp", "kSweepMax")
    assert build.K_RP_SWAP_PAD == _constant("mhs_bwd.hpp", "kRPSwapPad")
    m = re.search(r"constexpr int kBCGroup2 = kQuads \* 16 \+ 16;", (CSRC / "mhs_fwd.hpp").read_text())
    assert m and _constant("mhs_common.hpp", "kQuads") * 16 + 16 == 80


def test_lds_sizes_of_the_training_plan():
    """d_state 16 (NPL 2, G 4): forward 29,696 B (B and C in the broadcast
    tile); backward 46,208 B with the
    row-partial sums and the swapped B / C copies (3 blocks per CU fit the
    160 KiB of gfx950); carry pass 39,424 B; swept backward 52,288 B (the
    swapped copies and the sweep's state slots, no row partials)."""
    assert build.scan_lds_bytes("fwd", 4, 2) == 4 * 2 * (1024 + 8 * 80 + 4 * 512) == 29696
    assert build.scan_lds_bytes("bwd_carry", 4, 2) == 39424
    assert build.scan_lds_bytes("bwd_sweep", 4, 2) == 47616 + 4 * 2 * (2 * 288 + 8) == 52288
    rp = build.scan_lds_bytes("bwd", 4, 2)
    assert rp == 4 * (2 * (2048 + 2 * 288 + 2 * 288 + 8) + 4096 + 4 * (16 * 16 + 4))
    assert 3 * rp <= build.LDS_PER_CU and 3 * build.scan_lds_bytes("bwd_sweep", 4, 2) <= 160 * 1024
