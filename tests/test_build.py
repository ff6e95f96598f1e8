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
    assert build.K_CM_ROW == _constant("mhs_common.hpp", "kCmRow")
    assert "return carry ? CmLayout::kSwizzled : CmLayout::kPadded;" in (
        CSRC / "mhs_bwd.hpp").read_text()
    m = re.search(r"constexpr int kBCGroup2 = kQuads \* 16 \+ 16;", (CSRC / "mhs_common.hpp").read_text())
    assert m and _constant("mhs_common.hpp", "kQuads") * 16 + 16 == build.K_BC_GROUP2 == 80
    m = re.search(r"constexpr int kBCGroupQ = kQuads \* 16 \+ 8;", (CSRC / "mhs_common.hpp").read_text())
    assert m and _constant("mhs_common.hpp", "kQuads") * 16 + 8 == build.K_BC_GROUPQ == 72


def test_lds_sizes_of_the_training_plan():
    """d_state 16 (NPL 2, G 4): forward 34,304 B (B and C in the row
    broadcast tile, the two staged checkpoint tiles of 32 rows of 18 floats);
    backward 45,632 B with the row-partial sums, the padded
    channel-major tiles (4 x 32 rows of 20 floats per staging buffer) and B /
    C in the quad broadcast tile (3 blocks per CU fit the 160 KiB of gfx950);
    carry pass 39,424 B (swizzled channel-major tiles, per-group B / C tiles:
    4 blocks per CU); swept backward 47,616 B (the quad broadcast tile and
    the sweep's two state slots, no row partials)."""
    assert build.scan_lds_bytes("fwd", 4, 2) == 4 * (2 * (1024 + 8 * 80 + 4 * 512) + 2 * 576) == 34304
    assert build.scan_lds_bytes("fwd_nock", 4, 2) == 4 * 2 * (1024 + 8 * 80 + 4 * 512) == 29696
    assert build.scan_lds_bytes("bwd_carry", 4, 2) == 4 * (2 * (2048 + 2 * 288) + 4096 + 512) == 39424
    sweep = build.scan_lds_bytes("bwd_sweep", 4, 2)
    assert sweep == 4 * (2 * (2560 + 8 * 72) + 4096 + 512 + 2 * 64 * 4 * 2) == 47616
    rp = build.scan_lds_bytes("bwd", 4, 2)
    assert rp == 4 * (2 * (2560 + 8 * 72) + 4096 + 4 * (16 * 16 + 4)) == 45632
    assert 3 * rp <= build.LDS_PER_CU and 3 * sweep <= 160 * 1024


def test_dpp_hazard_check_finds_short_wait_states():
    """The build's check of the device assembly (build.dpp_hazards): a DPP
    read, in an inline-asm block, of a VGPR needs 2 wait states after a VALU
    write of it."""
    def asm(*lines):   # lines in one inline-asm block
        return ["  ;;#ASMSTART", *lines, "  ;;#ASMEND"]
    ok = "\n".join([
        "k:",
        "  ds_read_b128 v[4:7], v1",
        "  s_waitcnt lgkmcnt(0)",
        *asm("  v_fmac_f32_dpp v8, v5, v9 quad_perm:[0,1,0,1] row_mask:0xf bank_mask:0xf"),
        "  v_mul_f32_e32 v10, v2, v3",
        *asm("  s_nop 1",
             "  v_fmac_f32_dpp v8, v10, v9 quad_perm:[1,0,1,0] row_mask:0xf bank_mask:0xf"),
        "  v_mul_f32_e32 v11, v2, v3",
        "  v_add_f32_e32 v12, v2, v3",
        "  v_add_f32_e32 v13, v2, v3",
        *asm("  v_mul_f32_dpp v14, v11, v9 quad_perm:[2,3,2,3] row_mask:0xf bank_mask:0xf"),
        # the compiler's own DPP is padded by the compiler and not checked
        "  v_mul_f32_e32 v15, v2, v3",
        "  v_mul_f32_dpp v16, v15, v9 quad_perm:[2,3,2,3] row_mask:0xf bank_mask:0xf",
        ".LBB0_2:",
        "  v_add_f32_dpp v0, v3, v3 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf",
    ])
    assert build.dpp_hazards(ok) == []
    planted = {
        "no wait": ["  v_mul_f32_e32 v10, v2, v3",
                    *asm("  v_fmac_f32_dpp v8, v10, v9 quad_perm:[0,1,0,1] row_mask:0xf "
                         "bank_mask:0xf")],
        "one wait state": ["  v_mul_f32_e32 v10, v2, v3",
                           *asm("  s_nop 0",
                                "  v_add_f32_dpp v8, v10, v10 row_ror:8 row_mask:0xf bank_mask:0x3")],
        "inside the block": asm("  v_add_f32_dpp v10, v3, v3 row_ror:8 row_mask:0xf bank_mask:0x3",
                                "  v_add_f32_dpp v8, v10, v10 row_shl:4 row_mask:0xf bank_mask:0x5"),
        "64-bit write": ["  v_lshlrev_b64 v[10:11], 2, v[2:3]", "  v_add_f32_e32 v12, v2, v3",
                         *asm("  v_mov_b32_dpp v8, v11 quad_perm:[1,0,3,2] row_mask:0xf "
                              "bank_mask:0xf")],
        "after a label": [".LBB0_1:",
                          *asm("  v_fmac_f32_dpp v8, v10, v9 quad_perm:[0,1,0,1] row_mask:0xf "
                               "bank_mask:0xf")],
    }
    for name, body in planted.items():
        found = build.dpp_hazards("\n".join(["k:", *body]))
        assert len(found) == 1, (name, found)
