"""Pre-tuned fp32 GEMM solutions for the TinyMamba train step on gfx950.

Outside the scan and the conv, a TinyMamba train step is fp32 GEMMs (the
in/out/dt/B/C projections and the 32768-way head). ``gemm_tuning_gfx950.csv``
holds, for each GEMM shape of the 80M configuration (batch 16 x seq 512), the
fastest of the rocBLAS / hipBLASLt fp32 solutions found by PyTorch's
TunableOp on MI355X. ``use_tuned_gemms()`` loads it with tuning switched off,
so a run pays no tuning time; shapes not in the table use the default
solution. All candidates are ordinary fp32 GEMMs: results differ from the
default only by summation order.
"""
from __future__ import annotations

from pathlib import Path

import torch

TABLE = Path(__file__).resolve().with_name("gemm_tuning_gfx950.csv")


def use_tuned_gemms(table: Path = TABLE) -> bool:
    """Enable TunableOp with the shipped table (no on-line tuning). Returns
    False (and changes nothing) when the table does not apply here."""
    if not (torch.cuda.is_available() and torch.version.hip is not None and table.exists()):
        return False
    arch = torch.cuda.get_device_properties(0).gcnArchName
    if not arch.startswith("gfx950"):
        return False
    torch.cuda.tunable.enable(True)
    torch.cuda.tunable.tuning_enable(False)
    torch.cuda.tunable.record_untuned_enable(False)
    ok = torch.cuda.tunable.read_file(str(table))
    if not ok:
        torch.cuda.tunable.enable(False)
    return bool(ok)
