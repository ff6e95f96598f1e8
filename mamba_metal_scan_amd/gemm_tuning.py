"""Pre-tuned fp32 GEMM solutions for the TinyMamba train step on gfx950.

Outside the scan and the conv, a TinyMamba train step is fp32 GEMMs (the
in/out projections, the merged dt/B/C projection of the fused inner block,
and the 32768-way head). ``gemm_tuning_gfx950.csv``
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


def tune(out: Path, steps: int = 3, start: Path = TABLE) -> None:
    """Regenerate the table on a gfx950 device: run the 80M train step (batch
    16 x seq 512) with TunableOp tuning on, starting from ``start`` so that
    only shapes missing from it are tuned, and write the start table's rows
    plus the newly tuned ones to ``out``
    (``python -m mamba_metal_scan_amd.gemm_tuning OUT``)."""
    from .model import MambaConfig, TinyMamba
    torch.cuda.tunable.enable(True)
    torch.cuda.tunable.tuning_enable(True)
    torch.cuda.tunable.set_filename(str(out.with_suffix(".session.csv")))
    if start.exists():
        torch.cuda.tunable.read_file(str(start))
    torch.manual_seed(0)
    dev = torch.device("cuda", 0)
    cfg = MambaConfig(vocab_size=32768, d_model=640, n_layers=12, d_ff=2560, max_seq_len=512,
                      d_state=16, d_conv=4, scan_impl="hip")
    model = TinyMamba(cfg).to(dev)
    opt = torch.optim.AdamW(model.parameters(), lr=3e-4, fused=True)
    idx = torch.randint(0, cfg.vocab_size, (16, 513), device=dev)
    for step in range(steps):
        opt.zero_grad(set_to_none=True)
        _, loss = model(idx[:, :-1], idx[:, 1:])
        loss.backward()
        opt.step()
        torch.cuda.synchronize()
        print(f"tuning step {step + 1}/{steps} done, loss {loss.item():.4f}", flush=True)
    rows = {}
    if start.exists():
        for line in start.read_text().splitlines():
            f = line.split(",")
            if f and f[0] != "Validator" and len(f) >= 4:
                rows[(f[0], f[1])] = line
    for r in torch.cuda.tunable.get_results():
        f = [str(v) for v in r]
        rows[(f[0], f[1])] = ",".join(f)
    head = [f"Validator,{k},{v}" for k, v in torch.cuda.tunable.get_validators()]
    out.write_text("\n".join(head + sorted(rows.values())) + "\n")
    print(f"wrote {len(rows)} GEMM solutions to {out}", flush=True)


if __name__ == "__main__":
    import sys
    tune(Path(sys.argv[1]) if len(sys.argv) > 1 else TABLE)
