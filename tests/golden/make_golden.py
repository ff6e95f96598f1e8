"""Writes tests/golden/scan_golden.npz: small input/output vectors of the scan.

The reference ships no data files or vectors for the scan, so these are
produced by the float64 oracle (oracle/scan_oracle.c) after its CPU pins
(tests/test_oracle.py) pass. They freeze the oracle's answers so that the
GPU parity tests can check the HIP kernels against stored numbers as well as
against a live oracle run, and so that any later change to the oracle shows
up as a diff against them.

Each case k stores float32 inputs  k/x k/dt k/aneg k/B k/C k/dy k/dh_last and
float64 outputs k/y k/ckpt k/h_last k/dx k/ddt k/daneg k/dB k/dC (gradients of
sum(y*dy) + sum(h_last*dh_last)), plus k/chunk.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import oracle  # noqa: E402

# (name, (batch, T, d_inner, d_state), chunk, input style, seed)
CASES = [
    ("tiny", (1, 20, 8, 4), 16, "ref", 101),
    ("ragged", (2, 37, 33, 16), 7, "bench", 102),
    ("odd_state", (1, 16, 32, 5), 16, "bench", 103),
    ("one_step", (3, 1, 40, 8), 16, "ref", 104),
    ("wide_state", (1, 19, 24, 40), 5, "ref", 105),
]


def make() -> dict:
    out = {}
    for name, shape, chunk, style, seed in CASES:
        x, dt, aneg, b_in, c_in = oracle.make_inputs(*shape, seed=seed, style=style)
        rng = np.random.default_rng(seed + 1)
        dy = rng.standard_normal(x.shape, dtype=np.float32)
        dh = rng.standard_normal((shape[0], shape[2], shape[3]), dtype=np.float32)
        y, ckpt, h_last = oracle.scan_fwd(x, dt, aneg, b_in, c_in, chunk=chunk)
        dx, ddt, daneg, db, dc = oracle.scan_bwd(x, dt, aneg, b_in, c_in, dy, dh_last=dh)
        vals = dict(x=x, dt=dt, aneg=aneg, B=b_in, C=c_in, dy=dy, dh_last=dh, y=y, ckpt=ckpt,
                    h_last=h_last, dx=dx, ddt=ddt, daneg=daneg, dB=db, dC=dc,
                    chunk=np.array(chunk))
        for k, v in vals.items():
            out[f"{name}/{k}"] = v
    return out


if __name__ == "__main__":
    oracle.build()
    np.savez_compressed(Path(__file__).with_name("scan_golden.npz"), **make())
    print("wrote", Path(__file__).with_name("scan_golden.npz"))
