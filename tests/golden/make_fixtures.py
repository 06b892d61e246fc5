"""Writes the committed golden vectors of the Block AttnRes operator.

The reference (sabdulmajid/blackwell-switchyard) commits no fixtures: its
tests draw seeded inputs and compare against an on-the-fly float64 oracle
(tests/test_triton_op.py:47-52). These fixtures freeze that procedure so the
CPU suite and the GPU parity tests see identical bytes on every machine.

Inputs are drawn with numpy's PCG64 and rounded to bfloat16 (so they are exact
in every dtype the operator accepts); expected outputs are float64 from the C
oracle (oracle/attnres_oracle.c) and must agree with the torch restatement
(oracle/reference.py) to 1e-12 before anything is written.

Run from the repository root:  python tests/golden/make_fixtures.py
"""

from __future__ import annotations

import pathlib
import sys

import numpy as np
import torch

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import c_oracle  # noqa: E402
from oracle import reference as oref  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent / "attnres_golden.npz"

# (name, N, B, T, D, ||w||, S): the reference's odd shapes (D=63, N=17), a
# representative D, and a saturated query.
CASES = [
    ("small", 4, 1, 8, 64, 1.0, 3),
    ("odd", 3, 2, 5, 63, 1.0, 2),
    ("deep", 17, 1, 3, 40, 2.0, 2),
    ("wide", 9, 1, 2, 512, 1.0, 4),
    ("saturated", 5, 1, 4, 32, 40.0, 1),
    ("single", 1, 1, 3, 16, 1.0, 1),
]


def bf16_round(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(torch.bfloat16).double().numpy()


def main() -> None:
    rng = np.random.Generator(np.random.PCG64(20260312))
    arrays: dict[str, np.ndarray] = {}
    for name, n, b, t, d, scale, s in CASES:
        v = bf16_round(rng.standard_normal((n, b, t, d)))
        w = rng.standard_normal(d)
        w = bf16_round(w / np.linalg.norm(w) * scale)
        g = bf16_round(rng.standard_normal((b, t, d)))
        q = rng.standard_normal((s, d))
        q = bf16_round(q / np.linalg.norm(q, axis=1, keepdims=True))
        vt = v.reshape(n, b * t, d)
        out = c_oracle.forward(vt, w).reshape(b, t, d)
        dv, dw = c_oracle.backward(vt, w, g.reshape(b * t, d))
        batched = c_oracle.batched(vt, q).reshape(s, b, t, d)
        # Cross-check against the torch restatement before freezing anything.
        out_t = oref.block_attn_res_reference(torch.from_numpy(v), torch.from_numpy(w)).numpy()
        dv_t, dw_t = oref.oracle_grads(torch.from_numpy(v), torch.from_numpy(w), torch.from_numpy(g))
        assert np.abs(out - out_t).max() < 1e-12, name
        assert np.abs(dv.reshape(v.shape) - dv_t.numpy()).max() < 1e-12, name
        assert np.abs(dw - dw_t.numpy()).max() < 1e-12, name
        for key, arr in (("v", v), ("w", w), ("g", g), ("q", q), ("out", out),
                         ("dv", dv.reshape(v.shape)), ("dw", dw), ("batched", batched)):
            arrays[f"{name}/{key}"] = arr
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main()
