"""Writes tests/golden/edge_f64.npz: float64 expected outputs for the edge-shape sweep.

Shapes [1, 2, N, D] with N in {1, 17, 33, 70} (not multiples of any tile) and D in {16, 32, 64}.
Inputs q, k, v, do are drawn from a seeded CPU generator in float32 and rounded to float16, so the
same values are exact in both supported dtypes. Expected O, M and dQ/dK/dV for causal and
non-causal are computed by oracle.exact (float64 brute force) and stored as float32.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import exact  # noqa: E402

NS = (1, 17, 33, 70)
DS = (16, 32, 64)
OUT = Path(__file__).with_name("edge_f64.npz")


def main() -> None:
    import torch

    arrays: dict[str, np.ndarray] = {}
    for n in NS:
        for d in DS:
            g = torch.Generator().manual_seed(1000 * n + d)
            q, k, v, do = (torch.randn(1, 2, n, d, generator=g).half().numpy() for _ in range(4))
            tag = f"n{n}_d{d}"
            for name, t in (("q", q), ("k", k), ("v", v), ("do", do)):
                arrays[f"{tag}_{name}"] = t
            for causal in (False, True):
                ctag = f"{tag}_c{int(causal)}"
                o, m = exact.attention_fwd(q, k, v, causal)
                dq, dk, dv = exact.attention_bwd(q, k, v, do, causal)
                for name, t in (("o", o), ("m", m), ("dq", dq), ("dk", dk), ("dv", dv)):
                    arrays[f"{ctag}_{name}"] = t.astype(np.float32)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main()
