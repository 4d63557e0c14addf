"""The committed float64 fixtures agree with the oracle (CPU only)."""

import pytest
import torch

from helpers import golden
from oracle.reference import tiled_backward, tiled_forward

CASES = [(n, d, c) for n in (1, 17, 33, 70) for d in (16, 32, 64) for c in (0, 1)]


@pytest.mark.parametrize("n,d,causal", CASES)
def test_oracle_matches_fixture(n, d, causal):
    g = golden()
    tag = f"n{n}_d{d}"
    q, k, v, do = (torch.from_numpy(g[f"{tag}_{x}"]).float() for x in ("q", "k", "v", "do"))
    o, m = tiled_forward(q, k, v, bool(causal))
    ctag = f"{tag}_c{causal}"
    torch.testing.assert_close(o, torch.from_numpy(g[f"{ctag}_o"]), atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(m, torch.from_numpy(g[f"{ctag}_m"]), atol=1e-5, rtol=1e-5)
    grads = tiled_backward(q, k, v, o, m, do, bool(causal))
    for name, got in zip(("dq", "dk", "dv"), grads):
        torch.testing.assert_close(got, torch.from_numpy(g[f"{ctag}_{name}"]), atol=2e-5, rtol=2e-5)


def test_published_accuracy_fixture_covers_the_benchmark():
    """tests/golden/t4_accuracy.json (written by make_t4_accuracy.py from the reference's published
    results): forward errors at every benchmark length, both masks; gradients at 1024 and 4096."""
    import json
    from pathlib import Path

    e = json.loads((Path(__file__).parent / "golden" / "t4_accuracy.json").read_text())["entries"]
    fwd = {(x["seq"], x["causal"]) for x in e if "grad" not in x}
    assert fwd == {(n, c) for n in (512, 1024, 2048, 4096, 8192, 16384) for c in (False, True)}
    grads = {(x["seq"], x["causal"], x["grad"]) for x in e if "grad" in x}
    assert grads == {(n, c, g) for n in (1024, 4096) for c in (False, True) for g in ("dq", "dk", "dv")}
    assert all(0 < x["max_abs_err"] < 2e-3 for x in e)
