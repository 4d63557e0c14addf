"""Shared helpers for the test suite."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden" / "edge_f64.npz"


def rand(shape, dtype, seed, device="cpu"):
    """Seeded N(0,1) drawn on the CPU in float32, then cast and moved (the reference's recipe,
    tests/test_attention.py:16-18), so values are identical on every machine."""
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(device, dtype)


def golden():
    return np.load(GOLDEN, allow_pickle=False)


def gpu_ready() -> bool:
    if not torch.cuda.is_available() or torch.version.hip is None:
        return False
    from tattn import hip_available

    return hip_available(torch.device("cuda:0"))
