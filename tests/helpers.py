"""Shared helpers for the test suite."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

from oracle.reference import LOG2E

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


def emulated_backward(q, k, v, o, m, do, causal, scale):
    """The backward with the reference kernels' rounding points (kernels.py:151-337), in
    float32 on materialised matrices: delta from the stored (rounded) O, P = exp2(S c - M) from
    the saved M, P and dS rounded to the input dtype before the products that use them.
    Returns (dq, dk, dv) and, per element, the change that one-ulp flips of those rounded
    operands can cause (2u sum |dS||K| |scale|, 2u sum |dS||Q| |scale|, 2u sum |P||dO|): a last-bit
    difference upstream (summation order of S) may move a value across a rounding boundary."""
    dt = q.dtype
    qf, kf, vf, dof = (t.float() for t in (q, k, v, do))
    c = scale * LOG2E
    s = qf @ kf.transpose(-1, -2).contiguous() * c
    if causal:
        n = q.shape[-2]
        s = s.masked_fill(torch.ones(n, n, device=q.device, dtype=torch.bool).triu(1), float("-inf"))
    p = torch.exp2(s - m[..., None])
    delta = (dof * o.float()).sum(-1)
    dv = p.to(dt).float().transpose(-1, -2).contiguous() @ dof
    dp = dof @ vf.transpose(-1, -2).contiguous()
    ds = (p * (dp - delta[..., None])).to(dt).float()
    dq = ds @ kf * scale
    dk = ds.transpose(-1, -2).contiguous() @ qf * scale
    two_u = 2.0 ** -10 if dt == torch.float16 else 2.0 ** -7
    bq = two_u * abs(scale) * (ds.abs() @ kf.abs())
    bk = two_u * abs(scale) * (ds.abs().transpose(-1, -2).contiguous() @ qf.abs())
    bv = two_u * (p.transpose(-1, -2).contiguous() @ dof.abs())
    return (dq, dk, dv), (bq, bk, bv)
