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


# The error envelope the port is held to (the reference's stated maxima, docs/SPEC.md:23 and
# README.md:58-63 of amaanmithani/triton-attn): max abs error against float32 materialised
# attention and its autograd.
F16_MAX = 2e-3
F32_MAX = 1e-5
# Gradients in 16 bits are held to max(envelope, E + margin), where E is the max abs error, against
# the same float32 reference, of the reference's own backward algorithm with its rounding points
# (oracle.reference.rounded_backward) run on the backward's inputs: q, k, v, dO and the forward's
# saved O and M. Where that algorithm stays within the envelope the flat envelope holds; where it
# does not (causal rows that see few keys reach |grad| of 4-8, where the 16-bit store alone costs up
# to half an ulp), the kernel may exceed the algorithm's own error by the margin only. The margin
# covers one last-place flip at the store: kernel and algorithm sum in different orders, so a value
# near a rounding midpoint can land on the other neighbour, moving the error by at most the
# distance of the exact value from that midpoint (measured up to 3.3e-4 at |dv| in [4, 8)).
# 5e-4 in fp16, 8x that in bf16 (3 fewer mantissa bits).
GRAD_ENVELOPE = {torch.float16: F16_MAX, torch.bfloat16: 8 * F16_MAX}
GRAD_MARGIN = {torch.float16: 5e-4, torch.bfloat16: 8 * 5e-4}


def max_err(got, want) -> float:
    return (got.float() - want.float()).abs().max().item() if got.numel() else 0.0


def check_max(label: str, got, want, bound: float) -> float:
    """Flat check max |got - want| <= bound; prints the measured maximum."""
    err = max_err(got, want)
    print(f"{label}: max abs err {err:.3e} (bound {bound:.0e})", flush=True)
    assert err <= bound, f"{label}: max abs error {err:.3e} exceeds {bound:.0e}"
    return err


def check_grads_pinned(tag: str, got, want, emulated, dtype, exact_m=None) -> list[tuple[float, float, float]]:
    """16-bit gradients (dq, dk, dv) against the float32 reference `want`, bounded by
    max(envelope, E + margin) with E the error of `emulated` (the reference's backward algorithm
    with its rounding points on the same inputs, oracle.reference.rounded_backward with the
    forward's O and M) against the same `want`. Prints the kernel's error, E, the bound, the
    kernel's distance to the emulation and, when given, the error of `exact_m` (the same algorithm
    from the exact log-sum-exp and the exactly rounded O: the reference's whole pipeline); returns
    (err, E, bound) per gradient."""
    out = []
    for i, (name, g, w, e) in enumerate(zip(("dq", "dk", "dv"), got, want, emulated)):
        err, emu = max_err(g, w), max_err(e, w)
        bound = max(GRAD_ENVELOPE[dtype], emu + GRAD_MARGIN[dtype])
        extra = f", reference pipeline (exact M) {max_err(exact_m[i], w):.3e}" if exact_m is not None else ""
        print(f"{tag} {name}: max abs err {err:.3e}, reference algorithm {emu:.3e}, bound {bound:.3e}, "
              f"kernel vs reference algorithm {max_err(g, e):.3e}{extra}", flush=True)
        assert err <= bound, f"{tag} {name}: max abs error {err:.3e} exceeds {bound:.3e} (reference algorithm {emu:.3e})"
        out.append((err, emu, bound))
    return out


def emulated_backward(q, k, v, o, m, do, causal, scale):
    """The backward with the reference kernels' rounding points (kernels.py:151-337), in
    float32 on materialised matrices: delta from the stored (rounded) O, P = exp2(S c - M) from
    the saved M, P and dS rounded to the input dtype before the products that use them.
    Returns (dq, dk, dv) and, per element, the change that one-ulp flips of those rounded
    operands can cause (2u sum |dS||K| |scale|, 2u sum |dS||Q| |scale|, 2u sum |P||dO|): a last-bit
    difference upstream (summation order of S) may move a value across a rounding boundary.
    Callers cap that allowance with a flat bound (flip_cap)."""
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


def flip_cap(dtype, scale: float) -> float:
    """Flat cap on the one-ulp flip allowance of emulated_backward: one more error envelope of
    the dtype, scaled like dq and dk by |scale| against the default 1/8 (near one-hot rows at a
    large scale turn a flipped dS into a proportionally larger dq, dk)."""
    env = F16_MAX if dtype == torch.float16 else 8 * F16_MAX
    return env * max(1.0, abs(scale) / 0.125)
