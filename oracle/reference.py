"""CPU restatement of the reference's PyTorch attention algorithms (test infrastructure only).

Follows `src/tattn/reference.py` of amaanmithani/triton-attn:
- `naive_attention`   <- reference.py:18-26 (materialised softmax(Q K^T * s) V, triu(1) mask)
- `tiled_forward`     <- reference.py:29-64 (online softmax in base 2, returns O and M)
- `tiled_backward`    <- reference.py:67-102 (FlashAttention-2 backward, dK/dV per key block,
                          dQ per query block, P rebuilt from M, causal lower bound rounding)
- `rounded_backward`  <- kernels.py:142-146, 151-239, 242-337 (the fused kernels' gradients
                          with their rounding points: P and dS rounded to the input dtype as
                          GEMM operands, delta from the stored O, gradients rounded at the store)
- `flops`             <- bench/bench.py:31-35

All arithmetic is float32, like the reference (it upcasts at reference.py:41 and :83);
`rounded_backward` rounds to the input dtype exactly where the reference's kernels do.
"""

from __future__ import annotations

import math

import torch

LOG2E = 1.4426950408889634


def _scale(d: int, sm_scale: float | None) -> float:
    return sm_scale if sm_scale is not None else 1.0 / math.sqrt(d)


def naive_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
                    sm_scale: float | None = None) -> torch.Tensor:
    """The definition, materialising the [N, N] score matrix (reference.py:18-26)."""
    s = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) * _scale(q.shape[-1], sm_scale)
    if causal:
        n = q.shape[-2]
        above = torch.ones(n, n, dtype=torch.bool, device=q.device).triu(1)
        s = s.masked_fill(above, float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), v.float()).to(q.dtype)


def tiled_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
                  sm_scale: float | None = None, block_m: int = 16,
                  block_n: int = 16) -> tuple[torch.Tensor, torch.Tensor]:
    """Online-softmax forward over [*, N, D] tensors (reference.py:29-64).

    Scores are scaled by sm_scale*log2(e) and exponentiated with exp2; M = running max +
    log2(running sum) per query row, float32. Causal query blocks stop at their own last row.
    """
    *lead, n, d = q.shape
    c = _scale(d, sm_scale) * LOG2E
    qf, kf, vf = q.float(), k.float(), v.float()
    o = torch.empty(*lead, n, d, dtype=torch.float32, device=q.device)
    lse = torch.empty(*lead, n, dtype=torch.float32, device=q.device)
    for r0 in range(0, n, block_m):
        r1 = min(r0 + block_m, n)
        rows = torch.arange(r0, r1, device=q.device)
        qb = qf[..., r0:r1, :]
        run_max = torch.full((*lead, r1 - r0), float("-inf"), device=q.device)
        run_sum = torch.zeros(*lead, r1 - r0, device=q.device)
        acc = torch.zeros(*lead, r1 - r0, d, device=q.device)
        stop = r1 if causal else n
        for c0 in range(0, stop, block_n):
            c1 = min(c0 + block_n, n)
            cols = torch.arange(c0, c1, device=q.device)
            s = torch.matmul(qb, kf[..., c0:c1, :].transpose(-1, -2)) * c
            if causal:
                s = s.masked_fill(cols[None, :] > rows[:, None], float("-inf"))
            new_max = torch.maximum(run_max, s.amax(dim=-1))
            p = torch.exp2(s - new_max.unsqueeze(-1))
            corr = torch.exp2(run_max - new_max)
            run_sum = run_sum * corr + p.sum(dim=-1)
            acc = acc * corr.unsqueeze(-1) + torch.matmul(p, vf[..., c0:c1, :])
            run_max = new_max
        o[..., r0:r1, :] = acc / run_sum.unsqueeze(-1)
        lse[..., r0:r1] = run_max + torch.log2(run_sum)
    return o.to(q.dtype), lse


def tiled_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                   lse: torch.Tensor, do: torch.Tensor, causal: bool = False,
                   sm_scale: float | None = None, block_m: int = 16,
                   block_n: int = 16) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """FlashAttention-2 backward (reference.py:67-102).

    delta = rowsum(dO * O) from the stored (rounded) O; for each key block, query blocks from
    lo = floor(c0 / block_m) * block_m (causal) or 0; P = exp2(S*s*log2e - M) with the causal
    mask; dV += P^T dO; dS = P (dO V^T - delta); dK += s dS^T Q; dQ += s dS K.
    """
    *_, n, d = q.shape
    sm = _scale(d, sm_scale)
    c = sm * LOG2E
    qf, kf, vf, dof = q.float(), k.float(), v.float(), do.float()
    delta = (dof * o.float()).sum(dim=-1)
    dq = torch.zeros_like(qf)
    dk = torch.zeros_like(kf)
    dv = torch.zeros_like(vf)
    for c0 in range(0, n, block_n):
        c1 = min(c0 + block_n, n)
        cols = torch.arange(c0, c1, device=q.device)
        first = (c0 // block_m) * block_m if causal else 0
        for r0 in range(first, n, block_m):
            r1 = min(r0 + block_m, n)
            rows = torch.arange(r0, r1, device=q.device)
            s = torch.matmul(qf[..., r0:r1, :], kf[..., c0:c1, :].transpose(-1, -2)) * c
            p = torch.exp2(s - lse[..., r0:r1].unsqueeze(-1))
            if causal:
                p = p.masked_fill(cols[None, :] > rows[:, None], 0.0)
            dv[..., c0:c1, :] += torch.matmul(p.transpose(-1, -2), dof[..., r0:r1, :])
            dp = torch.matmul(dof[..., r0:r1, :], vf[..., c0:c1, :].transpose(-1, -2))
            ds = p * (dp - delta[..., r0:r1].unsqueeze(-1))
            dk[..., c0:c1, :] += torch.matmul(ds.transpose(-1, -2), qf[..., r0:r1, :]) * sm
            dq[..., r0:r1, :] += torch.matmul(ds, kf[..., c0:c1, :]) * sm
    return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype)


def rounded_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, do: torch.Tensor,
                     causal: bool = False, sm_scale: float | None = None, o: torch.Tensor | None = None,
                     lse: torch.Tensor | None = None,
                     max_scores: int = 1 << 28) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The gradients the reference's fused kernels produce, evaluated in float32 on materialised
    [N, N] matrices with the kernels' rounding points (src/tattn/kernels.py):
    - M is the exact base-2 log-sum-exp of the float32 scores S * s * log2(e) (`:143`), and the
      stored O = softmax(S) V is rounded to the input dtype (`:142-146`); a given `o` and `lse`
      (a forward's stored O and M, the backward's inputs at `api.py:102-105`) replace them;
    - delta = rowsum(dO * O) over that stored O, in float32 (`:324-337`);
    - P = exp2(S * s * log2(e) - M), 0 above the diagonal when causal (`:221-224`, `:309-312`);
      P is rounded to the dtype only as the operand of P^T dO (`:225`);
    - dS = P (dO V^T - delta) in float32 (`:226-227`, `:313-314`), rounded to the dtype as the
      operand of dS^T Q and dS K (`:228`, `:315`);
    - dK and dQ are scaled by s in float32 (`:232`, `:319`), and every gradient is rounded to the
      dtype at its store (`:230-238`, `:317-321`).
    In float32 every rounding point is the identity, so the result is the exact gradient up to
    float32 summation. Leading dimensions are processed in chunks of at most `max_scores` score
    elements. Returns (dq, dk, dv) in the input dtype."""
    *lead, n, d = q.shape
    dt = q.dtype
    sm = _scale(d, sm_scale)
    c = sm * LOG2E
    flat = [t.reshape(-1, n, d) for t in (q, k, v, do)]
    o_flat = o.reshape(-1, n, d) if o is not None else None
    m_flat = lse.reshape(-1, n) if lse is not None else None
    outs = [torch.empty(flat[0].shape, dtype=dt, device=q.device) for _ in range(3)]
    above = torch.ones(n, n, dtype=torch.bool, device=q.device).triu(1) if causal else None
    per = max(1, max_scores // (n * n))
    for s0 in range(0, flat[0].shape[0], per):
        qf, kf, vf, dof = (t[s0:s0 + per].float() for t in flat)
        x = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * c
        if above is not None:
            x = x.masked_fill(above, float("-inf"))
        if m_flat is None:
            m = torch.logsumexp(x / LOG2E, dim=-1) * LOG2E  # base-2 log-sum-exp of the base-2 scores
        else:
            m = m_flat[s0:s0 + per].float()
        p = torch.exp2(x - m.unsqueeze(-1))
        del x
        if o_flat is None:
            of = torch.matmul(p, vf).to(dt).float()
        else:
            of = o_flat[s0:s0 + per].float()
        delta = (dof * of).sum(dim=-1)
        outs[2][s0:s0 + per] = torch.matmul(p.to(dt).float().transpose(-1, -2).contiguous(), dof).to(dt)
        dp = torch.matmul(dof, vf.transpose(-1, -2).contiguous())
        ds = (p * (dp - delta.unsqueeze(-1))).to(dt).float()
        del p, dp
        outs[0][s0:s0 + per] = (torch.matmul(ds, kf) * sm).to(dt)
        outs[1][s0:s0 + per] = (torch.matmul(ds.transpose(-1, -2).contiguous(), qf) * sm).to(dt)
        del ds
    return tuple(t.reshape(*lead, n, d) for t in outs)


def flops(b: int, h: int, n: int, d: int, causal: bool, mode: str) -> float:
    """Counted work of the reference benchmark (bench/bench.py:31-35): 4*B*H*N^2*D for QK^T
    and PV (2 flops per multiply-add), halved when causal, times 3.5 for fwd+bwd."""
    f = 4.0 * b * h * n * n * d
    if causal:
        f *= 0.5
    return f * (3.5 if mode == "fwd+bwd" else 1.0)
