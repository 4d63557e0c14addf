"""Float64 numpy brute force for attention (test infrastructure only).

Independent of torch: pins `oracle.reference` and the GPU kernels against the mathematics.
- `attention_fwd`: O = softmax(Q K^T * s) V with the causal `key > query` mask, and
  M = log2(sum_j exp(s_ij)) computed as max + log2(sum 2^(x - max)) over base-2 scores
  x = s * log2(e) -- the quantity the reference's kernels save (src/tattn/kernels.py:143).
- `attention_bwd`: closed-form gradients of O with respect to Q, K, V for an upstream dO:
  dV = P^T dO, dP = dO V^T, dS = P * (dP - rowsum(dO * O)), dQ = s dS K, dK = s dS^T Q.
  These are the textbook softmax-attention gradients; the reference's backward restates them
  in tiles (src/tattn/reference.py:67-102).
"""

from __future__ import annotations

import math

import numpy as np

LOG2E = 1.4426950408889634


def _scale(d: int, sm_scale: float | None) -> float:
    return sm_scale if sm_scale is not None else 1.0 / math.sqrt(d)


def _probs(q: np.ndarray, k: np.ndarray, causal: bool, sm_scale: float | None) -> tuple[np.ndarray, np.ndarray]:
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    n = q.shape[-2]
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * _scale(q.shape[-1], sm_scale)
    if causal:
        above = np.triu(np.ones((n, n), dtype=bool), 1)
        s = np.where(above, -np.inf, s)
    x = s * LOG2E
    mx = x.max(axis=-1, keepdims=True)
    e = np.exp2(x - mx)
    tot = e.sum(axis=-1, keepdims=True)
    lse2 = (mx + np.log2(tot))[..., 0]
    return e / tot, lse2


def attention_fwd(q, k, v, causal: bool = False, sm_scale: float | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Returns (O, M) in float64; M is the base-2 log-sum-exp of the scaled scores."""
    p, lse2 = _probs(q, k, causal, sm_scale)
    return np.matmul(p, np.asarray(v, dtype=np.float64)), lse2


def attention_bwd(q, k, v, do, causal: bool = False,
                  sm_scale: float | None = None) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Closed-form (dQ, dK, dV) in float64 for loss = sum(O * dO)."""
    q64, k64, v64, do64 = (np.asarray(t, dtype=np.float64) for t in (q, k, v, do))
    s = _scale(q64.shape[-1], sm_scale)
    p, _ = _probs(q64, k64, causal, sm_scale)
    o = np.matmul(p, v64)
    dv = np.matmul(np.swapaxes(p, -1, -2), do64)
    dp = np.matmul(do64, np.swapaxes(v64, -1, -2))
    delta = (do64 * o).sum(axis=-1, keepdims=True)
    ds = p * (dp - delta)
    dq = np.matmul(ds, k64) * s
    dk = np.matmul(np.swapaxes(ds, -1, -2), q64) * s
    return dq, dk, dv
