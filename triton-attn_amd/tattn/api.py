"""Public API: `attention(q, k, v, causal=False, sm_scale=None)` with autograd.

Drop-in for src/tattn/api.py of amaanmithani/triton-attn: same argument checks and messages
(api.py:45-56), same default scale (api.py:182), same autograd contract (saves q, k, v, o, M;
`once_differentiable` backward returning no grads for `causal` and `scale`, api.py:149-173), and
the same internal `_forward` / `_backward` entry points with a `config=` override
(api.py:78-146). The work runs in hand-written HIP kernels for gfx950 through the C ABI of
libtattn_hip.so. There is no CPU path: on any device other than a ROCm gfx950 GPU the call
raises instead of computing.
"""

from __future__ import annotations

import contextlib
import math
import os
from typing import Any, Callable, Union

import torch
from torch.autograd.function import once_differentiable

from tattn import _lib

Config = Union[int, dict, None]

_DTYPES = {torch.float16: _lib.F16, torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


def hip_available(device: torch.device) -> bool:
    """True if `device` is a ROCm GPU this library runs on (gfx950) and the library loads."""
    device = torch.device(device)
    if device.type != "cuda" or torch.version.hip is None or not torch.cuda.is_available():
        return False
    try:
        lib = _lib.load()
    except (_lib.LibraryMissing, OSError):
        return False
    with torch.cuda.device(device):
        return bool(lib.tattn_device_supported())


def triton_available(device: torch.device) -> bool:
    """The reference's backend probe (src/tattn/api.py:35-42), kept for drop-in callers: reports
    whether the fused kernels (here: HIP for gfx950, not Triton) run on `device`."""
    return hip_available(device)


def _check(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """Input validation with the reference's messages (src/tattn/api.py:45-56)."""
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(
            f"expected q, k, v of equal shape [batch, heads, seq, dim]; got {q.shape}, {k.shape}, {v.shape}"
        )
    if not (q.device == k.device == v.device):
        raise ValueError(f"q, k, v must be on one device, got {q.device}, {k.device}, {v.device}")
    d = q.shape[-1]
    if d not in (16, 32, 64, 128):
        raise ValueError(f"head dim must be 16, 32, 64 or 128, got {d}")
    # bfloat16 is accepted in addition to the reference's float16 / float32 (api.py:55-56).
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in _DTYPES:
        raise ValueError(
            f"q, k, v must share dtype float16, bfloat16 or float32, got {q.dtype}, {k.dtype}, {v.dtype}"
        )


def _bucket(n: int) -> int:
    """Next power of two of a sequence length: the reference's autotune key (api.py:59-62)."""
    return 1 << max(0, (n - 1).bit_length())


_device_ok: dict[int, bool] = {}  # device index -> hip_available (fixed for the process)


def _require_gpu(t: torch.Tensor) -> None:
    idx = t.get_device()
    if _device_ok.get(idx):
        return
    ok = hip_available(t.device)
    if idx >= 0:
        _device_ok[idx] = ok
    if not ok:
        if t.device.type != "cuda":
            raise RuntimeError(
                f"tattn runs on a ROCm gfx950 (MI355X) GPU; got tensors on {t.device}"
            )
        _lib.load()  # raises with the build instructions if the library is missing
        raise RuntimeError(f"tattn: device {t.device} is not a gfx950 (MI355X) GPU")


def _kernel_layout(t: torch.Tensor) -> torch.Tensor:
    """The kernels read rows with 16-byte vector loads: unit d stride, 16-byte aligned rows and
    base. Anything else is copied to a contiguous tensor (same values)."""
    if t.is_contiguous() and t.data_ptr() % 16 == 0:  # rows of 16+ elements: 16-byte multiples
        return t
    vec = 16 // t.element_size()
    ok = (
        t.stride(-1) == 1
        and all(s % vec == 0 for s in t.stride()[:3])
        and t.data_ptr() % 16 == 0
    )
    return t if ok else t.contiguous()


def _resolve(kernel: int, d: int, dtype: torch.dtype, config: Config, causal: bool, n: int) -> int:
    """Maps the reference-style `config=` to a table index: None -> the library's pick; an int is
    the index; a dict may give "id" or any of block_m / block_n / waves / tiles / kind / ring
    (upper-case BLOCK_M / BLOCK_N as in the reference are accepted) and must match at least one
    entry. Of several matches of one kind, the lowest index is taken; matches
    of different kinds (a persistent entry shares its tiles with a pipelined one) are ambiguous
    unless the dict gives "kind", and raise ValueError."""
    if config is None:
        return -1
    if isinstance(config, int):
        return config
    if "id" in config:
        return int(config["id"])
    want = {k.lower(): int(v) for k, v in config.items()
            if k.lower() in ("block_m", "block_n", "waves", "tiles", "kind", "ring")}
    code = _DTYPES[dtype]
    descs = [_lib.config_desc(kernel, d, code, c) for c in range(_lib.num_configs(kernel, d, code))]
    hits = [c for c, desc in enumerate(descs) if all(desc[key] == val for key, val in want.items())]
    if not hits:
        raise ValueError(f"config {config} matches 0 {_lib.KERNEL_NAMES[kernel]} table entries")
    kinds = sorted({descs[c]["kind"] for c in hits})
    if len(kinds) > 1:
        raise ValueError(
            f"config {config} matches {_lib.KERNEL_NAMES[kernel]} table entries {hits} of kinds {kinds} "
            f"(0 generic, 1 pipelined, 2 persistent, 3 paired-wave): give \"kind\" or \"id\""
        )
    return hits[0]


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_current_device = getattr(torch._C, "_cuda_getDevice", torch.cuda.current_device)


def _stream(t: torch.Tensor) -> int:
    """Handle of the current stream of t's device (the stream torch enqueues on)."""
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def _on_device(t: torch.Tensor):
    """Device guard for the library call: a no-op when t's device is already current."""
    idx = t.get_device()
    return contextlib.nullcontext() if idx == _current_device() else torch.cuda.device(idx)


# Optional first-use timing of the tile table. The reference autotunes on the first call of each
# (N bucket, head dim, causal) key (src/tattn/kernels.py:57-61, 151-155, 242-246); here the
# measured picks of the library are the default and timing is opt-in: TATTN_AUTOTUNE=1 in the
# environment, or set_autotune(True). The first call of a key then times every table entry on
# the caller's stream (HIP events; skipped while a graph is being captured) and keeps the
# fastest for that key.
_autotune = os.environ.get("TATTN_AUTOTUNE", "0") not in ("", "0")
_tuned: dict[tuple[int, int, int, int, int, bool], int] = {}  # (kernel, device, N bucket, D, dtype, causal)


def set_autotune(on: bool) -> None:
    """Turn first-use timing of the tile table on or off (the cache is kept)."""
    global _autotune
    _autotune = bool(on)


def autotune_cache() -> dict[str, dict[str, int]]:
    """Entries chosen by timing so far: {kernel: {"device=.., n_bucket=.., d=.., dtype=..,
    causal=..": table id}} (the analog of the reference bench's dump of its autotune caches)."""
    out: dict[str, dict[str, int]] = {name: {} for name in _lib.KERNEL_NAMES.values()}
    for (kernel, dev, bucket, d, code, causal), cid in _tuned.items():
        dtype = str({c: t for t, c in _DTYPES.items()}[code]).removeprefix("torch.")
        key = f"device={dev}, n_bucket={bucket}, d={d}, dtype={dtype}, causal={causal}"
        out[_lib.KERNEL_NAMES[kernel]][key] = cid
    return out


def _tuned_id(kernel: int, t: torch.Tensor, d: int, causal: bool, n: int,
              launch: Callable[[int], int]) -> int:
    """The table entry for this call: -1 (the library's pick) unless autotuning is on; then the
    fastest entry for the key, timed on first use by running `launch(id)` for every entry."""
    if not _autotune or torch.cuda.is_current_stream_capturing():
        return -1
    code = _DTYPES[t.dtype]
    key = (kernel, t.device.index or 0, _bucket(n), d, code, causal)
    if key not in _tuned:
        stream = torch.cuda.current_stream(t.device)
        best, best_ms = -1, float("inf")
        for cid in range(_lib.num_configs(kernel, d, code)):
            if launch(cid) != 0:  # not usable for this call: skip
                continue
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            for _ in range(3):
                launch(cid)
            end.record(stream)
            end.synchronize()
            ms = start.elapsed_time(end)
            if ms < best_ms:
                best, best_ms = cid, ms
        _tuned[key] = best
    return _tuned[key]


def _forward(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool, scale: float,
    config: Config = None, *, save_lse: bool = True,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """(O, M): O in q's layout, M = [Z, H, N] float32 base-2 log-sum-exp (api.py:78-99).
    save_lse=False (no backward will follow) skips M: neither allocated nor stored, M is None."""
    _require_gpu(q)
    lib = _lib.load()
    q, k, v = _kernel_layout(q), _kernel_layout(k), _kernel_layout(v)
    z, h, n, d = q.shape
    o = torch.empty_like(q)
    m = q.new_empty((z, h, n), dtype=torch.float32) if save_lse else None
    cid = -1 if config is None else _resolve(_lib.K_FWD, d, q.dtype, config, causal, n)
    if q.numel() == 0:  # no rows: nothing to launch (the reference's empty grid launches nothing)
        return o, m
    _, (sq, sk, sv, so) = _lib.stride_block(q, k, v, o)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), m.data_ptr() if m is not None else None,
            sq, sk, sv, so, z, h, n, d, _DTYPES[q.dtype], int(causal), float(scale))
    with _on_device(q):
        stream = _stream(q)
        if config is None and _autotune:
            cid = _tuned_id(_lib.K_FWD, q, d, causal, n, lambda c: lib.tattn_fwd(*args, c, stream))
        rc = lib.tattn_fwd(*args, cid, stream)
    _lib.check(rc, "tattn_fwd")
    return o, m


def _backward(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor, m: torch.Tensor,
    do: torch.Tensor, causal: bool, scale: float, config: Config = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dQ, dK, dV), contiguous, in the inputs' dtype (api.py:102-146). `config` is an index
    valid in both backward tables, or a dict {"dkdv": id, "dq": id}."""
    _require_gpu(q)
    lib = _lib.load()
    z, h, n, d = q.shape
    if do.dtype != q.dtype:
        do = do.to(q.dtype)
    q, k, v, do, o = q.contiguous(), k.contiguous(), v.contiguous(), do.contiguous(), o.contiguous()
    m = m.contiguous()
    delta = q.new_empty((z, h, n), dtype=torch.float32)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    if q.numel() == 0:
        return dq, dk, dv
    code = _DTYPES[q.dtype]
    _, (st,) = _lib.stride_block(q)
    if config is None and not _autotune:
        # The whole backward in one library call: preprocess, dK/dV, dQ in stream order.
        with _on_device(q):
            rc = lib.tattn_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
                               dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), m.data_ptr(), delta.data_ptr(), st,
                               z, h, n, d, code, int(causal), float(scale), -1, _stream(q))
        _lib.check(rc, "tattn_bwd")
        return dq, dk, dv
    if isinstance(config, dict) and ("dkdv" in config or "dq" in config):
        kid = _resolve(_lib.K_BWD_DKDV, d, q.dtype, config.get("dkdv"), causal, n)
        qid = _resolve(_lib.K_BWD_DQ, d, q.dtype, config.get("dq"), causal, n)
    else:
        kid = _resolve(_lib.K_BWD_DKDV, d, q.dtype, config, causal, n)
        qid = _resolve(_lib.K_BWD_DQ, d, q.dtype, config, causal, n)
    dkdv_args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                 m.data_ptr(), delta.data_ptr(), st, z, h, n, d, code, int(causal), float(scale))
    dq_args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(), dq.data_ptr(), m.data_ptr(),
               delta.data_ptr(), st, z, h, n, d, code, int(causal), float(scale))
    with _on_device(q):
        stream = _stream(q)
        _lib.check(lib.tattn_bwd_preprocess(o.data_ptr(), do.data_ptr(), delta.data_ptr(), st,
                                            z, h, n, d, code, stream), "tattn_bwd_preprocess")
        if config is None:
            kid = _tuned_id(_lib.K_BWD_DKDV, q, d, causal, n, lambda c: lib.tattn_bwd_dkdv(*dkdv_args, c, stream))
            qid = _tuned_id(_lib.K_BWD_DQ, q, d, causal, n, lambda c: lib.tattn_bwd_dq(*dq_args, c, stream))
        _lib.check(lib.tattn_bwd_dkdv(*dkdv_args, kid, stream), "tattn_bwd_dkdv")
        _lib.check(lib.tattn_bwd_dq(*dq_args, qid, stream), "tattn_bwd_dq")
    return dq, dk, dv


class _Attention(torch.autograd.Function):
    """Autograd wrapper (src/tattn/api.py:149-173)."""

    @staticmethod
    def forward(ctx: Any, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool,
                scale: float) -> torch.Tensor:
        o, m = _forward(q, k, v, causal, scale)
        ctx.save_for_backward(q, k, v, o, m)
        ctx.causal, ctx.scale = causal, scale
        return o

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, do: torch.Tensor) -> tuple[torch.Tensor | None, ...]:
        q, k, v, o, m = ctx.saved_tensors
        dq, dk, dv = _backward(q, k, v, o, m, do, ctx.causal, ctx.scale)
        return dq, dk, dv, None, None


def attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
    sm_scale: float | None = None,
) -> torch.Tensor:
    """Fused attention over [batch, heads, seq, dim] tensors (src/tattn/api.py:176-184):
    softmax(q k^T * sm_scale [causal: key <= query]) v, sm_scale defaulting to 1/sqrt(dim)."""
    _check(q, k, v)
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(q.shape[-1])
    if not (torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)):
        # Inference: no autograd context and no log-sum-exp to save (the reference always saves
        # both, api.py:161); the output is the same.
        return _forward(q, k, v, causal, scale, save_lse=False)[0]
    out: torch.Tensor = _Attention.apply(q, k, v, causal, scale)
    return out


def configs(kernel: str, head_dim: int, dtype: torch.dtype) -> list[dict[str, int]]:
    """Every gfx950 tile-table entry for `kernel` in ("fwd", "bwd_dkdv", "bwd_dq")."""
    kid = {v: k for k, v in _lib.KERNEL_NAMES.items()}[kernel]
    code = _DTYPES[dtype]
    return [_lib.config_desc(kid, head_dim, code, c) for c in range(_lib.num_configs(kid, head_dim, code))]
