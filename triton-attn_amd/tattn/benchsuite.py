"""Comparison suite: tattn against PyTorch's attention backends on the same GPU.

Serves the purpose of the reference's benchmark script (bench/bench.py of
amaanmithani/triton-attn): speed, memory and accuracy of the fused kernels next to the stock
implementations, at a fixed token count per batch. Measurement semantics follow it where they
must be comparable: the FLOP convention (4*B*H*N^2*D, halved when causal, fwd+bwd = 3.5x fwd),
a cold-cache median timer (tattn.timing.do_bench) and peak memory above the inputs.

The suite is a grid of cells: every implementation x sequence length x mask x pass (forward,
forward+backward). Implementations are plain callables (q, k, v, causal) -> o; an
implementation that cannot run a cell (backend missing for this GPU or dtype, out of memory) is
recorded with its status, not fatal. Errors are measured separately on the same inputs: every
implementation's forward output against float32 materialised attention, and tattn's gradients
against float32 autograd at N = 1024 and 4096 (batch 0).

    python -m tattn.benchsuite [--seqs 512,...,16384] [--tokens 16384] [--heads 16] [--dim 64]
                               [--autotune] [--out results/<arch>.json]

Result schema "tattn-suite/1":
    device   {name, arch, memory_gib, torch, hip, python}
    method   {tokens, heads, dim, dtype, timer, flops, data}
    cells    [{impl, n, b, mask: "none"|"causal", pass: "fwd"|"fwd+bwd", status: "ok"|"oom"|
               "unsupported", ms, tflops, peak_mib, note}]
    errors   [{impl, n, mask, tensor: "o"|"dq"|"dk"|"dv", max_abs, mean_abs}]
    gemm_tflops, picks {n/mask: {kernel: table id}}, autotuned (or null)

Render it with `python -m tattn.report FILE`.
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import math
import platform
from pathlib import Path
from typing import Any, Callable, Iterable

import torch

REPO = Path(__file__).resolve().parents[2]
PASSES = ("fwd", "fwd+bwd")
MASKS = ("none", "causal")


def counted_flops(b: int, h: int, n: int, d: int, causal: bool, passes: str) -> float:
    """The reference's FLOP convention (bench/bench.py:31-35)."""
    per_fwd = 4.0 * b * h * n * n * d * (0.5 if causal else 1.0)
    return per_fwd * (3.5 if passes == "fwd+bwd" else 1.0)


@dataclasses.dataclass(frozen=True)
class Impl:
    name: str
    label: str
    fn: Callable[[torch.Tensor, torch.Tensor, torch.Tensor, bool], torch.Tensor]


def materialised(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool) -> torch.Tensor:
    """softmax(Q K^T / sqrt(D)) V with the N x N matrix in memory; softmax in float32, products in
    the inputs' dtype."""
    s = torch.matmul(q, k.transpose(-2, -1).contiguous()) / math.sqrt(q.shape[-1])
    if causal:
        n = q.shape[-2]
        s = s.masked_fill(torch.ones(n, n, dtype=torch.bool, device=q.device).triu(1), float("-inf"))
    return torch.matmul(torch.softmax(s.float(), dim=-1).to(q.dtype), v)


def default_impls() -> list[Impl]:
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from . import attention

    def backend(which):
        def run(q, k, v, causal):
            with sdpa_kernel(which):
                return F.scaled_dot_product_attention(q, k, v, is_causal=causal)
        return run

    return [
        Impl("tattn", "tattn (HIP, gfx950)", lambda q, k, v, causal: attention(q, k, v, causal=causal)),
        Impl("sdpa_flash", "SDPA flash", backend(SDPBackend.FLASH_ATTENTION)),
        Impl("sdpa_efficient", "SDPA mem-efficient", backend(SDPBackend.EFFICIENT_ATTENTION)),
        Impl("sdpa_math", "SDPA math", backend(SDPBackend.MATH)),
        Impl("materialised", "materialised", materialised),
    ]


@dataclasses.dataclass
class Inputs:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    do: torch.Tensor

    @property
    def b(self) -> int:
        return self.q.shape[0]


def make_inputs(n: int, tokens: int, heads: int, dim: int, device, dtype=torch.float16) -> Inputs:
    """N(0,1) values from a generator on `device` seeded with N (dO from the same stream)."""
    g = torch.Generator(device=device).manual_seed(n)
    shape = (max(1, tokens // n), heads, n, dim)
    return Inputs(*(torch.randn(shape, device=device, dtype=dtype, generator=g) for _ in range(4)))


def call_for(impl: Impl, x: Inputs, causal: bool, passes: str) -> tuple[Callable[[], None], Callable[[], None]]:
    """(the call to time, a reset that drops what a previous call left behind)."""
    if passes == "fwd":
        def fwd() -> None:
            with torch.no_grad():
                impl.fn(x.q, x.k, x.v, causal)
        return fwd, lambda: None
    leaves = [t.detach().clone().requires_grad_() for t in (x.q, x.k, x.v)]

    def reset() -> None:
        for t in leaves:
            t.grad = None

    def fwd_bwd() -> None:
        reset()
        impl.fn(*leaves, causal).backward(x.do)
    return fwd_bwd, reset


Timer = Callable[[Callable[[], None], Callable[[], None]], tuple[float, float]]


def gpu_timer(call: Callable[[], None], reset: Callable[[], None]) -> tuple[float, float]:
    """(median ms with a cold cache, MiB allocated at peak beyond what was live before the call)."""
    from .timing import do_bench

    call()
    reset()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    live = torch.cuda.memory_allocated()
    call()
    torch.cuda.synchronize()
    peak = (torch.cuda.max_memory_allocated() - live) / 2**20
    return do_bench(call), peak


def _status_of(exc: BaseException) -> tuple[str, str]:
    if isinstance(exc, torch.OutOfMemoryError):
        return "oom", "out of memory"
    first = (str(exc).strip().splitlines() or [type(exc).__name__])[0]
    return "unsupported", first[:160]


def sweep_cells(impls: Iterable[Impl], inputs: dict[int, Inputs], heads: int, dim: int, timer: Timer,
                after_cell: Callable[[], None] = lambda: None) -> list[dict[str, Any]]:
    """Times every (implementation, N, mask, pass) cell; failures become a status, not an error."""
    cells = []
    for n, x in inputs.items():
        for mask in MASKS:
            causal = mask == "causal"
            for impl in impls:
                for passes in PASSES:
                    cell: dict[str, Any] = {"impl": impl.name, "n": n, "b": x.b, "mask": mask, "pass": passes}
                    try:
                        call, reset = call_for(impl, x, causal, passes)
                        ms, peak = timer(call, reset)
                        cell.update(status="ok", ms=ms, peak_mib=peak,
                                    tflops=counted_flops(x.b, heads, n, dim, causal, passes) / (ms * 1e-3) / 1e12)
                    except (RuntimeError, torch.OutOfMemoryError) as exc:
                        status, note = _status_of(exc)
                        cell.update(status=status, note=note)
                    after_cell()
                    cells.append(cell)
                    print(json.dumps(cell), flush=True)
    return cells


def measure_errors(impls: Iterable[Impl], inputs: dict[int, Inputs], grad_seqs=(1024, 4096)) -> list[dict[str, Any]]:
    """Forward error of every implementation against float32 materialised attention (all heads),
    and tattn's gradient error against float32 autograd on batch 0 at `grad_seqs`."""
    out: list[dict[str, Any]] = []
    impls = list(impls)
    for n, x in inputs.items():
        for mask in MASKS:
            causal = mask == "causal"
            with torch.no_grad():
                ref = torch.cat([materialised(x.q[i:i + 1].float(), x.k[i:i + 1].float(), x.v[i:i + 1].float(), causal)
                                 for i in range(x.b)])
                for impl in impls:
                    try:
                        err = (impl.fn(x.q, x.k, x.v, causal).float() - ref).abs()
                        out.append({"impl": impl.name, "n": n, "mask": mask, "tensor": "o",
                                    "max_abs": err.max().item(), "mean_abs": err.mean().item()})
                        del err
                    except (RuntimeError, torch.OutOfMemoryError):
                        pass
                del ref
            tattn = next((i for i in impls if i.name == "tattn"), None)
            if tattn is None or n not in grad_seqs:
                continue
            q, k, v, do = (t[:1].detach().clone() for t in (x.q, x.k, x.v, x.do))
            got = [t.clone().requires_grad_() for t in (q, k, v)]
            tattn.fn(*got, causal).backward(do)
            want = [t.float().requires_grad_() for t in (q, k, v)]
            materialised(*want, causal).backward(do.float())
            for name, a, b in zip(("dq", "dk", "dv"), got, want):
                e = (a.grad.float() - b.grad).abs()
                out.append({"impl": "tattn", "n": n, "mask": mask, "tensor": name,
                            "max_abs": e.max().item(), "mean_abs": e.mean().item()})
    return out


def device_info() -> dict[str, Any]:
    p = torch.cuda.get_device_properties(0)
    return {"name": p.name, "arch": getattr(p, "gcnArchName", ""), "memory_gib": round(p.total_memory / 2**30, 1),
            "torch": torch.__version__, "hip": torch.version.hip, "python": platform.python_version()}


def gemm_rate() -> float:
    """TFLOP/s of a plain fp16 4096^3 matmul on the same timer (a GEMM-rate yardstick)."""
    from .timing import do_bench

    a, b = (torch.randn(4096, 4096, device="cuda", dtype=torch.float16) for _ in range(2))
    return 2 * 4096**3 / (do_bench(lambda: a @ b) * 1e-3) / 1e12


def table_picks(seqs: Iterable[int], dim: int) -> dict[str, dict[str, int]]:
    from . import _lib

    return {f"{n}/{mask}": {name: _lib.pick_config(kid, dim, _lib.F16, mask == "causal", n)
                            for kid, name in _lib.KERNEL_NAMES.items()}
            for n in seqs for mask in MASKS}


def run(seqs: list[int], tokens: int, heads: int, dim: int, autotune: bool = False,
        impls: list[Impl] | None = None) -> dict[str, Any]:
    from . import autotune_cache, set_autotune

    impls = impls if impls is not None else default_impls()
    set_autotune(autotune)
    inputs = {n: make_inputs(n, tokens, heads, dim, "cuda") for n in seqs}
    cells = sweep_cells(impls, inputs, heads, dim, gpu_timer, after_cell=torch.cuda.empty_cache)
    errors = measure_errors(impls, inputs)
    return {
        "schema": "tattn-suite/1",
        "device": device_info(),
        "method": {
            "tokens": tokens, "heads": heads, "dim": dim, "dtype": "float16",
            "timer": "tattn.timing.do_bench: 256 MB cache flush before each call, median, ~25 ms warm-up, ~100 ms",
            "flops": "4*B*H*N^2*D (halved when causal); fwd+bwd = 3.5x fwd",
            "data": "N(0,1), device generator seeded with N (dO from the same generator)",
        },
        "cells": cells,
        "errors": errors,
        "gemm_tflops": gemm_rate(),
        "picks": table_picks(seqs, dim),
        "autotuned": autotune_cache() if autotune else None,
    }


def main(argv: list[str] | None = None) -> None:
    ap = argparse.ArgumentParser(description="tattn against PyTorch's attention backends")
    ap.add_argument("--seqs", default="512,1024,2048,4096,8192,16384")
    ap.add_argument("--tokens", type=int, default=16384, help="batch * seq per cell")
    ap.add_argument("--heads", type=int, default=16)
    ap.add_argument("--dim", type=int, default=64)
    ap.add_argument("--autotune", action="store_true", help="time the tile table on first use")
    ap.add_argument("--out", default=None)
    a = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("needs a ROCm GPU")
    res = run([int(s) for s in a.seqs.split(",")], a.tokens, a.heads, a.dim, a.autotune)
    arch = res["device"]["arch"].split(":")[0] or res["device"]["name"].replace(" ", "_").lower()
    out = Path(a.out) if a.out else REPO / "results" / f"{arch}.json"
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(res, indent=1) + "\n")
    print("wrote", out)


if __name__ == "__main__":
    main()
