"""Comparison benchmark: tattn against PyTorch's attention backends on this GPU.

The counterpart of the reference's benchmark (bench/bench.py:1-206): for every sequence length
(batch x seq held at a fixed token count), causal and not, forward and forward+backward, it
times

  - tattn (this package's HIP kernels, table-picked tiles, or with --autotune the fastest
    table entry timed on first use; the picks are recorded as the reference records its
    autotune caches, bench/bench.py:176-201),
  - torch SDPA with each backend (flash, memory-efficient, math), one at a time,
  - naive materialised attention (the definition),

with the reference's timer (tattn.timing.do_bench: cache flushed before each call, median over
~100 ms after ~25 ms of warm-up) and records peak extra memory per call. It then measures the
output error of every implementation against float32 materialised attention at every length
(the float32 reference fits in HBM at 16k tokens here), tattn's gradient error against float32
autograd at N = 1024 and 4096, and a plain fp16 4096^3 matmul as a GEMM-rate reference. Cells an
implementation cannot run (unsupported backend, out of memory) are recorded, not fatal.

    python -m tattn.benchsuite [--seqs 512,...,16384] [--tokens 16384] [--heads 16] [--dim 64]
                               [--autotune] [--out results/<gpu>.json]

Render the result with `python -m tattn.report results/<gpu>.json`.
"""

from __future__ import annotations

import argparse
import json
import math
import platform
from pathlib import Path
from typing import Any, Callable

import torch
import torch.nn.functional as F

from . import attention, autotune_cache, set_autotune
from . import _lib
from .timing import do_bench

IMPLS = ("tattn", "sdpa_flash", "sdpa_efficient", "sdpa_math", "naive")
REPO = Path(__file__).resolve().parents[2]


def flops(b: int, h: int, n: int, d: int, causal: bool, mode: str) -> float:
    """The reference's FLOP convention (bench/bench.py:31-35)."""
    f = 4.0 * b * h * n * n * d
    if causal:
        f *= 0.5
    return f * (3.5 if mode == "fwd+bwd" else 1.0)


def naive(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool) -> torch.Tensor:
    """softmax(Q K^T / sqrt(D)) V, materialised, in the inputs' dtype (the comparator the
    reference calls naive)."""
    s = torch.matmul(q, k.transpose(-2, -1).contiguous()) * (1.0 / math.sqrt(q.shape[-1]))
    if causal:
        n = q.shape[-2]
        s = s.masked_fill(torch.ones(n, n, dtype=torch.bool, device=q.device).triu(1), float("-inf"))
    return torch.matmul(torch.softmax(s.float(), dim=-1).to(q.dtype), v)


def _sdpa(backend) -> Callable[..., torch.Tensor]:
    from torch.nn.attention import sdpa_kernel

    def run(q, k, v, causal):
        with sdpa_kernel(backend):
            return F.scaled_dot_product_attention(q, k, v, is_causal=causal)

    return run


def implementations() -> dict[str, Callable[..., torch.Tensor]]:
    from torch.nn.attention import SDPBackend

    return {
        "tattn": lambda q, k, v, causal: attention(q, k, v, causal=causal),
        "sdpa_flash": _sdpa(SDPBackend.FLASH_ATTENTION),
        "sdpa_efficient": _sdpa(SDPBackend.EFFICIENT_ATTENTION),
        "sdpa_math": _sdpa(SDPBackend.MATH),
        "naive": naive,
    }


def measure(fn: Callable[[], Any], clear: Callable[[], None] = lambda: None) -> dict[str, Any]:
    """Median ms and peak memory above the baseline of one call; `clear` drops state left by the
    warm-up call (gradients) before the baseline is taken."""
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    try:
        fn()
        clear()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        fn()
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated() - base
        return {"ms": do_bench(fn), "peak_extra_mib": peak / 2**20}
    except torch.OutOfMemoryError:
        torch.cuda.empty_cache()
        return {"oom": True}
    except RuntimeError as e:  # backend unavailable for this GPU, dtype or shape
        torch.cuda.empty_cache()
        return {"error": str(e).splitlines()[0][:200]}


def run(seqs: list[int], tokens: int, heads: int, dim: int, autotune: bool = False) -> dict[str, Any]:
    dev = torch.device("cuda")
    _lib.load()
    props = torch.cuda.get_device_properties(dev)
    impls = implementations()
    rows: list[dict[str, Any]] = []
    accuracy: list[dict[str, Any]] = []
    picks: dict[str, dict[str, int]] = {}
    set_autotune(autotune)
    for n in seqs:
        b = max(1, tokens // n)
        for causal in (False, True):
            g = torch.Generator(device=dev).manual_seed(n)
            q, k, v, do = (torch.randn(b, heads, n, dim, device=dev, dtype=torch.float16, generator=g)
                           for _ in range(4))
            for name, f in impls.items():
                for mode in ("fwd", "fwd+bwd"):
                    clear: Callable[[], None] = lambda: None  # noqa: E731
                    if mode == "fwd":
                        def fn(f=f, q=q, k=k, v=v, causal=causal) -> None:
                            with torch.no_grad():
                                f(q, k, v, causal)
                    else:
                        qg, kg, vg = (t.detach().clone().requires_grad_() for t in (q, k, v))

                        def fn(f=f, qg=qg, kg=kg, vg=vg, do=do, causal=causal) -> None:
                            qg.grad = kg.grad = vg.grad = None
                            f(qg, kg, vg, causal).backward(do)

                        def clear(qg=qg, kg=kg, vg=vg) -> None:
                            qg.grad = kg.grad = vg.grad = None
                    r = measure(fn, clear)
                    if "ms" in r:
                        r["tflops"] = flops(b, heads, n, dim, causal, mode) / (r["ms"] * 1e-3) / 1e12
                    rows.append({"impl": name, "seq": n, "batch": b, "causal": causal, "mode": mode, **r})
                    print(json.dumps(rows[-1]), flush=True)
            # Output error against float32 materialised attention (all heads, every length).
            with torch.no_grad():
                ref = naive(q.float(), k.float(), v.float(), causal)
                for name, f in impls.items():
                    try:
                        out = f(q, k, v, causal).float()
                        accuracy.append({"impl": name, "seq": n, "causal": causal, "reference": "naive fp32",
                                         "max_abs_err": (out - ref).abs().max().item(),
                                         "mean_abs_err": (out - ref).abs().mean().item()})
                        del out
                    except (RuntimeError, torch.OutOfMemoryError) as e:
                        accuracy.append({"impl": name, "seq": n, "causal": causal,
                                         "error": str(e).splitlines()[0][:120]})
                del ref
            # tattn gradients against float32 autograd of the definition.
            if n in (1024, 4096):
                qs, ks, vs, dos = (t[:1].detach().clone() for t in (q, k, v, do))
                qg, kg, vg = (t.clone().requires_grad_() for t in (qs, ks, vs))
                attention(qg, kg, vg, causal=causal).backward(dos)
                qr, kr, vr = (t.float().requires_grad_() for t in (qs, ks, vs))
                naive(qr, kr, vr, causal).backward(dos.float())
                for label, got, want in (("dq", qg.grad, qr.grad), ("dk", kg.grad, kr.grad),
                                         ("dv", vg.grad, vr.grad)):
                    accuracy.append({"impl": "tattn", "seq": n, "causal": causal, "grad": label,
                                     "max_abs_err": (got.float() - want).abs().max().item()})
            picks[f"{n}{'_causal' if causal else ''}"] = {
                name: _lib.pick_config(kid, dim, _lib.F16, causal, n) for kid, name in _lib.KERNEL_NAMES.items()}
            del q, k, v, do
            torch.cuda.empty_cache()
    a_ = torch.randn(4096, 4096, device=dev, dtype=torch.float16)
    b_ = torch.randn(4096, 4096, device=dev, dtype=torch.float16)
    mm_ms = do_bench(lambda: a_ @ b_)
    return {
        "env": {
            "gpu": props.name,
            "arch": getattr(props, "gcnArchName", ""),
            "memory_gib": round(props.total_memory / 2**30, 1),
            "torch": torch.__version__,
            "hip": torch.version.hip,
            "python": platform.python_version(),
        },
        "config": {
            "tokens": tokens, "heads": heads, "dim": dim, "dtype": "float16",
            "timer": "tattn.timing.do_bench: 256 MB cache flush before each call, median, warm-up ~25 ms, rep ~100 ms",
            "flops": "4*B*H*N^2*D (halved when causal); fwd+bwd = 3.5x fwd",
            "data": "N(0,1), device generator seeded with N (dO from the same generator)",
        },
        "fp16_matmul_4096_tflops": 2 * 4096**3 / (mm_ms * 1e-3) / 1e12,
        "rows": rows,
        "accuracy": accuracy,
        "table_picks": picks,
        "tuned_configs": autotune_cache() if autotune else None,
    }


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--seqs", default="512,1024,2048,4096,8192,16384")
    ap.add_argument("--tokens", type=int, default=16384, help="batch * seq held constant")
    ap.add_argument("--heads", type=int, default=16)
    ap.add_argument("--dim", type=int, default=64)
    ap.add_argument("--autotune", action="store_true", help="time the tile table on first use")
    ap.add_argument("--out", default=None)
    a = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit("needs a ROCm GPU")
    res = run([int(x) for x in a.seqs.split(",")], a.tokens, a.heads, a.dim, a.autotune)
    name = res["env"]["arch"].split(":")[0] or res["env"]["gpu"].replace(" ", "_").lower()
    out = Path(a.out) if a.out else REPO / "results" / f"{name}.json"
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(res, indent=2) + "\n")
    print("wrote", out)


if __name__ == "__main__":
    main()
