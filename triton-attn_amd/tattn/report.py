"""Markdown report of a tattn.benchsuite result (the counterpart of the reference's
bench/report.py:21-226, which renders the same tables into its README).

    python -m tattn.report results/gfx950.json [--out results/gfx950.md] [--check]

Sections: environment and method; TFLOP/s per implementation for forward and forward+backward,
non-causal and causal; peak extra memory of forward+backward; implementations that did not
run; output and gradient error against float32; tattn's speed-up over each SDPA backend.
`--check` only verifies that the file parses and has rows.
"""

from __future__ import annotations

import argparse
import json
from pathlib import Path
from typing import Any

IMPLS = ["tattn", "sdpa_flash", "sdpa_efficient", "sdpa_math", "naive"]
LABEL = {
    "tattn": "tattn (HIP, gfx950)",
    "sdpa_flash": "SDPA flash",
    "sdpa_efficient": "SDPA mem-efficient",
    "sdpa_math": "SDPA math",
    "naive": "naive",
}
PEAK_F16_TFLOPS = 2516.6


def _find(rows: list[dict[str, Any]], **kv: Any) -> dict[str, Any] | None:
    return next((r for r in rows if all(r.get(k) == v for k, v in kv.items())), None)


def _cell(r: dict[str, Any] | None, key: str) -> str:
    if r is None:
        return "–"
    if r.get("oom"):
        return "OOM"
    if "error" in r:
        return "n/a"
    return f"{r[key]:,.0f}" if key == "peak_extra_mib" else f"{r[key]:.1f}"


def table(res: dict[str, Any], mode: str, causal: bool, key: str) -> str:
    rows = [r for r in res["rows"] if r["mode"] == mode and r["causal"] == causal]
    present = [i for i in IMPLS if any(r["impl"] == i for r in rows)]
    lines = ["| seq (batch) | " + " | ".join(LABEL[i] for i in present) + " |",
             "|---" * (len(present) + 1) + "|"]
    for n in sorted({r["seq"] for r in rows}):
        b = next(r["batch"] for r in rows if r["seq"] == n)
        cells = [_cell(_find(rows, seq=n, impl=i), key) for i in present]
        lines.append(f"| {n:,} ({b}) | " + " | ".join(cells) + " |")
    return "\n".join(lines)


def unavailable(res: dict[str, Any]) -> str:
    notes: dict[str, str] = {}
    for r in res["rows"]:
        if "error" in r:
            notes.setdefault(r["impl"], r["error"])
        elif r.get("oom"):
            notes.setdefault(r["impl"], "out of memory at some lengths")
    return "\n".join(f"- {LABEL[k]} did not run everywhere: `{v}`" for k, v in notes.items())


def accuracy(res: dict[str, Any]) -> str:
    fwd = [e for e in res["accuracy"] if "grad" not in e and "max_abs_err" in e]
    lines = ["Reference: float32 materialised attention at every length (all heads).", "",
             "| impl | worst max abs error (fwd, all lengths) | worst mean abs error |", "|---|---|---|"]
    for i in IMPLS:
        es = [e for e in fwd if e["impl"] == i]
        if es:
            lines.append(f"| {LABEL[i]} | {max(e['max_abs_err'] for e in es):.2e} | "
                         f"{max(e['mean_abs_err'] for e in es):.2e} |")
    grads = [e for e in res["accuracy"] if "grad" in e]
    if grads:
        g = ", ".join(f"{e['grad']} {e['max_abs_err']:.1e} (seq {e['seq']}, {'causal' if e['causal'] else 'full'})"
                      for e in grads)
        lines += ["", f"tattn gradients vs float32 autograd (batch 1), max abs error: {g}."]
    return "\n".join(lines)


def speedups(res: dict[str, Any]) -> str:
    lines = ["| vs | fwd (min–max over lengths, causal and not) | fwd+bwd |", "|---|---|---|"]
    for other in ("sdpa_flash", "sdpa_efficient", "sdpa_math", "naive"):
        cells = []
        for mode in ("fwd", "fwd+bwd"):
            ratios = []
            for r in res["rows"]:
                if r["impl"] == "tattn" and r["mode"] == mode and "tflops" in r:
                    o = _find(res["rows"], impl=other, mode=mode, seq=r["seq"], causal=r["causal"])
                    if o and "tflops" in o:
                        ratios.append(r["tflops"] / o["tflops"])
            cells.append(f"{min(ratios):.2f}–{max(ratios):.2f}×" if ratios else "–")
        lines.append(f"| {LABEL[other]} | " + " | ".join(cells) + " |")
    return "\n".join(lines)


def render(res: dict[str, Any]) -> str:
    e, c = res["env"], res["config"]
    best = max((r["tflops"] for r in res["rows"] if r["impl"] == "tattn" and r["mode"] == "fwd" and "tflops" in r),
               default=float("nan"))
    out = [
        f"# tattn benchmark on {e['gpu']} ({e['arch']})",
        "",
        f"{e['gpu']} ({e['memory_gib']} GiB), torch {e['torch']}, HIP {e['hip']}, Python {e['python']}. fp16, head "
        f"dim {c['dim']}, {c['heads']} heads, batch × seq = {c['tokens']:,} tokens. Timer: {c['timer']}. "
        f"FLOPs: {c['flops']}. Data: {c['data']}.",
        "",
        f"Best tattn forward: {best:.1f} TFLOP/s ({100 * best / PEAK_F16_TFLOPS:.1f}% of the {PEAK_F16_TFLOPS} "
        f"TFLOP/s dense fp16 MFMA peak). A plain fp16 4096³ matmul reached "
        f"{res['fp16_matmul_4096_tflops']:.1f} TFLOP/s in the same run.",
        "",
        "## tattn speed-up",
        "",
        speedups(res),
        "",
    ]
    for mode, title in (("fwd", "Forward"), ("fwd+bwd", "Forward + backward")):
        for causal in (False, True):
            out += [f"## {title}, {'causal' if causal else 'non-causal'}: TFLOP/s", "",
                    table(res, mode, causal, "tflops"), ""]
    out += ["## Peak extra memory, forward + backward, non-causal (MiB)", "",
            table(res, "fwd+bwd", False, "peak_extra_mib"), ""]
    na = unavailable(res)
    if na:
        out += [na, ""]
    out += ["## Accuracy", "", accuracy(res), ""]
    if res.get("table_picks"):
        out += ["## Table picks (fwd / bwd_dkdv / bwd_dq entry ids)", "",
                ", ".join(f"{k}: {v['fwd']}/{v['bwd_dkdv']}/{v['bwd_dq']}" for k, v in res["table_picks"].items()),
                ""]
    return "\n".join(out)


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("result")
    ap.add_argument("--out", default=None)
    ap.add_argument("--check", action="store_true")
    a = ap.parse_args()
    res = json.loads(Path(a.result).read_text())
    if a.check:
        assert res["rows"], "empty results"
        print("ok", len(res["rows"]), "rows")
        return
    text = render(res)
    out = Path(a.out) if a.out else Path(a.result).with_suffix(".md")
    out.write_text(text + "\n")
    print("wrote", out)


if __name__ == "__main__":
    main()
