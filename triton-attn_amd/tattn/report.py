"""Markdown rendering of a tattn.benchsuite result (schema "tattn-suite/1").

Serves the purpose of the reference's report script (bench/report.py of
amaanmithani/triton-attn): the suite's numbers as tables for a README. Layout here: one table
per pass (forward, forward+backward) with a row per (mask, N) and a column per implementation,
the ratio of tattn to the fastest stock implementation of that row, fwd+bwd peak memory per N,
forward error and tattn's gradient error per N, the cells that did not run, and the tile-table
picks.

    python -m tattn.report results/gfx950.json [--out results/gfx950.md]
    python -m tattn.report results/gfx950.json --check   # schema check only, exit 1 on a problem
"""

from __future__ import annotations

import argparse
import json
import math
import sys
from pathlib import Path
from typing import Any

PEAK_F16_TFLOPS = 2516.6
ORDER = ("tattn", "sdpa_flash", "sdpa_efficient", "sdpa_math", "materialised")
LABELS = {"tattn": "tattn", "sdpa_flash": "SDPA flash", "sdpa_efficient": "SDPA mem-eff", "sdpa_math": "SDPA math",
          "materialised": "materialised"}
CELL_KEYS = ("impl", "n", "b", "mask", "pass", "status")


def problems(res: dict[str, Any]) -> list[str]:
    """Everything wrong with a result file's structure (empty list: it renders)."""
    out = []
    if res.get("schema") != "tattn-suite/1":
        out.append(f"schema is {res.get('schema')!r}, expected 'tattn-suite/1'")
    for key in ("device", "method", "cells", "errors"):
        if key not in res:
            out.append(f"missing {key!r}")
    cells = res.get("cells") or []
    if not cells:
        out.append("no cells")
    for i, c in enumerate(cells):
        missing = [k for k in CELL_KEYS if k not in c]
        if missing:
            out.append(f"cell {i} lacks {missing}")
        elif c["status"] == "ok" and not (c.get("ms", 0) > 0 and c.get("tflops", 0) > 0):
            out.append(f"cell {i} ({c['impl']}, N={c['n']}) is ok without a positive time and rate")
    for i, e in enumerate(res.get("errors") or []):
        if not all(isinstance(e.get(k), (int, float)) and math.isfinite(e[k]) for k in ("max_abs", "mean_abs")):
            out.append(f"error row {i} has non-finite values")
    return out


def _impls(cells: list[dict[str, Any]]) -> list[str]:
    seen = {c["impl"] for c in cells}
    return [i for i in ORDER if i in seen] + sorted(seen - set(ORDER))


def _index(cells: list[dict[str, Any]]) -> dict[tuple, dict[str, Any]]:
    return {(c["impl"], c["n"], c["mask"], c["pass"]): c for c in cells}


def _rate(c: dict[str, Any] | None) -> str:
    if c is None:
        return ""
    if c["status"] != "ok":
        return {"oom": "OOM"}.get(c["status"], "—")
    return f"{c['tflops']:.0f}"


def pass_table(res: dict[str, Any], passes: str) -> str:
    cells = res["cells"]
    idx = _index(cells)
    impls = _impls(cells)
    head = "| mask | N (B) | " + " | ".join(LABELS.get(i, i) for i in impls) + " | tattn ÷ fastest other | tattn % of peak |"
    rows = [head, "|" + "---|" * (len(impls) + 4)]
    for mask in ("none", "causal"):
        for n in sorted({c["n"] for c in cells}):
            row = [idx.get((i, n, mask, passes)) for i in impls]
            if not any(row):
                continue
            b = next(c["b"] for c in row if c)
            mine = idx.get(("tattn", n, mask, passes))
            others = [c["tflops"] for c in row if c and c["impl"] != "tattn" and c["status"] == "ok"]
            ratio = (f"{mine['tflops'] / max(others):.2f}×" if mine and mine["status"] == "ok" and others else "")
            pct = f"{100 * mine['tflops'] / PEAK_F16_TFLOPS:.1f}%" if mine and mine["status"] == "ok" else ""
            rows.append(f"| {mask} | {n:,} ({b}) | " + " | ".join(_rate(c) for c in row) + f" | {ratio} | {pct} |")
    return "\n".join(rows)


def memory_table(res: dict[str, Any]) -> str:
    cells = [c for c in res["cells"] if c["pass"] == "fwd+bwd" and c["mask"] == "none"]
    impls = _impls(cells)
    idx = _index(cells)
    rows = ["| N | " + " | ".join(LABELS.get(i, i) for i in impls) + " |", "|" + "---|" * (len(impls) + 1)]
    for n in sorted({c["n"] for c in cells}):
        vals = []
        for i in impls:
            c = idx.get((i, n, "none", "fwd+bwd"))
            vals.append(f"{c['peak_mib']:.0f}" if c and c["status"] == "ok" else _rate(c))
        rows.append(f"| {n:,} | " + " | ".join(vals) + " |")
    return "\n".join(rows)


def error_tables(res: dict[str, Any]) -> str:
    errs = res["errors"]
    fwd = [e for e in errs if e["tensor"] == "o"]
    impls = [i for i in _impls(fwd)]
    lines = ["Forward output against float32 materialised attention, max abs error (all heads):", "",
             "| mask | N | " + " | ".join(LABELS.get(i, i) for i in impls) + " |",
             "|" + "---|" * (len(impls) + 2)]
    for mask in ("none", "causal"):
        for n in sorted({e["n"] for e in fwd}):
            got = {e["impl"]: e for e in fwd if e["n"] == n and e["mask"] == mask}
            if got:
                lines.append(f"| {mask} | {n:,} | " + " | ".join(
                    f"{got[i]['max_abs']:.2e}" if i in got else "" for i in impls) + " |")
    grads = [e for e in errs if e["tensor"] != "o"]
    if grads:
        lines += ["", "tattn gradients against float32 autograd (batch 0), max abs error:", "",
                  "| mask | N | dq | dk | dv |", "|---|---|---|---|---|"]
        for mask in ("none", "causal"):
            for n in sorted({e["n"] for e in grads}):
                got = {e["tensor"]: e["max_abs"] for e in grads if e["n"] == n and e["mask"] == mask}
                if got:
                    lines.append(f"| {mask} | {n:,} | " + " | ".join(f"{got.get(t, float('nan')):.2e}"
                                                                     for t in ("dq", "dk", "dv")) + " |")
    return "\n".join(lines)


def not_run(res: dict[str, Any]) -> str:
    seen: dict[tuple[str, str], list[str]] = {}
    for c in res["cells"]:
        if c["status"] != "ok":
            seen.setdefault((c["impl"], c["status"]), []).append(f"{c['n']}/{c['mask']}/{c['pass']}"
                                                                  + (f" ({c['note']})" if c.get("note") else ""))
    return "\n".join(f"- {LABELS.get(i, i)}, {s}: " + "; ".join(v[:4]) + (" …" if len(v) > 4 else "")
                     for (i, s), v in seen.items())


def render(res: dict[str, Any]) -> str:
    d, m = res["device"], res["method"]
    parts = [
        f"# tattn on {d['name']} ({d['arch']})",
        "",
        f"torch {d['torch']}, HIP {d['hip']}, Python {d['python']}, {d['memory_gib']} GiB. {m['dtype']}, "
        f"H = {m['heads']}, D = {m['dim']}, B·N = {m['tokens']:,} tokens per cell. Timer: {m['timer']}. "
        f"Counted work: {m['flops']}. Inputs: {m['data']}. Peak: {PEAK_F16_TFLOPS} TFLOP/s dense fp16 MFMA"
        + (f"; a 4096³ fp16 matmul ran at {res['gemm_tflops']:.0f} TFLOP/s on the same timer." if res.get("gemm_tflops")
           else "."),
    ]
    for passes, title in (("fwd", "Forward"), ("fwd+bwd", "Forward + backward")):
        parts += ["", f"## {title}, TFLOP/s", "", pass_table(res, passes)]
    parts += ["", "## Peak memory above the inputs, forward + backward, no mask (MiB)", "", memory_table(res),
              "", "## Accuracy", "", error_tables(res)]
    missing = not_run(res)
    if missing:
        parts += ["", "## Cells that did not run", "", missing]
    if res.get("picks"):
        parts += ["", "## Tile-table entries used (forward / dK-dV / dQ)", "",
                  ", ".join(f"{k}: {v['fwd']}/{v['bwd_dkdv']}/{v['bwd_dq']}" for k, v in res["picks"].items())]
    return "\n".join(parts) + "\n"


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description="render a tattn.benchsuite result as markdown")
    ap.add_argument("result")
    ap.add_argument("--out", default=None)
    ap.add_argument("--check", action="store_true", help="only check the file's structure")
    a = ap.parse_args(argv)
    res = json.loads(Path(a.result).read_text())
    bad = problems(res)
    if a.check or bad:
        for p in bad:
            print("problem:", p, file=sys.stderr)
        if not bad:
            print(f"ok: {len(res['cells'])} cells, {len(res['errors'])} error rows")
        return 1 if bad else 0
    out = Path(a.out) if a.out else Path(a.result).with_suffix(".md")
    out.write_text(render(res))
    print("wrote", out)
    return 0


if __name__ == "__main__":
    sys.exit(main())
