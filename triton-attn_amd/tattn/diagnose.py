"""ISA and hardware-counter evidence for the tattn kernels on gfx950.

The counterpart of the reference's bench/diagnose.py:1-80, which counts `mma.sync`, `ldmatrix`
and fp32 `fma` in the PTX Triton emits. Here the evidence is our own gfx950 assembly (code built
in this repository, read as text) and rocprofv3 counter output:

    python -m tattn.diagnose [--sources fwd.hip,fwd_persist_causal.hip,bwd.hip,bwd_dq_persist.hip,bwd_split.hip] [--kernel SUBSTR] [--out FILE]
    python -m tattn.diagnose --counters DIR [DIR ...]

ISA mode compiles the library's kernel sources to assembly with the build's flags and reports,
per kernel: registers (VGPR, AGPR, SGPR), scratch bytes per lane, static LDS bytes, occupancy,
code size, and instruction counts (MFMA by opcode, LDS reads / transposed reads / writes, LDS
DMA loads, other global loads, v_exp / FMA / dot2 / pack VALU, barriers, full `vmcnt(0)` waits,
scratch accesses), for the whole kernel and for its main loop (the loop with the most MFMAs).
Counter mode prints, per kernel, the mean of every counter collected in rocprofv3 `--pmc` output
directories (the `counters_collection` table of their `.db` files) and the mean
dispatch time when the run also traced kernels.
"""

from __future__ import annotations

import argparse
import collections
import glob
import json
import re
import sqlite3
import subprocess
import sys
from pathlib import Path
from typing import Any

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / "csrc"

# Instruction classes counted in the assembly (opcode regexes, matched at the start of a line).
CLASSES: dict[str, str] = {
    "mfma": r"v_mfma_\w+",
    "ds_read": r"ds_read_b(?:32|64|96|128)\b",
    "ds_read_tr": r"ds_read_b64_tr_b16\b",
    "ds_write": r"ds_write_\w+",
    "lds_dma": r"(?:buffer_load_\w+|global_load_lds_\w+)\b.*\blds\b|global_load_lds_\w+",
    "global_load": r"(?:buffer_load_\w+|global_load_\w+)(?!.*\blds\b)",
    "global_store": r"(?:buffer_store_\w+|global_store_\w+)",
    "v_exp": r"v_exp_f32\w*",
    "v_fma": r"v_(?:fma|fmac|fmaak|fmamk)_f32\w*",
    "v_dot2": r"v_dot2\w*",
    "v_cvt_pk": r"v_cvt_pk_\w+",
    "valu": r"v_(?!mfma)\w+",
    "s_barrier": r"s_barrier\b",
    "wait_vmcnt0": r"s_waitcnt\b.*\bvmcnt\(0\)",
    "scratch": r"scratch_\w+",
}
_CLASS_RE = {k: re.compile(r"^\s*(?:" + v + ")") for k, v in CLASSES.items()}
_INFO_KEYS = {
    "TotalNumSgprs": "sgprs", "NumVgprs": "vgprs", "NumAgprs": "agprs", "TotalNumVgprs": "total_vgprs",
    "ScratchSize": "scratch_bytes_per_lane", "LDSByteSize": "lds_bytes", "Occupancy": "occupancy",
    "codeLenInByte": "code_bytes",
}


def build_flags() -> list[str]:
    from . import _build

    return [*_build.COMMON_FLAGS, f"-I{_build.INCLUDE}", f"-I{_build.CSRC}"]


def compile_asm(source: Path, extra: list[str] | None = None) -> str:
    """gfx950 assembly of one kernel source, compiled with the library's flags."""
    from . import _build

    flags = build_flags() + list(extra or []) + _build.SOURCE_FLAGS.get(source.name, [])
    cmd = [_build.hipcc(), *flags, "--cuda-device-only", "-S", str(source), "-o", "-"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{r.stderr[-3000:]}")
    return r.stdout


def _counts(lines: list[str]) -> dict[str, Any]:
    out: dict[str, Any] = {k: 0 for k in CLASSES}
    mfma_ops: collections.Counter[str] = collections.Counter()
    for line in lines:
        if not line.startswith(("\t", " ")) or line.lstrip().startswith(";"):
            continue
        for k, rx in _CLASS_RE.items():
            if rx.match(line):
                out[k] += 1
        if _CLASS_RE["mfma"].match(line):
            mfma_ops[line.split()[0]] += 1
    out["mfma_by_opcode"] = dict(mfma_ops)
    return out


_TEMPLATE_ARG = re.compile(r"DF16_|DF16b|f|Li(-?\d+)E|Lb([01])E")
_TYPE_NAMES = {"DF16_": "_Float16", "DF16b": "__bf16", "f": "float"}


def _short_demangle(name: str) -> str:
    """`ns::kernel<args>` for this library's kernels (a namespace, a kernel template over element
    types, ints and bools), which older c++filt builds leave mangled (no `DF16_` support)."""
    m = re.match(r"_ZN(\d+)(\w+)", name)
    if not m:
        return name
    ns_len = int(m.group(1))
    ns, rest = m.group(2)[:ns_len], m.group(2)[ns_len:]
    mm = re.match(r"(\d+)", rest)
    if not mm:
        return name
    fn_len = int(mm.group(1))
    fn, rest = rest[len(mm.group(1)):][:fn_len], rest[len(mm.group(1)) + fn_len:]
    if not rest.startswith("I"):
        return f"{ns}::{fn}"
    args, pos = [], 1
    while pos < len(rest) and rest[pos] != "E":
        t = _TEMPLATE_ARG.match(rest, pos)
        if not t:
            return name
        tok = t.group(0)
        args.append(_TYPE_NAMES.get(tok) or t.group(1) or ("true" if t.group(2) == "1" else "false"))
        pos = t.end()
    return f"{ns}::{fn}<{', '.join(args)}>"


def _demangle(names: list[str]) -> dict[str, str]:
    try:
        r = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True, check=True)
        out = dict(zip(names, r.stdout.splitlines()))
    except (OSError, subprocess.CalledProcessError):
        out = {}
    return {n: out[n] if out.get(n, n) != n else _short_demangle(n) for n in names}


def isa_stats(asm: str, name_filter: str = "") -> dict[str, dict[str, Any]]:
    """Per-kernel statistics parsed from assembly text."""
    lines = asm.splitlines()
    label = re.compile(r"^(_Z\w+):")
    kernels: dict[str, dict[str, Any]] = {}
    i = 0
    while i < len(lines):
        m = label.match(lines[i])
        if not m or name_filter not in m.group(1):
            i += 1
            continue
        name, body = m.group(1), []
        j = i + 1
        while j < len(lines) and "-- End function" not in lines[j]:
            body.append(lines[j])
            j += 1
        info: dict[str, Any] = {}
        k = j
        while k < len(lines) and k < j + 80 and not label.match(lines[k]):
            mm = re.match(r"^; (\w+)(?: \[[^\]]*\])?(?::| =) (\d+)", lines[k])
            if mm and mm.group(1) in _INFO_KEYS:
                info[_INFO_KEYS[mm.group(1)]] = int(mm.group(2))
            k += 1
        # Main loop: the loop with the most MFMAs. Loop membership comes from the compiler's block
        # notes: a header block says "Loop Header", every other block of a loop says
        # "in Loop: Header=BBx_y" (its innermost loop); a loop's lines are its header block and
        # the blocks whose innermost loop it is.
        blocks: list[tuple[str | None, list[str]]] = []  # (innermost loop header, lines)
        for line in body:
            m_lab = re.match(r"^\.L(BB\d+_\d+):", line)
            if m_lab or re.match(r"^; %bb\.\d+:", line):
                m_in = re.search(r"in Loop: Header=(BB\d+_\d+)", line)
                own = m_lab.group(1) if m_lab and "Loop Header" in line else None
                blocks.append((own or (m_in.group(1) if m_in else None), [line]))
            elif blocks:
                if "Loop Header" in line and blocks[-1][1][0].startswith(".L"):  # note on the next line
                    lab = re.match(r"^\.L(BB\d+_\d+):", blocks[-1][1][0])
                    blocks[-1] = (lab.group(1) if lab else blocks[-1][0], blocks[-1][1])
                blocks[-1][1].append(line)
        loops: dict[str, list[str]] = collections.defaultdict(list)
        for head, lines_ in blocks:
            if head:
                loops[head].extend(lines_)
        main_loop = None
        for lines_ in loops.values():
            c = _counts(lines_)
            if main_loop is None or c["mfma"] > main_loop["mfma"]:
                main_loop = c
        kernels[name] = {**info, "all": _counts(body), "main_loop": main_loop}
        i = j + 1
    names = _demangle(list(kernels))
    for mangled, st in kernels.items():
        st["name"] = names.get(mangled, mangled)
    return kernels


def counter_means(dirs: list[str]) -> dict[str, dict[str, float]]:
    """Mean of each collected counter (and of the dispatch time, when traced) per kernel."""
    acc: dict[str, dict[str, list[float]]] = collections.defaultdict(lambda: collections.defaultdict(list))
    for d in dirs:
        for db in glob.glob(str(Path(d) / "**" / "*.db"), recursive=True):
            con = sqlite3.connect(db)
            tables = {r[0] for r in con.execute("select name from sqlite_master")}
            if "counters_collection" in tables:
                per: dict[tuple[int, str], dict[str, float]] = collections.defaultdict(dict)
                for did, kname, cname, val in con.execute(
                        "select dispatch_id, kernel_name, counter_name, value from counters_collection"):
                    cur = per[(did, kname)]
                    cur[cname] = cur.get(cname, 0.0) + val  # sum over dimension instances
                for (_, kname), cs in per.items():
                    for cname, val in cs.items():
                        acc[kname.split("(")[0]][cname].append(val)
            if "kernels" in tables:
                for kname, dur in con.execute("select name, duration from kernels"):
                    acc[kname.split("(")[0]]["duration_us"].append(dur / 1e3)
            con.close()
    return {k: {c: sum(v) / len(v) for c, v in cs.items()} for k, cs in acc.items()}


def derived(cs: dict[str, float]) -> dict[str, float]:
    """Ratios from counter means (each present only when its counters were collected):
    mfma_busy: MFMA-busy SIMD cycles per SIMD cycle of the CUs' busy time (4 SIMDs per CU);
    lds_bank_conflict_per_lds_cycle: bank-conflict cycles per cycle with an LDS instruction active;
    valu_per_mfma: VALU instructions per MFMA instruction;
    lds_load_bytes: LDS read bytes (SQ_INSTS_LDS_LOAD_BANDWIDTH counts 64-byte units);
    lds_bytes_per_cu_cycle: those bytes per busy CU cycle (a CU's LDS returns at most 128 B per
    cycle: one ds_read_b128 of a wave64 takes 8 cycles)."""
    out: dict[str, float] = {}
    if cs.get("SQ_BUSY_CU_CYCLES") and "SQ_VALU_MFMA_BUSY_CYCLES" in cs:
        out["mfma_busy"] = cs["SQ_VALU_MFMA_BUSY_CYCLES"] / (4 * cs["SQ_BUSY_CU_CYCLES"])
    if cs.get("SQ_ACTIVE_INST_LDS") and "SQ_LDS_BANK_CONFLICT" in cs:
        out["lds_bank_conflict_per_lds_cycle"] = cs["SQ_LDS_BANK_CONFLICT"] / cs["SQ_ACTIVE_INST_LDS"]
    if cs.get("SQ_INSTS_MFMA") and "SQ_INSTS_VALU" in cs:
        out["valu_per_mfma"] = cs["SQ_INSTS_VALU"] / cs["SQ_INSTS_MFMA"]
    if "SQ_INSTS_LDS_LOAD_BANDWIDTH" in cs:
        out["lds_load_bytes"] = cs["SQ_INSTS_LDS_LOAD_BANDWIDTH"] * 64
        if cs.get("SQ_BUSY_CU_CYCLES"):
            out["lds_bytes_per_cu_cycle"] = out["lds_load_bytes"] / cs["SQ_BUSY_CU_CYCLES"]
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--sources", default="fwd.hip,fwd_persist_causal.hip,bwd.hip,bwd_dq_persist.hip,bwd_split.hip", help="kernel sources under csrc/")
    ap.add_argument("--kernel", default="pipe_kernel", help="substring of the mangled kernel names")
    ap.add_argument("--counters", nargs="*", help="rocprofv3 --pmc output directories (counter mode)")
    ap.add_argument("--out", default=None, help="write the JSON result here")
    a = ap.parse_args()
    if a.counters:
        means = counter_means(a.counters)
        names = _demangle(list(means))
        res: dict[str, Any] = {"counters": {names[k]: {**cs, "derived": derived(cs)} for k, cs in means.items()}}
    else:
        res = {"arch": "gfx950", "kernels": {}}
        for src in a.sources.split(","):
            res["kernels"].update(isa_stats(compile_asm(CSRC / src), a.kernel))
    text = json.dumps(res, indent=2)
    if a.out:
        Path(a.out).parent.mkdir(parents=True, exist_ok=True)
        Path(a.out).write_text(text + "\n")
    print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
