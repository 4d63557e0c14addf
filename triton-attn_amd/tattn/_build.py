"""Builds libtattn_hip.so in-tree with hipcc for gfx950.

The library is a plain C-ABI shared object (include/tattn.h); Python loads it with ctypes.
Packed fp32 VALU instructions are disabled for every HIP translation unit.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / "csrc"
REPO = PKG.parent.parent
INCLUDE = REPO / "include"
LIB = PKG / "libtattn_hip.so"
SOURCES = ["abi.hip", "fwd.hip", "fwd_persist_causal.hip", "bwd.hip", "bwd_dq_persist.hip", "bwd_dkdv_persist.hip",
           "bwd_split.hip"]
# Per-source flags. fwd.hip: keep each step's softmax work in the step that issues the
# independent MFMAs it interleaves with (machine sinking would move it to its first use).
# fwd_persist_causal.hip (persistent causal forward, two tiles per wave), bwd_dq_persist.hip
# (persistent dQ) and bwd_split.hip (paired-wave dK/dV and dQ) hold one kernel family each so
# that they can take the LLVM instruction scheduler that measured fastest for them; the other
# kernels are slower under either.
SOURCE_FLAGS = {
    "fwd.hip": ["-mllvm", "-disable-machine-sink"],
    "fwd_persist_causal.hip": ["-mllvm", "-disable-machine-sink", "-mllvm", "-amdgpu-sched-strategy=iterative-ilp"],
    "bwd_dq_persist.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
    "bwd_split.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"],
}
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _compile(src: Path, obj: Path, extra: list[str]) -> None:
    cmd = [hipcc(), *COMMON_FLAGS, *extra, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def build(verbose: bool = False, extra: list[str] | None = None) -> Path:
    """Compiles every source (in parallel) and links LIB. Always rebuilds."""
    extra = extra or []
    out = REPO / "_build"
    out.mkdir(exist_ok=True)
    objs = [out / (Path(s).stem + ".o") for s in SOURCES]
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        futs = [ex.submit(_compile, CSRC / s, o, extra + SOURCE_FLAGS.get(s, [])) for s, o in zip(SOURCES, objs)]
        for f in futs:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
