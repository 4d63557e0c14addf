"""Writes t4_accuracy.json: the accuracy the reference published for its own kernels
(results/t4.json of amaanmithani/triton-attn, entries with impl "tattn": forward max/mean abs error
against float32 at every benchmark length, causal and not, and dq/dk/dv max abs error against
float32 autograd at N=1024 and 4096). Data only; run from the repository root:

    python tests/golden/make_t4_accuracy.py /root/reference/results/t4.json
"""

import json
import sys
from pathlib import Path


def main() -> None:
    src = json.loads(Path(sys.argv[1]).read_text())
    keep = [{k: e[k] for k in ("seq", "causal", "grad", "reference", "max_abs_err", "mean_abs_err") if k in e}
            for e in src["accuracy"] if e.get("impl") == "tattn"]
    out = {"source": "results/t4.json (NVIDIA T4, Triton kernels), accuracy entries of impl tattn",
           "env": src["env"], "entries": keep}
    Path(__file__).with_name("t4_accuracy.json").write_text(json.dumps(out, indent=1) + "\n")
    print(len(keep), "entries")


if __name__ == "__main__":
    main()
