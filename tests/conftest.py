"""Test configuration: the `gpu` marker and import paths for the package and the oracle."""

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "triton-attn_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm gfx950 GPU (MI355X) and the built HIP library")
