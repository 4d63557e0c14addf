"""bench.py's output contract: one JSON line with the metric, whole-job value, roofline of the
forward kernel and the CPU baseline; a single GPU only."""

import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_recorded_traffic_is_read_from_the_profile():
    sys.path.insert(0, str(ROOT))
    import bench

    t = bench.measured_traffic()
    algorithmic = 4 * 33554432 + 1048576  # Q, K, V read, O written (16k tokens x 16 heads x 64 fp16), M
    # Q, K, V read once and O, M written once at N <= 8192; at N = 16384 a third of K/V is read
    # twice (profiles/fwd_persist_traffic_fp16_d64_headline.md): 1.03x on average.
    assert t is not None and algorithmic <= t < 1.05 * algorithmic


def test_cpu_baseline_threads_follow_the_host_budget(monkeypatch):
    sys.path.insert(0, str(ROOT))
    import bench

    import os

    cores = len(os.sched_getaffinity(0))
    monkeypatch.delenv("OMP_NUM_THREADS", raising=False)
    assert bench.cpu_threads()[:2] == (cores, cores)
    if cores > 1:
        monkeypatch.setenv("OMP_NUM_THREADS", "1")
        got = bench.cpu_threads()
        assert got[:2] == (cores, 1) and "OMP_NUM_THREADS=1" in got[2]


@pytest.mark.gpu
def test_default_contract_on_one_gpu():
    """A short run of the headline step (no sweep) prints one JSON line with every required key."""
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--no-sweep", "--steps", "2", "--warmup", "1"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [line for line in r.stdout.splitlines() if line.strip()]
    assert len(lines) == 1
    out = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in out, key
    assert out["n_gpus"] == 1 and out["steps"] == 2 and out["warmup"] == 1 and out["unit"] == "TFLOP/s"
    assert out["higher_is_better"] is True and out["vs_baseline"] is None and "workload" in out["config"]
    roof = out["roofline"]
    assert roof["bound"] == "mfma" and roof["unit"] == "TFLOP/s" and roof["peak"] == 2516.6
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-9 and 0 < roof["frac"] < 1
    assert roof["traffic"] is not None and roof["launches"] == 2 * 6
    assert [r["seq"] for r in roof["per_n"]] == [512, 1024, 2048, 4096, 8192, 16384]
    assert all(0 < r["frac"] < 1 and r["avg_launch_us"] > 0 for r in roof["per_n"])
    cpu = out["cpu_baseline"]
    assert cpu["kind"] == "port" and cpu["cores"] >= 1 and cpu["value"] > 0 and cpu["sample"]
    assert cpu["threads"] == cpu["cores"] <= cpu["affinity_cores"] and cpu["thread_choice"]
    assert 0 < out["value"] < 2516.6


@pytest.mark.gpu
def test_backward_roofline_and_copy_yardstick():
    """bench.py's backward-kernel roofline (tattn_bwd whole and its dK/dV alone, the fused dQ as
    their difference) and its HBM copy yardstick: every length present, fractions of peak in
    (0, 1), the parts adding up to the whole, and a copy rate below the 8 TB/s HBM peak."""
    import torch

    sys.path.insert(0, str(ROOT))
    import bench

    data = {n: bench._inputs(n, torch.device("cuda:0")) for n in bench.SEQS}
    roof = bench.backward_roofline(data, causal_modes=(False,))
    assert [r["seq"] for r in roof["per_n"]] == list(bench.SEQS)
    for r in roof["per_n"]:
        print(r, flush=True)
        for name in ("dkdv", "dq"):
            assert 0 < r[name]["frac"] < 1 and r[name]["us"] > 0
        assert 0 < r["tattn_bwd"]["frac"] < 1
        assert abs(r["tattn_bwd"]["us"] - r["dkdv"]["us"] - r["dq"]["us"]) < 0.05
    copy = bench.hbm_copy_tbps(64)
    print(copy, flush=True)
    assert 0.5 < copy["tbps"] < 8.0
