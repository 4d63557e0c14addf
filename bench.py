#!/usr/bin/env python3
"""Benchmark of the tattn attention path on one MI355X.

Metric: fwd & fwd+bwd TFLOP/s (fp16, d64, H16, 16k tokens) + % of MI355X dense fp16 MFMA peak.
Counted work follows the reference's benchmark (bench/bench.py:31-35 of amaanmithani/triton-attn):
4*B*H*N^2*D flops per forward, halved when causal, fwd+bwd counted as 3.5x fwd.

A timed step is one forward pass (non-causal, fp16) over each of the six 16,384-token shapes
[B=16384/N, H=16, N, D=64] for N in 512..16384; inputs stay resident in HBM. `value` is the
step's counted flops divided by its time. The same line carries the roofline of the forward
kernel (HIP events around every forward launch of the timed steps, on the launch stream), the
per-N sweep (forward, causal and non-causal; fwd+bwd, causal and non-causal, with peak extra
memory) timed like the reference's tables (tattn.timing.do_bench: cache flushed before each
call, median over ~100 ms), the roofline of the two backward kernels per N and mask
(`roofline.bwd`: HIP events around warm launches of tattn_bwd whole and of its dK/dV alone), a
measured HBM yardstick (`roofline.hbm_copy_tbps`: a 256 MiB device copy, the memory analog of
the reference's GEMM yardstick, bench/bench.py:173-175), the accuracy of each shape as the
reference's benchmark measures it (bench/bench.py:128-171: forward max / mean abs error against
float32 attention at every N and both masks, dq/dk/dv max abs error against float32 autograd at
N = 1024 and 4096, batch 0) plus causal gradients over the whole N = 512 tensors beside the
error of the reference's own algorithm on them, and a CPU baseline: the oracle's tiled forward
timed on the host cores on a bounded sample.

Usage: python bench.py [--gpus 1] [--steps 10] [--warmup 3] [--no-cpu-baseline] [--no-accuracy]
       (profiling: --no-sweep --seqs N --causal --backward --head-dim D)
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "triton-attn_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "fwd & fwd+bwd TFLOP/s (fp16,d64,H16,16k tok) + % of MI355X fp16 MFMA peak"
PEAK_F16_TFLOPS = 2516.6  # MI355X dense fp16 MFMA (256 CUs x 2.4 GHz x 4096 flop/clk/CU)
TOKENS, HEADS, DIM = 16384, 16, 64
SEQS = (512, 1024, 2048, 4096, 8192, 16384)


def flops(b: int, h: int, n: int, d: int, causal: bool, mode: str) -> float:
    f = 4.0 * b * h * n * n * d
    if causal:
        f *= 0.5
    return f * (3.5 if mode == "fwd+bwd" else 1.0)


def _inputs(n: int, dev):
    import torch

    b = TOKENS // n
    g = torch.Generator(device=dev).manual_seed(n)
    q, k, v, do = (torch.randn(b, HEADS, n, DIM, device=dev, dtype=torch.float16, generator=g)
                   for _ in range(4))
    return b, q, k, v, do


TRAFFIC_FILE = ROOT / "profiles" / "fwd_persist_traffic_fp16_d64_headline.md"


def measured_traffic() -> int | None:
    """HBM bytes per forward launch of the default headline workload, as measured with rocprofv3
    FETCH_SIZE / WRITE_SIZE counters (calibrated on a plain copy) and recorded in TRAFFIC_FILE.
    Counters cannot be read from inside the timed run, so the recorded figure is reported."""
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_threads() -> tuple[int, int, str]:
    """(cores this process may run on, threads to use, why they differ). The thread count is the
    host's per-process thread budget when one is set (OMP_NUM_THREADS: a GPU box gives each GPU a
    share of its cores), else every core of the affinity mask."""
    cores = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and 0 < int(env) < cores:
        return cores, int(env), f"OMP_NUM_THREADS={env}: the host's thread budget for this process"
    return cores, cores, "every core of the affinity mask"


def cpu_baseline() -> dict:
    """The oracle's tiled forward (restatement of the reference's CPU path) on the host CPU."""
    import torch

    from oracle.reference import tiled_forward

    affinity, threads, why = cpu_threads()
    torch.set_num_threads(threads)
    b, h, n, d = 1, 4, 8192, DIM
    g = torch.Generator().manual_seed(8192)
    q, k, v = (torch.randn(b, h, n, d, generator=g).half() for _ in range(3))
    run = lambda: tiled_forward(q, k, v, False, None, block_m=128, block_n=128)  # noqa: E731
    run()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    sec = statistics.median(times)
    return {
        "value": flops(b, h, n, d, False, "fwd") / sec / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "threads": threads,
        "affinity_cores": affinity,
        "thread_choice": why,
        "kind": "port",
        "sample": f"oracle tiled_forward (fp32 math on fp16 inputs), [B={b},H={h},N={n},D={d}] non-causal, "
                  f"128x128 blocks, median of 3 after 1 warm-up, {sec:.3f} s per run",
    }


def _reference_out(q, k, v, causal):
    """float32 materialised attention, a few heads at a time (~1 GiB of scores per chunk)."""
    import torch

    from oracle.reference import naive_attention

    z, h, n, _ = q.shape
    per = max(1, (1 << 28) // (z * n * n))
    return torch.cat([naive_attention(q[:, i:i + per].float(), k[:, i:i + per].float(), v[:, i:i + per].float(),
                                      causal=causal) for i in range(0, h, per)], dim=1)


def accuracy(data) -> list[dict]:
    """The reference benchmark's accuracy recipe (bench/bench.py:128-171) on the benchmark's own
    inputs: forward max / mean abs error against float32 attention for every N and mask (all
    heads up to N = 4096, the first two heads of batch 0 beyond); dq, dk, dv max abs error
    against float32 autograd on batch 0 at N = 1024 and 4096 (dO from the same generator)."""
    import torch

    from oracle.reference import naive_attention
    from tattn import attention

    rows = []
    for causal in (False, True):
        for n in SEQS:
            _, q, k, v, do = data[n]
            if n > 4096:
                q, k, v = (t[:1, :2].contiguous() for t in (q, k, v))
            with torch.inference_mode():
                err = (attention(q, k, v, causal=causal).float() - _reference_out(q, k, v, causal)).abs()
            rows.append({"seq": n, "causal": causal, "what": "o", "max_abs_err": float(f"{err.max().item():.4g}"),
                         "mean_abs_err": float(f"{err.mean().item():.4g}")})
            del err
        for n in (1024, 4096):
            _, q, k, v, do = data[n]
            q, k, v, do = (t[:1].clone() for t in (q, k, v, do))
            qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
            attention(qg, kg, vg, causal=causal).backward(do)
            qr, kr, vr = (t.float().requires_grad_() for t in (q, k, v))
            naive_attention(qr, kr, vr, causal=causal).backward(do.float())
            for name, got, want in (("dq", qg.grad, qr.grad), ("dk", kg.grad, kr.grad), ("dv", vg.grad, vr.grad)):
                rows.append({"seq": n, "causal": causal, "what": name,
                             "max_abs_err": float(f"{(got.float() - want).abs().max().item():.4g}")})
    rows += full_tensor_causal_grads(data, 512)
    return rows


def full_tensor_causal_grads(data, n: int) -> list[dict]:
    """Causal dq, dk, dv over the whole [B, 16, N, 64] tensors (all batches and heads) against float32
    autograd, with beside each the error of the reference's own backward algorithm with its
    kernels' rounding points (oracle.reference.rounded_backward) on the same inputs (q, k, v, dO
    and the forward's O and M), and of the reference's whole pipeline (the same algorithm from the
    exact log-sum-exp). The bound is max(2e-3, the algorithm's error + 5e-4)."""
    import torch

    from oracle.reference import naive_attention, rounded_backward
    from tattn import attention
    from tattn.api import _forward

    _, q, k, v, do = data[n]
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
    attention(qg, kg, vg, causal=True).backward(do)
    got = (qg.grad, kg.grad, vg.grad)
    o, m = _forward(q, k, v, True, 1.0 / math.sqrt(DIM))
    emulated = rounded_backward(q, k, v, do, causal=True, o=o, lse=m)
    pipeline = rounded_backward(q, k, v, do, causal=True)
    err, emu, pipe = [0.0] * 3, [0.0] * 3, [0.0] * 3
    per = max(1, (1 << 28) // (q.shape[1] * n * n))  # batches per chunk: ~1 GiB of scores
    for b0 in range(0, q.shape[0], per):
        sl = slice(b0, b0 + per)
        qr, kr, vr = (t[sl].float().requires_grad_() for t in (q, k, v))
        naive_attention(qr, kr, vr, causal=True).backward(do[sl].float())
        for i, want in enumerate((qr.grad, kr.grad, vr.grad)):
            err[i] = max(err[i], (got[i][sl].float() - want).abs().max().item())
            emu[i] = max(emu[i], (emulated[i][sl].float() - want).abs().max().item())
            pipe[i] = max(pipe[i], (pipeline[i][sl].float() - want).abs().max().item())
        del qr, kr, vr
    return [{"seq": n, "causal": True, "what": name, "scope": "all batches and heads",
             "max_abs_err": float(f"{e:.4g}"), "reference_algorithm_max_abs_err": float(f"{r:.4g}"),
             "reference_pipeline_max_abs_err": float(f"{pp:.4g}"),
             "bound": float(f"{max(2e-3, r + 5e-4):.4g}")}
            for name, e, r, pp in zip(("dq", "dk", "dv"), err, emu, pipe)]


def backward_roofline(data, causal_modes=(False, True), reps: int = 10) -> dict:
    """The two backward kernels of the default path, timed like the forward roofline: HIP events
    around every launch on the launch stream, back to back with the inputs resident (3 untimed
    launches first), average duration. Per N and mask: tattn_bwd as one call (dQ computing delta
    itself, then dK/dV: the backward every fwd+bwd cell runs) and tattn_bwd_dkdv alone with the
    same pick; the fused dQ is their difference. Executed matrix-core work per launch: dK/dV 4
    GEMMs per 32 x 32 block (S, dP, dV, dK) = 2 x the forward's flops, dQ 3 (S, dP, dQ) = 1.5 x;
    the reference's convention counts the backward as 2.5 x the forward (bench/bench.py:31-35)."""
    import torch

    from tattn import _lib
    from tattn.api import _forward

    lib = _lib.load()
    scale = 1.0 / math.sqrt(DIM)

    def avg_ms(fn) -> float:
        for _ in range(3):
            fn()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for e0, e1 in ev:
            e0.record()
            fn()
            e1.record()
        torch.cuda.synchronize()
        return sum(e0.elapsed_time(e1) for e0, e1 in ev) / reps

    rows = []
    for causal in causal_modes:
        for n in SEQS:
            b, q, k, v, do = data[n]
            o, m = _forward(q, k, v, causal, scale)
            st = _lib.strides4(q)
            stream = torch.cuda.current_stream().cuda_stream
            delta = torch.empty((b, HEADS, n), device=q.device, dtype=torch.float32)
            dq, dk, dv = (torch.empty_like(q) for _ in range(3))
            shape = (b, HEADS, n, DIM, _lib.F16, int(causal), scale, -1, stream)

            def whole() -> None:
                _lib.check(lib.tattn_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
                                         dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), m.data_ptr(), delta.data_ptr(),
                                         st, *shape), "tattn_bwd")

            def dkdv() -> None:
                _lib.check(lib.tattn_bwd_dkdv(q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(), dk.data_ptr(),
                                              dv.data_ptr(), m.data_ptr(), delta.data_ptr(), st, *shape),
                           "tattn_bwd_dkdv")

            f = flops(b, HEADS, n, DIM, causal, "fwd")
            t_all = avg_ms(whole)  # also leaves delta computed for dkdv()
            t_kv = avg_ms(dkdv)
            t_q = max(t_all - t_kv, 1e-6)
            row = {"seq": n, "batch": b, "causal": causal}
            for name, ms, work, kern in (("dkdv", t_kv, 2.0 * f, _lib.K_BWD_DKDV), ("dq", t_q, 1.5 * f, _lib.K_BWD_DQ)):
                tf = work / (ms * 1e-3) / 1e12
                row[name] = {"entry": _lib.pick_config(kern, DIM, _lib.F16, causal, n), "us": round(1e3 * ms, 2),
                             "exec_tflops": round(tf, 1), "frac": round(tf / PEAK_F16_TFLOPS, 4)}
            counted = 2.5 * f / (t_all * 1e-3) / 1e12
            row["tattn_bwd"] = {"us": round(1e3 * t_all, 2), "counted_tflops": round(counted, 1),
                                "frac": round(counted / PEAK_F16_TFLOPS, 4)}
            rows.append(row)
            print(json.dumps({"bwd_roofline": row}), file=sys.stderr, flush=True)
            del o, m, delta, dq, dk, dv
    return {"bound": "mfma", "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
            "timer": f"HIP events around each launch on the launch stream, {reps} back-to-back launches after 3 untimed, "
                     "inputs resident; dq = tattn_bwd - tattn_bwd_dkdv (dQ computes delta itself)",
            "work": "dkdv: 2x forward flops, dq: 1.5x (executed GEMMs); tattn_bwd: 2.5x (the reference's count)",
            "per_n": rows}


def hbm_copy_tbps(mib: int = 256, reps: int = 20) -> dict:
    """Measured HBM bandwidth yardstick: device-to-device copies of `mib` MiB (torch's copy, the
    runtime's copy kernel), HIP events around each of `reps` back-to-back copies after 3 untimed
    ones, average; bytes moved = read + write."""
    import torch

    src = torch.empty(mib * 2**18, device="cuda", dtype=torch.float32)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for e0, e1 in ev:
        e0.record()
        dst.copy_(src)
        e1.record()
    torch.cuda.synchronize()
    ms = sum(e0.elapsed_time(e1) for e0, e1 in ev) / reps
    del src, dst
    return {"mib": mib, "us": round(1e3 * ms, 2), "tbps": round(2 * mib * 2**20 / (ms * 1e-3) / 1e12, 3),
            "peak_tbps": 8.0, "timer": f"HIP events around each of {reps} back-to-back copies, average"}


def main() -> int:
    global DIM
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[1])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-accuracy", action="store_true", help="skip the per-shape error measurement")
    ap.add_argument("--no-sweep", action="store_true", help="only the headline forward step")
    ap.add_argument("--seqs", default=",".join(map(str, SEQS)),
                    help="sequence lengths of the step (16,384 tokens each); default: all six")
    ap.add_argument("--causal", action="store_true", help="headline step with the causal mask")
    ap.add_argument("--backward", action="store_true",
                    help="headline step runs forward + backward (for profiling the backward kernels)")
    ap.add_argument("--head-dim", type=int, default=DIM, choices=(16, 32, 64, 128),
                    help="head dim of every shape (default 64, the benchmark's; others for profiling)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also run a plain device copy of this many MiB, 5 times (HBM-counter calibration)")
    a = ap.parse_args()
    DIM = a.head_dim
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (the attention path has no multi-GPU part); got --gpus {a.gpus}",
              file=sys.stderr)
        return 2

    import torch

    from tattn import attention, hip_available
    from tattn.api import _forward
    from tattn.timing import do_bench

    dev = torch.device("cuda:0")
    if not hip_available(dev):
        raise RuntimeError("tattn HIP library not usable on cuda:0")
    torch.cuda.set_device(dev)
    seqs = tuple(int(x) for x in a.seqs.split(","))
    data = {n: _inputs(n, dev) for n in (seqs if a.no_sweep else sorted(set(SEQS) | set(seqs)))}
    scale = 1.0 / math.sqrt(DIM)
    head_mode = "fwd+bwd" if a.backward else "fwd"

    if a.copy_mib:
        src = torch.empty(a.copy_mib * 2**18, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # ---- headline: forward (or fwd+bwd) over the step's shapes ---------------------------
    grads = {}
    if a.backward:
        for n in seqs:
            _, q, k, v, _ = data[n]
            grads[n] = tuple(t.detach().clone().requires_grad_() for t in (q, k, v))

    # Forward mode: every launch of the timed steps is bracketed by events on the launch stream;
    # their durations give the roofline's average launch time over the timed region.
    launch_events: list[tuple[int, object, object]] = []

    def step(record: bool = False) -> None:
        for n in seqs:
            _, q, k, v, do = data[n]
            if a.backward:
                qg, kg, vg = grads[n]
                qg.grad = kg.grad = vg.grad = None
                attention(qg, kg, vg, causal=a.causal).backward(do)
            elif record:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                _forward(q, k, v, a.causal, scale)
                e1.record()
                launch_events.append((n, e0, e1))
            else:
                _forward(q, k, v, a.causal, scale)

    step_flops = sum(flops(data[n][0], HEADS, n, DIM, a.causal, head_mode) for n in seqs)
    with torch.inference_mode(not a.backward):
        for _ in range(a.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            step(record=True)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / a.steps
    value = step_flops / (ms_per_step * 1e-3) / 1e12

    # ---- roofline of the forward kernel over the timed region ----------------------------
    if not launch_events:  # fwd+bwd headline: time the forward launches of the same shapes
        with torch.inference_mode():
            for _ in range(a.steps):
                for n in seqs:
                    _, q, k, v, _ = data[n]
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    _forward(q, k, v, a.causal, scale)
                    e1.record()
                    launch_events.append((n, e0, e1))
        torch.cuda.synchronize()
    durations = [e0.elapsed_time(e1) for _, e0, e1 in launch_events]
    fwd_flops = sum(flops(data[n][0], HEADS, n, DIM, a.causal, "fwd") for n, _, _ in launch_events)
    kernel_ms = sum(durations) / len(durations)  # average launch duration
    achieved = fwd_flops / len(durations) / (kernel_ms * 1e-3) / 1e12
    traffic = None
    if seqs == SEQS and not a.causal and DIM == 64:
        traffic = measured_traffic()
    # Per shape: the table entry the forward runs, its average launch time and roofline fraction.
    from tattn import _lib

    def entry_name(n: int) -> str:
        cfg = _lib.config_desc(_lib.K_FWD, DIM, _lib.F16, _lib.pick_config(_lib.K_FWD, DIM, _lib.F16, a.causal, n))
        kind = {2: f"fwd_persist_kernel, ring {cfg['ring']}", 1: "fwd_pipe_kernel"}.get(cfg["kind"], "fwd_generic_kernel")
        return f"{kind}, {cfg['waves']} waves x {cfg['tiles']} tiles ({cfg['block_m']} query rows per workgroup)"

    per_n = []
    for n in seqs:
        ds = [e0.elapsed_time(e1) for m, e0, e1 in launch_events if m == n]
        f = flops(data[n][0], HEADS, n, DIM, a.causal, "fwd")
        tf = f / (sum(ds) / len(ds) * 1e-3) / 1e12
        per_n.append({"seq": n, "batch": data[n][0], "entry": entry_name(n),
                      "avg_launch_us": round(1e3 * sum(ds) / len(ds), 2),
                      "tflops": round(tf, 1), "frac": round(tf / PEAK_F16_TFLOPS, 4)})
    names = sorted({entry_name(n) for n in seqs})
    roofline = {"bound": "mfma", "achieved": achieved, "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                "frac": achieved / PEAK_F16_TFLOPS, "traffic": traffic,
                "kernel": f"tattn::{' / '.join(names)} (fp16, D={DIM}, {'causal' if a.causal else 'non-causal'})",
                "avg_launch_ms": kernel_ms, "launches": len(durations),
                "flops_per_launch": fwd_flops / len(durations), "per_n": per_n}

    if not a.no_sweep and seqs == SEQS and DIM == 64:
        roofline["bwd"] = backward_roofline(data)
        roofline["hbm_copy"] = hbm_copy_tbps(256)
        roofline["hbm_copy_tbps"] = roofline["hbm_copy"]["tbps"]

    # ---- sweep: per N, forward and fwd+bwd, causal and non-causal -------------------------
    sweep = []
    agg = {}
    if not a.no_sweep:
        for causal in (False, True):
            for mode in ("fwd", "fwd+bwd"):
                tot_f = tot_ms = 0.0
                for n in SEQS:
                    b, q, k, v, do = data[n]
                    if mode == "fwd":
                        with torch.inference_mode():
                            ms = do_bench(lambda: attention(q, k, v, causal=causal))
                        peak_mib = None
                    else:
                        qg, kg, vg = (t.detach().clone().requires_grad_() for t in (q, k, v))

                        def fb() -> None:
                            qg.grad = kg.grad = vg.grad = None
                            attention(qg, kg, vg, causal=causal).backward(do)

                        fb()
                        qg.grad = kg.grad = vg.grad = None
                        torch.cuda.synchronize()
                        torch.cuda.reset_peak_memory_stats()
                        base = torch.cuda.memory_allocated()
                        fb()
                        torch.cuda.synchronize()
                        peak_mib = (torch.cuda.max_memory_allocated() - base) / 2**20
                        ms = do_bench(fb)
                        del qg, kg, vg
                    f = flops(b, HEADS, n, DIM, causal, mode)
                    tf = f / (ms * 1e-3) / 1e12
                    tot_f += f
                    tot_ms += ms
                    row = {"seq": n, "batch": b, "causal": causal, "mode": mode, "ms": round(ms, 4),
                           "tflops": round(tf, 1), "pct_of_peak": round(100 * tf / PEAK_F16_TFLOPS, 2)}
                    if peak_mib is not None:
                        row["peak_extra_mib"] = round(peak_mib, 1)
                    sweep.append(row)
                    print(json.dumps(row), file=sys.stderr, flush=True)
                key = f"{mode}_{'causal' if causal else 'non_causal'}"
                tflops = tot_f / (tot_ms * 1e-3) / 1e12
                agg[key] = {"tflops": round(tflops, 1), "pct_of_peak": round(100 * tflops / PEAK_F16_TFLOPS, 2)}

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic N(0,1), device generator seeded with N",
        "config": {
            "workload": f"attention {head_mode}, fp16, {'causal' if a.causal else 'non-causal'}, H=16, D={DIM}, "
                        f"one pass over each of N={','.join(map(str, seqs))} with B=16384/N",
            "tokens_per_shape": TOKENS, "heads": HEADS, "head_dim": DIM, "seqs": list(seqs),
        },
        "pct_of_peak": round(100 * value / PEAK_F16_TFLOPS, 2),
        "aggregates": agg,
        "roofline": roofline,
        "sweep": sweep,
    }
    if not a.no_accuracy and not a.no_sweep:
        out["accuracy"] = accuracy(data)
        recipe = [r for r in out["accuracy"] if "scope" not in r]
        full = [r for r in out["accuracy"] if "scope" in r]
        out["accuracy_worst"] = {
            "fwd_max_abs_err": max(r["max_abs_err"] for r in recipe if r["what"] == "o"),
            "fwd_mean_abs_err": max(r["mean_abs_err"] for r in recipe if r["what"] == "o"),
            "grad_max_abs_err": max(r["max_abs_err"] for r in recipe if r["what"] != "o"),
            "envelope": 2e-3,
            "full_tensor_causal_grad_max_abs_err": max(r["max_abs_err"] for r in full),
            "full_tensor_causal_reference_algorithm": max(r["reference_algorithm_max_abs_err"] for r in full),
            "full_tensor_causal_within_bound": all(r["max_abs_err"] <= r["bound"] for r in full),
        }
    if not a.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
