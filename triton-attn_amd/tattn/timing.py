"""GPU timing with the reference benchmark's method.

The reference times every cell with `triton.testing.do_bench(fn, warmup=25, rep=100,
return_mode="median")` (bench/bench.py:52): a 256 MB buffer is overwritten before each timed
call, so L2 and the last-level cache start cold, each call is bracketed by its own pair of
events, and the median is reported. `do_bench` below is that method in plain PyTorch (no
Triton): warm-up and repetition counts come from a 5-call estimate, events are recorded on the
current stream (the stream the library launches on).
"""

from __future__ import annotations

import statistics
from typing import Callable

FLUSH_BYTES = 256 * 2**20


def do_bench(fn: Callable[[], object], warmup_ms: float = 25.0, rep_ms: float = 100.0,
             flush_bytes: int = FLUSH_BYTES) -> float:
    """Median milliseconds of one `fn()` call with the cache flushed before each call."""
    import torch

    flush = torch.empty(flush_bytes // 4, dtype=torch.int32, device="cuda")
    fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(5):
        flush.zero_()
        fn()
    t1.record()
    t1.synchronize()
    est = max(t0.elapsed_time(t1) / 5, 1e-3)
    n_warm = max(1, int(warmup_ms / est))
    n_rep = max(1, int(rep_ms / est))
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n_rep)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n_rep)]
    for _ in range(n_warm):
        fn()
    for i in range(n_rep):
        flush.zero_()
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    del flush
    return statistics.median(s.elapsed_time(e) for s, e in zip(starts, ends))
