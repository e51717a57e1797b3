"""hipEvent timers and the HBM copy calibration for MI355X.

``gpu_ms`` restates the reference's validated timer (extra_bench.py:8-20,
timer_fix.py:4-14): events around a loop of calls on the current stream, the
loop length sized so the loop takes ~300 ms, clamped to [5, 200] calls.
``median_us`` is the reference's ``T`` (extra_bench.py:22): the median of 3
such loops, in microseconds.  torch.cuda.Event records on torch's current
stream, which is the stream every launch of this library goes to.

``copy_calibration`` replaces the reference's A100 sanity check
(timer_fix.py:17-24, 8192^2 fp32 copy against a hard-coded 1555 GB/s) with a
copy larger than MI355X's 256 MB Infinity Cache, checked against 8 TB/s.
"""
from __future__ import annotations

import statistics
from typing import Callable, Dict, List

import torch

HBM_PEAK_GBPS = 8000.0


def gpu_ms(fn: Callable[[], object], warmup: int = 10, target_ms: float = 300.0, min_iters: int = 5,
           max_iters: int = 200) -> float:
    """Mean milliseconds per call of `fn` over an event-timed loop."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    fn()
    e1.record()
    torch.cuda.synchronize()
    one = max(e0.elapsed_time(e1), 1e-3)
    iters = max(min_iters, min(max_iters, int(target_ms / one)))
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(iters):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def median_us(fn: Callable[[], object], rounds: int = 3, **kw) -> float:
    """Median over `rounds` event loops, microseconds per call."""
    return statistics.median(gpu_ms(fn, **kw) for _ in range(rounds)) * 1000.0


class CacheFlusher:
    """Evicts q/k/v/o by reading a buffer larger than the 256 MB Infinity Cache.

    Reading leaves the caches holding clean lines.  Writing the buffer instead
    leaves up to a cache's worth of dirty lines, whose write-back then runs
    inside the next measured kernel and competes with its reads: at B4 H16
    S4096 D64 that added 10-26 us to the banded kernels' cold times (local
    45.0 against 55.6 us, block-diagonal 39.0 against 56.5 us).  Reading a 1 GB
    buffer, or two 512 MB buffers in turn, gives the same times as this one.
    """

    def __init__(self, nbytes: int = 512 << 20, device: str = "cuda"):
        self.buf = torch.ones(nbytes // 4, dtype=torch.float32, device=device)
        self.acc = torch.zeros(1, dtype=torch.float32, device=device)

    def __call__(self) -> None:
        torch.sum(self.buf, dim=(0,), out=self.acc[0])


def cold_us(fn: Callable[[], object], reps: int = 20, flusher: CacheFlusher = None) -> float:
    """Median microseconds of single calls, each after a cache-evicting write."""
    flusher = flusher or CacheFlusher()
    fn()
    torch.cuda.synchronize()
    times: List[float] = []
    for _ in range(reps):
        flusher()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1000.0)
    return statistics.median(times)


def copy_calibration(nbytes: int = 2 << 30, device: str = "cuda") -> Dict[str, float]:
    """Device-to-device copy of `nbytes` (read + write = 2*nbytes moved)."""
    n = nbytes // 4
    x = torch.empty(n, dtype=torch.float32, device=device).fill_(1.0)
    y = torch.empty_like(x)
    ms = gpu_ms(lambda: y.copy_(x), warmup=3, target_ms=200.0, min_iters=5, max_iters=50)
    gbps = 2 * nbytes / (ms * 1e-3) / 1e9
    del x, y
    return {"bytes": 2 * nbytes, "us": ms * 1000.0, "GBps": gbps, "frac_of_peak": gbps / HBM_PEAK_GBPS}
