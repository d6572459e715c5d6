"""Wall-clock timing of host-CPU callables (the CPU baseline).

Same statistics as reference mlx/scripts/timing.py:31-72 (`time_mlx`): untimed
warmup, then `iters` timed calls, times sorted, median = times[n // 2].  The
reference timed MLX on the Apple GPU; here the timed callable is the
registry's Model spec on the host CPU (MLX is not available on this platform).
"""
from __future__ import annotations

import os
import time
from typing import Any, Callable


def cpu_threads() -> int:
    try:
        import torch
        return torch.get_num_threads()
    except Exception:
        return os.cpu_count() or 1


def use_all_cores() -> int:
    """Give torch's CPU kernels every host core (its default is the physical
    core count, which may be fewer); returns the thread count."""
    try:
        import torch
        n = os.cpu_count() or 1
        if torch.get_num_threads() != n:
            torch.set_num_threads(n)
        return torch.get_num_threads()
    except Exception:
        return os.cpu_count() or 1


def warm(fn: Callable[..., Any], *args, n: int = 1) -> None:
    for _ in range(n):
        fn(*args)


def time_cpu(fn: Callable[..., Any], *args, warmup: int = 1, iters: int = 5) -> dict:
    """Time `fn(*args)` with time.perf_counter (reference timing.py:54-58), on
    every host core."""
    use_all_cores()
    if iters <= 0:
        iters = 1
    for _ in range(warmup):
        fn(*args)
    times: list[float] = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn(*args)
        times.append((time.perf_counter() - t0) * 1000.0)
    times.sort()
    return {
        "min_ms": times[0],
        "median_ms": times[len(times) // 2],
        "mean_ms": sum(times) / len(times),
        "iters": iters,
        "threads": cpu_threads(),
    }
