"""Slope timing of the fused-block benchmarks (bench-timing.js:22-97).

N iterations are run behind one fence (``Device.sync``), then 2N; the fixed
fence and launch-pipeline cost appears in both and cancels:

    per_iteration = (t(2N) - t(N)) / N

N is calibrated per run to make a batch about TARGET_BATCH_MS long; the two
paths of a pair share one N (sized to the slower) and are measured
interleaved, one batch pair of A then one of B, so drift in machine state
lands on both.  Wall clock on purpose: host dispatch overhead is part of what
fusion removes.
"""
from __future__ import annotations

import time
from typing import Callable, Dict, List

TARGET_BATCH_MS = 30.0
MIN_N = 2
MAX_N = 200
REPEATS = 7
WARM_MS = 400.0


def _now_ms() -> float:
    return time.perf_counter() * 1e3


def measure_pair(device, run_a: Callable[[], None], run_b: Callable[[], None],
                 repeats: int = REPEATS, warm_ms: float = WARM_MS) -> Dict[str, List[float]]:
    """Per-iteration ms of two paths, ``repeats`` samples each (interleaved)."""

    def time_batch(run, count):
        t0 = _now_ms()
        for _ in range(count):
            run()
        device.sync()
        return _now_ms() - t0

    warm_until = _now_ms() + warm_ms
    while _now_ms() < warm_until:
        run_a()
        run_b()
        device.sync()

    def calibrate(run):
        c1 = time_batch(run, 2)
        c2 = time_batch(run, 4)
        per = max((c2 - c1) / 2.0, 1e-5)
        return max(MIN_N, min(MAX_N, int(round(TARGET_BATCH_MS / per))))

    n = min(calibrate(run_a), calibrate(run_b))

    def slope(run):
        t_n = time_batch(run, n)
        t_2n = time_batch(run, 2 * n)
        return (t_2n - t_n) / n

    a, b = [], []
    for _ in range(repeats):
        a.append(slope(run_a))
        b.append(slope(run_b))
    return {"a": a, "b": b}


def measure_one(device, run: Callable[[], None], repeats: int = REPEATS,
                warm_ms: float = WARM_MS) -> List[float]:
    """Absolute per-iteration ms of one path (measurePair with A = B)."""
    return measure_pair(device, run, run, repeats, warm_ms)["a"]


def median(xs: List[float]) -> float:
    s = sorted(xs)
    return s[len(s) // 2]
