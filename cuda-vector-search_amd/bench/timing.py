"""Timing and recall helpers for the benchmark tools (bench/timing.py of the
reference defines the same two measurements: median wall time of a synced call,
and recall@k as the averaged fraction of reference ids found)."""

from __future__ import annotations

import statistics
import time


def time_call(fn, sync=None, target_s: float = 0.3, max_reps: int = 100, warmup: int = 2,
              slow_s: float = 1.0):
    """(median ms, repetitions) of ``fn(); sync()`` after ``warmup`` untimed calls
    (one when a call takes longer than ``slow_s``), repeated until ``target_s``
    seconds or ``max_reps`` calls, and at least 3 calls unless a call is slow."""

    def run_once():
        t0 = time.perf_counter()
        fn()
        if sync is not None:
            sync()
        return time.perf_counter() - t0

    first = run_once()
    for _ in range(warmup - 1 if first < slow_s else 0):
        run_once()
    samples = []
    while len(samples) < max_reps:
        samples.append(run_once())
        if samples[-1] > slow_s:
            break
        if sum(samples) >= target_s and len(samples) >= 3:
            break
    return 1000.0 * statistics.median(samples), len(samples)


def recall(got_ids, ref_ids) -> float:
    """Mean over queries of |got & ref| / |ref| (lists of id lists)."""
    found = sum(len(set(g) & set(r)) for g, r in zip(got_ids, ref_ids))
    total = sum(len(r) for r in ref_ids)
    return found / total if total else 0.0
