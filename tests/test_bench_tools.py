"""The benchmark tools under cuda-vector-search_amd/bench (CPU: report rendering,
timing, sweep summary; GPU: one tiny grid run with the reference's row schema)."""

from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import pytest

BENCH = Path(__file__).resolve().parents[1] / "cuda-vector-search_amd" / "bench"


def load(name):
    if str(BENCH) not in sys.path:
        sys.path.insert(0, str(BENCH))
    spec = importlib.util.spec_from_file_location(f"cvs_bench_{name}", BENCH / f"{name}.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


ROWS = [
    {"n": 100000, "d": 384, "batch": 1, "k": 10, "method": "fused", "ms": 0.05, "recall_vs_fp32": 1.0},
    {"n": 100000, "d": 384, "batch": 1, "k": 10, "method": "torch", "ms": 0.2, "recall_vs_fp32": 1.0},
    {"n": 100000, "d": 384, "batch": 1, "k": 10, "method": "twopass", "error": "OOM"},
    {"n": 1000000, "d": 384, "batch": 256, "k": 10, "method": "fused", "ms": 0.25, "recall_vs_fp32": 1.0},
    {"n": 1000000, "d": 384, "batch": 256, "k": 10, "method": "torch", "ms": 1.5, "recall_vs_fp32": 0.99},
    {"n": 4000000, "d": 768, "skipped": "memory"},
]
GEMM = [{"n": 1000000, "d": 384, "batch": 256, "custom_ms": 0.3, "cublas_ms": 0.45, "custom_tflops": 650.0,
         "cublas_tflops": 437.0}]


def test_report_tables():
    report = load("report")
    text = report.render({"gpu": "MI355X", "arch": "gfx950", "sm_count": 256}, ROWS, GEMM)
    assert "| 100k | 10 | 1 | **0.05** | OOM | 0.2 | 4.00x |" in text
    assert "| 1M | 10 | 256 | **0.25** |  | 1.5 | 6.00x |" in text
    assert "| 1M | 384 | 256 | 0.3 | 0.45 | 650.0 | 437.0 |" in text
    assert "| torch | 0.9900 | 0.9950 |" in text
    assert "skipped" not in text


def test_report_merges_files(tmp_path):
    import json

    report = load("report")
    a, b = tmp_path / "a.json", tmp_path / "b.json"
    a.write_text(json.dumps({"env": {"gpu": "x"}, "rows": ROWS[:2], "gemm": GEMM}))
    b.write_text(json.dumps({"env": {"gpu": "y", "cpu_count": 8}, "rows": ROWS[3:5]}))
    env, rows, gemm = report.merge([a, b])
    assert env == {"gpu": "x", "cpu_count": 8} and len(rows) == 4 and len(gemm) == 1


def test_timing_helpers():
    timing = load("timing")
    calls = []
    ms, reps = timing.time_call(lambda: calls.append(1), target_s=0.0)
    assert reps == 3 and len(calls) == 3 + 2 and ms >= 0
    assert timing.recall([[1, 2, 3], [4, 5, 6]], [[1, 2, 9], [4, 5, 6]]) == pytest.approx(5 / 6)


def test_sweep_summary():
    sweep = load("sweep")
    rows = [{"batch": 256, "k": 10, "bq": 0, "chunks": 0, "plan": [256, 253], "auto": [256, 253], "ms": 0.25},
            {"batch": 256, "k": 10, "bq": 128, "chunks": 126, "plan": [128, 126], "auto": [256, 253], "ms": 0.4},
            {"batch": 256, "k": 10, "bq": 256, "chunks": 126, "plan": [256, 128], "auto": [256, 253], "ms": 0.24}]
    (b, k, best, auto_ms), = sweep.best_vs_auto(rows)
    assert (b, k, best["ms"], auto_ms) == (256, 10, 0.24, 0.25)


@pytest.mark.gpu
def test_bench_grid_row_schema(eng):
    import torch

    bench = load("bench_gpu")
    rows, gemm = bench.bench_grid([20000], [128], [1, 8], [10], ["fused", "twopass", "torch"],
                                  target_s=0.01, log=lambda s: None)
    assert len(rows) == 6 and len(gemm) == 1
    for r in rows:
        assert set(r) >= {"n", "d", "batch", "k", "method", "extra_mem_mb", "recall_vs_fp32", "ms", "qps", "reps"}
    assert all(r["recall_vs_fp32"] == 1.0 for r in rows if r["method"] == "fused")
    assert set(gemm[0]) >= {"custom_ms", "cublas_ms", "custom_tflops", "cublas_tflops"}
    torch.cuda.synchronize()
