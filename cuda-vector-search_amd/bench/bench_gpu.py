"""Method grid on one MI355X: fused / twopass / torch over corpus sizes, widths,
batches and k, plus the raw score-matrix kernel against hipBLASLt.

    python cuda-vector-search_amd/bench/bench_gpu.py --out results/mi355x.json

Writes ``{"env": ..., "rows": [...], "gemm": [...]}`` with the row schema of the
reference's bench/bench_gpu.py (keys n, d, batch, k, method, extra_mem_mb,
recall_vs_fp32, ms, qps, reps; gemm rows n, d, batch, custom_ms, cublas_ms,
custom_tflops, cublas_tflops, where "cublas" is the vendor BLAS behind
torch.matmul, hipBLASLt here), so its report tooling reads these files too.
Data: seeded unit vectors per 2^18-row chunk (cuda_vector_search.synthetic), an
``ip`` index, recall checked on the first 8 queries against the exact fp32
reference.
"""

from __future__ import annotations

import argparse
import datetime as dt
import functools
import itertools
import json
import os
import platform
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path[:0] = [str(HERE.parent), str(HERE)]

import torch  # noqa: E402

from cuda_vector_search import Index, _ext, exact_topk_fp32, synthetic  # noqa: E402
from timing import recall, time_call  # noqa: E402

N_REF = 8


def int_list(s: str):
    return [int(float(v)) for v in s.split(",") if v.strip()]


def env_info() -> dict:
    p = torch.cuda.get_device_properties(0)
    rocm = Path("/opt/rocm/.info/version")
    return {
        "date": dt.datetime.now(dt.timezone.utc).strftime("%Y-%m-%d %H:%M UTC"),
        "gpu": p.name,
        "arch": getattr(p, "gcnArchName", ""),
        "gpu_mem_gb": round(p.total_memory / 2**30, 1),
        "sm_count": p.multi_processor_count,  # compute units
        "torch": torch.__version__,
        "torch_hip": torch.version.hip,
        "rocm": rocm.read_text().strip() if rocm.exists() else "n/a",
        "python": platform.python_version(),
        "cpu_count": os.cpu_count(),
    }


def _mb(nbytes: int) -> float:
    return round(nbytes / 2**20, 1)


def measure_cell(index, q, k, method, ref_ids, target_s):
    """One grid cell: peak extra device memory of a first call, recall of its ids
    on the reference's queries, then the median synced wall time.  Returns the
    row fields (or {"error": "OOM"})."""
    sync = torch.cuda.synchronize
    run = functools.partial(index.search, q, k, method=method)
    sync()
    before = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    try:
        ids = run()[1]
        sync()
        extra = torch.cuda.max_memory_allocated() - before
        checked = min(len(ref_ids), q.shape[0])
        found = recall(ids[:checked].cpu().tolist(), [r[:k] for r in ref_ids[:checked]])
        ms, reps = time_call(run, sync, target_s=target_s)
    except torch.cuda.OutOfMemoryError:
        torch.cuda.empty_cache()
        return {"error": "OOM"}
    return {"extra_mem_mb": _mb(extra), "recall_vs_fp32": found, "ms": round(ms, 4),
            "qps": round(q.shape[0] * 1000.0 / ms, 1), "reps": reps}


def score_kernel_vs_blas(index, q, target_s):
    """The gfx950 score kernel (fp16 score matrix) against the vendor BLAS behind
    torch.matmul on the same prepared operands."""
    eng = _ext.load()
    qp = index._prep_queries(q)
    sync = torch.cuda.synchronize
    ours, _ = time_call(lambda: eng.scores(qp, index._x, False), sync, target_s=target_s)
    blas, _ = time_call(lambda: torch.matmul(qp, index._x.T), sync, target_s=target_s)
    n, d, b = len(index), index.dim, q.shape[0]
    tera = 2.0 * b * n * d / 1e12
    return {"n": n, "d": d, "batch": b, "custom_ms": round(ours, 3), "cublas_ms": round(blas, 3),
            "custom_tflops": round(tera / (ours / 1e3), 2), "cublas_tflops": round(tera / (blas / 1e3), 2),
            "blas": "hipBLASLt (torch.matmul)"}


def bench_grid(sizes, dims, batches, ks, methods, seed=0, target_s=0.3, log=print):
    """Every (n, d) corpus that fits, then every (batch, k, method) cell on it;
    one score-kernel comparison per corpus at the largest batch."""
    rows, gemm = [], []
    dev_bytes = torch.cuda.get_device_properties(0).total_memory
    for d, n in itertools.product(dims, sizes):
        # fp16 corpus + int8 companion + the largest score matrix + slack
        if 3 * n * d + 4 * max(batches) * n + (1 << 30) > dev_bytes:
            rows.append({"n": n, "d": d, "skipped": "memory"})
            continue
        torch.cuda.empty_cache()
        index = Index(synthetic.unit_corpus(n, d, seed=seed + d, device="cuda"), metric="ip", copy=False)
        queries = synthetic.unit_queries(max(batches), d, seed=seed + 1, device="cuda")
        ref_ids = exact_topk_fp32(queries[:N_REF], index.embeddings, max(ks))[1].cpu().tolist()
        for b, k, method in itertools.product(batches, ks, methods):
            row = {"n": n, "d": d, "batch": b, "k": k, "method": method}
            row.update(measure_cell(index, queries[:b].contiguous(), k, method, ref_ids, target_s))
            log(json.dumps(row))
            rows.append(row)
        gemm.append(score_kernel_vs_blas(index, queries, target_s))
        log(json.dumps(gemm[-1]))
        del index, queries
        torch.cuda.empty_cache()
    return rows, gemm


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--sizes", default="100000,1000000,4000000")
    ap.add_argument("--dims", default="384,768")
    ap.add_argument("--batches", default="1,32,256")
    ap.add_argument("--ks", default="10,100")
    ap.add_argument("--methods", default="auto,fused,int8,twopass,torch")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--target-s", type=float, default=0.3)
    ap.add_argument("--out", default="results/gpu.json")
    args = ap.parse_args()
    _ext.load()
    env = env_info()
    print(json.dumps(env), flush=True)
    rows, gemm = bench_grid(int_list(args.sizes), int_list(args.dims), int_list(args.batches),
                            int_list(args.ks), [m for m in args.methods.split(",") if m],
                            seed=args.seed, target_s=args.target_s, log=lambda s: print(s, flush=True))
    out = Path(args.out)
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps({"env": env, "rows": rows, "gemm": gemm}, indent=1))
    print("wrote", out, flush=True)


if __name__ == "__main__":
    main()
