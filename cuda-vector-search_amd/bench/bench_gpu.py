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


def bench_grid(sizes, dims, batches, ks, methods, seed=0, target_s=0.3, log=print):
    sync = torch.cuda.synchronize
    rows, gemm = [], []
    total_mem = torch.cuda.get_device_properties(0).total_memory
    for d in dims:
        for n in sizes:
            need = 3 * n * d + 4 * max(batches) * n + (1 << 30)  # fp16 corpus + int8 companion + scores
            if need > total_mem:
                rows.append({"n": n, "d": d, "skipped": "memory"})
                continue
            torch.cuda.empty_cache()
            x = synthetic.unit_corpus(n, d, seed=seed + d, device="cuda")
            index = Index(x, metric="ip", copy=False)
            qall = synthetic.unit_queries(max(batches), d, seed=seed + 1, device="cuda")
            _, ref_i = exact_topk_fp32(qall[:N_REF], x, max(ks))
            ref_i = ref_i.cpu()
            for b in batches:
                q = qall[:b].contiguous()
                for k in ks:
                    for m in methods:
                        row = {"n": n, "d": d, "batch": b, "k": k, "method": m}
                        try:
                            sync()
                            torch.cuda.reset_peak_memory_stats()
                            base = torch.cuda.memory_allocated()
                            _, ids = index.search(q, k, method=m)
                            sync()
                            row["extra_mem_mb"] = round((torch.cuda.max_memory_allocated() - base) / 2**20, 1)
                            nr = min(N_REF, b)
                            row["recall_vs_fp32"] = recall(ids[:nr].cpu().tolist(), ref_i[:nr, :k].tolist())
                            ms, reps = time_call(lambda: index.search(q, k, method=m), sync, target_s=target_s)
                            row.update(ms=round(ms, 4), qps=round(b / (ms / 1000), 1), reps=reps)
                        except torch.cuda.OutOfMemoryError:
                            row["error"] = "OOM"
                            torch.cuda.empty_cache()
                        log(json.dumps(row))
                        rows.append(row)
            b = max(batches)
            qp = index._prep_queries(qall[:b].contiguous())
            eng = _ext.load()
            ms_c, _ = time_call(lambda: eng.scores(qp, index._x, False), sync, target_s=target_s)
            ms_b, _ = time_call(lambda: qp @ index._x.T, sync, target_s=target_s)
            flops = 2.0 * b * n * d
            g = {"n": n, "d": d, "batch": b, "custom_ms": round(ms_c, 3), "cublas_ms": round(ms_b, 3),
                 "custom_tflops": round(flops / ms_c / 1e9, 2), "cublas_tflops": round(flops / ms_b / 1e9, 2),
                 "blas": "hipBLASLt (torch.matmul)"}
            log(json.dumps(g))
            gemm.append(g)
            del x, index, qall, qp
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
