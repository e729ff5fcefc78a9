"""Plan sweep of the fused path on gfx950: query block (bq) x corpus chunks.

    python cuda-vector-search_amd/bench/sweep.py --out results/sweep.json

The reference sweeps its CUDA tile knobs (bench/sweep.py); here the knobs are
the gfx950 plan: bq in {16, 32, 64, 128, 256} where the width allows it and
the chunk count at 1/4 .. 4x of the automatic plan.  Prints the best plan per
(batch, k) next to the automatic one.
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path[:0] = [str(HERE.parent), str(HERE)]

import torch  # noqa: E402

from cuda_vector_search import _ext, synthetic  # noqa: E402
from timing import time_call  # noqa: E402


def sweep(n, d, batches=(1, 32, 256), ks=(10, 100, 256), target_s=0.15, log=print):
    eng = _ext.load()
    x = synthetic.unit_corpus(n, d, seed=d, device="cuda")
    qall = synthetic.unit_queries(max(batches), d, seed=1, device="cuda")
    rows = []
    for b in batches:
        q = qall[:b].contiguous()
        for k in ks:
            auto = [int(v) for v in eng.fused_topk(q, x, k)[2].tolist()]
            ms, _ = time_call(lambda: eng.fused_topk(q, x, k), torch.cuda.synchronize, target_s=target_s)
            r = {"n": n, "d": d, "batch": b, "k": k, "bq": 0, "chunks": 0, "plan": auto, "auto": auto,
                 "ms": round(ms, 4)}
            log(json.dumps(r))
            rows.append(r)
            for bq in (16, 32, 64, 128, 256):
                if bq > 16 and b < bq // 2:
                    continue
                for f in (0.25, 0.5, 1, 2, 4):
                    chunks = max(1, int(auto[1] * f))
                    try:
                        plan = [int(v) for v in eng.fused_topk(q, x, k, bq, chunks)[2].tolist()]
                        ms, _ = time_call(lambda: eng.fused_topk(q, x, k, bq, chunks), torch.cuda.synchronize,
                                          target_s=target_s)
                    except RuntimeError as e:  # plan not available at this width / k
                        log(f"skip b={b} k={k} bq={bq} chunks={chunks}: {e}")
                        continue
                    r = {"n": n, "d": d, "batch": b, "k": k, "bq": bq, "chunks": chunks, "plan": plan,
                         "auto": auto, "ms": round(ms, 4)}
                    log(json.dumps(r))
                    rows.append(r)
    return rows


def best_vs_auto(rows):
    """[(batch, k, best row, auto-plan ms or None)] for every (batch, k)."""
    out = []
    for key in sorted({(r["batch"], r["k"]) for r in rows}):
        cand = [r for r in rows if (r["batch"], r["k"]) == key]
        best = min(cand, key=lambda r: r["ms"])
        auto = [r["ms"] for r in cand if r["plan"] == r["auto"]]
        out.append((key[0], key[1], best, min(auto) if auto else None))
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--n", type=int, default=1000000)
    ap.add_argument("--d", type=int, default=384)
    ap.add_argument("--out", default="results/sweep.json")
    args = ap.parse_args()
    rows = sweep(args.n, args.d, log=lambda s: print(s, flush=True))
    Path(args.out).parent.mkdir(parents=True, exist_ok=True)
    Path(args.out).write_text(json.dumps(rows, indent=1))
    for b, k, best, auto_ms in best_vs_auto(rows):
        print(f"b={b:4d} k={k:4d} best bq={best['bq']} chunks={best['chunks']} {best['ms']:.3f} ms; "
              f"auto {best['auto']} {auto_ms if auto_ms is not None else 'n/a'} ms", flush=True)


if __name__ == "__main__":
    main()
