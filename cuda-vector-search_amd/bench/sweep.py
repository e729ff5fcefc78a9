"""Plan sweep of the fused path on gfx950: query block (bq) x corpus chunks.

    python cuda-vector-search_amd/bench/sweep.py --out results/sweep.json

The reference sweeps its CUDA tile knobs (bench/sweep.py); here the knobs are
the gfx950 plan: bq in {16, 32, 64, 128, 256} where the width allows it and
the chunk count at 1/4 .. 4x of the automatic plan.  Prints the best plan per
(batch, k) next to the automatic one.
"""

from __future__ import annotations

import argparse
import itertools
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path[:0] = [str(HERE.parent), str(HERE)]

import torch  # noqa: E402

from cuda_vector_search import _ext, synthetic  # noqa: E402
from timing import time_call  # noqa: E402


def candidate_plans(auto_chunks: int, batch: int):
    """Forced (bq, chunks) plans around the automatic one: every query block the
    batch can fill at least half of (16 always), chunk counts from a quarter to
    four times the automatic count in powers of two."""
    blocks = [bq for bq in (16, 32, 64, 128, 256) if bq == 16 or 2 * batch >= bq]
    scales = [2.0 ** e for e in range(-2, 3)]
    return [(bq, max(1, int(auto_chunks * f))) for bq in blocks for f in scales]


def sweep(n, d, batches=(1, 32, 256), ks=(10, 100, 256), target_s=0.15, log=print):
    eng = _ext.load()
    x = synthetic.unit_corpus(n, d, seed=d, device="cuda")
    qall = synthetic.unit_queries(max(batches), d, seed=1, device="cuda")
    sync = torch.cuda.synchronize
    rows = []

    def timed(q, k, bq, chunks):
        plan = [int(v) for v in eng.fused_topk(q, x, k, bq, chunks)[2].tolist()]
        ms, _ = time_call(lambda: eng.fused_topk(q, x, k, bq, chunks), sync, target_s=target_s)
        return plan, round(ms, 4)

    for b, k in itertools.product(batches, ks):
        q = qall[:b].contiguous()
        auto, auto_ms = timed(q, k, 0, 0)
        cells = [(0, 0, auto, auto_ms)]
        for bq, chunks in candidate_plans(auto[1], b):
            try:
                cells.append((bq, chunks, *timed(q, k, bq, chunks)))
            except RuntimeError as e:  # no kernel for this block at this width / k
                log(f"skip b={b} k={k} bq={bq} chunks={chunks}: {e}")
        for bq, chunks, plan, ms in cells:
            rows.append({"n": n, "d": d, "batch": b, "k": k, "bq": bq, "chunks": chunks, "plan": plan,
                         "auto": auto, "ms": ms})
            log(json.dumps(rows[-1]))
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
