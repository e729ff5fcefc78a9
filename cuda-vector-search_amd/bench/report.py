"""Markdown tables (and, with matplotlib, latency charts) from benchmark JSON.

    python cuda-vector-search_amd/bench/report.py results/mi355x.json [more.json] --md results/mi355x.md

Reads files with the reference's row schema (bench_gpu.py here, or the
reference's own bench_gpu.py / bench_baselines.py outputs) and prints, per
width: median ms per batch for every method present (fastest in bold) with the
fused-vs-torch speed-up; the score-matrix kernel against the vendor BLAS; and
recall@k against the fp32 exact search.
"""

from __future__ import annotations

import argparse
import json
from pathlib import Path

METHOD_ORDER = ["auto", "fused", "int8", "twopass", "torch", "faiss_gpu_fp16", "faiss_gpu_fp32", "faiss_cpu", "numpy"]


def short_n(n: int) -> str:
    return f"{n / 1e6:g}M" if n >= 1_000_000 else f"{n // 1000}k"


def merge(paths):
    """(env, rows, gemm) of several result files: rows and score-kernel rows of
    all of them (grid rows only: skipped corpora carry no method), and the
    environment with the first file's value wherever two files disagree."""
    docs = [json.loads(Path(p).read_text()) for p in paths]
    env = {}
    for doc in reversed(docs):
        env.update(doc.get("env", {}))
    rows = [r for doc in docs for r in doc.get("rows", []) if "method" in r]
    gemm = [g for doc in docs for g in doc.get("gemm", [])]
    return env, rows, gemm


def _cell(v, best):
    if v is None:
        return ""
    if isinstance(v, str):
        return v
    txt = f"{v:.3g}" if v < 100 else f"{v:.0f}"
    return f"**{txt}**" if v == best else txt


def latency_tables(rows):
    by_key = {(r["n"], r["d"], r["batch"], r["k"], r["method"]): r for r in rows}
    methods = [m for m in METHOD_ORDER if any(r["method"] == m for r in rows)]
    methods += sorted({r["method"] for r in rows} - set(methods))
    lines = []
    for d in sorted({r["d"] for r in rows}):
        lines += ["", f"**width {d}**: median ms per batch (lower is better, fastest in bold)", "",
                  "| corpus | k | batch | " + " | ".join(methods) + " | fused vs torch |",
                  "|---|---|---|" + "---|" * (len(methods) + 1)]
        for n in sorted({r["n"] for r in rows if r["d"] == d}):
            for k in sorted({r["k"] for r in rows if r["d"] == d}):
                for b in sorted({r["batch"] for r in rows if r["d"] == d}):
                    vals = {}
                    for m in methods:
                        r = by_key.get((n, d, b, k, m))
                        vals[m] = None if r is None else r.get("error", r.get("ms"))
                    nums = [v for v in vals.values() if isinstance(v, (int, float))]
                    if not nums:
                        continue
                    best = min(nums)
                    f, t = vals.get("fused"), vals.get("torch")
                    ratio = f"{t / f:.2f}x" if isinstance(f, (int, float)) and isinstance(t, (int, float)) else ""
                    lines.append(f"| {short_n(n)} | {k} | {b} | " + " | ".join(_cell(vals[m], best) for m in methods)
                                 + f" | {ratio} |")
    return lines


def gemm_table(gemm):
    ok = [g for g in gemm if "error" not in g]
    if not ok:
        return []
    lines = ["", "**Score matrix only** (fp16 output, no top-k): custom kernel vs vendor BLAS", "",
             "| corpus | width | batch | custom ms | BLAS ms | custom TFLOP/s | BLAS TFLOP/s |",
             "|---|---|---|---|---|---|---|"]
    for g in ok:
        lines.append(f"| {short_n(g['n'])} | {g['d']} | {g['batch']} | {g['custom_ms']} | {g['cublas_ms']} | "
                     f"{g['custom_tflops']} | {g['cublas_tflops']} |")
    return lines


def recall_table(rows):
    per = {}
    for r in rows:
        if "recall_vs_fp32" in r:
            per.setdefault(r["method"], []).append(r["recall_vs_fp32"])
    if not per:
        return []
    lines = ["", "**Recall@k vs the exact fp32 search** (first 8 queries of each config)", "",
             "| method | min | mean |", "|---|---|---|"]
    for m in [m for m in METHOD_ORDER if m in per] + sorted(set(per) - set(METHOD_ORDER)):
        v = per[m]
        lines.append(f"| {m} | {min(v):.4f} | {sum(v) / len(v):.4f} |")
    return lines


def render(env, rows, gemm) -> str:
    rows = [r for r in rows if "method" in r]  # skipped configs carry no method
    head = []
    if env:
        head = [f"GPU: {env.get('gpu', '?')} ({env.get('arch', '')}, {env.get('sm_count', '?')} CUs), "
                f"torch {env.get('torch', '?')}, ROCm {env.get('rocm', env.get('torch_hip', '?'))}, "
                f"{env.get('date', '')}"]
    return "\n".join(head + latency_tables(rows) + gemm_table(gemm) + recall_table(rows)) + "\n"


def charts(rows, outdir: Path):
    """One PNG per width: ms vs batch per (corpus size, k) panel and method."""
    import matplotlib

    matplotlib.use("Agg")
    import matplotlib.pyplot as plt

    files = []
    for d in sorted({r["d"] for r in rows}):
        ns = sorted({r["n"] for r in rows if r["d"] == d})
        ks = sorted({r["k"] for r in rows if r["d"] == d})
        fig, axes = plt.subplots(len(ks), len(ns), figsize=(4 * len(ns), 3.2 * len(ks)), squeeze=False)
        for i, k in enumerate(ks):
            for j, n in enumerate(ns):
                ax = axes[i][j]
                for m in METHOD_ORDER:
                    pts = sorted((r["batch"], r["ms"]) for r in rows
                                 if r["d"] == d and r["n"] == n and r["k"] == k and r["method"] == m and "ms" in r)
                    if pts:
                        ax.plot([p[0] for p in pts], [p[1] for p in pts], marker="o", label=m)
                ax.set_xscale("log")
                ax.set_yscale("log")
                ax.set_title(f"{short_n(n)} x {d}, k={k}", fontsize=9)
                ax.set_xlabel("batch")
                ax.set_ylabel("ms / batch")
        axes[0][0].legend(fontsize=7)
        fig.tight_layout()
        path = outdir / f"latency_d{d}.png"
        fig.savefig(path, dpi=110)
        plt.close(fig)
        files.append(path)
    return files


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("inputs", nargs="+")
    ap.add_argument("--md", help="also write the tables to this file")
    ap.add_argument("--charts", help="directory for PNG charts (needs matplotlib)")
    args = ap.parse_args()
    env, rows, gemm = merge(args.inputs)
    text = render(env, rows, gemm)
    print(text)
    if args.md:
        Path(args.md).write_text(text)
    if args.charts:
        Path(args.charts).mkdir(parents=True, exist_ok=True)
        for f in charts(rows, Path(args.charts)):
            print("wrote", f)


if __name__ == "__main__":
    main()
