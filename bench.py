"""Benchmark of the exact top-k hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs C2,C1,C3,C4,C5]

A step is one ``Index.search(queries, k)`` over one batch with the corpus and the
queries already resident in HBM (the reference's methodology,
bench/bench_gpu.py:105,124: an ``ip`` index over unit vectors, so cosine
without per-call query normalisation).  The headline workload is benchmark
config C2 (1M x 384 corpus, batch 256, k=10); the other configs are reported in
``configs_detail``.  One JSON line goes to stdout:

* value / ms_per_step: host-timed whole-batch throughput (queries/s) over K steps
  bracketed by device synchronisation;
* roofline: the dominant kernel of the path ``Index.search`` takes (the fp16
  MFMA scan / GEMV, or their int8 pre-filter forms over the int8 companion of
  the corpus where "auto" picks it) timed with HIP events that the library
  records on the stream it launches on, over a second timed region of K
  back-to-back calls, against its algorithmic bytes (corpus read once +
  queries, in the kernel's element type) and the MI355X peaks (8 TB/s HBM;
  2.5 PFLOP/s dense fp16 / 5.0 POP/s int8 MFMA as mfma_frac).  Each config row
  also times the other exact path on the same batch.  ``traffic`` is the kernel's
  measured HBM bytes per launch: two child runs of this script under
  ``rocprofv3 --pmc`` (FETCH_SIZE, then WRITE_SIZE), each scaled by what the
  same counter reads for a plain 1 GiB device copy in the same child;
* configs_detail: one row per config with the same W warm-up and K timed calls:
  ms per batch, queries/s, per-stage device times, the dominant kernel's
  fraction of its roofline on its own bytes, and the end-to-end roofline of
  the whole search (achieved = max(F/P_fp16, B/BW) / t with F = 2 b n d,
  B = 2 n d + 2 b d + 12 b k, both component fractions), plus that config's
  CPU baseline;
* cpu_baseline: the reference's CPU search path (fp32 torch matmul + topk,
  reference.py:8-15) and the numpy baseline (bench/bench_baselines.py:45-50),
  both as restated in oracle/, timed on this host on a bounded sample of each
  config's batch (time_call semantics of bench/timing.py:9-34 with the CPU
  settings of bench/bench_baselines.py:125-127); their results double as the
  recall check of the GPU output.

Clock settling: the GPU's clocks take ~20 ms of sustained MFMA work to settle
(measured per call after 2 s idle: the C2 search 176-199 -> 146-149 us over its
first ~100 calls, a hipBLASLt 4096^3 fp16 GEMM 147 -> 121 us the same way, a
384 MB device copy flat at 153-156 us).  Before its W warm-up steps each config
therefore runs its step untimed for --settle-ms (default 30) of wall time
(``settle_calls`` in its row); the timed region is still exactly K steps.
Beside the settled figure each row carries ``cold_ms_per_batch``: the mean of
the first 20 back-to-back searches after 2 s of idle, with no settling (the
ramp a process that searches a few times after idling sees).
"""

from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (str(REPO), str(REPO / "cuda-vector-search_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "queries/sec at 1M×384 b256 k10; ms/batch + HBM GB/s at 4M×768 b1"
HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK = 2.5e15
MFMA_INT8_PEAK = 5.0e15
REF_T4_QPS_C2 = 13178.5  # reference fused kernel on a Tesla T4 at C2 (results/t4.json:380-391, README.md:113)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_bytes(n, d, b):
    """Algorithmic HBM bytes of one fp16 scan/GEMV launch: corpus once + queries."""
    return 2 * n * d + 2 * b * d


def kernel_bytes_q8(n, dq, b):
    """Algorithmic HBM bytes of one int8 scan/GEMV launch: int8 corpus once + int8 queries."""
    return n * dq + b * dq


def end_to_end(n, d, b, k, ms, int8, dq):
    """The whole search against its roofline max(F/P, B/BW) with
    F = 2 b n d (fp16 MFMA peak) and B = 2 n d + 2 b d + 12 b k (the fp16
    corpus read once), whatever path ran; both component fractions."""
    f = 2.0 * b * n * d
    nbytes = 2.0 * n * d + 2.0 * b * d + 12.0 * b * k
    t_mfma = f / MFMA_FP16_PEAK
    t_hbm = nbytes / (HBM_PEAK_GBS * 1e9)
    t = ms * 1e-3
    out = {"flops": f, "bytes": nbytes, "t_mfma_us": round(t_mfma * 1e6, 2), "t_hbm_us": round(t_hbm * 1e6, 2),
           "achieved": round(max(t_mfma, t_hbm) / t, 4), "mfma_frac": round(t_mfma / t, 4),
           "hbm_frac": round(t_hbm / t, 4)}
    if int8:
        out["note"] = (f"the int8 path streams n*{dq} bytes of int8 companion instead of the 2*n*d fp16 bytes "
                       "counted in B, plus the fp16 rows of the candidates it rescores")
    return out


def run_config(name, steps, warmup, eng, torch, synthetic, Index, settle_ms=30.0, cold_idle_s=2.0, cold_calls=20):
    from cuda_vector_search.index import q8_row_bytes

    n, d, b, k, ties = synthetic.CONFIGS[name]
    log(f"[{name}] generating n={n} d={d} b={b} k={k} near_ties={ties}")
    x = synthetic.unit_corpus(n, d, seed=d, device="cuda")
    if ties:
        synthetic.inject_near_ties(x, seed=7)
    q = synthetic.unit_queries(b, d, seed=1, device="cuda")
    index = Index(x, metric="ip", copy=False)
    torch.cuda.synchronize()

    def step():
        return index.search(q, k)

    # Cold calls: one untimed call (first-use allocations), cold_idle_s of idle,
    # then the first cold_calls searches back to back, each event-timed: the
    # unsettled clocks a process sees after idling (module docstring).
    step()
    torch.cuda.synchronize()
    time.sleep(cold_idle_s)
    cold_ev = [torch.cuda.Event(enable_timing=True) for _ in range(cold_calls + 1)]
    cold_ev[0].record()
    for i in range(cold_calls):
        step()
        cold_ev[i + 1].record()
    torch.cuda.synchronize()
    cold_ms = [cold_ev[i].elapsed_time(cold_ev[i + 1]) for i in range(cold_calls)]

    settle_calls = 0  # untimed, until the clocks have settled (module docstring)
    t_settle = time.perf_counter() + settle_ms / 1000.0
    while settle_calls < 1 or time.perf_counter() < t_settle:
        step()
        settle_calls += 1
        if settle_calls % 8 == 0:
            torch.cuda.synchronize()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        out = step()
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1000.0 / steps
    dev_ms = e0.elapsed_time(e1) / steps

    # Second timed region: the same K calls back to back, through the path
    # Index.search took, with the library recording HIP events between its
    # launches on the stream it uses.
    int8 = index._int8_wins(b, k)
    qq = index._prep_queries(q)
    width = index._x.shape[1]

    def marked(ev):
        if int8:
            return eng.q8_topk(qq, index._x, index._xq, k, marks=ev)
        return eng.fused_topk_marked(qq, index._x, k, ev)

    marks = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(steps)]
    torch.cuda.synchronize()
    for i in range(steps):
        _, _, plan = marked(marks[i])
    torch.cuda.synchronize()
    per_step = [[m[j].elapsed_time(m[j + 1]) for j in range(4)] for m in marks]
    stage_ms = [statistics.fmean(s[j] for s in per_step) for j in range(4)]
    kern_ms = stage_ms[2]
    dq = q8_row_bytes(width)
    nbytes = kernel_bytes_q8(n, dq, b) if int8 else kernel_bytes(n, width, b)
    gbs = nbytes / (kern_ms * 1e-3) / 1e9
    flops = 2.0 * b * n * (dq if int8 else d)
    mfma_peak = MFMA_INT8_PEAK if int8 else MFMA_FP16_PEAK

    # The other exact path on the same batch, for comparison (not the value).
    def alt():
        if int8:
            return eng.fused_topk(qq, index._x, k)
        return eng.q8_topk(qq, index._x, index._xq, k) if index._xq is not None else None

    alt_ms = None
    if alt() is not None:
        for _ in range(warmup):  # the same warm-up as the timed path
            alt()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(steps):
            alt()
        torch.cuda.synchronize()
        alt_ms = (time.perf_counter() - t1) * 1000.0 / steps
    row = {
        "config": name, "n": n, "d": d, "batch": b, "k": k, "near_ties": ties,
        "plan": [int(v) for v in plan.tolist()],
        "settle_calls": settle_calls,
        "cold_ms_per_batch": round(statistics.fmean(cold_ms), 4),
        "cold_first_last_ms": [round(cold_ms[0], 4), round(cold_ms[-1], 4)],
        "cold_sample": f"{cold_calls} back-to-back calls after {cold_idle_s:g} s idle, no settling; event-timed",
        "ms_per_batch": round(wall_ms, 4), "device_ms_per_batch": round(dev_ms, 4),
        "qps": round(b / (wall_ms / 1000.0), 1),
        "path": "int8" if int8 else "fused",
        "stage_ms": {"sample_pass": round(stage_ms[0], 4), "threshold_select": round(stage_ms[1], 4),
                     "scan" if b > 1 else "gemv": round(kern_ms, 4),
                     "rescore_select" if int8 else "final_select": round(stage_ms[3], 4)},
        "kernel": (("scan (int8 MFMA)" if int8 else "scan (MFMA)") if plan.tolist()[0] != 1
                   else ("gemv (int8 v_dot4)" if int8 else "gemv (v_dot2)")),
        "kernel_bytes": nbytes,
        "kernel_hbm_gbs": round(gbs, 1), "kernel_hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "kernel_mfma_frac": round(flops / (kern_ms * 1e-3) / mfma_peak, 4),
        "roofline_floor_us": round(max(flops / mfma_peak, nbytes / (HBM_PEAK_GBS * 1e9)) * 1e6, 2),
        "end_to_end": end_to_end(n, d, b, k, wall_ms, int8, dq),
        "other_path": {"path": "fused" if int8 else "int8",
                       "ms_per_batch": round(alt_ms, 4) if alt_ms is not None else None},
    }
    log(f"[{name}] {json.dumps(row)}")
    return row, (index, q, k, out)


# Demangled names of the dominant kernel's dispatches (mode 0 = candidate append).
DOMINANT = {"scan": re.compile(r"scan_kernel<(?:\d+,\s*){5}0\b"), "gemv": re.compile(r"gemv_kernel<\d+,\s*0>"),
            "scan_q8": re.compile(r"scan_kernel<(?:\d+,\s*){5}4\b|q8scan384_kernel"),
            "gemv_q8": re.compile(r"gemv_kernel<\d+,\s*4>")}
COPY_KERNEL = re.compile(r"copyBuffer")  # torch copy_ between device tensors = hipMemcpyAsync
COPY_BYTES = 1 << 30


def pmc_child(name, method="auto"):
    """Body of one ``rocprofv3 --pmc`` child: a few searches of config `name`
    (Index.search with `method`), then a plain device copy of COPY_BYTES for the
    counter's calibration."""
    import torch

    from cuda_vector_search import Index, synthetic

    n, d, b, k, ties = synthetic.CONFIGS[name]
    x = synthetic.unit_corpus(n, d, seed=d, device="cuda")
    if ties:
        synthetic.inject_near_ties(x, seed=7)
    q = synthetic.unit_queries(b, d, seed=1, device="cuda")
    index = Index(x, metric="ip", copy=False)
    for _ in range(3):
        index.search(q, k, method=method)
    torch.cuda.synchronize()
    del index, x
    src = torch.ones(COPY_BYTES // 2, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"pmc child {name}: 3 searches (method {method}), 3 copies of {COPY_BYTES} bytes", flush=True)


def dominant_key(name):
    """Which kernel dominates config `name` on the path Index.search takes."""
    from cuda_vector_search.index import PAD, int8_auto
    from cuda_vector_search.synthetic import CONFIGS

    n, d, b, k, _ = CONFIGS[name]
    key = "gemv" if b == 1 else "scan"
    return key + "_q8" if int8_auto(n, d + (-d) % PAD, b, k) else key


def measure_traffic(name):
    """HBM bytes per launch of the dominant kernel from two rocprofv3 --pmc child
    runs; None (with the reason) when rocprofv3 is absent or a run fails."""
    import csv
    import shutil
    import subprocess
    import tempfile

    if shutil.which("rocprofv3") is None:
        return None, "rocprofv3 not on PATH"
    pat = DOMINANT[dominant_key(name)]
    env = dict(os.environ, TMPDIR="/tmp")
    res = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        out_dir = tempfile.mkdtemp(prefix=f"cvs_pmc_{counter}_", dir="/tmp")
        cmd = ["timeout", "-k", "10", "-s", "KILL", "240", "rocprofv3", "--pmc", counter, "-f", "csv",
               "-d", out_dir, "-o", "pmc", "--", sys.executable, str(REPO / "bench.py"),
               "--pmc-child", name]
        log(f"[traffic] rocprofv3 --pmc {counter} child run ...")
        t0 = time.perf_counter()
        r = subprocess.run(cmd, cwd="/tmp", env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                           text=True)
        log(f"[traffic] {counter}: exit {r.returncode} after {time.perf_counter() - t0:.1f} s")
        files = sorted(Path(out_dir).rglob("*counter_collection.csv"))
        if r.returncode != 0 or not files:
            tail = "\n".join(r.stdout.splitlines()[-5:])
            shutil.rmtree(out_dir, ignore_errors=True)
            return None, f"rocprofv3 --pmc {counter} failed (exit {r.returncode}): {tail}"
        kern, copy = [], []
        for f in files:
            with open(f, newline="") as fh:
                for row in csv.DictReader(fh):
                    if row.get("Counter_Name") != counter:
                        continue
                    kname = row.get("Kernel_Name", "")
                    if pat.search(kname):
                        kern.append(float(row["Counter_Value"]))
                    elif COPY_KERNEL.search(kname):
                        copy.append(float(row["Counter_Value"]))
        shutil.rmtree(out_dir, ignore_errors=True)
        # the calibration copies are the child's largest (corpus set-up copies less)
        big_copies = [c for c in copy if copy and c >= 0.75 * max(copy)]
        if not kern or not big_copies:
            return None, f"{counter}: no dispatches matched (kernel {len(kern)}, copy {len(big_copies)})"
        scale = COPY_BYTES / (statistics.median(big_copies) * 1024.0)
        res[counter] = {"kib_per_launch": statistics.median(kern), "copy_kib": statistics.median(big_copies),
                        "scale": round(scale, 4)}
    traffic = sum(v["kib_per_launch"] * 1024.0 * v["scale"] for v in res.values())
    return int(round(traffic)), res


def _host_facts(torch):
    cpu_model = ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    blas = ""
    try:
        import numpy as np

        cfg = np.show_config(mode="dicts")
        blas = cfg.get("Build Dependencies", {}).get("blas", {}).get("name", "")
    except Exception:  # noqa: BLE001 - informational only
        pass
    return {"host_cpu": cpu_model, "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
            "numpy_blas": blas}


def _mem_available_bytes():
    try:
        for line in Path("/proc/meminfo").read_text().splitlines():
            if line.startswith("MemAvailable:"):
                return int(line.split()[1]) * 1024
    except OSError:
        pass
    return None


def time_cpu(fn, target_s=1.0, max_reps=20):
    """Median seconds per call with bench/timing.py:9-34's semantics at the CPU
    settings of bench/bench_baselines.py:125-127: 2 warm-up calls (1 if a call
    takes more than a second), then calls until target_s or max_reps, at least 3."""
    t0 = time.perf_counter()
    res = fn()
    if time.perf_counter() - t0 <= 1.0:
        res = fn()
    times = []
    t_end = time.perf_counter() + target_s
    while (time.perf_counter() < t_end and len(times) < max_reps) or len(times) < 3:
        t1 = time.perf_counter()
        res = fn()
        times.append(time.perf_counter() - t1)
    return statistics.median(times), len(times), res


def cpu_baseline(index, q, k, gpu_ids, torch, sample_q=64):
    """The reference's CPU paths for one config on a bounded sample: every
    corpus row, the first `sample_q` queries of the batch.  Restated in oracle/
    (kind "port"): the CPU Index's fp32 torch matmul + topk (reference.py:8-15,
    index.py:69) and numpy matmul + argpartition (bench_baselines.py:45-50)."""
    import numpy as np

    import oracle

    n, dim = index.embeddings.shape
    need = n * dim * 4 * 2  # the fp32 corpus, and headroom for its score rows and copies
    avail = _mem_available_bytes()
    if avail is not None and need > 0.5 * avail:
        return {"value": None, "unit": "queries/s", "kind": "port",
                "skipped": f"fp32 corpus {n}x{dim} needs ~{need / 1e9:.1f} GB; host has {avail / 1e9:.1f} GB "
                           "available"}
    threads = torch.get_num_threads()
    sq = min(sample_q, q.shape[0])
    xf = index.embeddings.float().cpu().contiguous()
    qf = q[:sq, :dim].float().cpu().contiguous()
    xn, qn = xf.numpy(), qf.numpy()
    t_torch, reps_t, (tv, ti) = time_cpu(lambda: oracle.torch_topk_cpu(qf, xf, k))
    t_np, reps_n, _ = time_cpu(lambda: oracle.numpy_search(qn, xn, k))
    gi = gpu_ids[:sq].cpu().numpy()
    recall = float(np.mean([len(set(a) & set(b)) / k for a, b in zip(gi.tolist(), ti.numpy().tolist())]))
    del xf, xn
    return {
        "value": round(sq / t_torch, 2), "unit": "queries/s", "cores": threads, "kind": "port",
        "sample": f"{sq} of the batch's {q.shape[0]} queries against the full corpus ({n}x{dim} fp32); "
                  f"torch matmul+topk (reference.py:8-15), median of {reps_t}",
        "ms_per_query": round(t_torch / sq * 1e3, 4),
        "numpy_argpartition_qps": round(sq / t_np, 2),
        "numpy_sample": f"same sample, numpy matmul+argpartition (bench_baselines.py:45-50), median of {reps_n}",
        "gpu_recall_vs_cpu_torch": round(recall, 5),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20,
                    help="untimed steps before each config's timed ones")
    ap.add_argument("--configs", default="C2,C1,C3,C4,C5",
                    help="first entry is the headline workload")
    ap.add_argument("--settle-ms", type=float, default=30.0,
                    help="untimed wall time of each config's step before its warm-up (clock settling)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-queries", type=int, default=64,
                    help="queries of each batch in the CPU baseline's sample (all of a smaller batch)")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 --pmc child runs that measure roofline.traffic")
    ap.add_argument("--pmc-child", metavar="CONFIG", help=argparse.SUPPRESS)
    ap.add_argument("--pmc-method", default="auto", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.pmc_child:
        pmc_child(args.pmc_child, args.pmc_method)
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on exactly one GPU (asked for --gpus {args.gpus}, WORLD_SIZE={world}): "
              "the exact top-k engine is a single-GPU build; multi-GPU sharding is design-only.",
              file=sys.stderr, flush=True)
        sys.exit(2)

    names = [c.strip() for c in args.configs.split(",") if c.strip()]
    # Counter runs first, in child processes, before this process touches the GPU.
    traffic, traffic_detail = (None, "skipped (--no-traffic)")
    if not args.no_traffic:
        traffic, traffic_detail = measure_traffic(names[0])
        log(f"[traffic] {traffic} bytes/launch: {traffic_detail}")

    import torch

    from cuda_vector_search import Index, _ext, synthetic

    if not _ext.available():
        print("bench.py needs an AMD Instinct MI355X (gfx950) GPU", file=sys.stderr)
        sys.exit(1)
    eng = _ext.load()

    rows = []
    cpu = None
    for i, name in enumerate(names):
        # every config gets the same warm-up and timed steps
        row, state = run_config(name, args.steps, args.warmup, eng, torch, synthetic, Index, args.settle_ms)
        if not args.no_cpu_baseline:
            index, q, k, out = state
            log(f"[{name}] cpu baseline ...")
            row["cpu_baseline"] = cpu_baseline(index, q, k, out[1], torch, sample_q=args.cpu_queries)
            log(f"[{name}] cpu baseline {json.dumps(row['cpu_baseline'])}")
            if i == 0:
                cpu = dict(row["cpu_baseline"], **_host_facts(torch))
        rows.append(row)
        del state
        torch.cuda.empty_cache()

    row = rows[0]
    n, d, b, k = row["n"], row["d"], row["batch"], row["k"]
    kern_ms = row["stage_ms"]["scan" if b > 1 else "gemv"]
    out = {
        "metric": METRIC,
        "value": row["qps"],
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": row["ms_per_batch"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(row["qps"] / REF_T4_QPS_C2, 3) if row["config"] == "C2" else None,
        "vs_baseline_ref": "reference fused kernel on a Tesla T4 (results/t4.json:380-391), not MI355X",
        "dtype": ("int8 pre-filter (int32 accumulate, rigorous bound) + exact fp16 rescoring (fp32 accumulate)"
                  if row["path"] == "int8" else "fp16 in, fp32 accumulate"),
        "data": "synthetic: seeded N(0,1) rows, L2-normalised, stored fp16 (cuda_vector_search.synthetic)",
        "config": {"workload": f"{row['config']}: exact top-{k} over {n}x{d} fp16 corpus, batch {b}, "
                               "cosine on unit vectors (ip index)",
                   "n": n, "d": d, "batch": b, "k": k, "plan": row["plan"]},
        "roofline": {
            "bound": "hbm",
            "kernel": row["kernel"],
            "achieved": row["kernel_hbm_gbs"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": row["kernel_hbm_frac"],
            "traffic": traffic,
            "traffic_detail": traffic_detail,
            "kernel_ms": kern_ms,
            "algorithmic_bytes": row["kernel_bytes"],
            "mfma_frac": row["kernel_mfma_frac"],
            "end_to_end": row["end_to_end"],
        },
        "cpu_baseline": cpu,
        "configs_detail": rows,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
