"""Writes the golden top-k vectors under tests/golden/ (run once; outputs are committed).

The reference ships no golden vectors (its tests recompute everything from fp32
torch math, ``tests/test_search.py:11-44``), so these fixtures come from an
independent brute force: float64 numpy scores of the fp16 inputs and a full
lexicographic sort by (score desc, id asc), the order of ``kernels.cu:277-279``.
They pin the C oracle and the HIP path on the edge cases the reference tests:
k=1, k=n, duplicated rows (exact ties), non-unit vectors with large scores,
widths that are not a multiple of 64, and near-duplicates at the k-th place.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent


def unit(rng, m, d):
    a = rng.standard_normal((m, d)).astype(np.float32)
    return (a / np.linalg.norm(a, axis=1, keepdims=True)).astype(np.float16)


def brute(q16, x16, k):
    s = q16.astype(np.float64) @ x16.astype(np.float64).T
    ids = np.broadcast_to(np.arange(x16.shape[0]), s.shape)
    order = np.lexsort((ids, -s), axis=-1)[:, :k]
    return np.take_along_axis(s, order, 1).astype(np.float32), order.astype(np.int64)


def case_random(rng):
    x, q = unit(rng, 300, 64), unit(rng, 5, 64)
    return dict(q=q, x=x, k=10)


def case_duplicates(rng):
    x = unit(rng, 200, 32)
    src = rng.choice(200, 20, replace=False)
    dst = rng.choice(np.setdiff1d(np.arange(200), src), 20, replace=False)
    x[dst] = x[src]
    q = np.concatenate([x[src[:3]], unit(rng, 1, 32)])  # queries that hit the duplicated rows
    return dict(q=q, x=x, k=15)


def case_k_equals_n(rng):
    return dict(q=unit(rng, 3, 64), x=unit(rng, 50, 64), k=50)


def case_k_one(rng):
    return dict(q=unit(rng, 7, 128), x=unit(rng, 500, 128), k=1)


def case_raw_ip(rng):
    x = rng.standard_normal((400, 96)).astype(np.float16)
    q = rng.standard_normal((3, 96)).astype(np.float16)
    return dict(q=q, x=x, k=20)


def case_near_ties(rng):
    n, d = 1000, 384
    x = unit(rng, n, d)
    src = rng.choice(n, 50, replace=False)
    dst = rng.choice(np.setdiff1d(np.arange(n), src), 50, replace=False)
    pert = x[src].astype(np.float32) + 1e-4 * rng.standard_normal((50, d)).astype(np.float32)
    pert /= np.linalg.norm(pert, axis=1, keepdims=True)
    x[dst[:25]] = x[src[:25]]
    x[dst[25:]] = pert[25:].astype(np.float16)
    q = np.concatenate([x[src[:4]], unit(rng, 4, d)])
    return dict(q=q, x=x, k=100)


CASES = {
    "random_n300_d64_b5_k10": case_random,
    "duplicates_n200_d32_k15": case_duplicates,
    "k_equals_n_n50_d64": case_k_equals_n,
    "k_one_n500_d128": case_k_one,
    "raw_ip_n400_d96_k20": case_raw_ip,
    "near_ties_n1000_d384_k100": case_near_ties,
}


def main():
    for i, (name, fn) in enumerate(CASES.items()):
        rng = np.random.default_rng(1000 + i)
        c = fn(rng)
        v, ids = brute(c["q"], c["x"], c["k"])
        np.savez_compressed(OUT / f"{name}.npz", q=c["q"], x=c["x"], k=np.int64(c["k"]),
                            scores=v, ids=ids)
        print("wrote", name, c["x"].shape, c["q"].shape, "k", c["k"])


if __name__ == "__main__":
    main()
