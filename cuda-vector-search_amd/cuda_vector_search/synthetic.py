"""Seeded synthetic workloads of the benchmark configurations.

Data follow the reference benchmark's distribution (``bench/bench_gpu.py:36-49``):
rows drawn N(0, 1), L2-normalised in fp32, stored fp16, generated 2^18 rows at a
time with seed ``seed * 100003 + chunk``.  The generator runs on ``device``
(CPU for bit-reproducible test inputs, the GPU for the large bench corpora).

``inject_near_ties`` builds the selection-stress variant of configuration C5:
a fraction of rows replaced by exact copies or sigma-perturbed, renormalised
copies of other rows, so that many queries have ties and near-ties at the
k-th place.
"""

from __future__ import annotations

import torch

CHUNK = 1 << 18

# name -> (n, d, batch, k, near_ties)
CONFIGS = {
    "C1": (100_000, 384, 32, 10, False),
    "C2": (1_000_000, 384, 256, 10, False),
    "C3": (4_000_000, 768, 1, 10, False),
    "C4": (1_000_000, 768, 256, 100, False),
    "C5": (100_000, 384, 256, 100, True),
}


def unit_corpus(n: int, d: int, seed: int, device="cpu") -> torch.Tensor:
    """[n, d] fp16 unit vectors, chunk c drawn with seed*100003 + c."""
    x = torch.empty(n, d, dtype=torch.float16, device=device)
    for c, lo in enumerate(range(0, n, CHUNK)):
        g = torch.Generator(device=device).manual_seed(seed * 100003 + c)
        blk = torch.randn(min(CHUNK, n - lo), d, device=device, generator=g)
        x[lo:lo + blk.shape[0]] = (blk / blk.norm(dim=1, keepdim=True)).half()
    return x


def unit_queries(b: int, d: int, seed: int, device="cpu") -> torch.Tensor:
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(b, d, device=device, generator=g)
    return (q / q.norm(dim=1, keepdim=True)).half()


def inject_near_ties(x: torch.Tensor, frac: float = 0.05, sigma: float = 1e-4, seed: int = 0,
                     exact_share: float = 0.5) -> torch.Tensor:
    """Replace ``frac`` of the rows (in place) with copies of other rows.

    The first ``exact_share`` of the replaced rows are exact copies (bit-identical
    scores: ties), the rest are copies perturbed by N(0, sigma^2) per coordinate
    and renormalised (near-ties).  Sources and targets are disjoint, chosen by a
    seeded permutation.
    """
    n = x.shape[0]
    m = int(round(frac * n))
    if m == 0:
        return x
    g = torch.Generator(device="cpu").manual_seed(seed)
    perm = torch.randperm(n, generator=g)
    dst, src = perm[:m].to(x.device), perm[m:2 * m].to(x.device)
    n_exact = int(round(exact_share * m))
    x[dst[:n_exact]] = x[src[:n_exact]]
    if n_exact < m:
        gd = torch.Generator(device=x.device).manual_seed(seed + 1)
        base = x[src[n_exact:]].float()
        noisy = base + sigma * torch.randn(base.shape, device=x.device, generator=gd)
        x[dst[n_exact:]] = (noisy / noisy.norm(dim=1, keepdim=True)).half()
    return x


def make_config(name: str, seed: int = 0, device="cpu"):
    """(corpus fp16 [n, d], queries fp16 [b, d], k) for a benchmark configuration."""
    n, d, b, k, ties = CONFIGS[name]
    x = unit_corpus(n, d, seed + d, device)
    if ties:
        inject_near_ties(x, seed=seed + 7)
    q = unit_queries(b, d, seed + 1, device)
    return x, q, k
