"""The seeded benchmark workloads (cuda_vector_search.synthetic) on the CPU."""

from __future__ import annotations

import torch

from cuda_vector_search import synthetic


def test_unit_corpus_is_reproducible_and_normalised():
    a = synthetic.unit_corpus(1000, 64, seed=3)
    b = synthetic.unit_corpus(1000, 64, seed=3)
    assert a.dtype == torch.float16 and torch.equal(a, b)
    assert torch.allclose(a.float().norm(dim=1), torch.ones(1000), atol=2e-3)
    assert not torch.equal(a, synthetic.unit_corpus(1000, 64, seed=4))


def test_chunk_seeding_matches_reference_pattern():
    # chunk c uses seed*100003 + c (bench/bench_gpu.py:36-43)
    x = synthetic.unit_corpus(synthetic.CHUNK + 10, 8, seed=2)
    g = torch.Generator().manual_seed(2 * 100003 + 1)
    blk = torch.randn(10, 8, generator=g)
    assert torch.equal(x[synthetic.CHUNK:], (blk / blk.norm(dim=1, keepdim=True)).half())


def test_near_tie_injection():
    x = synthetic.unit_corpus(2000, 32, seed=5)
    y = synthetic.inject_near_ties(x.clone(), frac=0.05, sigma=1e-4, seed=1)
    changed = (y != x).any(dim=1)
    assert 90 <= int(changed.sum()) <= 100
    # half exact copies: rows that equal some other row exactly
    uniq = torch.unique(y.view(torch.int16), dim=0).shape[0]
    assert uniq <= 2000 - 45
    assert torch.allclose(y.float().norm(dim=1), torch.ones(2000), atol=2e-3)


def test_configs_match_baseline():
    assert synthetic.CONFIGS["C2"] == (1_000_000, 384, 256, 10, False)
    assert synthetic.CONFIGS["C3"] == (4_000_000, 768, 1, 10, False)
    assert synthetic.CONFIGS["C5"][4] is True
