"""Rows wider than 1536 (needs an MI355X).

The reference accepts any width that is a multiple of 64: ``check_matrix``
tests only ``% 64`` (``csrc/kernels.cu:451-458``) and its score tile loops over
the whole width (``kernels.cu:150``).  Here rows wider than 1536 run scan
kernels whose query fragments ride through LDS beside the corpus rows instead
of staying in registers, a GEMV that takes the row 8 pieces at a time, and a
two-pass row preparation.  Everything is checked against the oracle at the
north star's bar (ids identical outside the 1e-3 near-tie band, scores within
1e-3; score matrices within 1e-3 fp32 / 3e-3 fp16), and ``Index.search``'s
"auto" must stay on the exact kernels at these widths.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from cuda_vector_search import Index, _ext
from cuda_vector_search import index as index_mod

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def make(n, d, b, seed=0):
    """Unit rows as tests/test_search.py:11-18."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, d, generator=g)
    q = torch.randn(b, d, generator=g)
    x = x / x.norm(dim=1, keepdim=True)
    q = q / q.norm(dim=1, keepdim=True)
    return x.half(), q.half()


@pytest.mark.parametrize("nq,n,d", [(37, 3001, 1600), (5, 1000, 2048), (32, 5000, 2048), (130, 2001, 3072),
                                    (3, 517, 4096), (257, 700, 1728), (64, 64, 4096)])
def test_wide_scores_match_oracle(eng, nq, n, d):
    say(f"wide scores nq={nq} n={n} d={d}")
    x, q = make(n, d, nq, seed=n + d)
    ref = oracle.scores(q, x)
    s = eng.scores(q.cuda(), x.cuda()).cpu().numpy()
    assert s.shape == (nq, n)
    np.testing.assert_allclose(s, ref, rtol=0, atol=1e-3)
    s16 = eng.scores(q.cuda(), x.cuda(), False)
    assert s16.dtype == torch.float16
    np.testing.assert_allclose(s16.float().cpu().numpy(), ref, rtol=0, atol=3e-3)


WIDE_FUSED = [
    (20000, 1600, 1, 10),     # batch-1 GEMV
    (20000, 2048, 16, 10),    # 16-query block (16x16x32 MFMA)
    (30000, 2048, 32, 100),   # 32-query block, 4 row splits
    (20000, 3072, 64, 256),   # 64-query block, k = 256
    (40000, 4096, 128, 64),   # 128-query block
    (20000, 1728, 256, 10),   # two 128-query groups, odd stage count (27)
    (5000, 4096, 3, 1),       # k = 1 (arg-max)
    (300, 2048, 5, 150),      # tiny corpus, k > tile rows
]


@pytest.mark.parametrize("n,d,b,k", WIDE_FUSED)
def test_wide_fused_matches_oracle(eng, n, d, b, k):
    say(f"wide fused n={n} d={d} b={b} k={k}")
    x, q = make(n, d, b, seed=n + d + b + k)
    index = Index(x.cuda(), metric="ip")
    v, i = index.search(q.cuda(), k, method="fused")
    assert oracle.check_exact(q, x, k, v, i) >= 0.999


@pytest.mark.parametrize("flags", [_ext.FLAG_NO_PREPASS, _ext.FLAG_FORCE_PREPASS])
def test_wide_prepass_does_not_change_results(eng, flags):
    n, d, b, k = 30000, 2048, 100, 20
    say(f"wide prepass flags={flags}")
    x, q = make(n, d, b, seed=7)
    qd, xd = q.cuda(), x.cuda()
    v0, i0, _ = eng.fused_topk(qd, xd, k)
    v1, i1, _ = eng.fused_topk(qd, xd, k, flags=flags)
    torch.cuda.synchronize()
    assert torch.equal(v0, v1) and torch.equal(i0, i1)
    oracle.check_exact(q, x, k, v0.cpu().numpy(), i0.cpu().numpy().astype(np.int64))


@pytest.mark.parametrize("d", [1600, 2048, 4096])
@pytest.mark.parametrize("k", [1, 10, 100])
def test_wide_gemv_matches_oracle_and_scan(eng, d, k):
    say(f"wide gemv d={d} k={k}")
    x, q = make(30011, d, 1, seed=d + k)
    qd, xd = q.cuda(), x.cuda()
    v, i, plan = eng.fused_topk(qd, xd, k)
    v2, i2, plan2 = eng.fused_topk(qd, xd, k, flags=_ext.FLAG_NO_GEMV)
    torch.cuda.synchronize()
    assert plan.tolist()[0] == 1 and plan2.tolist()[0] == 16
    v, i = v.cpu().numpy(), i.cpu().numpy().astype(np.int64)
    oracle.check_exact(q, x, k, v, i)
    np.testing.assert_allclose(v, v2.cpu().numpy(), rtol=0, atol=1e-5)


def test_wide_forced_plans(eng):
    say("wide forced plans")
    x, q = make(20000, 2048, 50, seed=4)
    qd, xd = q.cuda(), x.cuda()
    base_v, base_i, _ = eng.fused_topk(qd, xd, 10)
    for bq, chunks in [(16, 1), (32, 7), (64, 1000), (128, 3)]:
        v, i, plan = eng.fused_topk(qd, xd, 10, bq, chunks)
        assert plan.tolist()[0] == bq
        assert torch.allclose(v, base_v, atol=1e-5) and torch.equal(i, base_i)
    with pytest.raises(RuntimeError, match="not supported at width"):
        eng.fused_topk(qd, xd, 10, 256)


def test_wide_index_auto_stays_exact_on_the_kernels(eng, monkeypatch):
    """"auto" never takes the fp16 torch path on gfx950 at these widths: k <= 256
    runs the fused kernels, 256 < k <= 1024 the exact large-k path."""
    n, d, b = 20000, 2000, 40  # d pads to 2048 (prep kernel, wide rows)
    say(f"wide index auto n={n} d={d} b={b}")
    x, q = make(n, d, b, seed=12)

    def no_torch(*a, **kw):
        raise AssertionError("auto took the torch path")

    monkeypatch.setattr(index_mod, "torch_topk", no_torch)
    index = Index(x.cuda(), metric="cosine")
    assert index._x.shape[1] == 2048 and index._xq is None
    qq = index._prep_queries(q.cuda())[:, :d].cpu()
    xs = index.embeddings.cpu()
    for k in (10, 256, 300, 1024):
        v, i = index.search(q.cuda(), k)
        assert v.dtype == torch.float32 and i.dtype == torch.int64
        oracle.check_exact(qq, xs, k, v, i)
    s = index.scores(q.cuda())
    np.testing.assert_allclose(s.cpu().numpy(), oracle.scores(qq, xs), rtol=0, atol=1e-3)
    with pytest.raises(ValueError, match="widths up to 1536"):
        index.search(q.cuda(), 10, method="int8")


def test_wide_twopass(eng):
    n, d, b, k = 10000, 3072, 8, 10
    say("wide twopass")
    x, q = make(n, d, b, seed=13)
    index = Index(x.cuda(), metric="ip")
    v, i = index.search(q.cuda(), k, method="twopass")
    oracle.check_exact(q, x, k, v, i, tol=2e-3)


@pytest.mark.parametrize("n,d,width", [(100, 2000, 2048), (33, 4096, 4096), (5, 1537, 1600), (64, 1600, 1600)])
def test_wide_prep_rows_matches_oracle(eng, n, d, width):
    say(f"wide prep_rows n={n} d={d} width={width}")
    g = torch.Generator().manual_seed(n + d)
    x = (torch.randn(n, d, generator=g) * torch.rand(n, 1, generator=g) * 10).half()
    x[0] = 0
    src = x.cuda()
    out = torch.full((n, width), float("nan"), dtype=torch.float16, device="cuda")
    eng.prep_rows(src, out, True)
    torch.cuda.synchronize()
    want = oracle.normalize_rows(x.numpy(), width=width)
    got = out.cpu().numpy()
    a, b = got.astype(np.float32), want.astype(np.float32)
    ulp = np.maximum(np.abs(np.spacing(got)), np.abs(np.spacing(want))).astype(np.float32)
    assert np.all(np.abs(a - b) <= ulp)
    assert not got[:, d:].any() and not got[0].any()
    if width == d:
        inplace = x.cuda()
        eng.prep_rows(inplace, inplace, True)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(inplace.cpu().numpy(), got)


def test_wide_int8_is_refused_by_the_engine(eng):
    x = torch.zeros(128, 2048, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="widths up to 1536"):
        eng.q8_build(x)
    with pytest.raises(RuntimeError, match="widths up to 1536"):
        eng.q8_plan(4, 128, 2048, 10)
