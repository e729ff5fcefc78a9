"""Parity of the gfx950 HIP path with the CPU oracle (needs an MI355X).

Restates the reference's GPU tests (tests/test_search.py:47-169) against the
oracle instead of torch, and adds: the committed golden vectors, the batch-1
GEMV path, the sampling pre-pass on/off, list compaction under adversarial
ordering, exact ties, the benchmark configs at full size (every query at
C1, C3 and C5, 64 spread queries at C2 and C4, both exact paths), and an
int8 companion kept current when the corpus changes.

Bars (the north star's): ids identical except inside the 1e-3 near-tie band of
the k-th score, scores within 1e-3 (oracle.check_exact); score matrices within
1e-3 (fp32) / 3e-3 (fp16) of the exactly accumulated scores.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from cuda_vector_search import Index, _ext, synthetic

pytestmark = pytest.mark.gpu

GOLDEN = sorted((Path(__file__).parent / "golden").glob("*.npz"))


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def make(n, d, b, seed=0, normal=True):
    """tests/test_search.py:11-18."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, d, generator=g)
    q = torch.randn(b, d, generator=g)
    if normal:
        x = x / x.norm(dim=1, keepdim=True)
        q = q / q.norm(dim=1, keepdim=True)
    return x.half(), q.half()


def pad64(t: torch.Tensor) -> torch.Tensor:
    extra = (-t.shape[1]) % 64
    return torch.nn.functional.pad(t, (0, extra)) if extra else t


def run_fused(eng, q, x, k, **kw):
    """fused_topk on padded device copies; returns numpy (v, i, plan)."""
    qd = pad64(q).cuda().contiguous()
    xd = pad64(x).cuda().contiguous()
    v, i, plan = eng.fused_topk(qd, xd, k, **kw)
    torch.cuda.synchronize()
    return v.cpu().numpy(), i.cpu().numpy().astype(np.int64), plan.tolist()


# --------------------------------------------------------------------------- scores


@pytest.mark.parametrize("nq,n,d", [(37, 3001, 192), (5, 1000, 64), (100, 2000, 768),
                                    (3, 517, 1536), (16, 64, 384), (70, 130, 128),
                                    (300, 20000, 384), (200, 9999, 768), (129, 4097, 256),
                                    (257, 3, 64)])
def test_scores_kernel_matches_oracle(eng, nq, n, d):
    say(f"scores nq={nq} n={n} d={d}")
    x, q = make(n, d, nq, seed=n + d)
    s = eng.scores(q.cuda(), x.cuda()).cpu().numpy()
    ref = oracle.scores(q, x)
    assert s.shape == (nq, n)
    np.testing.assert_allclose(s, ref, rtol=0, atol=1e-3)
    s16 = eng.scores(q.cuda(), x.cuda(), False)
    assert s16.dtype == torch.float16
    np.testing.assert_allclose(s16.float().cpu().numpy(), ref, rtol=0, atol=3e-3)


# --------------------------------------------------------------------------- golden


@pytest.mark.parametrize("path", GOLDEN, ids=[p.stem for p in GOLDEN])
@pytest.mark.parametrize("flags", [0, _ext.FLAG_NO_GEMV])
def test_golden_vectors(eng, path, flags):
    z = np.load(path)
    k = int(z["k"])
    say(f"golden {path.stem} flags={flags}")
    v, i, _ = run_fused(eng, torch.from_numpy(z["q"]), torch.from_numpy(z["x"]), k, flags=flags)
    np.testing.assert_allclose(v, z["scores"], rtol=0, atol=1e-3 * max(1.0, float(np.abs(z["scores"]).max())))
    assert oracle.check_exact(z["q"], z["x"], k, v, i) >= 0.99
    # exact ties (bit-identical rows) come out in id order
    for r in range(v.shape[0]):
        for j in range(k - 1):
            if v[r, j] == v[r, j + 1]:
                assert i[r, j] < i[r, j + 1]


# --------------------------------------------------------------------------- reference cases


FUSED_CASES = [
    (1000, 64, 1, 1),
    (1000, 64, 3, 10),
    (4099, 128, 17, 10),
    (20000, 384, 1, 10),
    (20000, 384, 32, 100),
    (20000, 384, 100, 33),
    (20000, 768, 256, 64),
    (50000, 384, 70, 128),
    (30000, 384, 40, 256),
    (300, 96, 5, 150),
    (100, 64, 2, 100),
]


@pytest.mark.parametrize("n,d,b,k", FUSED_CASES)
def test_fused_matches_exact(eng, n, d, b, k):
    say(f"fused n={n} d={d} b={b} k={k}")
    x, q = make(n, d, b, seed=n + d + b + k)
    index = Index(x.cuda(), metric="ip")
    v, i = index.search(q.cuda(), k, method="fused")
    assert v.dtype == torch.float32 and i.dtype == torch.int64
    rec = oracle.check_exact(q, x, k, v, i)
    assert rec >= 0.999


def _random_fused_cases(count=16, seed=20261203):
    """Seeded random (nq, n, d, k) for the fp16 path: widths 8-4096 (zero-padded
    to multiples of 64; the wide path above 1536), batches 1-300 (the batch-1
    GEMV and every query-block size), log-uniform corpus sizes, k 1-256."""
    rng = np.random.default_rng(seed)
    batches = [1, 1, 3, 16, 17, 32, 64, 65, 128, 200, 256, 300]
    out = []
    while len(out) < count:
        d = int(rng.choice([int(rng.integers(1, 64)) * 8, int(rng.integers(1, 25)) * 64, int(rng.integers(25, 65)) * 64]))
        nq = int(rng.choice(batches))
        n = int(np.exp(rng.uniform(np.log(500), np.log(200000))))
        if nq * n * d > 4e9:
            continue
        k = int(min(n, rng.choice([1, 5, 10, 50, 100, 256])))
        out.append((nq, n, d, k))
    return out


@pytest.mark.parametrize("nq,n,d,k", _random_fused_cases())
def test_fused_random_shapes_match_oracle(eng, nq, n, d, k):
    say(f"fused random nq={nq} n={n} d={d} k={k}")
    x, q = make(n, d, nq, seed=nq * 104729 + n + d + k)
    v, i, _ = run_fused(eng, q, x, k)
    oracle.check_exact(q.numpy(), x.numpy(), k, v, i)


@pytest.mark.parametrize("n,d,b,k", [(5000, 384, 8, 10), (20000, 768, 64, 100)])
def test_twopass_and_torch_paths(eng, n, d, b, k):
    say(f"twopass/torch n={n} d={d} b={b} k={k}")
    x, q = make(n, d, b, seed=3)
    index = Index(x.cuda(), metric="ip")
    for method in ("twopass", "torch"):
        v, i = index.search(q.cuda(), k, method=method)
        oracle.check_exact(q, x, k, v, i, tol=2e-3)


def test_cosine_metric_unnormalised_input(eng):
    say("cosine unnormalised")
    x, q = make(8000, 384, 16, seed=7, normal=False)
    x = x * torch.rand(x.shape[0], 1).half() * 4
    index = Index(x.cuda(), metric="cosine")
    v, i = index.search(q.cuda(), 10)
    xn = x.float() / x.float().norm(dim=1, keepdim=True)
    qn = q.float() / q.float().norm(dim=1, keepdim=True)
    ref_v, _ = torch.topk(qn @ xn.T, 10, dim=1)
    assert torch.allclose(v.cpu(), ref_v, atol=3e-3)
    qq = index._prep_queries(q.cuda())[:, :index.dim]
    oracle.check_exact(qq, index.embeddings, 10, v, i)


def test_raw_ip_large_values(eng):
    say("raw ip large values")
    x, q = make(10000, 256, 9, seed=11, normal=False)
    index = Index(x.cuda(), metric="ip")
    v, i = index.search(q.cuda(), 50, method="fused")
    oracle.check_exact(q, x, 50, v, i)


def test_one_dim_query_and_large_k_fallback(eng):
    say("1-D query, k=400 fallback")
    x, q = make(5000, 128, 1, seed=2)
    index = Index(x.cuda(), metric="ip")
    v, i = index.search(q[0].cuda(), 5)
    assert v.shape == (1, 5)
    oracle.check_exact(q, x, 5, v, i)
    v, i = index.search(q.cuda(), 400)
    assert i.shape == (1, 400)


def test_fused_plan_overrides(eng):
    say("plan overrides")
    x, q = make(40000, 384, 50, seed=4)
    index = Index(x.cuda(), metric="ip")
    qq = index._prep_queries(q.cuda())
    base_v, base_i = index.search(q.cuda(), 10, method="fused")
    for bq, chunks in [(16, 1), (32, 7), (64, 1000), (128, 3), (256, 0)]:
        v, i, plan = eng.fused_topk(qq, index._x, 10, bq, chunks)
        assert plan.tolist()[0] == bq
        assert torch.allclose(v, base_v, atol=1e-5)
        assert torch.equal(i.long(), base_i)


@pytest.mark.parametrize("k,bq", [(100, 64), (256, 32), (200, 16), (40, 64)])
def test_fused_large_state_configs(eng, k, bq):
    say(f"large state k={k} bq={bq}")
    x, q = make(30000, 384, 70, seed=k + bq)
    index = Index(x.cuda(), metric="ip")
    qq = index._prep_queries(q.cuda())
    for chunks in (1, 5, 0):
        v, i, plan = eng.fused_topk(qq, index._x, k, bq, chunks)
        assert plan.tolist()[0] == bq
        oracle.check_exact(q, x, k, v, i.long())


def test_reference_error_behaviour(eng):
    say("errors")
    x, q = make(200, 64, 3, seed=1)
    xd, qd = x.cuda(), q.cuda()
    with pytest.raises(RuntimeError, match="1 <= k <= 256"):
        eng.fused_topk(qd, xd, 257)
    with pytest.raises(RuntimeError, match="corpus size"):
        eng.fused_topk(qd, xd[:5], 6)
    with pytest.raises(RuntimeError, match="bq must be"):
        eng.fused_topk(qd, xd, 10, 48)
    with pytest.raises(RuntimeError, match=r"bq \* ceil\(k/32\)"):
        eng.fused_topk(qd, xd, 200, 64)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        eng.fused_topk(qd[:, :32].contiguous(), xd[:, :32].contiguous(), 3)
    with pytest.raises(RuntimeError, match="float16"):
        eng.fused_topk(qd.float(), xd, 3)
    with pytest.raises(RuntimeError, match="contiguous"):
        eng.scores(qd, torch.cat([xd, xd], 1)[:, :64])


# --------------------------------------------------------------------------- engine paths


@pytest.mark.parametrize("d", [64, 384, 768, 1536])
@pytest.mark.parametrize("k", [1, 10, 100])
def test_gemv_path_matches_oracle_and_scan(eng, d, k):
    say(f"gemv d={d} k={k}")
    x, q = make(30011, d, 1, seed=d + k)
    v, i, plan = run_fused(eng, q, x, k)
    assert plan[0] == 1  # the batch-1 GEMV path ran
    oracle.check_exact(q, x, k, v, i)
    v2, i2, plan2 = run_fused(eng, q, x, k, flags=_ext.FLAG_NO_GEMV)
    assert plan2[0] == 16
    np.testing.assert_allclose(v, v2, rtol=0, atol=1e-5)


@pytest.mark.parametrize("flags", [0, _ext.FLAG_NO_PREPASS, _ext.FLAG_FORCE_PREPASS])
# (100000, 384, 32, 10) and the three after it sample up to 64 tiles, one maximum
# per (query, sampling workgroup), and the scan finds each query's threshold
# itself (one query group of <= 32); the last samples every tile of its corpus.
@pytest.mark.parametrize("n,d,b,k", [(60000, 384, 256, 10), (60000, 768, 200, 100), (9000, 256, 33, 64),
                                     (100000, 384, 32, 10), (40000, 384, 13, 32), (20000, 768, 5, 16),
                                     (3000, 128, 20, 5)])
def test_prepass_does_not_change_results(eng, flags, n, d, b, k):
    say(f"prepass flags={flags} n={n} d={d} b={b} k={k}")
    x, q = make(n, d, b, seed=n + b)
    v, i, _ = run_fused(eng, q, x, k, flags=flags)
    oracle.check_exact(q, x, k, v, i)
    v0, i0, _ = run_fused(eng, q, x, k, flags=_ext.FLAG_NO_PREPASS)
    np.testing.assert_array_equal(v, v0)
    np.testing.assert_array_equal(i, i0)


# (32, 100000, 10): the 4-wave kernel, 196 scanning + 8 threshold workgroups;
# (256, 100000, 100): the 8-wave kernel, 224 + 32, with near-duplicate rows;
# (256, 60013, 50): fewer chunks (4 -> 5 tiles each) to fit the threshold
# workgroups, a batch short of a multiple of the waves and a partial last tile;
# (256, 6000, 10): units barely above 2k.
@pytest.mark.parametrize("nq,n,k,ties", [(32, 100000, 10, False), (256, 100000, 100, True), (64, 60000, 10, False),
                                         (128, 80000, 32, False), (250, 60013, 50, False), (17, 30011, 5, False),
                                         (256, 6000, 10, False)])
def test_fused_thresholds_in_the_scan_match_the_threshold_launch(eng, nq, n, k, ties):
    """The fp16 scan at width 384 with one query group samples itself: every
    workgroup publishes its first tile's per-lane maxima as units, the grid's
    extra workgroups take each query's threshold from them (one query per
    wave), and every workgroup filters with it.  Bitwise the results of the
    separate sampling pass and threshold launch (FLAG_TAU_LAUNCH) and of no
    sampling at all, and the oracle's."""
    say(f"fp16 thresholds in the scan nq={nq} n={n} k={k} ties={ties}")
    x, q = make(n, 384, nq, seed=n + nq + k)
    if ties:
        synthetic.inject_near_ties(x, seed=7)
    v, i, plan = run_fused(eng, q, x, k)
    vl, il, planl = run_fused(eng, q, x, k, flags=_ext.FLAG_TAU_LAUNCH)
    vn, i_n, _ = run_fused(eng, q, x, k, flags=_ext.FLAG_NO_PREPASS)
    assert plan[0] == planl[0]
    np.testing.assert_array_equal(v, vl)
    np.testing.assert_array_equal(i, il)
    np.testing.assert_array_equal(v, vn)
    np.testing.assert_array_equal(i, i_n)
    sub = slice(0, 16)
    oracle.check_exact(q[sub], x, k, v[sub], i[sub])


@pytest.mark.parametrize("nq,n,k", [(32, 100000, 10), (256, 100000, 100)])
def test_fused_in_scan_waits_that_give_up_stay_exact(eng, nq, n, k):
    """The fp16 scan's waits for units and thresholds are bounded.
    CVS_FLAG_TAU_NOWAIT makes every wait not satisfied at once give up (units
    left out, thresholds -inf, lists compacted as they fill): the results stay
    bitwise those of the default search."""
    say(f"fp16 in-scan waits that give up nq={nq} n={n} k={k}")
    x, q = make(n, 384, nq, seed=n + k + 9)
    v, i, _ = run_fused(eng, q, x, k)
    vn, i_n, _ = run_fused(eng, q, x, k, flags=_ext.FLAG_TAU_NOWAIT)
    np.testing.assert_array_equal(v, vn)
    np.testing.assert_array_equal(i, i_n)


@pytest.mark.parametrize("n,d,b,k", [(100, 384, 5, 28), (65, 384, 3, 20), (65, 128, 3, 20), (100, 768, 5, 28),
                                     (130, 256, 40, 60), (70, 384, 200, 40)])
def test_forced_prepass_with_fewer_finite_units_than_k(eng, n, d, b, k):
    """A forced sampling pass over a corpus whose last tile is mostly past n:
    the sampled units outnumber k, but fewer than k of them hold a row (the
    rest are -inf), so the k-th largest maximum is -inf.  The truncated bit
    search of the threshold must then give -inf (every row a candidate), not
    a threshold no score reaches."""
    say(f"forced prepass, few finite units n={n} d={d} b={b} k={k}")
    x, q = make(n, d, b, seed=n + k)
    v, i, _ = run_fused(eng, q, x, k, flags=_ext.FLAG_FORCE_PREPASS)
    oracle.check_exact(q, x, k, v, i)
    v0, i0, _ = run_fused(eng, q, x, k, flags=_ext.FLAG_NO_PREPASS)
    np.testing.assert_array_equal(v, v0)
    np.testing.assert_array_equal(i, i0)
    qd = pad64(q).cuda().contiguous()
    xd = pad64(x).cuda().contiguous()
    v8, i8, _ = eng.q8_topk(qd, xd, eng.q8_build(xd), k, flags=_ext.FLAG_FORCE_PREPASS)
    torch.cuda.synchronize()
    v8, i8 = v8.cpu().numpy(), i8.cpu().numpy().astype(np.int64)
    np.testing.assert_allclose(v8, v, rtol=0, atol=2e-6)
    same = i8 == i
    assert same.all() or np.abs(v8 - v)[~same].max() < 2e-6


@pytest.mark.parametrize("n,d,b,k", [(100000, 384, 32, 10), (20000, 384, 13, 16), (5000, 256, 2, 1),
                                     (3000, 128, 32, 16), (129, 384, 20, 16), (60000, 320, 32, 7)])
def test_register_topk_scan_matches_the_sampled_threshold(eng, n, d, b, k):
    """The running top-k in registers (FLAG_REGISTER_TOPK: no sampling pass,
    each lane's k best kept in VGPRs, the workgroup's k-th best shared through
    LDS): the oracle's results, bitwise those of the default path."""
    say(f"register top-k n={n} d={d} b={b} k={k}")
    x, q = make(n, d, b, seed=n + b + k)
    v, i, _ = run_fused(eng, q, x, k, flags=_ext.FLAG_REGISTER_TOPK)
    oracle.check_exact(q, x, k, v, i)
    v0, i0, _ = run_fused(eng, q, x, k)
    np.testing.assert_array_equal(v, v0)
    np.testing.assert_array_equal(i, i0)


def test_register_topk_scan_with_exact_duplicates(eng):
    """Bit-identical rows across lanes and workgroups: ties come out in id order."""
    say("register top-k, duplicates")
    x, q = make(30000, 384, 24, seed=77)
    src = torch.arange(0, 30000, 97)
    x[src + 1] = x[src]  # pairs of equal rows
    x[src[:50] + 2] = x[src[:50]]
    v, i, _ = run_fused(eng, q, x, 16, flags=_ext.FLAG_REGISTER_TOPK)
    v0, i0, _ = run_fused(eng, q, x, 16)
    np.testing.assert_array_equal(v, v0)
    np.testing.assert_array_equal(i, i0)
    oracle.check_exact(q, x, 16, v, i)


@pytest.mark.parametrize("k", [10, 100])
def test_two_group_sampling_on_paired_xcds(eng, k):
    """d = 768 at b = 256 runs two 128-query groups; with 128 sampling
    workgroups per group (a multiple of 8) the sampling pass maps both groups
    of a chunk to one XCD, on the fp16 and the int8 path alike."""
    n, d, b = 200000, 768, 256
    say(f"paired sampling n={n} d={d} b={b} k={k}")
    x, q = make(n, d, b, seed=31 + k)
    v, i, plan = run_fused(eng, q, x, k)
    assert plan[0] == 128
    assert oracle.check_exact(q, x, k, v, i) >= 0.999
    qd = pad64(q).cuda().contiguous()
    xd = pad64(x).cuda().contiguous()
    v8, i8, _ = eng.q8_topk(qd, xd, eng.q8_build(xd), k)
    torch.cuda.synchronize()
    v8, i8 = v8.cpu().numpy(), i8.cpu().numpy().astype(np.int64)
    np.testing.assert_allclose(v8, v, rtol=0, atol=2e-6)
    same = i8 == i
    assert same.all() or np.abs(v8 - v)[~same].max() < 2e-6


@pytest.mark.parametrize("n,d,b,k", [(50000, 384, 256, 10), (70000, 768, 1, 10)])
def test_timed_and_marked_twins_match(eng, n, d, b, k):
    """The diagnostic entry points run the same launches as fused_topk: identical
    outputs, and stage times that account for the work (scan/GEMV > 0)."""
    say(f"timed/marked twins n={n} d={d} b={b} k={k}")
    x, q = make(n, d, b, seed=5)
    qd, xd = q.cuda(), x.cuda()
    v0, i0, p0 = eng.fused_topk(qd, xd, k)
    (v1, i1, p1), ms = eng.fused_topk_timed(qd, xd, k)
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
    v2, i2, p2 = eng.fused_topk_marked(qd, xd, k, marks)
    torch.cuda.synchronize()
    for v, i, p in ((v1, i1, p1), (v2, i2, p2)):
        assert torch.equal(v, v0) and torch.equal(i, i0) and p.tolist() == p0.tolist()
    ms2 = [marks[j].elapsed_time(marks[j + 1]) for j in range(4)]
    assert all(t >= 0 for t in ms + ms2) and ms[2] > 0 and ms2[2] > 0
    oracle.check_exact(q, x, k, v0.cpu().numpy(), i0.cpu().numpy().astype(np.int64))


@pytest.mark.parametrize("n,d,b,k", [(30000, 384, 64, 10), (50000, 768, 1, 25)])
def test_int64_ids_flag(eng, n, d, b, k):
    """CVS_FLAG_IDS_INT64 (what Index.search uses) writes the same ids as int64."""
    say(f"int64 ids n={n} d={d} b={b} k={k}")
    x, q = make(n, d, b, seed=9)
    qd, xd = q.cuda(), x.cuda()
    v32, i32, _ = eng.fused_topk(qd, xd, k)
    v64, i64, _ = eng.fused_topk(qd, xd, k, flags=_ext.FLAG_IDS_INT64)
    torch.cuda.synchronize()
    assert i32.dtype == torch.int32 and i64.dtype == torch.int64
    assert torch.equal(v32, v64) and torch.equal(i32.long(), i64)
    index = Index(xd, metric="ip", copy=False)
    vi, ii = index.search(qd, k)
    assert ii.dtype == torch.int64 and torch.equal(ii, i64) and torch.equal(vi, v64)


@pytest.mark.parametrize("b,k", [(1, 10), (1, 200), (64, 10), (256, 100), (16, 256)])
def test_compaction_under_ascending_scores(eng, b, k):
    """Rows ordered so that every tile beats all previous ones: without a
    pre-pass every score is a candidate and the lists must compact repeatedly."""
    say(f"compaction b={b} k={k}")
    d, n = 128, 12000
    g = torch.Generator().manual_seed(b * 1000 + k)
    q = torch.randn(b, d, generator=g)
    q = q / q.norm(dim=1, keepdim=True)
    base = q.mean(0, keepdim=True)
    base = base / base.norm()
    t = torch.linspace(0.0, 1.0, n)[:, None]
    noise = torch.randn(n, d, generator=g)
    x = t * base + (1 - t) * noise / noise.norm(dim=1, keepdim=True)
    x = (x / x.norm(dim=1, keepdim=True)).half()
    q = q.half()
    for flags in (_ext.FLAG_NO_PREPASS, 0):
        v, i, _ = run_fused(eng, q, x, k, flags=flags)
        oracle.check_exact(q, x, k, v, i)


def test_exact_duplicates_and_near_ties(eng):
    say("near ties")
    x = synthetic.unit_corpus(40000, 384, seed=5)
    synthetic.inject_near_ties(x, frac=0.05, sigma=1e-4, seed=3)
    q = torch.cat([x[:32], synthetic.unit_queries(32, 384, seed=9)])  # queries on duplicated rows too
    for k in (10, 100):
        v, i, _ = run_fused(eng, q, x, k)
        oracle.check_exact(q, x, k, v, i)
        ov, oi = oracle.topk(q, x, k)
        # the engine's scores are fp32 sums in another order: above the band of
        # the k-th score its ids are the oracle's, in the oracle's order except
        # among rows whose scores agree to 1e-5; exact ties come in id order
        oracle.check_order(v, i, ov, oi)
        for r in range(q.shape[0]):
            for j in range(k - 1):
                if v[r, j] == v[r, j + 1]:
                    assert i[r, j] < i[r, j + 1]


# --------------------------------------------------------------------------- full-size shapes


def _spread_queries(b: int, want: int = 64) -> np.ndarray:
    """Query indices for the parity check of a full-size batch: every query when
    b <= 256 and the oracle is cheap enough (the caller decides), else ``want``
    spread over every query group and wave of the scan (32 consecutive queries
    per wave) with a different lane column in each."""
    if b <= want:
        return np.arange(b)
    per = max(1, want // (b // 32))
    sel = [32 * w + (7 * j + 3 * w) % 32 for w in range(b // 32) for j in range(per)]
    return np.unique(np.asarray(sel))[:want]


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4", "C5"])
def test_baseline_configs_full_size(eng, name):
    """The five benchmark configs at full size, through Index.search (auto: the
    int8 pre-filter at C2-C4, the fp16 scan at C1/C5) and method="fused":
    every query at C1, C3 and C5 (the near-tie config), 64 queries spread over
    every query group, wave and lane column at C2 and C4; ids and scores at the
    oracle's bar, ids in the oracle's order above the near-tie band, and the
    int8 path's ids equal the fp16 path's except between scores within 2e-6."""
    n, d, b, k, ties = synthetic.CONFIGS[name]
    say(f"baseline config {name}: n={n} d={d} b={b} k={k}")
    x = synthetic.unit_corpus(n, d, seed=d, device="cuda")
    if ties:
        synthetic.inject_near_ties(x, seed=7)
    q = synthetic.unit_queries(b, d, seed=1, device="cuda")
    index = Index(x, metric="cosine", copy=False)
    qq = index._prep_queries(q)
    va, ia = index.search(q, k)
    vf, i_f = index.search(q, k, method="fused")
    torch.cuda.synchronize()
    for v, i in ((va, ia), (vf, i_f)):  # size-independent properties over every query
        assert bool((v[:, :-1] >= v[:, 1:]).all())
        ii = i.cpu()
        assert all(len(set(r)) == k for r in ii.tolist())
        assert int(ii.min()) >= 0 and int(ii.max()) < n
    # the two exact paths agree (they differ only in the fp32 sum order)
    va_, ia_, vf_, if_ = (t.cpu().numpy() for t in (va, ia, vf, i_f))
    np.testing.assert_allclose(va_, vf_, rtol=0, atol=2e-6)
    same = ia_ == if_
    assert same.all() or np.abs(va_ - vf_)[~same].max() < 2e-6
    sel = np.arange(b) if name in ("C1", "C3", "C5") else _spread_queries(b)
    say(f"  oracle on {len(sel)} of {b} queries")
    xc = index.embeddings.cpu()
    qc = qq[torch.from_numpy(sel).cuda(), :index.dim].cpu()
    full = oracle.scores(qc, xc)
    ov, oi = oracle.topk(qc, xc, k)
    for v, i in ((va_, ia_), (vf_, if_)):
        oracle.check_exact(qc, xc, k, v[sel], i[sel], full=full)
        oracle.check_order(v[sel], i[sel], ov, oi)
    del x, index, full
    torch.cuda.empty_cache()


# --------------------------------------------------------------------------- row preparation


def within_one_ulp(a16, b16):
    """|a - b| <= one fp16 ulp at the larger of the two magnitudes (a quotient
    just past a rounding midpoint may round either way between fp32 sums)."""
    a, b = a16.astype(np.float32), b16.astype(np.float32)
    ulp = np.maximum(np.abs(np.spacing(a16)), np.abs(np.spacing(b16))).astype(np.float32)
    return np.abs(a - b) <= ulp


@pytest.mark.parametrize("n,d,width", [(1, 1, 64), (1000, 100, 128), (4097, 384, 384), (513, 768, 768),
                                       (77, 1536, 1536), (300, 700, 704)])
def test_prep_rows_matches_oracle(eng, n, d, width):
    """cvs_prep_rows (cosine normalisation + zero padding, index.py:27-41) within
    one fp16 ulp of the oracle; pass-through and padding bit-exact; in place."""
    say(f"prep_rows n={n} d={d} width={width}")
    g = torch.Generator().manual_seed(n + d)
    x = (torch.randn(n, d, generator=g) * torch.rand(n, 1, generator=g) * 10).half()
    x[0] = 0  # a zero row stays zero
    src = x.cuda()
    out = torch.full((n, width), float("nan"), dtype=torch.float16, device="cuda")
    eng.prep_rows(src, out, True)
    copy = torch.full((n, width), float("nan"), dtype=torch.float16, device="cuda")
    eng.prep_rows(src, copy, False)
    torch.cuda.synchronize()
    want = oracle.normalize_rows(x.numpy(), width=width)
    got = out.cpu().numpy()
    assert np.all(within_one_ulp(got, want))
    assert not got[:, d:].any() and not got[0].any()
    c = copy.cpu().numpy()
    np.testing.assert_array_equal(c[:, :d], x.numpy())
    assert not c[:, d:].any()
    if width == d:  # in place
        inplace = x.cuda()
        eng.prep_rows(inplace, inplace, True)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(inplace.cpu().numpy(), got)


def test_prep_rows_errors(eng):
    x = torch.zeros(4, 64, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="destination width"):
        eng.prep_rows(x, torch.zeros(4, 32, dtype=torch.float16, device="cuda"), True)
    # any width is accepted now (rows wider than 1536 take the two-pass kernel);
    # a source stride shorter than the row is still refused, before any launch
    wide = torch.zeros(4, 2048, dtype=torch.float16, device="cuda")
    rc = eng.lib.cvs_prep_rows(wide.data_ptr(), wide.data_ptr(), 4, 2048, 1000, 2048, 1,
                               wide.device.index, None)
    assert rc != 0 and b"source row stride" in eng.lib.cvs_last_error()
    with pytest.raises(RuntimeError, match="fp16 CUDA"):
        eng.prep_rows(x.float(), x, True)


def test_cosine_index_uses_the_prep_kernel_and_stays_exact(eng):
    """Index(metric="cosine") normalises the corpus (in place, like the reference
    with copy=False) and each query batch with cvs_prep_rows; search stays exact
    against the stored rows, and a width that is not a multiple of 64 is padded."""
    say("cosine index prep")
    g = torch.Generator().manual_seed(21)
    x = (torch.randn(20000, 200, generator=g) * 3).half()
    q = (torch.randn(40, 200, generator=g) * 5).half()
    xd = x.cuda()
    index = Index(xd, metric="cosine", copy=False)
    assert index._x.shape == (20000, 256)
    want = oracle.normalize_rows(x.numpy())
    stored = index.embeddings.cpu().numpy()
    assert np.all(within_one_ulp(stored, want))
    np.testing.assert_array_equal(xd.cpu().numpy(), stored)  # caller's tensor normalised in place
    v, i = index.search(q.cuda(), 10)
    qn = index._prep_queries(q.cuda())
    assert qn.shape == (40, 256) and not qn[:, 200:].any()
    oracle.check_exact(qn[:, :200], index.embeddings, 10, v.cpu().numpy(), i.cpu().numpy())


# --------------------------------------------------------------------------- large k


@pytest.mark.parametrize("nq,n,k", [(3, 5000, 1), (7, 20000, 300), (2, 3000, 1024), (5, 1024, 1024),
                                    (2, 200000, 100), (1, 1 << 20, 1024)])
def test_topk_rows_matches_sorted_rows(eng, nq, n, k):
    """cvs_topk_rows equals a stable sort of each row (value desc, column asc),
    including exact ties (the matrix holds repeated values)."""
    say(f"topk_rows nq={nq} n={n} k={k}")
    g = torch.Generator().manual_seed(n + k)
    s = torch.randint(-500, 500, (nq, n), generator=g).float() / 64  # many exact ties
    v, i = eng.topk_rows(s.cuda(), k)
    v64, i64 = eng.topk_rows(s.cuda(), k, flags=_ext.FLAG_IDS_INT64)
    torch.cuda.synchronize()
    sn = s.numpy()
    order = np.lexsort((np.broadcast_to(np.arange(n), sn.shape), -sn), axis=1)[:, :k]
    np.testing.assert_array_equal(i.cpu().numpy(), order)
    np.testing.assert_array_equal(v.cpu().numpy(), np.take_along_axis(sn, order, axis=1))
    assert i64.dtype == torch.int64 and torch.equal(i64.cpu(), i.cpu().long()) and torch.equal(v64, v)


@pytest.mark.parametrize("nq,n,k", [(4, 30000, 10), (3, 9000, 200), (4, 50000, 64)])
def test_topk_rows_with_infinite_scores(eng, nq, n, k):
    """Rows holding -inf and +inf scores, one with fewer than k finite ones, go
    through the selects' histogram cuts (whose score span is then infinite):
    the result is still the stable sort, -inf ties in column order."""
    say(f"topk_rows infinite nq={nq} n={n} k={k}")
    g = torch.Generator().manual_seed(7 * n + k)
    s = torch.randint(-500, 500, (nq, n), generator=g).float() / 64
    s[0, ::3] = -float("inf")
    s[1, : n - k // 2] = -float("inf")  # only k/2 finite scores
    s[2, ::1000] = float("inf")
    s[3 % nq, 5::7] = -float("inf")
    v, i = eng.topk_rows(s.cuda(), k)
    torch.cuda.synchronize()
    sn = s.numpy()
    order = np.lexsort((np.broadcast_to(np.arange(n), sn.shape), -sn), axis=1)[:, :k]
    np.testing.assert_array_equal(i.cpu().numpy(), order)
    np.testing.assert_array_equal(v.cpu().numpy(), np.take_along_axis(sn, order, axis=1))


def test_topk_rows_errors(eng):
    s = torch.zeros(2, 100, device="cuda")
    with pytest.raises(RuntimeError, match="1 <= k <= 1024"):
        eng.topk_rows(s, 1025)
    with pytest.raises(RuntimeError, match="must not exceed"):
        eng.topk_rows(s, 101)
    with pytest.raises(RuntimeError, match="float32"):
        eng.topk_rows(s.half(), 5)


@pytest.mark.parametrize("b,k", [(5, 300), (40, 1024), (1, 700)])
def test_large_k_search_is_exact(eng, b, k):
    """Index.search with 256 < k <= 1024 runs the score kernel + row top-k on the
    GPU (the reference falls back to torch fp16 scores) and is exact."""
    say(f"large-k search b={b} k={k}")
    x, q = make(20000, 128, b, seed=k)
    index = Index(x.cuda(), metric="ip")
    v, i = index.search(q.cuda(), k)
    assert v.dtype == torch.float32 and i.dtype == torch.int64 and v.shape == (b, k)
    oracle.check_exact(q, x, k, v.cpu().numpy(), i.cpu().numpy())


# --------------------------------------------------------------------------- int8 pre-filter


@pytest.mark.gpu
@pytest.mark.parametrize("n,d", [(1000, 384), (130, 320), (4097, 768), (64, 1536), (70, 64)])
def test_q8_build_matches_oracle(eng, n, d):
    say(f"q8 build n={n} d={d}")
    rng = np.random.default_rng(n + d)
    x = (rng.standard_normal((n, d)) * rng.uniform(0.01, 2, (n, 1))).astype(np.float16)
    x[n // 3:n // 3 + min(70, n // 2)] = x[5]  # equal maxima, across a block boundary: stable order
    xd = pad64(torch.from_numpy(x)).cuda().contiguous()
    xq = eng.q8_build(xd)
    torch.cuda.synchronize()
    ref_q, ref_m, ref_p = oracle.q8_companion(xd.cpu().numpy())
    raw = xq.cpu().numpy()
    body = raw[:ref_q.size].view(np.int8).reshape(ref_q.shape)
    assert np.array_equal(body, ref_q)
    nblk = ref_m.shape[0]
    off = -(-ref_q.size // 256) * 256
    meta = raw[off:off + 16 * nblk].view(np.float32).reshape(nblk, 4)
    assert np.array_equal(meta[:, 0].astype(np.float64), ref_m[:, 0])
    for j in (1, 2):  # norms rounded up, by less than 0.2%
        assert (meta[:, j] >= ref_m[:, j]).all()
        assert (meta[:, j] <= ref_m[:, j] * 1.002 + 1e-30).all()
    xmax = raw[off + 16 * nblk:off + 16 * nblk + 4].view(np.float32)[0]
    assert xmax == meta[:, 2].max()
    off_perm = -(-(off + 16 * nblk + 16) // 256) * 256
    perm = raw[off_perm:off_perm + 4 * ref_p.size].view(np.int32)
    assert np.array_equal(perm, ref_p) and raw.size == off_perm + 4 * ref_p.size


Q8_CASES = [(1, 30000, 384, 10), (7, 20000, 320, 5), (33, 25000, 384, 64), (65, 30000, 512, 10),
            (129, 20000, 768, 100), (256, 40000, 384, 10), (300, 20000, 1024, 256), (40, 20000, 1536, 1),
            # 8-wave int8 kernels with a sampled threshold and a partial last tile
            # (the int8 sampling pass, one unit per workgroup row split and lane group)
            (256, 300001, 384, 10), (200, 262193, 768, 16), (256, 200003, 768, 100),
            # the 384-byte-row scan (batches above 128): a ragged last query group, d < 384
            (129, 70001, 320, 7), (255, 65536, 384, 33),
            # batch 1: the int8 GEMV sampling pass, whole-block units and 8 per block
            (1, 200003, 768, 3), (1, 100000, 1536, 256), (1, 64000, 384, 100)]


@pytest.mark.gpu
@pytest.mark.parametrize("nq,n,d,k", Q8_CASES)
def test_q8_topk_matches_fused(eng, nq, n, d, k):
    say(f"q8 topk nq={nq} n={n} d={d} k={k}")
    x, q = make(n, d, nq, seed=n + k)
    qd = pad64(q).cuda().contiguous()
    xd = pad64(x).cuda().contiguous()
    xq = eng.q8_build(xd)
    v8, i8, plan8 = eng.q8_topk(qd, xd, xq, k)
    v, i, _ = eng.fused_topk(qd, xd, k)
    torch.cuda.synchronize()
    v8, i8, v, i = v8.cpu().numpy(), i8.cpu().numpy().astype(np.int64), v.cpu().numpy(), i.cpu().numpy()
    assert oracle.check_exact(q.numpy(), x.numpy(), k, v8, i8) >= 0.99
    # same rows as the fused path; scores agree to fp32 rounding of the sum order
    np.testing.assert_allclose(v8, v, rtol=0, atol=2e-6)
    same = (i8 == i)
    assert same.mean() > 0.999 or np.abs(v8 - v)[~same].max() < 2e-6


def _random_q8_cases(count=16, seed=20261202):
    """Seeded random (nq, n, d, k): widths 64-1536, batches 1-300 (the batch-1
    GEMV, the 4- and 8-wave scans, the 384-byte-row scan), corpora with partial
    last tiles, k 1-256; nq * n * d bounded so the oracle check takes seconds."""
    rng = np.random.default_rng(seed)
    widths = [64, 128, 192, 256, 320, 384, 448, 512, 640, 768, 896, 1024, 1536]
    batches = [1, 1, 2, 5, 17, 64, 100, 129, 200, 256, 300]
    out = []
    while len(out) < count:
        d = int(rng.choice(widths))
        nq = int(rng.choice(batches))
        n = int(np.exp(rng.uniform(np.log(2000), np.log(250000))))  # log-uniform
        if nq * n * d > 4e9:
            continue
        k = int(min(n, rng.choice([1, 3, 10, 32, 64, 100, 200, 256])))
        out.append((nq, n, d, k))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("nq,n,d,k", _random_q8_cases())
def test_q8_random_shapes_match_fused_and_oracle(eng, nq, n, d, k):
    say(f"q8 random nq={nq} n={n} d={d} k={k}")
    x, q = make(n, d, nq, seed=nq * 7919 + n + d + k)
    qd = pad64(q).cuda().contiguous()
    xd = pad64(x).cuda().contiguous()
    xq = eng.q8_build(xd)
    v8, i8, _ = eng.q8_topk(qd, xd, xq, k)
    v, i, _ = eng.fused_topk(qd, xd, k)
    torch.cuda.synchronize()
    v8, i8, v, i = v8.cpu().numpy(), i8.cpu().numpy().astype(np.int64), v.cpu().numpy(), i.cpu().numpy()
    assert oracle.check_exact(q.numpy(), x.numpy(), k, v8, i8) >= 0.99
    np.testing.assert_allclose(v8, v, rtol=0, atol=2e-6)
    same = (i8 == i)
    assert same.mean() > 0.999 or np.abs(v8 - v)[~same].max() < 2e-6


@pytest.mark.gpu
def test_q8_overflowing_lists_are_rescanned(eng):
    """4000 copies of the best row: every copy passes the int8 bound, the
    candidate lists overflow, and the select rescans their ranges exactly."""
    say("q8 overflow")
    x, q = make(30000, 384, 3, seed=11)
    x[5000:9000] = q[0]
    x[20000:20050] = q[1]
    qd = pad64(q).cuda().contiguous()
    xd = pad64(x).cuda().contiguous()
    xq = eng.q8_build(xd)
    for k in (10, 200):
        v8, i8, _ = eng.q8_topk(qd, xd, xq, k)
        v, i, _ = eng.fused_topk(qd, xd, k)
        torch.cuda.synchronize()
        assert np.array_equal(i8.cpu().numpy(), i.cpu().numpy())
        np.testing.assert_allclose(v8.cpu().numpy(), v.cpu().numpy(), rtol=0, atol=2e-6)
        assert i8[0].cpu().tolist() == list(range(5000, 5000 + k))
        # (the exact-set recall is not asserted: with thousands of exact ties the
        # oracle's reference set is any k of them; check_exact's own rules apply)
        oracle.check_exact(q.numpy(), x.numpy(), k, v8.cpu().numpy(), i8.cpu().numpy())
        # batch 1 runs the int8 GEMV, whose per-wave lists overflow the same way
        v1, i1, plan1 = eng.q8_topk(qd[:1].contiguous(), xd, xq, k)
        assert plan1[0].item() == 1
        assert i1[0].cpu().tolist() == list(range(5000, 5000 + k))
        np.testing.assert_allclose(v1.cpu().numpy(), v8[:1].cpu().numpy(), rtol=0, atol=2e-6)


@pytest.mark.gpu
def test_q8_overflow_in_the_batch_scan(eng):
    """The 384-byte-row int8 scan of batches above 128 (a ragged group of 200
    queries): 3000 copies of query 0 and 40 of query 150 overflow those
    queries' lists, the select rescans the overflowed chunks exactly, and every
    other query is unaffected."""
    say("q8 overflow, batch scan")
    x, q = make(70001, 384, 200, seed=23)
    x[10000:13000] = q[0]
    x[50000:50040] = q[150]
    qd = pad64(q).cuda().contiguous()
    xd = pad64(x).cuda().contiguous()
    xq = eng.q8_build(xd)
    for k in (10, 64):
        v8, i8, plan = eng.q8_topk(qd, xd, xq, k)
        v, i, _ = eng.fused_topk(qd, xd, k)
        torch.cuda.synchronize()
        assert plan[0].item() == 256
        assert i8[0].cpu().tolist() == list(range(10000, 10000 + k))
        assert set(i8[150, :min(k, 40)].cpu().tolist()) == set(range(50000, 50000 + min(k, 40)))
        np.testing.assert_allclose(v8.cpu().numpy(), v.cpu().numpy(), rtol=0, atol=2e-6)
        same = (i8 == i).cpu().numpy()
        assert same.all() or np.abs((v8 - v).cpu().numpy())[~same].max() < 2e-6
        oracle.check_exact(q.numpy(), x.numpy(), k, v8.cpu().numpy(), i8.cpu().numpy().astype(np.int64))


@pytest.mark.gpu
@pytest.mark.parametrize("nq,k", [(1, 10), (64, 100), (160, 10), (160, 100)])
def test_q8_loose_bounds_reorder_candidates(eng, nq, k):
    """A block holding a very long row gets a coarse int8 scale, so its other
    rows carry score bounds near 1 while their exact scores are ordinary (the
    companion orders rows by their largest magnitude: the five long rows share
    the last block with the 59 ordinary rows of largest magnitude): the k
    candidates of largest bound, which the select rescores first, are not the
    top k, and the exact result has to come from the remaining candidates.
    Batches below 128 rescore every candidate before the select; from 128 on
    the select rescores the k of largest bound first, then only the rest that
    can still enter."""
    say(f"q8 loose bounds nq={nq} k={k}")
    x, q = make(40000, 384, nq, seed=17 + nq + k)
    for blk in (10, 150, 300, 450, 600):
        x[blk * 64] = 0
        x[blk * 64, blk % 384] = 30.0
    qd = pad64(q).cuda().contiguous()
    xd = pad64(x).cuda().contiguous()
    xq = eng.q8_build(xd)
    v8, i8, _ = eng.q8_topk(qd, xd, xq, k)
    v, i, _ = eng.fused_topk(qd, xd, k)
    torch.cuda.synchronize()
    v8, i8, v, i = v8.cpu().numpy(), i8.cpu().numpy().astype(np.int64), v.cpu().numpy(), i.cpu().numpy()
    # a missed row would open a gap in the sorted scores; ids may differ only
    # between rows whose fp32 scores agree to the rounding of the sum order
    np.testing.assert_allclose(v8, v, rtol=0, atol=2e-6)
    same = i8 == i
    say(f"  id mismatches {int((~same).sum())}")
    assert same.all() or np.abs(v8 - v)[~same].max() < 2e-6
    assert oracle.check_exact(q.numpy(), x.numpy(), k, v8, i8) >= 0.99
    # the loose block's ordinary rows are not what the search returns
    order = oracle.q8_row_order(pad64(x).numpy())
    spikes = {blk * 64 for blk in (10, 150, 300, 450, 600)}
    assert set(order[-5:].tolist()) == spikes
    loose = set(order[-64:-5].tolist())
    assert np.isin(i8, list(loose)).mean() < 0.2


@pytest.mark.gpu
@pytest.mark.parametrize("k", [10, 100])
def test_q8_equal_bounds_fall_back_to_the_exact_cut(eng, k):
    """Six 64-row runs of copies of one row close to query 0, far apart in the
    corpus; its largest magnitude (0.9) exceeds every other row's, so the
    companion's row order puts the 384 copies into its last six blocks, with
    equal block metadata: 384 candidates in ordinary lists (none overflows)
    share one score bound, so the select's histogram cut cannot isolate k of
    them and takes the exact cut; the result is the k copies of smallest id."""
    say(f"q8 equal bounds k={k}")
    x, q = make(40000, 384, 160, seed=23 + k)
    row = q[0].clone()
    j = int(row.abs().argmax())
    row[j] = 0.9 if row[j] > 0 else -0.9
    assert float(x.abs().max()) < 0.9
    blocks = (20, 140, 260, 380, 500, 620)
    for blk in blocks:
        x[blk * 64:(blk + 1) * 64] = row
    qd = pad64(q).cuda().contiguous()
    xd = pad64(x).cuda().contiguous()
    xq = eng.q8_build(xd)
    v8, i8, _ = eng.q8_topk(qd, xd, xq, k)
    v, i, _ = eng.fused_topk(qd, xd, k)
    torch.cuda.synchronize()
    v8, i8, v, i = v8.cpu().numpy(), i8.cpu().numpy().astype(np.int64), v.cpu().numpy(), i.cpu().numpy()
    copies = [blk * 64 + r for blk in blocks for r in range(64)]
    assert i8[0].tolist() == copies[:k]
    np.testing.assert_allclose(v8, v, rtol=0, atol=2e-6)
    same = i8 == i
    assert same.all() or np.abs(v8 - v)[~same].max() < 2e-6
    oracle.check_exact(q.numpy(), x.numpy(), k, v8, i8)


@pytest.mark.gpu
@pytest.mark.parametrize("flags", [_ext.FLAG_NO_PREPASS, _ext.FLAG_FORCE_PREPASS, _ext.FLAG_IDS_INT64,
                                   _ext.FLAG_NO_GEMV])
def test_q8_flags(eng, flags):
    say(f"q8 flags={flags}")
    for nq in (1, 20):
        x, q = make(6000, 384, nq, seed=flags + nq)
        qd = pad64(q).cuda().contiguous()
        xd = pad64(x).cuda().contiguous()
        xq = eng.q8_build(xd)
        v8, i8, _ = eng.q8_topk(qd, xd, xq, 10, flags=flags)
        v, i, _ = eng.fused_topk(qd, xd, 10)
        torch.cuda.synchronize()
        assert i8.dtype == (torch.int64 if flags & _ext.FLAG_IDS_INT64 else torch.int32)
        assert np.array_equal(i8.cpu().numpy().astype(np.int64), i.cpu().numpy().astype(np.int64))
        np.testing.assert_allclose(v8.cpu().numpy(), v.cpu().numpy(), rtol=0, atol=2e-6)


@pytest.mark.gpu
def test_q8_errors(eng):
    x, q = make(1000, 384, 4, seed=3)
    qd = pad64(q).cuda().contiguous()
    xd = pad64(x).cuda().contiguous()
    xq = eng.q8_build(xd)
    with pytest.raises(RuntimeError, match="int8 corpus too small"):
        eng.q8_topk(qd, xd, xq[:1000], 10)
    with pytest.raises(RuntimeError, match="1 <= k <= 256"):
        eng.q8_topk(qd, xd, xq, 300)
    with pytest.raises(RuntimeError, match="k must not exceed"):
        eng.q8_topk(qd, xd[:5], eng.q8_build(xd[:5].contiguous()), 10)
    with pytest.raises(RuntimeError, match="xq must be"):
        eng.q8_topk(qd, xd, xq.float(), 10)
    assert eng.q8_corpus_bytes(1000, 384) == xq.numel()


@pytest.mark.gpu
def test_index_int8_method_matches_fused():
    say("index int8 method")
    x, q = make(50000, 300, 6, seed=21)
    idx = Index(x, metric="cosine", int8_prefilter=True)
    assert idx._xq is not None and idx._x.shape[1] == 320
    v8, i8 = idx.search(q, 10, method="int8")
    v, i = idx.search(q, 10, method="fused")
    assert i8.dtype == torch.int64
    assert torch.equal(i8, i)
    torch.testing.assert_close(v8, v, rtol=0, atol=2e-6)
    # batch 1 goes to the int8 path under "auto" once the companion exists
    assert idx._int8_wins(1, 10) and not idx._int8_wins(6, 10)
    va, ia = idx.search(q[:1], 10)
    assert torch.equal(ia, i[:1])
    # no companion: "auto" stays on the fp16 path, "int8" builds one on demand
    idx2 = Index(x, metric="cosine", int8_prefilter=False)
    assert idx2._xq is None and not idx2._int8_wins(1, 10)
    v2, i2 = idx2.search(q, 10, method="int8")
    assert torch.equal(i2, i) and idx2._xq is not None
    with pytest.raises(ValueError, match="int8 search supports k <= 256"):
        idx.search(q, 300, method="int8")


@pytest.mark.gpu
def test_index_auto_int8_at_size_is_exact():
    n = (1 << 19) + 123
    say(f"index auto int8 n={n}")
    x, q = make(n, 384, 8, seed=5)
    idx = Index(x, metric="ip")
    assert idx._xq is not None and idx._int8_wins(8, 10) and idx._int8_wins(8, 100)
    assert idx._int8_wins(256, 16) and idx._int8_wins(256, 100) and idx._int8_wins(64, 100)
    assert not idx._int8_wins(128, 100) and not idx._int8_wins(8, 300)
    v, i = idx.search(q, 10)
    vf, i_f = idx.search(q, 10, method="fused")
    assert torch.equal(i, i_f)
    assert oracle.check_exact(q.numpy(), x.numpy(), 10, v.cpu().numpy(), i.cpu().numpy()) >= 0.99


@pytest.mark.gpu
@pytest.mark.parametrize("nq,n,d,k", [(1, 1, 64, 1), (3, 70, 128, 5), (1000, 3000, 384, 20), (2, 5000, 768, 256),
                                      (5, 129, 1536, 129)])
def test_q8_edge_shapes(eng, nq, n, d, k):
    """Tiny corpora (no pre-pass: every list overflows and is rescanned), a
    partial last block, many query groups, k = 256 and k > rows per block."""
    say(f"q8 edge nq={nq} n={n} d={d} k={k}")
    x, q = make(n, d, nq, seed=nq + n)
    qd = pad64(q).cuda().contiguous()
    xd = pad64(x).cuda().contiguous()
    xq = eng.q8_build(xd)
    v8, i8, _ = eng.q8_topk(qd, xd, xq, k)
    v, i, _ = eng.fused_topk(qd, xd, k)
    torch.cuda.synchronize()
    v8, i8 = v8.cpu().numpy(), i8.cpu().numpy().astype(np.int64)
    assert oracle.check_exact(q.numpy(), x.numpy(), k, v8, i8) >= 0.99
    np.testing.assert_allclose(v8, v.cpu().numpy(), rtol=0, atol=2e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("nq,n,d,k", [(40, 5000, 384, 256), (200, 9000, 768, 200), (256, 70000, 384, 100)])
def test_q8_forced_sampling_with_few_units(eng, nq, n, d, k):
    """The int8 sampling pass forced onto small corpora (fewer sampled rows or
    units than k leave the threshold at -inf) and at k = 100 over 70k rows: the
    same results as without the pass and as the fused path."""
    say(f"q8 forced sampling nq={nq} n={n} d={d} k={k}")
    x, q = make(n, d, nq, seed=n + k + 1)
    qd = pad64(q).cuda().contiguous()
    xd = pad64(x).cuda().contiguous()
    xq = eng.q8_build(xd)
    v8, i8, _ = eng.q8_topk(qd, xd, xq, k, flags=_ext.FLAG_FORCE_PREPASS)
    v0, i0, _ = eng.q8_topk(qd, xd, xq, k, flags=_ext.FLAG_NO_PREPASS)
    v, i, _ = eng.fused_topk(qd, xd, k)
    torch.cuda.synchronize()
    assert torch.equal(i8, i0) and torch.equal(v8, v0)
    np.testing.assert_allclose(v8.cpu().numpy(), v.cpu().numpy(), rtol=0, atol=2e-6)
    same = (i8 == i).cpu().numpy()
    assert same.all() or np.abs((v8 - v).cpu().numpy())[~same].max() < 2e-6
    assert oracle.check_exact(q.numpy(), x.numpy(), k, v8.cpu().numpy(), i8.cpu().numpy().astype(np.int64)) >= 0.99


@pytest.mark.gpu
@pytest.mark.parametrize("nq,n,k,forced", [(256, 300000, 10, False), (200, 150000, 10, False), (150, 200000, 32, False),
                                           (256, 120000, 100, False), (300, 200000, 10, False), (256, 9000, 250, True),
                                           (137, 5000, 40, True)])
def test_q8_thresholds_in_the_scan_match_the_threshold_launch(eng, nq, n, k, forced):
    """The 384-byte int8 scan samples the first tiles of each chunk and
    computes each query's threshold itself (one query per 4 waves of a
    workgroup; units and thresholds published to the other workgroups through
    64-bit words): bitwise the same results as the sampling pass with its
    separate threshold launch (FLAG_TAU_LAUNCH), and the fused path's.  Covers
    one and two query groups, the batches whose candidates are rescored by a
    kernel of their own (fewer than 160 queries: it reads the thresholds the
    scan stored), and forced sampling over corpora with fewer sampled rows
    than k (threshold -inf)."""
    say(f"q8 thresholds in the scan nq={nq} n={n} k={k} forced={forced}")
    x, q = make(n, 384, nq, seed=n + nq + k)
    qd = q.cuda().contiguous()
    xd = x.cuda().contiguous()
    xq = eng.q8_build(xd)
    f = _ext.FLAG_FORCE_PREPASS if forced else 0
    v8, i8, _ = eng.q8_topk(qd, xd, xq, k, flags=f)
    vl, il, _ = eng.q8_topk(qd, xd, xq, k, flags=f | _ext.FLAG_TAU_LAUNCH)
    v, i, _ = eng.fused_topk(qd, xd, k)
    torch.cuda.synchronize()
    assert torch.equal(v8, vl) and torch.equal(i8, il)
    np.testing.assert_allclose(v8.cpu().numpy(), v.cpu().numpy(), rtol=0, atol=2e-6)
    same = (i8 == i).cpu().numpy()
    assert same.all() or np.abs((v8 - v).cpu().numpy())[~same].max() < 2e-6
    sub = slice(0, 16)  # (the CPU oracle on 16 queries; the rest are pinned to the fused path above)
    oracle.check_exact(q[sub].numpy(), x.numpy(), k, v8[sub].cpu().numpy(), i8[sub].cpu().numpy().astype(np.int64))


@pytest.mark.gpu
@pytest.mark.parametrize("n,k", [(150000, 10), (120000, 100)])
def test_q8_in_scan_waits_that_give_up_stay_exact(eng, n, k):
    """The 384-byte int8 scan's workgroups wait for each other's unit and
    threshold words with a bounded wait (a GPU shared with other work may not
    hold them all at once).  CVS_FLAG_TAU_NOWAIT makes every wait that is not
    satisfied at once give up: units left out, thresholds -inf, lists that
    overflow and are rescanned by the select.  The results stay bitwise those
    of the default search."""
    say(f"q8 in-scan waits that give up n={n} k={k}")
    x, q = make(n, 384, 256, seed=n + k + 5)
    qd = q.cuda().contiguous()
    xd = x.cuda().contiguous()
    xq = eng.q8_build(xd)
    v8, i8, _ = eng.q8_topk(qd, xd, xq, k)
    vn, i_n, _ = eng.q8_topk(qd, xd, xq, k, flags=_ext.FLAG_TAU_NOWAIT)
    torch.cuda.synchronize()
    assert torch.equal(v8, vn) and torch.equal(i8, i_n)
    sub = slice(0, 8)
    oracle.check_exact(q[sub].numpy(), x.numpy(), k, vn[sub].cpu().numpy(), i_n[sub].cpu().numpy().astype(np.int64))


@pytest.mark.gpu
def test_q8_zero_queries_and_rows(eng):
    """All-zero queries (scale 0) and all-zero corpus blocks: every score is 0 and
    ties order by id."""
    say("q8 zeros")
    x, q = make(3000, 384, 4, seed=9)
    x[64:256] = 0
    q[1] = 0
    qd = pad64(q).cuda().contiguous()
    xd = pad64(x).cuda().contiguous()
    xq = eng.q8_build(xd)
    v8, i8, _ = eng.q8_topk(qd, xd, xq, 10)
    v, i, _ = eng.fused_topk(qd, xd, 10)
    torch.cuda.synchronize()
    assert torch.equal(i8.cpu(), i.cpu())
    assert i8[1].cpu().tolist() == list(range(10)) and (v8[1] == 0).all()


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["fused", "int8", "gemv"])
def test_graph_capture_replays_match_eager(eng, path):
    """The search issues no memset, allocation or synchronisation, so a HIP graph
    captures it: every replay (with eager searches and syncs in between) returns
    exactly the eager result."""
    say(f"graph capture {path}")
    nq = 1 if path == "gemv" else 64
    x, q = make(40000, 384, nq, seed=17)
    qd = q.cuda().contiguous()
    xd = x.cuda().contiguous()
    xq = eng.q8_build(xd) if path == "int8" else None
    fn = (lambda: eng.q8_topk(qd, xd, xq, 10)) if path == "int8" else (lambda: eng.fused_topk(qd, xd, 10))
    ref = fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    for _ in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[0], ref[0]) and torch.equal(out[1], ref[1])
        again = fn()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(again[1], ref[1])


@pytest.mark.gpu
def test_concurrent_searches_on_threads_and_streams(eng):
    """Re-entrant entry points: four threads, each on its own stream, search
    different query batches at once; results equal the sequential ones."""
    import threading

    say("concurrent streams")
    x, _ = make(30000, 384, 1, seed=23)
    xd = x.cuda().contiguous()
    xq = eng.q8_build(xd)
    batches = [make(1, 384, nq, seed=100 + t)[1].cuda().contiguous() for t, nq in enumerate((1, 40, 130, 256))]
    expect = [(eng.q8_topk(b, xd, xq, 16)[1].cpu(), eng.fused_topk(b, xd, 16)[1].cpu()) for b in batches]
    torch.cuda.synchronize()
    results, errors = [None] * len(batches), []

    def work(t):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                got = []
                for _ in range(5):
                    got.append((eng.q8_topk(batches[t], xd, xq, 16)[1], eng.fused_topk(batches[t], xd, 16)[1]))
                s.synchronize()
            results[t] = [(a.cpu(), b.cpu()) for a, b in got]
        except Exception as exc:  # reported below
            errors.append(exc)

    threads = [threading.Thread(target=work, args=(t,)) for t in range(len(batches))]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    for t, res in enumerate(results):
        for a, b in res:
            assert torch.equal(a, expect[t][0]) and torch.equal(b, expect[t][1])


@pytest.mark.gpu
def test_int8_companion_follows_corpus_changes(eng):
    """With copy=False the index stores the caller's tensor (as the reference
    does); rows changed in place afterwards, through that tensor or through
    Index.embeddings, must not leave the int8 companion stale: "auto" and
    "int8" rebuild it and stay exact against the current rows, also when
    several threads search at once after a change."""
    import threading

    n, d = (1 << 18) + 77, 384
    say(f"int8 companion after corpus changes n={n}")
    x = synthetic.unit_corpus(n, d, seed=3, device="cuda")
    q = synthetic.unit_queries(8, d, seed=4, device="cuda")
    index = Index(x, metric="ip", copy=False)
    assert index._x.data_ptr() == x.data_ptr() and index._xq is not None
    assert index.int8_bytes == eng.q8_corpus_bytes(n, d)
    index.search(q, 10, method="int8")  # companion of the original rows in use
    x[123457] = q[0]          # through the caller's tensor
    index.embeddings[98765] = q[1]  # through the stored rows' view
    for method in ("auto", "int8"):
        nq = 1 if method == "auto" else 8  # batch 1: "auto" takes the int8 GEMV here
        v, i = index.search(q[:nq], 10, method=method)
        assert int(i[0, 0]) == 123457
        if nq > 1:
            assert int(i[1, 0]) == 98765
        oracle.check_exact(q[:nq].cpu(), x.cpu(), 10, v, i)
    x[5] = q[2]
    results, errors = [None] * 4, []

    def work(t):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                r = index.search(q, 10, method="int8")
                s.synchronize()
            results[t] = r
        except Exception as exc:  # reported below
            errors.append(exc)

    threads = [threading.Thread(target=work, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    for v, i in results:
        assert int(i[2, 0]) == 5
        oracle.check_exact(q.cpu(), x.cpu(), 10, v, i)


@pytest.mark.gpu
@pytest.mark.parametrize("n,d,b,k", [(100_000, 384, 32, 10), (200_000, 384, 256, 10), (100_000, 384, 256, 100)])
def test_searches_on_a_garbage_workspace(eng, n, d, b, k):
    """The workspace needs no initialisation: searches right after its memory
    held random bits (the caching allocator hands the same block back) are
    exact and repeat bit for bit, on the fp16 and int8 paths."""
    say(f"garbage workspace n={n} d={d} b={b} k={k}")
    x, q = make(n, d, b, seed=b + k)
    qd, xd = q.cuda(), x.cuda()
    xq = eng.q8_build(xd)
    _, ws16 = eng.plan(b, n, d, k, device=qd.device.index)
    _, ws8 = eng.q8_plan(b, n, d, k, device=qd.device.index)
    outs = []
    for _ in range(3):
        for nbytes in (ws16, ws8):
            junk = torch.randint(-2**62, 2**62, (max(nbytes, 256) // 8 + 1,), dtype=torch.int64, device="cuda")
            del junk
            outs.append(eng.fused_topk(qd, xd, k) if nbytes == ws16 else eng.q8_topk(qd, xd, xq, k))
    torch.cuda.synchronize()
    v0, i0, _ = outs[0]
    oracle.check_exact(q, x, k, v0.cpu().numpy(), i0.cpu().numpy().astype(np.int64))
    for v, i, _ in outs[1:]:
        np.testing.assert_allclose(v.cpu().numpy(), v0.cpu().numpy(), rtol=0, atol=2e-6)
        same = (i == i0).cpu().numpy()
        assert same.all() or np.abs((v - v0).cpu().numpy())[~same].max() < 2e-6
