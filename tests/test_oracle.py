"""Pins the CPU oracle before anything is compared against it (CPU only).

Each check is chosen so that a plausible oracle bug (wrong fp16 decoding, a
dropped term, a wrong tie order, an off-by-one in the heap, transposed
operands) fails at least one of them:

* fp16 decoding: exhaustive over all 65536 bit patterns vs numpy.
* golden vectors (tests/golden/*.npz): independent float64 brute force.
* closed forms: k=1 is the arg-max (first index on ties), k=n is a full sort,
  an identity corpus returns the query's own coordinates, duplicated rows tie
  and are ordered by id, a transposed-operand score matrix is detected.
* cross-checks against the numpy restatement of reference.py:18-34 and the
  reference's CPU baselines (torch matmul+topk, numpy argpartition).
* the acceptance rule (tests/test_search.py:21-44 + id parity) rejects planted
  mistakes.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = sorted((Path(__file__).parent / "golden").glob("*.npz"))


def unit(rng, m, d):
    a = rng.standard_normal((m, d)).astype(np.float32)
    return (a / np.linalg.norm(a, axis=1, keepdims=True)).astype(np.float16)


def test_half_decoding_exhaustive():
    L = oracle.lib()
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([L.cvs_oracle_half_to_float(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.parametrize("path", GOLDEN, ids=[p.stem for p in GOLDEN])
def test_oracle_matches_golden(path):
    z = np.load(path)
    k = int(z["k"])
    v, i = oracle.topk(z["q"], z["x"], k)
    np.testing.assert_allclose(v, z["scores"], rtol=0, atol=1e-6)
    # ids identical except where two candidate scores are within 1e-6 (float64 vs
    # double-accumulated-then-rounded scores may round differently there)
    for r in range(v.shape[0]):
        diff = np.nonzero(i[r] != z["ids"][r])[0]
        for j in diff:
            assert abs(float(z["scores"][r, j]) - float(v[r, j])) < 1e-6
            near = np.abs(z["scores"][r] - z["scores"][r, j]) < 1e-6
            assert near.sum() >= 2, f"{path.stem}: row {r} pos {j} differs without a tie"


def test_golden_fixture_properties():
    # the committed fixtures exercise what they claim to
    names = {p.stem for p in GOLDEN}
    assert {"k_one_n500_d128", "k_equals_n_n50_d64", "duplicates_n200_d32_k15",
            "near_ties_n1000_d384_k100", "raw_ip_n400_d96_k20", "random_n300_d64_b5_k10"} <= names
    z = np.load(GOLDEN[[p.stem for p in GOLDEN].index("duplicates_n200_d32_k15")])
    s = z["scores"]
    assert (s[:, :-1] == s[:, 1:]).any(), "duplicates fixture must contain exact ties"


def test_k1_is_argmax():
    rng = np.random.default_rng(1)
    x, q = unit(rng, 777, 64), unit(rng, 9, 64)
    full = q.astype(np.float64) @ x.astype(np.float64).T
    v, i = oracle.topk(q, x, 1)
    assert np.array_equal(i[:, 0], np.argmax(full, axis=1))


def test_k_equals_n_is_full_sort():
    rng = np.random.default_rng(2)
    x, q = unit(rng, 64, 128), unit(rng, 4, 128)
    full = q.astype(np.float64) @ x.astype(np.float64).T
    v, i = oracle.topk(q, x, 64)
    for r in range(4):
        assert sorted(i[r].tolist()) == list(range(64))
        assert np.all(np.diff(v[r]) <= 0)
        np.testing.assert_array_equal(i[r], np.lexsort((np.arange(64), -full[r])))


def test_identity_corpus_returns_query_coordinates():
    rng = np.random.default_rng(3)
    d = 64
    x = np.eye(d, dtype=np.float16)
    q = rng.standard_normal((5, d)).astype(np.float16)
    v, i = oracle.topk(q, x, d)
    for r in range(5):
        np.testing.assert_array_equal(v[r], np.sort(q[r].astype(np.float32))[::-1])
        np.testing.assert_array_equal(q[r, i[r]].astype(np.float32), v[r])


def test_duplicates_tie_by_smaller_id():
    rng = np.random.default_rng(4)
    x = unit(rng, 50, 64)
    x[[7, 19, 33]] = x[40]
    q = x[40:41].copy()
    v, i = oracle.topk(q, x, 4)
    assert i[0].tolist() == [7, 19, 33, 40]
    assert v[0, 0] == v[0, 1] == v[0, 2] == v[0, 3]


def test_scores_not_transposed():
    rng = np.random.default_rng(5)
    x, q = unit(rng, 40, 64), unit(rng, 3, 64)
    s = oracle.scores(q, x)
    assert s.shape == (3, 40)
    ref = q.astype(np.float64) @ x.astype(np.float64).T
    np.testing.assert_allclose(s, ref, rtol=0, atol=1e-6)


def test_restated_reference_and_cpu_baselines_agree():
    rng = np.random.default_rng(6)
    x, q = unit(rng, 5000, 384), unit(rng, 7, 384)
    v, i = oracle.topk(q, x, 25)
    ev, ei = oracle.exact_topk_fp32(q, x, 25, chunk=1024)
    np.testing.assert_allclose(ev, v, atol=1e-5)
    nv, ni = oracle.numpy_search(q.astype(np.float32), x.astype(np.float32), 25)
    np.testing.assert_allclose(nv, v, atol=1e-5)
    import torch

    tv, ti = oracle.torch_topk_cpu(torch.from_numpy(q).float(), torch.from_numpy(x).float(), 25)
    np.testing.assert_allclose(tv.numpy(), v, atol=1e-5)
    for got in (ei, ni, ti.numpy()):
        assert oracle.check_exact(q, x, 25, v, got) >= 0.99


def test_check_exact_accepts_oracle_and_rejects_planted_mistakes():
    rng = np.random.default_rng(7)
    x, q = unit(rng, 3000, 128), unit(rng, 6, 128)
    k = 20
    v, i = oracle.topk(q, x, k)
    assert oracle.check_exact(q, x, k, v, i) == 1.0

    full = oracle.scores(q, x)
    worst = np.argsort(full, axis=1)[:, :1]
    bad = i.copy()
    bad[:, 3] = worst[:, 0]
    with pytest.raises(oracle.ParityError):
        oracle.check_exact(q, x, k, v, bad)          # an id outside the top-k
    with pytest.raises(oracle.ParityError):
        oracle.check_exact(q, x, k, v + 0.01, i)     # scores off by 1e-2
    with pytest.raises(oracle.ParityError):
        oracle.check_exact(q, x, k, v[:, ::-1].copy(), i[:, ::-1].copy())  # unsorted
    dup = i.copy()
    dup[:, 1] = dup[:, 0]
    dv = v.copy()
    dv[:, 1] = dv[:, 0]
    with pytest.raises(oracle.ParityError):
        oracle.check_exact(q, x, k, dv, dup)         # duplicate ids
    with pytest.raises(oracle.ParityError):
        oracle.check_exact(q, x, k - 1, v[:, :k - 1], i[:, 1:])  # best id missing


def test_check_order_accepts_oracle_and_rejects_planted_mistakes():
    """check_order: the oracle's own output and reorderings among near-equal
    scores pass; two well-separated ids swapped, or a returned set that is right
    but misordered above the band, fail."""
    rng = np.random.default_rng(11)
    x, q = unit(rng, 4000, 96), unit(rng, 5, 96)
    x[100] = x[200] = x[300] = q[0]  # three exact duplicates: the top three of query 0
    k = 15
    v, i = oracle.topk(q, x, k)
    oracle.check_order(v, i, v, i)
    assert i[0, :3].tolist() == [100, 200, 300]
    tie = i.copy()
    tie[0, :3] = [300, 100, 200]  # any order among the equal scores
    oracle.check_order(v, tie, v, i)
    swapped = i.copy()
    gaps = np.diff(v[1])
    j = int(np.argmin(gaps))  # the largest gap between neighbours (scores descend)
    assert v[1, j] - v[1, j + 1] > 1e-5 and v[1, j + 1] > v[1, -1] + 1e-3
    swapped[1, [j, j + 1]] = swapped[1, [j + 1, j]]
    with pytest.raises(oracle.ParityError):
        oracle.check_order(v, swapped, v, i)
    wrong = i.copy()
    wrong[2, 0] = i[2, -1]  # a band id in first place instead of the best
    with pytest.raises(oracle.ParityError):
        oracle.check_order(v, wrong, v, i)


# --------------------------------------------------------------------------- row preparation


def test_normalize_rows_closed_forms():
    """Pins oracle.normalize_rows: unit rows are fixed points, a zero row stays
    zero (the 1e-12 clamp), power-of-two scalings normalise to the same row,
    padding columns are zero, and the pass-through copies bit-exactly."""
    e = np.zeros((3, 5), dtype=np.float16)
    e[0, 0] = 1
    e[1, :2] = [0.6, 0.8]           # |.| = 1 up to fp16 rounding of 0.6, 0.8
    got = oracle.normalize_rows(e, width=64)
    assert got.shape == (3, 64) and not got[:, 5:].any()
    assert got[0, 0] == 1 and not got[0, 1:].any()
    assert not got[2].any()         # zero row: divided by the clamp, stays 0
    np.testing.assert_allclose(got[1, :2].astype(np.float32), [0.6, 0.8], atol=1e-3)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((50, 100)).astype(np.float16)
    a = oracle.normalize_rows(x)
    b = oracle.normalize_rows((x.astype(np.float32) * 8).astype(np.float16))
    np.testing.assert_array_equal(a, b)
    norms = np.linalg.norm(a.astype(np.float64), axis=1)
    np.testing.assert_allclose(norms, 1.0, atol=2e-3)
    np.testing.assert_array_equal(oracle.normalize_rows(x, width=128, normalize=False)[:, :100], x)


def test_normalize_rows_agrees_with_the_torch_restatement():
    """The package's torch path (index.py:35-41 restated with torch ops) and the
    oracle agree within one fp16 ulp."""
    import torch

    from cuda_vector_search.index import _normalize_

    rng = np.random.default_rng(4)
    x = (rng.standard_normal((200, 384)) * rng.uniform(0.1, 10, (200, 1))).astype(np.float16)
    t = _normalize_(torch.from_numpy(x.copy())).numpy()
    o = oracle.normalize_rows(x)
    ulp = np.maximum(np.abs(np.spacing(o)), np.abs(np.spacing(t))).astype(np.float32)
    assert np.all(np.abs(t.astype(np.float32) - o.astype(np.float32)) <= ulp)


# --------------------------------------------------------------------------- int8 pre-filter format


def test_q8_quantisation_closed_forms():
    # block max 127 -> scale exactly 1: integers stay, halves round to even
    x = np.zeros((3, 64), dtype=np.float16)
    x[0, 0] = 127
    x[0, 1:7] = [2.5, 3.5, -2.5, -0.5, 126.5, 1.25]
    x[1, :] = -127                      # saturates exactly, zero residual
    xq, meta = oracle.q8_quantize_blocks(x)
    assert xq.shape == (64, 384) and xq.dtype == np.int8
    assert xq[0, :7].tolist() == [127, 2, 4, -2, 0, 126, 1]
    assert (xq[1, :64] == -127).all() and (xq[2] == 0).all() and (xq[3:] == 0).all()
    assert (xq[:, 64:] == 0).all()      # zero padding columns
    assert meta[0, 0] == 1.0
    # residual: row 0 keeps 0.5, 0.5, 0.5, 0.5, 0.5, 0.25 away from the grid
    assert np.isclose(meta[0, 1], np.sqrt(5 * 0.25 + 0.0625))
    assert meta[0, 2] == 127 * 8          # the largest row norm of the block (row 1)
    # an all-zero block has scale 0 and no residual
    z, zm = oracle.q8_quantize_blocks(np.zeros((10, 128), dtype=np.float16))
    assert (z == 0).all() and (zm == 0).all()
    # queries: one scale per row
    q = np.array([[127, 63.5, -1], [0.5, 0.25, 0]], dtype=np.float16)
    q = np.pad(q, ((0, 0), (0, 61)))
    qq, qm = oracle.q8_quantize_queries(q)
    assert qq[0, :3].tolist() == [127, 64, -1]   # 63.5 -> 64 (even)
    assert qq[1, :2].tolist() == [127, 64]        # scale 0.5/127: 0.25 -> 63.5 -> 64
    assert qm[0, 0] == 1.0 and np.isclose(qm[0, 2], 0.5)
    assert np.isclose(qm[1, 0], np.float32(np.float32(0.5) / np.float32(127)))


def test_q8_row_order_closed_forms():
    # planted row maxima: ascending order of max |x_r|, negatives by magnitude
    x = np.zeros((6, 64), dtype=np.float16)
    x[0, 3] = 5.0
    x[1, 0] = -0.25
    x[2, 7] = 2.0
    x[3, 1] = -9.0
    x[4, 2] = 0.5
    x[4, 5] = -0.75       # max |x| 0.75
    # row 5: all zero (max 0)
    assert oracle.q8_row_order(x).tolist() == [5, 1, 4, 2, 0, 3]
    # equal maxima keep the corpus order (stable), also among copies
    y = np.zeros((7, 64), dtype=np.float16)
    y[:, 0] = [3, 1, 3, -1, 2, 3, 1]
    assert oracle.q8_row_order(y).tolist() == [1, 3, 6, 4, 0, 2, 5]
    # NaNs are skipped; an all-NaN row counts as 0
    z = np.ones((3, 64), dtype=np.float16)
    z[0, 5] = np.nan
    z[1, :] = np.nan
    z[2, 9] = 4
    assert oracle.q8_row_order(z).tolist() == [1, 0, 2]


def test_q8_companion_layout_and_order_invariants():
    rng = np.random.default_rng(9)
    n, d = 300, 128
    x = (rng.standard_normal((n, d)) * rng.uniform(0.1, 3, (n, 1))).astype(np.float16)
    x[40:60] = x[10]      # equal maxima
    xq, meta, perm = oracle.q8_companion(x)
    rows = -(-n // 64) * 64
    assert perm.dtype == np.int32 and perm.shape == (rows,)
    assert sorted(perm[:n].tolist()) == list(range(n))            # a permutation
    assert perm[n:].tolist() == list(range(n, rows))              # padding maps to itself
    mx = np.abs(x.astype(np.float32)).max(axis=1)
    assert (np.diff(mx[perm[:n]]) >= 0).all()                     # ascending maxima
    same = [c for c in range(n) if mx[perm[c]] == mx[10]]
    assert perm[same].tolist() == sorted(perm[same].tolist())      # stable among equals
    # the companion's rows are the corpus rows in that order, block-quantised
    xq2, meta2 = oracle.q8_quantize_blocks(x[perm[:n]])
    assert np.array_equal(xq, xq2) and np.array_equal(meta, meta2)
    # ordered blocks share their scale with rows of nearly the same maximum:
    # every block's scale is at most that of the same rows in corpus order
    _, meta_c = oracle.q8_quantize_blocks(x)
    assert meta[:, 0].sum() < meta_c[:, 0].sum()


def test_q8_bound_holds_and_needs_both_terms():
    rng = np.random.default_rng(5)
    # random rows of mixed scales, including heavy-tailed ones
    x = (rng.standard_normal((512, 384)) * rng.uniform(0.01, 3, (512, 1))).astype(np.float16)
    x[::7, rng.integers(0, 384)] *= 40
    q = rng.standard_normal((9, 384)).astype(np.float16)
    A, B, S = oracle.q8_bound(q, x)
    assert (np.abs(S - A) <= B).all()
    # ... and over the blocks of the companion's row order, where it is tighter
    A2, B2, S2 = oracle.q8_bound(q, x, order=oracle.q8_row_order(x))
    assert np.array_equal(S2, S) and (np.abs(S2 - A2) <= B2).all()
    assert B2.mean() < B.mean()
    # a query that is exactly representable (integers, max 127: e = 0) and
    # aligned with a row's residual f: |S - A| = |q.f| reaches |q^||f|, so the
    # bound without its f-term (|e||x| = 0) fails
    xq, meta = oracle.q8_quantize_blocks(x)
    f = x[0].astype(np.float64) - meta[0, 0] * xq[0, :384].astype(np.float64)
    qa = np.rint(127 * f / np.abs(f).max()).astype(np.float16)[None, :]
    A, B, S = oracle.q8_bound(qa, x[:64])
    _, qm = oracle.q8_quantize_queries(qa)
    assert qm[0, 2] == 0.0 and (np.abs(S - A) <= B).all()
    assert abs(S[0, 0] - A[0, 0]) > 0.5 * B[0, 0]
    without_f = qm[0, 2] * np.sqrt((x[:64].astype(np.float64) ** 2).sum(axis=1))
    assert (np.abs(S - A)[0] > without_f).any()
    # a row that is exactly representable (f = 0) and aligned with a query's
    # residual e: the bound without its e-term (|q^||f| = 0) fails
    qb = rng.standard_normal((1, 384)).astype(np.float16)
    qq, qm = oracle.q8_quantize_queries(qb)
    e = qb[0].astype(np.float64) - qm[0, 0] * qq[0, :384].astype(np.float64)
    xb = np.rint(127 * e / np.abs(e).max()).astype(np.float16)[None, :]
    A, B, S = oracle.q8_bound(qb, xb)
    _, mb = oracle.q8_quantize_blocks(xb)
    assert mb[0, 1] == 0.0 and abs(S[0, 0] - A[0, 0]) <= B[0, 0]
    assert abs(S[0, 0] - A[0, 0]) > 0.5 * B[0, 0] > 0
