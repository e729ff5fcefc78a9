"""CPU oracle for the exact top-k hot path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed CPU
baseline.  The shipped package (``cuda-vector-search_amd/cuda_vector_search``)
never imports it; its HIP path fails loudly instead of falling back here.

Contents, each restating one reference function (file:line into the reference):

* ``topk`` / ``scores``  - C restatement (``cvs_oracle.c``) of
  ``cuda_vector_search/reference.py:18-34`` (exact fp32 top-k over the stored
  fp16 values) with the total output order of ``csrc/kernels.cu:277-279``
  (score desc, id asc), and of the score matrix of ``csrc/kernels.cu:472-497``.
* ``exact_topk_fp32``    - numpy restatement of ``reference.py:18-34`` (chunked
  fp32 matmul + running top-k merge), ties ordered by id.
* ``torch_topk_cpu``     - the reference's CPU torch path ``reference.py:8-15``
  (fp32 ``q @ x.T`` + ``torch.topk``), used as a CPU baseline.
* ``numpy_search``       - ``bench/bench_baselines.py:45-50`` (matmul +
  argpartition + argsort), used as a CPU baseline.
* ``normalize_rows``     - ``index.py:35-41`` + ``index.py:27-32`` (cosine
  normalisation and zero-padding of fp16 rows).
* ``q8_row_order`` / ``q8_quantize_blocks`` / ``q8_companion`` /
  ``q8_quantize_queries`` / ``q8_bound`` - the int8 pre-filter's data format
  (this build's own design; no reference counterpart): corpus rows in
  ascending order of their largest magnitude (stable), symmetric int8 rows
  with one scale per 64-row block of that order or per query, and the
  Cauchy-Schwarz bound |q.x - A| <= |q^| |f| + |e| |x| that keeps the
  pre-filter exact.  Pinned by closed forms (scales, saturation, ties-to-even,
  the order of rows with planted maxima, stability of equal maxima) and by the
  bound holding, and failing without either term, on random data.
* ``check_exact``        - the acceptance rule of ``tests/test_search.py:21-44``
  plus the id-parity rule (ids identical except inside the near-tie band of the
  k-th score).
* ``check_order``        - the same parity position by position: above the band,
  the ids come in the oracle's order (score desc, id asc, ``kernels.cu:277-279``)
  except among rows whose scores agree closer than the fp32 sum-order error.

Pinning (see ``tests/test_oracle.py``): fp16 decoding is checked exhaustively
against numpy; ``topk`` is checked against committed golden vectors made by an
independent float64 brute force (``tests/golden/make_golden.py``), against the
closed forms k=1 (arg-max), k=n (full sort), identity corpora (score = query
coordinate), exact duplicates (ties by id) and planted mistakes that
``check_exact`` must reject.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "libcvs_oracle.so"
_lock = threading.Lock()
_lib = None


def build(force: bool = False) -> Path:
    """Compile ``libcvs_oracle.so`` with the Makefile beside this file."""
    import subprocess

    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(_DIR), "-B" if force else "all"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not _LIB_PATH.exists():
                build()
            L = ctypes.CDLL(str(_LIB_PATH))
            L.cvs_oracle_half_to_float.restype = ctypes.c_float
            L.cvs_oracle_half_to_float.argtypes = [ctypes.c_uint16]
            L.cvs_oracle_topk.restype = ctypes.c_int
            L.cvs_oracle_topk.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                          ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                          ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
            L.cvs_oracle_scores.restype = ctypes.c_int
            L.cvs_oracle_scores.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                            ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                            ctypes.c_int]
            _lib = L
    return _lib


def _threads(threads):
    return int(threads) if threads else (os.cpu_count() or 1)


def _as_half(a) -> np.ndarray:
    """fp16 numpy view of a numpy array or a torch tensor (any device)."""
    if hasattr(a, "detach"):  # torch tensor
        import torch

        a = a.detach().to("cpu", torch.float16).contiguous().numpy()
    a = np.ascontiguousarray(a)
    if a.dtype != np.float16:
        a = a.astype(np.float16)
    return a


def topk(q, x, k: int, threads: int | None = None):
    """Exact top-k of fp32(q . x) over fp16 inputs.  Returns (f32 [b,k], int64 [b,k]).

    Restates ``reference.py:18-34`` with score-desc / id-asc order
    (``kernels.cu:277-279``).
    """
    q16, x16 = _as_half(q), _as_half(x)
    if q16.ndim == 1:
        q16 = q16[None]
    nq, d = q16.shape
    n = x16.shape[0]
    if x16.shape[1] != d:
        raise ValueError("width mismatch")
    k = int(k)
    v = np.empty((nq, k), np.float32)
    i = np.empty((nq, k), np.int64)
    rc = lib().cvs_oracle_topk(q16.ctypes.data, x16.ctypes.data, nq, n, d, k,
                               v.ctypes.data, i.ctypes.data, _threads(threads))
    if rc != 0:
        raise ValueError(f"oracle topk rejected nq={nq} n={n} d={d} k={k}")
    return v, i


def scores(q, x, threads: int | None = None) -> np.ndarray:
    """fp32(q . x) for every pair (``kernels.cu:472-497``), exactly accumulated."""
    q16, x16 = _as_half(q), _as_half(x)
    nq, d = q16.shape
    n = x16.shape[0]
    out = np.empty((nq, n), np.float32)
    rc = lib().cvs_oracle_scores(q16.ctypes.data, x16.ctypes.data, nq, n, d, out.ctypes.data,
                                 _threads(threads))
    if rc != 0:
        raise ValueError("oracle scores rejected its arguments")
    return out


def _order(v: np.ndarray, ids: np.ndarray):
    """Sort each row by (score desc, id asc)."""
    sel = np.lexsort((ids, -v.astype(np.float64)), axis=-1)
    return np.take_along_axis(v, sel, -1), np.take_along_axis(ids, sel, -1)


def exact_topk_fp32(q, x, k: int, chunk: int = 1 << 18):
    """numpy restatement of ``reference.py:18-34``: chunked fp32 matmul, running merge.

    Ties are ordered by id so that the result is a function of its inputs.
    """
    qf = _as_half(q).astype(np.float32)
    xh = _as_half(x)
    best_v = best_i = None
    for start in range(0, xh.shape[0], chunk):
        s = qf @ xh[start:start + chunk].astype(np.float32).T
        kk = min(k, s.shape[1])
        ids = np.broadcast_to(np.arange(start, start + s.shape[1], dtype=np.int64), s.shape)
        v, i = _order(s, ids)
        v, i = v[:, :kk], i[:, :kk]
        if best_v is not None:
            v = np.concatenate([best_v, v], axis=1)
            i = np.concatenate([best_i, i], axis=1)
            v, i = _order(v, i)
            v, i = v[:, :k], i[:, :k]
        best_v, best_i = v, i
    return best_v, best_i


def torch_topk_cpu(q, x, k: int):
    """The reference's CPU search path ``reference.py:8-15``: fp32 matmul + torch.topk."""
    import torch

    s = q @ x.T
    v, i = torch.topk(s, k, dim=1)
    return v.float(), i


def numpy_search(q: np.ndarray, x: np.ndarray, k: int):
    """``bench/bench_baselines.py:45-50``: matmul, argpartition, argsort of the k."""
    s = q @ x.T
    part = np.argpartition(-s, k - 1, axis=1)[:, :k]
    pv = np.take_along_axis(s, part, 1)
    order = np.argsort(-pv, axis=1)
    return np.take_along_axis(pv, order, 1), np.take_along_axis(part, order, 1)


def normalize_rows(x, width: int | None = None, normalize: bool = True) -> np.ndarray:
    """Restates ``index.py:35-41`` (``_normalize_``: fp16 rows to fp32, divide by
    the L2 norm clamped at 1e-12, round to fp16) and ``index.py:27-32``
    (``_pad_width``: zero columns up to ``width``).  The norm is accumulated in
    float64 and rounded once to fp32 (any fp32 summation order is within its own
    rounding error of it), so a GPU result may differ from this by one fp16 ulp
    where the quotient sits at an fp16 rounding boundary."""
    x16 = _as_half(x)
    n, d = x16.shape
    width = d if width is None else int(width)
    f = x16.astype(np.float32)
    if normalize:
        nrm = np.sqrt((f.astype(np.float64) ** 2).sum(axis=1)).astype(np.float32)
        f = f / np.maximum(nrm, np.float32(1e-12))[:, None]
    out = np.zeros((n, width), dtype=np.float16)
    out[:, :d] = f.astype(np.float16)
    return out


def q8_row_bytes(d: int) -> int:
    """int8 row bytes for fp16 rows of width d: 384, 768 or 1536."""
    return 384 if d <= 384 else 768 if d <= 768 else 1536


def _q8_rows(f32: np.ndarray):
    """Quantise rows sharing one scale: s = fp32(max|x|) / 127 and
    x~ = clip(rint(x * fp32(127 / max)), -127, 127), all in fp32 (rint ties to
    even), as the GPU kernels do.  Returns (x~ as float64, s)."""
    m = np.float32(np.abs(f32).max()) if f32.size else np.float32(0)
    s = np.float32(m / np.float32(127))
    inv = np.float32(np.float32(127) / m) if m > 0 else np.float32(0)
    qv = np.clip(np.rint(f32 * inv), -127, 127)
    return qv.astype(np.float64), s


def q8_row_order(x) -> np.ndarray:
    """Row order of the int8 companion (``cvs_q8.hip`` ``q8_rowkey_kernel`` and
    its stable radix sort): corpus rows by ascending max_j |x_rj| compared as
    fp16 bit patterns (NaNs skipped, an all-NaN row counts as 0), equal maxima
    in corpus order.  Entry c is the corpus row at companion row c."""
    x16 = _as_half(x)
    m = np.fmax.reduce(np.abs(x16), axis=1, initial=np.float16(0)) if x16.size else \
        np.zeros(x16.shape[0], dtype=np.float16)
    return np.argsort(m.astype(np.float16).view(np.uint16), kind="stable")


def q8_quantize_blocks(x, block: int = 64, order=None):
    """int8 companion rows of an fp16 corpus (``cvs_q8.hip`` ``q8_build_kernel``),
    taking the rows in ``order`` (companion row c = corpus row order[c]; None:
    corpus order).

    Returns ``(xq, meta)``: ``xq`` int8 ``[ceil(n/64)*64, q8_row_bytes(d)]`` (zero
    padding columns and rows) and ``meta`` float64 ``[ceil(n/64), 3]`` = (block
    scale s_b as the fp32 value the GPU stores, exact max_r |f_r|_2, exact
    max_r |x_r|_2) with f_r = x_r - s_b x~_r.  The GPU stores the two norms
    rounded up; a test checks they are >= these and within 0.2%."""
    x16 = _as_half(x)
    if order is not None:
        x16 = x16[np.asarray(order)]
    n, d = x16.shape
    dq = q8_row_bytes(d)
    nblk = -(-n // block)
    xq = np.zeros((nblk * block, dq), dtype=np.int8)
    meta = np.zeros((nblk, 3), dtype=np.float64)
    xf = x16.astype(np.float32)
    for b in range(nblk):
        rows = xf[b * block:(b + 1) * block]
        qv, s = _q8_rows(rows)
        xq[b * block:b * block + rows.shape[0], :d] = qv.astype(np.int8)
        f = rows.astype(np.float64) - np.float64(s) * qv
        meta[b, 0] = s
        meta[b, 1] = np.sqrt((f * f).sum(axis=1)).max()
        meta[b, 2] = np.sqrt((rows.astype(np.float64) ** 2).sum(axis=1)).max()
    return xq, meta


def q8_companion(x, block: int = 64):
    """The whole int8 companion as ``cvs_q8_build`` writes it: ``(xq, meta,
    perm)`` with the rows in ``q8_row_order`` and ``perm`` int32
    ``[ceil(n/64)*64]`` (companion row -> corpus row; padding rows map to
    themselves)."""
    order = q8_row_order(x)
    xq, meta = q8_quantize_blocks(x, block, order)
    perm = np.arange(xq.shape[0], dtype=np.int32)
    perm[:order.size] = order
    return xq, meta, perm


def q8_quantize_queries(q):
    """Per-row int8 queries (``q8_query_kernel``): ``(qq, meta)`` with ``qq`` int8
    ``[nq, q8_row_bytes(d)]`` and ``meta`` float64 ``[nq, 3]`` = (s_q as stored,
    exact |q^|_2 = s_q |q~|_2, exact |e|_2 with e = q - q^)."""
    q16 = _as_half(q)
    nq, d = q16.shape
    dq = q8_row_bytes(d)
    qq = np.zeros((nq, dq), dtype=np.int8)
    meta = np.zeros((nq, 3), dtype=np.float64)
    qf = q16.astype(np.float32)
    for r in range(nq):
        qv, s = _q8_rows(qf[r])
        qq[r, :d] = qv.astype(np.int8)
        e = qf[r].astype(np.float64) - np.float64(s) * qv
        meta[r] = (s, np.float64(s) * np.sqrt((qv * qv).sum()), np.sqrt((e * e).sum()))
    return qq, meta


def q8_bound(q, x, block: int = 64, order=None):
    """(A, B, S): the int8 estimate A = s_q s_b sum(q~ x~), the bound B =
    |q^| |f_r| + |e| |x_r| (per row, exact), and the exact scores S = q.x in
    float64, for every (query, corpus row) pair, with the blocks formed over
    the rows in ``order`` (as ``q8_quantize_blocks``)."""
    x16, q16 = _as_half(x), _as_half(q)
    n, d = x16.shape
    xq, meta = q8_quantize_blocks(x16, block, order)
    qq, qm = q8_quantize_queries(q16)
    pos = np.arange(n) if order is None else np.argsort(np.asarray(order))  # companion row of each corpus row
    xs = np.repeat(meta[:, 0], block)[pos]
    xf = x16.astype(np.float64)
    xt = xq[pos, :d].astype(np.float64)
    A = (qq[:, :d].astype(np.float64) @ xt.T) * qm[:, :1] * xs[None, :]
    f = xf - xs[:, None] * xt
    B = qm[:, 1:2] * np.sqrt((f * f).sum(axis=1))[None, :] + qm[:, 2:3] * np.sqrt((xf * xf).sum(axis=1))[None, :]
    S = q16.astype(np.float64) @ xf.T
    return A, B, S


class ParityError(AssertionError):
    pass


def check_exact(q, x, k: int, scores_got, ids_got, tol: float = 1e-3, full=None):
    """Acceptance rule of ``tests/test_search.py:21-44`` plus id parity.

    ``q``/``x`` are the prepared (normalised, unpadded) fp16 queries and stored
    corpus.  Checks, against fp32 scores of the stored values:
      * shape, id range, unique ids per row;
      * every returned id scores at least the true k-th - tol*scale;
      * returned scores match their ids' true scores within tol*scale;
      * rows sorted (1e-6 slack, as the reference);
      * id parity: every true top-k id whose score is above the k-th by more
        than tol*scale is returned (so ids differ only inside the near-tie band).
    Returns the exact-set recall (informational, as the reference).
    """
    v_got = np.asarray(scores_got.detach().cpu() if hasattr(scores_got, "detach") else scores_got,
                       dtype=np.float32)
    i_got = np.asarray(ids_got.detach().cpu() if hasattr(ids_got, "detach") else ids_got).astype(np.int64)
    if full is None:
        full = scores(q, x)
    b, n = full.shape
    if v_got.shape != (b, k) or i_got.shape != (b, k):
        raise ParityError(f"shape {v_got.shape}/{i_got.shape} != {(b, k)}")
    if (i_got < 0).any() or (i_got >= n).any():
        raise ParityError("id out of range")
    part = np.argpartition(-full, k - 1, axis=1)[:, :k]       # a true top-k (any tie order)
    kth = np.take_along_axis(full, part, 1).min(axis=1, keepdims=True)
    got_true = np.take_along_axis(full, i_got, 1)
    scale = max(1.0, float(np.abs(full).max()))
    band = tol * scale
    if not (got_true >= kth - band).all():
        raise ParityError("returned an id outside the true top-k")
    if not (np.abs(v_got - got_true) <= band).all():
        raise ParityError("scores do not match their ids")
    if not (v_got[:, :-1] >= v_got[:, 1:] - 1e-6).all():
        raise ParityError("results not sorted")
    for row in i_got:
        if len(set(row.tolist())) != k:
            raise ParityError("duplicate ids")
    for r in range(b):
        must = np.nonzero(full[r] > kth[r, 0] + band)[0]
        if not set(must.tolist()).issubset(set(i_got[r].tolist())):
            raise ParityError(f"row {r}: a true top-k id outside the near-tie band is missing")
    hit = sum(len(set(a) & set(c)) for a, c in zip(i_got.tolist(), part.tolist()))
    return hit / i_got.size


def check_order(v_got, i_got, ov, oi, band: float = 1e-3, eps: float = 1e-5) -> None:
    """Ids equal the oracle's position by position above the near-tie band of
    the k-th score (``kernels.cu:277-279`` order), except that rows whose oracle
    scores lie within ``eps`` of each other (exact duplicates, perturbations
    closer than the fp32 sum-order error) may come in either order among
    themselves: each such run of positions must hold the same ids.  A run that
    reaches into the band belongs to the band (``check_exact`` covers it).
    ``v_got``/``i_got`` from the engine, ``ov``/``oi`` from ``topk``; [b, k]."""
    i_got, ov, oi = (np.asarray(a) for a in (i_got, ov, oi))
    b, k = ov.shape
    if np.asarray(v_got).shape != (b, k) or i_got.shape != (b, k):
        raise ParityError("shape mismatch")
    for r in range(b):
        m = int((ov[r] > ov[r, -1] + band).sum())  # a prefix: ov is sorted
        j = 0
        while j < m:
            e = j + 1
            while e < k and ov[r, e - 1] - ov[r, e] <= eps:
                e += 1
            if e <= m and sorted(i_got[r, j:e].tolist()) != sorted(oi[r, j:e].tolist()):
                raise ParityError(f"row {r}: positions {j}..{e - 1} hold {i_got[r, j:e].tolist()}, "
                                  f"the oracle {oi[r, j:e].tolist()}")
            j = e
