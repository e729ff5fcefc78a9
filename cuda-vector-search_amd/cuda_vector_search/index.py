"""``Index``: exact top-k search over an fp16 corpus resident in GPU memory.

Public behaviour is that of the reference's ``cuda_vector_search/index.py:44-155``
(constructor arguments, copy/aliasing rules, in-place cosine normalisation,
zero-padding of the width to a multiple of 64, method dispatch, error types and
messages, ``.npy`` + ``<path>.json`` persistence).  The difference is underneath:
``method="fused"``/``"twopass"`` and ``scores()`` run the gfx950 HIP engine
(``libcvs_hip.so`` through ``_ext``), never a CUDA extension.
"""

from __future__ import annotations

import json
import threading
from pathlib import Path

import numpy as np
import torch

from . import _ext
from .reference import torch_topk

PAD = 64            # widths are zero-padded to a multiple of this (the MFMA depth step x 2)
MAX_FUSED_K = 256   # largest k of the fused path
MAX_EXACT_K = 1024  # largest k of the exact large-k path (score matrix + row top-k)
_SCORE_BLOCK_BYTES = 1 << 31  # fp32 score rows computed per block on the large-k path
Q8_MAX_WIDTH = 1536  # widest (padded) rows the int8 companion covers; wider corpora use the fp16 scan
_NORM_CHUNK = 1 << 18
# int8 pre-filter (an int8 companion of the corpus scanned instead of the fp16
# rows; exact results).  Built by default for corpora of at least Q8_MIN_ROWS
# rows wider than Q8_MIN_WIDTH; "auto" uses it where it measured faster than the
# fp16 scan (MI355X latency grid, 100k-4M rows x 384/768, k 10/100, batch
# 1-256): batch 1 (bandwidth-bound GEMV on half the bytes), and over at least
# Q8_BATCH_MIN_ROWS rows any batch with k <= Q8_MAX_K, batches of at most
# Q8_MAX_BATCH queries, and batches of at least Q8_TWO_PHASE_BATCH (where the
# select rescores the k candidates of largest bound first and then only those
# that can still enter).  Batches in between with larger k stay on the fp16
# path: there every candidate that passes the int8 bound (~3x the fp16 scan's)
# is rescored from its fp16 row.
Q8_MIN_ROWS = 1 << 18
Q8_MIN_WIDTH = 256
Q8_MAX_K = 16
Q8_MAX_BATCH = 64
Q8_TWO_PHASE_BATCH = 160
Q8_BATCH_MIN_ROWS = 1 << 19

METHODS = ("auto", "fused", "twopass", "torch", "int8")


def int8_builds(n: int, width: int) -> bool:
    """Whether Index builds the int8 companion by default (int8_prefilter=None)."""
    return n >= Q8_MIN_ROWS and Q8_MIN_WIDTH < width <= Q8_MAX_WIDTH


def _int8_faster(n: int, nq: int, k: int) -> bool:
    """Whether the int8 path measured faster than the fp16 scan for this shape."""
    return k <= MAX_FUSED_K and (nq == 1 or (n >= Q8_BATCH_MIN_ROWS and (
        k <= Q8_MAX_K or nq <= Q8_MAX_BATCH or nq >= Q8_TWO_PHASE_BATCH)))


def int8_auto(n: int, width: int, nq: int, k: int) -> bool:
    """Whether method="auto" runs the int8 path (default companion, k <= 256)."""
    return int8_builds(n, width) and _int8_faster(n, nq, k)


def q8_row_bytes(width: int) -> int:
    """Bytes of one int8 companion row (the smallest int8 scan width >= width)."""
    return 384 if width <= 384 else 768 if width <= 768 else 1536


def _as_tensor(a) -> torch.Tensor:
    return a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a))


def _padded(x: torch.Tensor) -> torch.Tensor:
    """Zero-pad the columns up to the next multiple of PAD (no copy when already aligned)."""
    extra = (-x.shape[1]) % PAD
    return torch.nn.functional.pad(x, (0, extra)) if extra else x


def _normalize_(x: torch.Tensor) -> torch.Tensor:
    """Unit-normalise the rows of ``x`` in place, converting at most 2^18 rows to fp32 at a time."""
    n = x.shape[0]
    for lo in range(0, n, _NORM_CHUNK):
        rows = x[lo:lo + _NORM_CHUNK]
        f = rows.float()
        f = f / f.norm(dim=1, keepdim=True).clamp_min(1e-12)
        rows.copy_(f.to(x.dtype))
    return x


class Index:
    """Brute-force (exact) top-k index.

    Args:
        embeddings: ``[n, d]`` array or tensor; stored as fp16 on a GPU, fp32 on the CPU.
        metric: ``"cosine"`` (rows and queries are L2-normalised) or ``"ip"``.
        device: ``"cuda"``, ``"cuda:1"``, ``"cpu"``...; defaults to the GPU when present.
        copy: with ``False`` a contiguous fp16 tensor already on the device is stored
            without a copy (and normalised in place for cosine).
        int8_prefilter: build the int8 companion used by ``method="int8"`` (and by
            "auto" where it is faster): None = when the corpus is large enough
            (>= 2^18 rows, padded width in (256, 1536]), True = always on a gfx950
            GPU (widths up to 1536), False = never.  It costs one byte per stored
            element plus 16 bytes per 64 rows (``int8_bytes``): +50% of the fp16
            corpus's HBM (1M x 768: +768 MB).  It is built here and rebuilt before
            the next int8 search whenever the stored rows have changed through
            torch (in-place ops on ``_x``, ``embeddings`` or, with ``copy=False``,
            the caller's tensor bump its version counter).  Writes that bypass
            torch (raw pointers, other libraries) are not seen: call
            ``refresh_int8()`` after them.
    """

    def __init__(self, embeddings, metric: str = "cosine", device=None, copy: bool = True,
                 int8_prefilter: bool | None = None):
        if metric not in ("cosine", "ip"):
            raise ValueError("metric must be 'cosine' or 'ip'")
        src = _as_tensor(embeddings)
        if src.dim() != 2:
            raise ValueError("embeddings must be 2-D [n, d]")
        if src.shape[0] == 0:
            raise ValueError("embeddings is empty")
        self.device = torch.device(device if device is not None else
                                   ("cuda" if torch.cuda.is_available() else "cpu"))
        self.metric = metric
        self.dim = int(src.shape[1])
        on_gpu = self.device.type == "cuda"

        x = src.to(self.device, torch.float16 if on_gpu else torch.float32)
        if copy and x.data_ptr() == src.data_ptr():  # .to() returned the caller's storage
            x = x.clone()
        x = x.contiguous()
        # The reference asks only _ext.available() here (index.py:78); available()
        # is False when the engine library cannot be loaded, and then the index
        # uses the torch path as the reference does without its kernels.
        self._use_kernels = on_gpu and _ext.available()
        if self._use_kernels:
            # one HIP pass each: normalise in place (the caller's tensor too when
            # copy=False, as in the reference), then zero-pad into a new tensor
            eng = _ext.load()
            if metric == "cosine" and x.shape[0] > 0:
                eng.prep_rows(x, x, True)
            width = x.shape[1] + (-x.shape[1]) % PAD
            if width != x.shape[1]:
                xp = torch.empty((x.shape[0], width), dtype=x.dtype, device=x.device)
                eng.prep_rows(x, xp, False)
                x = xp
            self._x = x
        else:
            if metric == "cosine":
                _normalize_(x)
            self._x = _padded(x) if on_gpu else x
        self._xq = None
        self._xq_stamp = None  # (version, data_ptr, shape) of _x when _xq was built
        self._xq_ready = None  # event recorded after the build of _xq
        self._xq_lock = threading.Lock()
        if self._use_kernels and int8_prefilter is not False and self._x.shape[1] <= Q8_MAX_WIDTH:
            if int8_prefilter or int8_builds(self._x.shape[0], self._x.shape[1]):
                self._build_int8()

    def _corpus_stamp(self):
        return (self._x._version, self._x.data_ptr(), tuple(self._x.shape))

    def _build_int8(self) -> None:
        stamp = self._corpus_stamp()
        xq = _ext.load().q8_build(self._x)  # enqueued on the current stream
        ready = torch.cuda.Event()
        ready.record()
        self._xq, self._xq_stamp, self._xq_ready = xq, stamp, ready

    def _int8_companion(self, build: bool):
        """The int8 companion, current with the stored rows: rebuilt when they
        changed since it was built (and built when ``build`` and there is none).
        Thread-safe, and safe across streams: the caller's stream waits for the
        build, and the companion's memory is held for that stream's work even if
        another thread replaces it meanwhile.  None when there is none and
        ``build`` is False."""
        with self._xq_lock:
            if self._xq is None and not build:
                return None
            if self._xq is None or self._xq_stamp != self._corpus_stamp():
                self._build_int8()
            xq, ready = self._xq, self._xq_ready
        stream = torch.cuda.current_stream(self.device)
        if not ready.query():  # still being built: order this stream after the build
            stream.wait_event(ready)
        xq.record_stream(stream)
        return xq

    def refresh_int8(self) -> None:
        """Rebuild the int8 companion from the stored rows (after writes torch did not see)."""
        with self._xq_lock:
            if self._xq is not None:
                self._build_int8()

    @property
    def int8_bytes(self) -> int:
        """Device bytes held by the int8 companion (0 when there is none)."""
        xq = self._xq
        return 0 if xq is None else int(xq.numel())

    # -- basics -------------------------------------------------------------
    def __len__(self) -> int:
        return int(self._x.shape[0])

    @property
    def embeddings(self) -> torch.Tensor:
        """The stored matrix (normalised for cosine), without the padding columns."""
        return self._x[:, :self.dim]

    def _prep_queries(self, queries) -> torch.Tensor:
        q = _as_tensor(queries)
        if q.dim() == 1:
            q = q.unsqueeze(0)
        if q.dim() != 2 or q.shape[1] != self.dim:
            raise ValueError(f"queries must be [b, {self.dim}]")
        q = q.to(self.device, self._x.dtype).contiguous()
        width = self._x.shape[1]
        if (self._use_kernels and q.shape[0] > 0
                and (self.metric == "cosine" or width != q.shape[1])):
            # normalise (cosine) + zero-pad in one HIP pass into a new tensor
            out = torch.empty((q.shape[0], width), dtype=q.dtype, device=q.device)
            _ext.load().prep_rows(q, out, self.metric == "cosine")
            return out
        if self.metric == "cosine":
            q = _normalize_(q.clone())
        return _padded(q) if self.device.type == "cuda" else q

    # -- search -------------------------------------------------------------
    def search(self, queries, k: int = 10, method: str = "auto"):
        """Top-k (scores ``[b, k]`` float32, ids ``[b, k]`` int64), best first.

        method:
            "fused"   - gfx950 engine: MFMA scores + threshold filter + exact select (k <= 256)
            "twopass" - gfx950 score kernel writes the fp16 matrix, then torch.topk
            "torch"   - torch matmul + torch.topk
            "int8"    - gfx950 engine over the int8 companion: int8 scan/GEMV with a
                        rigorous error bound, exact fp16 rescoring of what passes
                        (same results as "fused", k <= 256)
            "auto"    - int8 where it is faster (batch 1; over >= 2^19 rows, batches of
                        <= 64 queries or k <= 16), else fused, for k <= 256; exact
                        fp32 scores + row top-k for k <= 1024; else torch.  Any
                        width: rows wider than 1536 run the fp16 kernels (the int8
                        companion covers widths up to 1536)
        """
        if method not in METHODS:
            raise ValueError(f"method must be one of {METHODS}")
        k = int(k)
        if k < 1:
            raise ValueError("k must be >= 1")
        k = min(k, len(self))
        q = self._prep_queries(queries)
        if method == "auto":
            if self._use_kernels and k <= MAX_FUSED_K:
                method = "int8" if self._int8_wins(q.shape[0], k) else "fused"
            elif self._use_kernels and k <= MAX_EXACT_K:
                return self._search_large_k(q, k)
            else:
                method = "torch"
        if method in ("fused", "twopass", "int8") and not self._use_kernels:
            raise RuntimeError(f"method={method!r} needs an AMD Instinct MI355X (gfx950) GPU")
        if method == "int8":
            if k > MAX_FUSED_K:
                raise ValueError(f"int8 search supports k <= {MAX_FUSED_K}")
            if self._x.shape[1] > Q8_MAX_WIDTH:
                raise ValueError(f"int8 search supports widths up to {Q8_MAX_WIDTH}")
            xq = self._int8_companion(build=True)
            v, i, _ = _ext.load().q8_topk(q, self._x, xq, k, flags=_ext.FLAG_IDS_INT64)
            return v, i
        if method == "fused":
            if k > MAX_FUSED_K:
                raise ValueError(f"fused search supports k <= {MAX_FUSED_K}")
            # ids come out as int64 directly (index.py:126 widens int32 with .long())
            v, i, _ = _ext.load().fused_topk(q, self._x, k, flags=_ext.FLAG_IDS_INT64)
            return v, i
        if method == "twopass":
            s = _ext.load().scores(q, self._x, False)
            v, i = torch.topk(s, k, dim=1)
            return v.float(), i
        return torch_topk(q, self._x, k)

    def _int8_wins(self, nq: int, k: int) -> bool:
        """Whether "auto" sends a batch of nq queries with this k to the int8 path."""
        return self._xq is not None and _int8_faster(len(self), nq, k)

    def _search_large_k(self, q: torch.Tensor, k: int):
        """Exact top-k for MAX_FUSED_K < k <= MAX_EXACT_K on the GPU: fp32 score
        rows from the score kernel, then the exact row top-k, in query blocks of
        at most 2 GB of scores.  (The reference sends k > 256 to torch with fp16
        scores, index.py:118.)"""
        eng = _ext.load()
        n = len(self)
        if q.shape[0] == 0:
            return (torch.empty((0, k), dtype=torch.float32, device=q.device),
                    torch.empty((0, k), dtype=torch.int64, device=q.device))
        rows = max(1, _SCORE_BLOCK_BYTES // (4 * n))
        vs, ids = [], []
        for lo in range(0, q.shape[0], rows):
            s = eng.scores(q[lo:lo + rows], self._x, True)
            v, i = eng.topk_rows(s, k, flags=_ext.FLAG_IDS_INT64)
            vs.append(v)
            ids.append(i)
            del s
        if len(vs) == 1:
            return vs[0], ids[0]
        return torch.cat(vs), torch.cat(ids)

    def scores(self, queries, fp32: bool = True) -> torch.Tensor:
        """Full ``[b, n]`` score matrix (gfx950 score kernel on a GPU index)."""
        q = self._prep_queries(queries)
        if not self._use_kernels:
            return (q @ self._x.T).float()
        return _ext.load().scores(q, self._x, fp32)

    # -- persistence --------------------------------------------------------
    def save(self, path) -> None:
        """Write the stored vectors to ``path`` (``np.save``, fp16) and ``<path>.json`` metadata."""
        path = Path(path)
        np.save(path, self.embeddings.to(torch.float16).cpu().numpy())
        Path(f"{path}.json").write_text(json.dumps({"metric": self.metric, "dim": self.dim, "n": len(self)}))

    @classmethod
    def load(cls, path, metric: str | None = None, device=None) -> "Index":
        path = Path(path)
        if metric is None:
            side = Path(f"{path}.json")
            metric = json.loads(side.read_text())["metric"] if side.exists() else "cosine"
        return cls(torch.from_numpy(np.load(path)), metric=metric, device=device, copy=False)
