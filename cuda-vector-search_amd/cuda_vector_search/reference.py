"""Plain PyTorch search paths of the public API (no custom kernels).

Same functions and behaviour as the reference's ``cuda_vector_search/reference.py``:

* ``torch_topk`` (reference.py:8-15): one matmul then ``torch.topk``.  This is
  the ``method="torch"`` path and the fallback for CPU indexes and k > 256,
  exactly as in the reference (index.py:117-118,131).
* ``exact_topk_fp32`` (reference.py:18-34): fp32 ground truth, chunked over the
  corpus with a running top-k merge so a large fp16 corpus never needs a full
  fp32 copy.
"""

from __future__ import annotations

import torch


def torch_topk(queries: torch.Tensor, corpus: torch.Tensor, k: int):
    """Score matrix with one matmul, then ``torch.topk``; returns (fp32 scores, ids).

    On a GPU with fp16 inputs the scores are produced (and ranked) in fp16.
    """
    top_v, top_i = torch.topk(queries @ corpus.T, k, dim=1)
    return top_v.float(), top_i


def exact_topk_fp32(queries: torch.Tensor, corpus: torch.Tensor, k: int, chunk: int = 1 << 18):
    """Exact top-k with fp32 arithmetic on the stored values, ``chunk`` corpus rows at a time."""
    qf = queries.float()
    kept_v = kept_i = None
    n = corpus.shape[0]
    for lo in range(0, n, chunk):
        part = qf @ corpus[lo:lo + chunk].float().T
        v, i = torch.topk(part, min(k, part.shape[1]), dim=1)
        i = i + lo
        if kept_v is not None:
            v = torch.cat((kept_v, v), dim=1)
            i = torch.cat((kept_i, i), dim=1)
            v, pick = torch.topk(v, min(k, v.shape[1]), dim=1)
            i = torch.gather(i, 1, pick)
        kept_v, kept_i = v, i
    return kept_v, kept_i
