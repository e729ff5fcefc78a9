"""Exact top-k vector search on AMD Instinct MI355X (gfx950) with hand-written HIP kernels.

Drop-in for ``cuda_vector_search`` (reference ``__init__.py:3-7``): same names,
same behaviour, gfx950 engine underneath.
"""

from .index import Index
from .reference import exact_topk_fp32, torch_topk

__all__ = ["Index", "exact_topk_fp32", "torch_topk"]
__version__ = "0.1.0"
