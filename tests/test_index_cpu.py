"""Host-side behaviour of ``Index`` on the CPU, mirroring the reference's
contract (cuda_vector_search/index.py:44-155; tests/test_search.py:146-156).
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

import oracle
from cuda_vector_search import Index, exact_topk_fp32, torch_topk
from cuda_vector_search import __version__
from cuda_vector_search import index as index_mod


def make(n, d, b, seed=0, normal=True):
    """Data generator of tests/test_search.py:11-18 (CPU generator, fp16)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, d, generator=g)
    q = torch.randn(b, d, generator=g)
    if normal:
        x = x / x.norm(dim=1, keepdim=True)
        q = q / q.norm(dim=1, keepdim=True)
    return x.half(), q.half()


def test_public_surface():
    assert __version__ == "0.1.0"
    assert callable(exact_topk_fp32) and callable(torch_topk)
    # the reference's methods (index.py:104-131), plus the int8 pre-filter
    assert index_mod.METHODS[:4] == ("auto", "fused", "twopass", "torch")
    assert index_mod.METHODS[4:] == ("int8",)
    assert index_mod.PAD == 64 and index_mod.MAX_FUSED_K == 256


def test_save_load_roundtrip(tmp_path):
    # the reference's CPU-runnable test (tests/test_search.py:146-156)
    x, q = make(500, 64, 3, seed=1, normal=False)
    index = Index(x.float().numpy(), metric="cosine", device="cpu")
    path = tmp_path / "emb.npy"
    index.save(path)
    again = Index.load(path, device="cpu")
    assert again.metric == "cosine" and len(again) == 500 and again.dim == 64
    a = index.search(q.float().numpy(), 5, method="torch")
    b = again.search(q.float().numpy(), 5, method="torch")
    assert torch.equal(a[1].cpu(), b[1].cpu())
    assert np.load(path).dtype == np.float16
    meta = json.loads((tmp_path / "emb.npy.json").read_text())
    assert meta == {"metric": "cosine", "dim": 64, "n": 500}


def test_save_without_npy_suffix_keeps_reference_quirk(tmp_path):
    # np.save appends ".npy" but the sidecar is "<path>.json" (index.py:144-146)
    x, _ = make(20, 8, 1, seed=2)
    Index(x.numpy(), metric="ip", device="cpu").save(tmp_path / "emb")
    assert (tmp_path / "emb.npy").exists() and (tmp_path / "emb.json").exists()
    again = Index.load(tmp_path / "emb.npy", device="cpu")
    assert again.metric == "cosine"  # sidecar not found under "emb.npy.json": default


@pytest.mark.parametrize("kwargs,exc,msg", [
    (dict(metric="l2"), ValueError, "metric must be"),
])
def test_constructor_errors(kwargs, exc, msg):
    with pytest.raises(exc, match=msg):
        Index(np.ones((3, 4), np.float32), device="cpu", **kwargs)


def test_constructor_shape_errors():
    with pytest.raises(ValueError, match="2-D"):
        Index(np.ones(4, np.float32), device="cpu")
    with pytest.raises(ValueError, match="empty"):
        Index(np.ones((0, 4), np.float32), device="cpu")


def test_search_argument_errors():
    x, q = make(50, 16, 2, seed=3)
    idx = Index(x, metric="ip", device="cpu")
    with pytest.raises(ValueError, match="method must be one of"):
        idx.search(q, 3, method="faiss")
    with pytest.raises(ValueError, match="k must be >= 1"):
        idx.search(q, 0)
    with pytest.raises(ValueError, match=r"queries must be \[b, 16\]"):
        idx.search(q[:, :8], 3)
    for m in ("fused", "twopass"):
        with pytest.raises(RuntimeError, match="gfx950"):
            idx.search(q, 3, method=m)


def test_cpu_index_is_fp32_unpadded_and_auto_uses_torch():
    x, q = make(300, 96, 4, seed=4)
    idx = Index(x, metric="ip", device="cpu")
    assert idx._x.dtype == torch.float32 and idx._x.shape == (300, 96)
    assert idx._use_kernels is False
    v, i = idx.search(q, 7)
    assert v.dtype == torch.float32 and i.dtype == torch.int64 and v.shape == (4, 7)
    ov, oi = oracle.topk(q, x, 7)
    assert oracle.check_exact(q, x, 7, v, i) == 1.0


def test_k_is_clipped_and_1d_query_promoted():
    x, q = make(30, 8, 1, seed=5)
    idx = Index(x, metric="ip", device="cpu")
    v, i = idx.search(q[0], 100)
    assert v.shape == (1, 30) and i.shape == (1, 30)


def test_copy_semantics_and_inplace_cosine():
    x = torch.randn(10, 8) * 3
    keep = x.clone()
    Index(x, metric="cosine", device="cpu")          # copy=True: caller untouched
    assert torch.equal(x, keep)
    Index(x, metric="cosine", device="cpu", copy=False)  # fp32 CPU: aliasing, normalised in place
    np.testing.assert_allclose(x.norm(dim=1).numpy(), 1.0, rtol=1e-6)


def test_normalize_and_pad_helpers():
    x = (torch.randn(700, 96) * 5).half()
    y = index_mod._normalize_(x.clone())
    np.testing.assert_allclose(y.float().norm(dim=1).numpy(), 1.0, atol=2e-3)
    z = torch.zeros(3, 8, dtype=torch.float16)
    index_mod._normalize_(z)  # clamp_min keeps zero rows finite
    assert torch.isfinite(z.float()).all()
    p = index_mod._padded(y)
    assert p.shape == (700, 128) and torch.equal(p[:, :96], y) and not p[:, 96:].any()
    assert index_mod._padded(p) is p


def test_scores_cpu_fallback():
    x, q = make(40, 16, 3, seed=6)
    idx = Index(x, metric="ip", device="cpu")
    s = idx.scores(q)
    assert s.shape == (3, 40) and s.dtype == torch.float32
    np.testing.assert_allclose(s.numpy(), oracle.scores(q, x), atol=1e-5)


def test_exact_reference_helper_cpu():
    # tests/test_search.py:116-121 on the CPU: chunked fp32 ground truth == one topk
    x, q = make(7000, 128, 4, seed=9)
    v, i = exact_topk_fp32(q, x, 20, chunk=1024)
    ref_v, _ = torch.topk(q.float() @ x.float().T, 20, dim=1)
    assert torch.allclose(v, ref_v, atol=1e-5)
    ov, _ = oracle.topk(q, x, 20)
    np.testing.assert_allclose(v.numpy(), ov, atol=1e-5)
