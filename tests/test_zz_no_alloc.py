"""The allocation-free search entry point, cvs_fused_topk_noalloc (needs an MI355X).

It has no counterpart in the reference: it serves callers that cannot
allocate device memory at search time.  It runs cvs_fused_topk's kernels with
a library-owned scratch array instead of a workspace argument, so its results
must equal cvs_fused_topk's exactly.  Two calls in a row, the second on a
smaller input, check that nothing the first call left in the shared scratch
leaks into the second; a plan larger than the scratch is refused before any
launch.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

import oracle
from cuda_vector_search import _ext, synthetic

pytestmark = pytest.mark.gpu


def noalloc(eng, q, x, k, flags=0):
    """cvs_fused_topk_noalloc through the C-ABI; (rc, v, i, plan)."""
    nq, d = q.shape
    n = x.shape[0]
    v = torch.empty((nq, k), dtype=torch.float32, device=q.device)
    i = torch.empty((nq, k), dtype=torch.int64 if flags & _ext.FLAG_IDS_INT64 else torch.int32, device=q.device)
    plan = (ctypes.c_int64 * 2)()
    stream = ctypes.c_void_p(torch.cuda.current_stream(q.device).cuda_stream)
    rc = eng.lib.cvs_fused_topk_noalloc(q.data_ptr(), x.data_ptr(), nq, n, d, k, flags, v.data_ptr(),
                                        i.data_ptr(), plan, q.device.index, stream)
    return rc, v, i, [int(plan[0]), int(plan[1])]


def test_noalloc_equals_fused_on_two_calls_the_second_smaller(eng):
    cases = [(1_000_000, 384, 256, 10, 0),                 # the headline shape: 67.1 MB of scratch
             (50_000, 384, 40, 100, _ext.FLAG_IDS_INT64)]  # smaller, after it, other flags
    for n, d, b, k, flags in cases:
        print(f"noalloc n={n} d={d} b={b} k={k} flags={flags}", flush=True)
        x = synthetic.unit_corpus(n, d, seed=11, device="cuda")
        q = synthetic.unit_queries(b, d, seed=12, device="cuda")
        _, ws = eng.plan(b, n, d, k, flags=flags, device=q.device.index)
        assert ws <= _ext.NOALLOC_SCRATCH_BYTES
        rc, v, i, plan = noalloc(eng, q, x, k, flags)
        assert rc == 0, eng.lib.cvs_last_error()
        vf, i_f, pf = eng.fused_topk(q, x, k, flags=flags)
        torch.cuda.synchronize()
        assert plan == pf.tolist()
        assert torch.equal(v, vf) and torch.equal(i, i_f)
        sel = torch.arange(0, b, max(1, b // 16))
        oracle.check_exact(q[sel].cpu(), x.cpu(), k, v[sel].cpu(), i[sel].cpu())
        del x, q


def test_noalloc_refuses_a_plan_larger_than_its_scratch(eng):
    x = torch.zeros((1_000_000, 384), dtype=torch.float16, device="cuda")
    q = torch.zeros((4096, 384), dtype=torch.float16, device="cuda")
    _, ws = eng.plan(4096, 1_000_000, 384, 100, device=q.device.index)
    assert ws > _ext.NOALLOC_SCRATCH_BYTES
    rc, _, _, _ = noalloc(eng, q, x, 100)
    assert rc == 1 and b"allocation-free" in eng.lib.cvs_last_error()
