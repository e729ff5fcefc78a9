"""The C-ABI boundary on the CPU: the library builds, loads and exports exactly
what include/cvs.h declares; the Python loader mirrors the reference's
``_ext.available()/load()`` contract (cuda_vector_search/_ext.py:15-47).

No compute entry point is called here (there is no GPU in this container).
"""

from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest
import torch

from cuda_vector_search import _ext

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "cvs.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cvs_[a-z_0-9]+)\s*\(", text)))


def header_defines():
    return dict(re.findall(r"#define\s+(CVS_[A-Z_0-9]+)\s+(\d+)", HEADER.read_text()))


@pytest.fixture(scope="module")
def lib_path():
    if not _ext.LIBRARY.exists():
        _ext.build()
    return _ext.LIBRARY


def test_header_declares_the_reference_operations():
    names = declared_functions()
    for required in ("cvs_scores", "cvs_fused_topk", "cvs_fused_plan", "cvs_last_error",
                     "cvs_version", "cvs_device_supported"):
        assert required in names


def test_library_exports_every_declared_symbol(lib_path):
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib_path)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT\s+(cvs_[a-z_0-9]+)\b", out))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"declared in cvs.h but not exported: {missing}"


def test_library_imports_no_allocation_call(lib_path):
    """No entry point allocates or frees device or host memory through HIP:
    outputs and workspaces are the caller's, and the int8 companion build sorts
    inside the buffer it is given."""
    out = subprocess.run(["nm", "-D", "--undefined-only", str(lib_path)], capture_output=True,
                         text=True, check=True).stdout
    imported = {s.split("@")[0] for s in re.findall(r"\bU\s+(\S+)", out)}
    assert "hipLaunchKernel" in imported or any(s.startswith("__hipRegister") for s in imported)
    alloc = sorted(s for s in imported if re.match(r"hip(Ext)?(Malloc|Free|HostAlloc|HostMalloc|HostFree|"
                                                   r"MallocAsync|FreeAsync|MemPool|MallocManaged|"
                                                   r"MallocPitch|Malloc3D|MallocArray)", s))
    assert not alloc, f"libcvs_hip.so imports allocation calls: {alloc}"


def test_library_is_gfx950_code(lib_path):
    # the embedded offload bundle names its target triple; nothing else may be there
    blob = lib_path.read_bytes()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-f]+)", blob))
    assert targets == {b"gfx950"}


def test_library_loads_and_binds(lib_path):
    lib = _ext.open_library(lib_path)
    d = header_defines()
    assert lib.cvs_version() == int(d["CVS_VERSION"])
    assert isinstance(lib.cvs_last_error(), bytes)


def test_python_flags_match_header():
    d = header_defines()
    assert _ext.FLAG_NO_PREPASS == int(d["CVS_FLAG_NO_PREPASS"])
    assert _ext.FLAG_FORCE_PREPASS == int(d["CVS_FLAG_FORCE_PREPASS"])
    assert _ext.FLAG_NO_GEMV == int(d["CVS_FLAG_NO_GEMV"])
    assert _ext.FLAG_IDS_INT64 == int(d["CVS_FLAG_IDS_INT64"])
    assert _ext.FLAG_TAU_LAUNCH == int(d["CVS_FLAG_TAU_LAUNCH"])
    assert _ext.FLAG_REGISTER_TOPK == int(d["CVS_FLAG_REGISTER_TOPK"])
    assert _ext.FLAG_TAU_NOWAIT == int(d["CVS_FLAG_TAU_NOWAIT"])
    m = re.search(r"#define\s+CVS_NOALLOC_SCRATCH_BYTES\s+\((\d+)ll << (\d+)\)", HEADER.read_text())
    assert m and _ext.NOALLOC_SCRATCH_BYTES == int(m[1]) << int(m[2])


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU behaviour")
def test_available_and_load_without_gpu():
    assert _ext.available() is False
    with pytest.raises(RuntimeError, match="gfx950"):
        _ext.load()


def test_engine_rejects_non_gpu_tensors_like_the_reference(lib_path):
    eng = _ext.Engine(_ext.open_library(lib_path))
    q = torch.zeros(2, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        eng.fused_topk(q, q, 1)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        eng.scores(q, q)
