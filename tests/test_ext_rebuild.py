"""The stale-binary guard of ``_ext.load()`` (CPU only, no GPU needed).

``build()`` records the sha256 of the library's sources next to it; ``load()``
rebuilds when the tree's sources no longer match (as torch's JIT extensions,
which the reference's ``_ext.py:29-46`` uses, rebuild on a source change).
Checked on a copy of the package with the build and the library open faked.
"""

from __future__ import annotations

import importlib.util
import shutil
from pathlib import Path

import pytest

from cuda_vector_search import _ext

REPO = Path(__file__).resolve().parents[1]
PKG = REPO / "cuda-vector-search_amd"


def _build_module():
    spec = importlib.util.spec_from_file_location("_cvs_build_test", PKG / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_build_and_load_hash_the_same_files():
    assert _ext.source_hash() == _build_module().source_hash()
    names = {f.name for f in _ext.source_files()}
    assert {"cvs_scan.hip", "cvs_capi.hip", "cvs_common.h", "cvs.h", "build.py"} <= names


@pytest.fixture
def tree(tmp_path, monkeypatch):
    """A copy of the sources, an 'up-to-date' library and _ext pointed at them."""
    pkg = tmp_path / "cuda-vector-search_amd"
    shutil.copytree(PKG / "csrc", pkg / "csrc")
    shutil.copy(PKG / "build.py", pkg / "build.py")
    (tmp_path / "include").mkdir()
    shutil.copy(REPO / "include" / "cvs.h", tmp_path / "include" / "cvs.h")
    lib_dir = pkg / "cuda_vector_search"
    lib_dir.mkdir()
    monkeypatch.setattr(_ext, "_PKG_ROOT", pkg)
    monkeypatch.setattr(_ext, "_REPO", tmp_path)
    monkeypatch.setattr(_ext, "LIBRARY", lib_dir / "libcvs_hip.so")
    monkeypatch.setattr(_ext, "HASH_FILE", lib_dir / "libcvs_hip.srchash")
    monkeypatch.setattr(_ext, "_mod", None)
    monkeypatch.setattr(_ext, "device_supported", lambda: True)

    builds = []

    def fake_build(verbose=False):
        builds.append(_ext.source_hash())
        _ext.LIBRARY.write_bytes(b"\x7fELF")
        _ext.HASH_FILE.write_text(_ext.source_hash() + "\n")
        return _ext.LIBRARY

    class FakeLib:
        def cvs_device_supported(self, dev):
            return 1

    monkeypatch.setattr(_ext, "build", fake_build)
    monkeypatch.setattr(_ext, "open_library", lambda path=None: FakeLib())
    import torch

    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    fake_build()
    builds.clear()
    return pkg, builds


def _reload():
    _ext._mod = None
    return _ext.load()


def test_load_keeps_a_current_library(tree):
    pkg, builds = tree
    assert _ext.is_current()
    _reload()
    assert builds == []


def test_load_rebuilds_after_a_source_edit(tree):
    pkg, builds = tree
    src = pkg / "csrc" / "cvs_select.hip"
    src.write_text(src.read_text() + "\n// edited\n")
    assert not _ext.is_current()
    _reload()
    assert len(builds) == 1 and _ext.is_current()
    _reload()  # nothing changed since: no second build
    assert len(builds) == 1


def test_load_rebuilds_without_a_recorded_hash(tree):
    pkg, builds = tree
    _ext.HASH_FILE.unlink()
    assert not _ext.is_current()
    _reload()
    assert len(builds) == 1


def test_available_is_false_and_warns_when_load_fails(monkeypatch):
    monkeypatch.setattr(_ext, "_mod", None)
    monkeypatch.setattr(_ext, "_load_error", None)
    monkeypatch.setattr(_ext, "device_supported", lambda: True)

    def broken(verbose=False):
        raise RuntimeError("hipcc failed (1): simulated")

    monkeypatch.setattr(_ext, "load", broken)
    with pytest.warns(RuntimeWarning, match="simulated"):
        assert _ext.available() is False
    assert _ext.available() is False  # warned once
