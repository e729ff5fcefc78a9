"""Test configuration: import paths, the ``gpu`` marker, shared helpers."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG = REPO / "cuda-vector-search_amd"
for p in (str(REPO), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950) GPU")


@pytest.fixture(scope="module")
def eng():
    """The gfx950 engine through its C-ABI.  Skips only off an MI355X; on one, a
    library that fails to load, or was built from other sources than this
    tree's, fails the test instead of skipping it."""
    from cuda_vector_search import _ext

    if not _ext.device_supported():
        pytest.skip("needs an AMD Instinct MI355X (gfx950)")
    e = _ext.load()
    maps = Path("/proc/self/maps").read_text()
    assert str(_ext.LIBRARY) in maps, "libcvs_hip.so from this tree is not mapped"
    assert _ext.is_current(), "libcvs_hip.so was not built from this tree's sources"
    return e
