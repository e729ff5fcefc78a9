"""Host-side logic of bench.py (no GPU): the counter-run kernel matching, the
algorithmic byte count and the one-GPU guard."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import bench

REPO = Path(__file__).resolve().parents[1]


def test_dominant_kernel_patterns_match_the_append_launches_only():
    scan = bench.DOMINANT["scan"]
    assert scan.search("void cvs::(anonymous namespace)::scan_kernel<32, 4, 2, 2, 24, 0, true>(cvs::ScanArgs)")
    assert scan.search("void cvs::(anonymous namespace)::scan_kernel<16, 1, 1, 1, 12, 0, false>(cvs::ScanArgs)")
    assert not scan.search("void cvs::(anonymous namespace)::scan_kernel<32, 4, 2, 2, 24, 1, true>(cvs::ScanArgs)")
    assert not scan.search("void cvs::(anonymous namespace)::scan_kernel<32, 4, 2, 2, 24, 2, false>(cvs::ScanArgs)")
    gemv = bench.DOMINANT["gemv"]
    assert gemv.search("void cvs::(anonymous namespace)::gemv_kernel<12, 0>(cvs::GemvArgs)")
    assert not gemv.search("void cvs::(anonymous namespace)::gemv_kernel<12, 1>(cvs::GemvArgs)")
    assert bench.COPY_KERNEL.search("__amd_rocclr_copyBuffer")


def test_instantiated_kernels_are_the_ones_the_patterns_expect():
    src = (REPO / "cuda-vector-search_amd" / "csrc" / "cvs_scan.hip").read_text()
    assert "template <int MS, int QS, int QB, int RB, int KSMAX, int MODE, bool FULLW>" in src
    assert "kAppend = 0," in (REPO / "cuda-vector-search_amd" / "csrc" / "cvs_kernels.h").read_text()


def test_algorithmic_bytes():
    assert bench.kernel_bytes(1_000_000, 384, 256) == 2 * 1_000_000 * 384 + 2 * 256 * 384
    assert bench.kernel_bytes(4_000_000, 768, 1) == 6_144_001_536


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 2
    assert "exactly one GPU" in r.stderr
