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
    scan8 = bench.DOMINANT["scan_q8"]
    assert scan8.search("void cvs::(anonymous namespace)::scan_kernel<32, 8, 1, 2, 12, 4, true>(cvs::ScanArgs)")
    assert scan8.search("cvs::(anonymous namespace)::q8scan384_kernel(cvs::ScanArgs)")
    assert not scan8.search("void cvs::(anonymous namespace)::scan_kernel<32, 8, 1, 2, 24, 1, true>(cvs::ScanArgs)")
    gemv8 = bench.DOMINANT["gemv_q8"]
    assert gemv8.search("void cvs::(anonymous namespace)::gemv_kernel<6, 4>(cvs::GemvArgs)")
    assert not gemv8.search("void cvs::(anonymous namespace)::gemv_kernel<12, 1>(cvs::GemvArgs)")


def test_dominant_kernel_follows_the_auto_path():
    # C2 (1M x 384, b256, k10), C3 (b1) and C4 (1M x 768, b256, k100) take the
    # int8 pre-filter; C1 and C5 (100k rows) the fp16 fused path
    assert [bench.dominant_key(c) for c in ("C1", "C2", "C3", "C4", "C5")] == \
        ["scan", "scan_q8", "gemv_q8", "scan_q8", "scan"]


def test_instantiated_kernels_are_the_ones_the_patterns_expect():
    src = (REPO / "cuda-vector-search_amd" / "csrc" / "cvs_scan.hip").read_text()
    assert "template <int MS, int QS, int QB, int RB, int KSMAX, int MODE, bool FULLW>" in src
    lean = (REPO / "cuda-vector-search_amd" / "csrc" / "cvs_scan_q8.hip").read_text()
    assert "void q8scan384_kernel(ScanArgs a)" in lean
    hdr = (REPO / "cuda-vector-search_amd" / "csrc" / "cvs_kernels.h").read_text()
    assert "kAppend = 0," in hdr and "kAppendQ8 = 4," in hdr


def test_algorithmic_bytes():
    assert bench.kernel_bytes(1_000_000, 384, 256) == 2 * 1_000_000 * 384 + 2 * 256 * 384
    assert bench.kernel_bytes(4_000_000, 768, 1) == 6_144_001_536
    assert bench.kernel_bytes_q8(1_000_000, 384, 256) == 384_000_000 + 256 * 384


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 2
    assert "exactly one GPU" in r.stderr
