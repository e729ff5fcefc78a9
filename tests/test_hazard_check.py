"""The build's MFMA result-hazard check (cuda-vector-search_amd/hazard_check.py)
on planted assembly: a read one wait state short of passes + 4 is caught, in
straight-line code and across a branch; the same read at passes + 4, a read
of other registers and an accumulating MFMA are not reported."""

from __future__ import annotations

import importlib.util
from pathlib import Path

PKG = Path(__file__).resolve().parents[1] / "cuda-vector-search_amd"


def hc():
    spec = importlib.util.spec_from_file_location("cvs_hazard_check", PKG / "hazard_check.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def kernel(body: str) -> str:
    return "_Z6kernelv:\n" + body + "\ts_endpgm\n.Lfunc_end0:\n"


MFMA = "\tv_mfma_f32_32x32x16_f16 v[0:15], v[16:19], a[0:3], v[0:15]\n"  # 8 passes: needs 12


def test_straight_line_read_one_short_is_caught():
    mod = hc()
    short = kernel(MFMA + "\ts_nop 7\n\ts_nop 1\n\tv_mov_b32_e32 v40, v0\n")    # 8 + 2 = 10 ... + 1
    ok = kernel(MFMA + "\ts_nop 7\n\ts_nop 3\n\tv_mov_b32_e32 v40, v0\n")       # 8 + 4 = 12
    eleven = kernel(MFMA + "\ts_nop 7\n\ts_nop 2\n\tv_cvt_pk_f16_f32 v41, v2, v3\n")  # 11
    assert len(mod.early_reads(*mod.kernels(short)["_Z6kernelv"])) == 1
    assert mod.early_reads(*mod.kernels(ok)["_Z6kernelv"]) == []
    (i, j, ws, need), = mod.early_reads(*mod.kernels(eleven)["_Z6kernelv"])
    assert (ws, need) == (11, 12)


def test_other_registers_and_accumulation_are_not_reported():
    mod = hc()
    other = kernel(MFMA + "\tv_mov_b32_e32 v40, v16\n")  # reads an operand, not the result
    chain = kernel(MFMA + "\tv_mfma_f32_32x32x16_f16 v[0:15], v[20:23], a[4:7], v[0:15]\n")
    assert mod.early_reads(*mod.kernels(other)["_Z6kernelv"]) == []
    assert mod.early_reads(*mod.kernels(chain)["_Z6kernelv"]) == []


def test_read_across_a_branch_is_caught():
    mod = hc()
    asm = kernel(MFMA + "\ts_cbranch_scc1 .LBB0_2\n\ts_nop 7\n\ts_nop 7\n"
                 ".LBB0_2:\n\tv_max_f32_e32 v40, v5, v5\n")
    (i, j, ws, need), = mod.early_reads(*mod.kernels(asm)["_Z6kernelv"])
    assert ws == 1 and need == 12


def test_built_scans_have_no_early_reads():
    import pytest

    for name in ("cvs_scan.s", "cvs_scan_q8.s"):
        asm = PKG / "_build" / name
        if not asm.exists():
            pytest.skip("library not built in this tree")
        assert hc().check(asm) == []
