"""Builds libcvs_hip.so (the gfx950 HIP engine) in-tree with hipcc.

    python cuda-vector-search_amd/build.py [--jobs N] [--verbose]

Objects go to cuda-vector-search_amd/_build/, the library to
cuda-vector-search_amd/cuda_vector_search/libcvs_hip.so, next to the Python
package that loads it, with the sha256 of its sources in libcvs_hip.srchash
(cuda_vector_search._ext.load() rebuilds when the tree no longer matches it).
Always rebuilds (the build check must compile).
"""

from __future__ import annotations

import argparse
import hashlib
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent))
import hazard_check  # noqa: E402

PKG_ROOT = Path(__file__).resolve().parent
REPO = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
INCLUDE = REPO / "include"
BUILD = PKG_ROOT / "_build"
LIB = PKG_ROOT / "cuda_vector_search" / "libcvs_hip.so"
HASH = LIB.with_name("libcvs_hip.srchash")  # source hash of the library built last

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# Packed fp32 VALU ops are disabled for all device code (the compiler would
# otherwise form v_pk_{add,mul,fma}_f32 from plain float code by itself).
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", f"-I{CSRC}",
]

SOURCES = ["cvs_scan.hip", "cvs_scan_q8.hip", "cvs_select.hip", "cvs_gemv.hip", "cvs_prep.hip", "cvs_q8.hip", "cvs_capi.hip"]

# Per-source extra flags.  The scan keeps its MFMA accumulators in VGPRs (the
# query fragments are pinned in AGPRs explicitly): the epilogue then reads the
# scores without 64 v_accvgpr_read per tile (measured 3-6% faster scan).
MFMA_SOURCES = ["cvs_scan.hip", "cvs_scan_q8.hip"]  # kernels whose MFMA results the build checks
EXTRA = {"cvs_scan.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"], "cvs_scan_q8.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _run(cmd, verbose):
    if verbose:
        print(" ".join(str(c) for c in cmd), flush=True)
    r = subprocess.run([str(c) for c in cmd], capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed ({r.returncode}): {' '.join(str(c) for c in cmd)}")
    return r


def source_hash() -> str:
    """sha256 over the sources the library is built from (same rule as
    cuda_vector_search._ext.source_hash, which load() compares with HASH)."""
    csrc = sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.h")))
    h = hashlib.sha256()
    for f in csrc + [INCLUDE / "cvs.h", Path(__file__).resolve()]:
        h.update(f.name.encode() + b"\0" + f.read_bytes() + b"\0")
    return h.hexdigest()


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    digest = source_hash()  # of the sources as they are when compilation starts
    BUILD.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *FLAGS, *EXTRA.get(src, []), "-c", CSRC / src, "-o", obj])
    # device assembly of the MFMA kernels, for the result-hazard check below
    asms = []
    for src in MFMA_SOURCES:
        asm = BUILD / (Path(src).stem + ".s")
        asms.append(asm)
        cmds.append([HIPCC, *FLAGS, *EXTRA[src], "--cuda-device-only", "-S", "-c", CSRC / src, "-o", asm])
    with ThreadPoolExecutor(max_workers=jobs or min(len(cmds), os.cpu_count() or 1)) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    early = [p for asm in asms for p in hazard_check.check(asm)]
    if early:
        raise RuntimeError(f"{len(early)} MFMA results read too early in the scan kernels, e.g. " + early[0])
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    os.replace(tmp, LIB)
    HASH.write_text(digest + "\n")
    return LIB


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose))


if __name__ == "__main__":
    main()
