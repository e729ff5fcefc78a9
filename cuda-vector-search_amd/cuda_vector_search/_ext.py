"""Loader for the gfx950 engine ``libcvs_hip.so`` (C ABI, see include/cvs.h).

Drop-in for the reference's ``cuda_vector_search/_ext.py:15-47``: the same two
functions, ``available()`` and ``load(verbose=False)``, and ``load()`` returns an
object with the reference extension's methods

    scores(q, x, out_fp32=True) -> Tensor[nq, n]                 (kernels.cu:472-497)
    fused_topk(q, x, k, bq=0, chunks=0) -> [v, i, plan]          (kernels.cu:501-582)

with the reference's argument checks and ``RuntimeError`` messages
(kernels.cu:451-470).  Underneath, torch only supplies device memory and the
current stream; every score and every selection is computed by the HIP
kernels.  There is no fallback inside this module: ``load()`` raises when the
library cannot be loaded, and ``available()`` (which ``Index`` consults, as the
reference's does at index.py:78) then returns False with a warning that carries
the cause, so an ``Index`` takes the reference's own torch path instead.

Stale binaries: ``build()`` records a hash of the sources it compiled
(``csrc/``, ``include/cvs.h``, ``build.py``) beside the library, and ``load()``
rebuilds when the tree's sources no longer match it, as torch's JIT extensions
(the reference's ``_ext.py:29-46``) rebuild on a source change.
"""

from __future__ import annotations

import ctypes
import hashlib
import threading
import warnings
from pathlib import Path

_lock = threading.Lock()
_mod = None
_load_error: str | None = None

LIBRARY = Path(__file__).with_name("libcvs_hip.so")
HASH_FILE = Path(__file__).with_name("libcvs_hip.srchash")
ARCH = "gfx950"
_PKG_ROOT = Path(__file__).resolve().parent.parent
_REPO = _PKG_ROOT.parent

# Flags of cvs_fused_topk (include/cvs.h).
FLAG_NO_PREPASS = 1
FLAG_FORCE_PREPASS = 2
FLAG_NO_GEMV = 4
FLAG_IDS_INT64 = 8  # ids as int64 (Index.search's dtype) instead of the reference's int32
FLAG_TAU_LAUNCH = 16  # the sampling pass and thresholds in launches of their own instead of in the scan
FLAG_REGISTER_TOPK = 32  # fp16 path: a running top-k per lane in registers instead of the sampled threshold
FLAG_TAU_NOWAIT = 64  # tests only: the scans' cross-workgroup waits give up at once (exact fallback)
NOALLOC_SCRATCH_BYTES = 96 << 20  # CVS_NOALLOC_SCRATCH_BYTES: scratch of cvs_fused_topk_noalloc per GPU


def device_supported() -> bool:
    """True when the current torch device is an MI355X-class (gfx950) GPU."""
    import torch

    if not torch.cuda.is_available():
        return False
    try:
        arch = torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName
    except Exception:  # pragma: no cover - exotic torch builds
        return False
    return str(arch).split(":")[0] == ARCH


def available() -> bool:
    """True when the engine can run here: a gfx950 GPU and a library that loads.

    Replaces ``_ext.py:15-21`` of the reference.  A load failure is reported once
    as a ``RuntimeWarning`` (with its cause) and makes this False."""
    if not device_supported():
        return False
    try:
        load()
        return True
    except Exception as e:  # noqa: BLE001 - any failure means "not available"
        global _load_error
        if _load_error is None:
            _load_error = str(e)
            warnings.warn(f"libcvs_hip could not be loaded; searches use the torch path: {e}",
                          RuntimeWarning, stacklevel=2)
        return False


def source_files() -> list[Path]:
    """The files whose contents the built library depends on."""
    csrc = _PKG_ROOT / "csrc"
    files = sorted(list(csrc.glob("*.hip")) + list(csrc.glob("*.h")))
    return files + [_REPO / "include" / "cvs.h", _PKG_ROOT / "build.py"]


def source_hash() -> str | None:
    """sha256 over the library's sources (None when they are not in this tree)."""
    files = source_files()
    if not all(f.exists() for f in files):
        return None
    h = hashlib.sha256()
    for f in files:
        h.update(f.name.encode() + b"\0" + f.read_bytes() + b"\0")
    return h.hexdigest()


def built_hash() -> str | None:
    """The source hash recorded when the library was built (None if unknown)."""
    try:
        return HASH_FILE.read_text().strip() or None
    except OSError:
        return None


def is_current() -> bool:
    """Whether the library exists and was built from the sources in this tree."""
    want = source_hash()
    return LIBRARY.exists() and (want is None or built_hash() == want)


def _bind(lib: ctypes.CDLL) -> ctypes.CDLL:
    i64, i32, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
    lib.cvs_version.restype = i32
    lib.cvs_version.argtypes = []
    lib.cvs_last_error.restype = ctypes.c_char_p
    lib.cvs_last_error.argtypes = []
    lib.cvs_device_supported.restype = i32
    lib.cvs_device_supported.argtypes = [i32]
    lib.cvs_scores.restype = i32
    lib.cvs_scores.argtypes = [vp, vp, i64, i64, i64, vp, i32, i32, vp]
    lib.cvs_fused_plan.restype = i32
    lib.cvs_fused_plan.argtypes = [i64, i64, i64, i64, i64, i64, i32, i32,
                                   ctypes.POINTER(i64), ctypes.POINTER(i64)]
    lib.cvs_fused_topk.restype = i32
    lib.cvs_fused_topk.argtypes = [vp, vp, i64, i64, i64, i64, i64, i64, i32, vp, i64,
                                   vp, vp, ctypes.POINTER(i64), i32, vp]
    lib.cvs_fused_topk_timed.restype = i32
    lib.cvs_fused_topk_timed.argtypes = [vp, vp, i64, i64, i64, i64, i64, i64, i32, vp, i64,
                                         vp, vp, ctypes.POINTER(i64), i32, vp,
                                         ctypes.POINTER(ctypes.c_float)]
    lib.cvs_fused_topk_noalloc.restype = i32
    lib.cvs_fused_topk_noalloc.argtypes = [vp, vp, i64, i64, i64, i64, i32, vp, vp, ctypes.POINTER(i64), i32, vp]
    lib.cvs_topk_rows.restype = i32
    lib.cvs_topk_rows.argtypes = [vp, i64, i64, i64, i32, vp, i64, vp, vp, i32, vp]
    lib.cvs_topk_rows_plan.restype = i32
    lib.cvs_topk_rows_plan.argtypes = [i64, i64, i64, i32, ctypes.POINTER(i64)]
    lib.cvs_prep_rows.restype = i32
    lib.cvs_prep_rows.argtypes = [vp, vp, i64, i64, i64, i64, i32, i32, vp]
    lib.cvs_fused_topk_marked.restype = i32
    lib.cvs_fused_topk_marked.argtypes = [vp, vp, i64, i64, i64, i64, i64, i64, i32, vp, i64,
                                          vp, vp, ctypes.POINTER(i64), i32, vp,
                                          ctypes.POINTER(vp)]
    lib.cvs_q8_corpus_bytes.restype = i32
    lib.cvs_q8_corpus_bytes.argtypes = [i64, i64, ctypes.POINTER(i64)]
    lib.cvs_q8_build.restype = i32
    lib.cvs_q8_build.argtypes = [vp, i64, i64, vp, i64, i32, vp]
    lib.cvs_q8_plan.restype = i32
    lib.cvs_q8_plan.argtypes = [i64, i64, i64, i64, i32, i32, ctypes.POINTER(i64), ctypes.POINTER(i64)]
    lib.cvs_q8_topk.restype = i32
    lib.cvs_q8_topk.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, i32, vp, i64, vp, vp,
                                ctypes.POINTER(i64), i32, vp]
    lib.cvs_q8_topk_marked.restype = i32
    lib.cvs_q8_topk_marked.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, i32, vp, i64, vp, vp,
                                       ctypes.POINTER(i64), i32, vp, ctypes.POINTER(vp)]
    return lib


def open_library(path: str | Path | None = None) -> ctypes.CDLL:
    """ctypes handle of the engine library with its signatures bound (no GPU needed)."""
    return _bind(ctypes.CDLL(str(path or LIBRARY)))


class Engine:
    """The object ``load()`` returns: the reference extension's two methods."""

    def __init__(self, lib: ctypes.CDLL):
        self.lib = lib
        self.path = str(LIBRARY)

    # -- helpers -------------------------------------------------------------
    def _error(self, rc: int) -> RuntimeError:
        msg = self.lib.cvs_last_error().decode("utf-8", "replace")
        return RuntimeError(msg or f"libcvs_hip error {rc}")

    @staticmethod
    def _check_matrix(t, name: str) -> None:
        import torch

        if not (isinstance(t, torch.Tensor) and t.is_cuda):
            raise RuntimeError(f"{name} must be a CUDA tensor")
        if t.dtype != torch.float16:
            raise RuntimeError(f"{name} must be float16")
        if t.dim() != 2:
            raise RuntimeError(f"{name} must be 2-D")
        if not t.is_contiguous():
            raise RuntimeError(f"{name} must be contiguous")
        if t.shape[1] % 64 != 0:
            raise RuntimeError(f"{name} width must be a multiple of 64 (zero-pad it)")
        if t.data_ptr() % 16 != 0:
            raise RuntimeError(f"{name} must be 16-byte aligned")

    def _check_pair(self, q, x) -> None:
        self._check_matrix(q, "queries")
        self._check_matrix(x, "corpus")
        if q.device != x.device:
            raise RuntimeError("queries and corpus must be on the same device")
        if q.shape[1] != x.shape[1]:
            raise RuntimeError("queries and corpus must have the same width")
        if x.shape[0] >= 2**31 - 1:
            raise RuntimeError("corpus must have fewer than 2^31 rows")
        if q.shape[0] >= 2**31 - 1:
            raise RuntimeError("too many queries")

    @staticmethod
    def _stream(dev):
        import torch

        return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    # -- row preparation (index.py:27-41 on the GPU) ----------------------------
    def prep_rows(self, src, dst, normalize: bool) -> None:
        """dst[:, :d] = src (L2-normalised when `normalize`), dst[:, d:] = 0, in one
        kernel.  src: [n, d] fp16 CUDA rows with unit column stride; dst: [n, w]
        contiguous fp16, w >= d; dst may be src itself (in place, w == d)."""
        import torch

        if not (src.is_cuda and dst.is_cuda and src.dtype == torch.float16 and dst.dtype == torch.float16):
            raise RuntimeError("prep_rows needs fp16 CUDA tensors")
        if src.dim() != 2 or dst.dim() != 2 or src.shape[0] != dst.shape[0] or src.stride(1) != 1:
            raise RuntimeError("prep_rows needs [n, d] rows with unit column stride")
        if not dst.is_contiguous():
            raise RuntimeError("prep_rows needs a contiguous destination")
        n, d = src.shape
        rc = self.lib.cvs_prep_rows(src.data_ptr(), dst.data_ptr(), n, d, src.stride(0), dst.shape[1],
                                    1 if normalize else 0, src.device.index, self._stream(src.device))
        if rc != 0:
            raise self._error(rc)

    def topk_rows(self, s, k: int, flags: int = 0):
        """Exact top-k (values desc, column asc) of each row of a fp32 CUDA
        matrix; ids int32 (int64 with FLAG_IDS_INT64)."""
        import torch

        if not (isinstance(s, torch.Tensor) and s.is_cuda and s.dtype == torch.float32 and s.dim() == 2
                and s.is_contiguous()):
            raise RuntimeError("topk_rows needs a contiguous 2-D float32 CUDA tensor")
        nq, n = s.shape
        k = int(k)
        ws_bytes = ctypes.c_int64(0)
        rc = self.lib.cvs_topk_rows_plan(nq, n, k, s.device.index, ctypes.byref(ws_bytes))
        if rc != 0:
            raise self._error(rc)
        v = torch.empty((nq, k), dtype=torch.float32, device=s.device)
        i = torch.empty((nq, k), dtype=torch.int64 if flags & FLAG_IDS_INT64 else torch.int32, device=s.device)
        ws = torch.empty(max(int(ws_bytes.value), 256), dtype=torch.uint8, device=s.device)
        rc = self.lib.cvs_topk_rows(s.data_ptr(), nq, n, k, flags, ws.data_ptr(), ws.numel(), v.data_ptr(),
                                    i.data_ptr(), s.device.index, self._stream(s.device))
        if rc != 0:
            raise self._error(rc)
        return v, i

    # -- reference API -------------------------------------------------------
    def scores(self, q, x, out_fp32: bool = True):
        import torch

        self._check_pair(q, x)
        nq, d = q.shape
        n = x.shape[0]
        out = torch.empty((nq, n), dtype=torch.float32 if out_fp32 else torch.float16, device=q.device)
        if nq == 0 or n == 0:
            return out
        rc = self.lib.cvs_scores(q.data_ptr(), x.data_ptr(), nq, n, d, out.data_ptr(),
                                 1 if out_fp32 else 0, q.device.index, self._stream(q.device))
        if rc != 0:
            raise self._error(rc)
        return out

    def plan(self, nq: int, n: int, d: int, k: int, bq: int = 0, chunks: int = 0, flags: int = 0,
             device: int = 0):
        """(plan[2], workspace_bytes) for these sizes, without running anything."""
        plan = (ctypes.c_int64 * 2)()
        ws = ctypes.c_int64(0)
        rc = self.lib.cvs_fused_plan(nq, n, d, k, bq, chunks, flags, device, plan, ctypes.byref(ws))
        if rc != 0:
            raise self._error(rc)
        return [int(plan[0]), int(plan[1])], int(ws.value)

    def fused_topk(self, q, x, k: int, bq: int = 0, chunks: int = 0, flags: int = 0):
        return self._fused(q, x, k, bq, chunks, flags, None)

    def fused_topk_timed(self, q, x, k: int, bq: int = 0, chunks: int = 0, flags: int = 0):
        """fused_topk plus per-stage device milliseconds (HIP events on the current
        stream): [sample pass, threshold select, scan/GEMV, final select].  Blocks."""
        ms = (ctypes.c_float * 4)()
        out = self._fused(q, x, k, bq, chunks, flags, ms)
        return out, [float(v) for v in ms]

    def fused_topk_marked(self, q, x, k: int, marks, bq: int = 0, chunks: int = 0, flags: int = 0):
        """fused_topk that records the five timing-enabled ``torch.cuda.Event``s in
        ``marks`` around its four stages on the current stream, without blocking
        (read them with ``marks[i].elapsed_time(marks[i + 1])`` after a sync)."""
        if len(marks) != 5:
            raise ValueError("marks must hold 5 events")
        for ev in marks:
            if not ev.cuda_event:  # torch creates the HIP event at its first record
                ev.record()
        handles = (ctypes.c_void_p * 5)(*[ev.cuda_event for ev in marks])
        return self._fused(q, x, k, bq, chunks, flags, None, handles)

    def _fused(self, q, x, k, bq, chunks, flags, stage_ms, marks=None):
        import torch

        self._check_pair(q, x)
        nq, d = q.shape
        n = x.shape[0]
        k, bq, chunks = int(k), int(bq), int(chunks)
        dev = q.device
        plan_c = (ctypes.c_int64 * 2)()
        ws_bytes = ctypes.c_int64(0)
        rc = self.lib.cvs_fused_plan(nq, n, d, k, bq, chunks, flags, dev.index, plan_c,
                                     ctypes.byref(ws_bytes))
        if rc != 0:
            raise self._error(rc)
        out_v = torch.empty((nq, k), dtype=torch.float32, device=dev)
        out_i = torch.empty((nq, k), dtype=torch.int64 if flags & FLAG_IDS_INT64 else torch.int32, device=dev)
        plan = torch.tensor([int(plan_c[0]), int(plan_c[1])], dtype=torch.int64)
        if nq == 0:
            return [out_v, out_i, plan]
        ws = torch.empty(max(int(ws_bytes.value), 256), dtype=torch.uint8, device=dev)
        args = (q.data_ptr(), x.data_ptr(), nq, n, d, k, bq, chunks, flags, ws.data_ptr(), ws.numel(),
                out_v.data_ptr(), out_i.data_ptr(), plan_c, dev.index, self._stream(dev))
        if marks is not None:
            rc = self.lib.cvs_fused_topk_marked(*args, marks)
        elif stage_ms is None:
            rc = self.lib.cvs_fused_topk(*args)
        else:
            rc = self.lib.cvs_fused_topk_timed(*args, stage_ms)
        if rc != 0:
            raise self._error(rc)
        return [out_v, out_i, plan]


    # -- int8 pre-filter (no counterpart in the reference) ------------------------
    def q8_corpus_bytes(self, n: int, d: int) -> int:
        out = ctypes.c_int64(0)
        rc = self.lib.cvs_q8_corpus_bytes(int(n), int(d), ctypes.byref(out))
        if rc != 0:
            raise self._error(rc)
        return int(out.value)

    def q8_build(self, x):
        """int8 companion of the fp16 corpus ``x`` (a uint8 tensor on its device)."""
        import torch

        self._check_matrix(x, "corpus")
        n, d = x.shape
        xq = torch.empty(self.q8_corpus_bytes(n, d), dtype=torch.uint8, device=x.device)
        rc = self.lib.cvs_q8_build(x.data_ptr(), n, d, xq.data_ptr(), xq.numel(), x.device.index,
                                   self._stream(x.device))
        if rc != 0:
            raise self._error(rc)
        return xq

    def q8_plan(self, nq: int, n: int, d: int, k: int, flags: int = 0, device: int = 0):
        plan = (ctypes.c_int64 * 2)()
        ws = ctypes.c_int64(0)
        rc = self.lib.cvs_q8_plan(nq, n, d, k, flags, device, plan, ctypes.byref(ws))
        if rc != 0:
            raise self._error(rc)
        return [int(plan[0]), int(plan[1])], int(ws.value)

    def q8_topk(self, q, x, xq, k: int, flags: int = 0, marks=None):
        """Exact top-k through the int8 pre-filter; same results as fused_topk.
        ``xq`` is ``q8_build(x)``.  With ``marks`` (five timing-enabled events)
        the stages are marked as in fused_topk_marked."""
        import torch

        self._check_pair(q, x)
        if not (isinstance(xq, torch.Tensor) and xq.dtype == torch.uint8 and xq.device == x.device
                and xq.is_contiguous()):
            raise RuntimeError("xq must be the contiguous uint8 tensor q8_build returned, on the corpus's device")
        nq, d = q.shape
        n = x.shape[0]
        k = int(k)
        dev = q.device
        plan_c = (ctypes.c_int64 * 2)()
        ws_bytes = ctypes.c_int64(0)
        rc = self.lib.cvs_q8_plan(nq, n, d, k, flags, dev.index, plan_c, ctypes.byref(ws_bytes))
        if rc != 0:
            raise self._error(rc)
        out_v = torch.empty((nq, k), dtype=torch.float32, device=dev)
        out_i = torch.empty((nq, k), dtype=torch.int64 if flags & FLAG_IDS_INT64 else torch.int32, device=dev)
        plan = torch.tensor([int(plan_c[0]), int(plan_c[1])], dtype=torch.int64)
        if nq == 0:
            return [out_v, out_i, plan]
        ws = torch.empty(max(int(ws_bytes.value), 256), dtype=torch.uint8, device=dev)
        args = (q.data_ptr(), x.data_ptr(), xq.data_ptr(), xq.numel(), nq, n, d, k, flags, ws.data_ptr(),
                ws.numel(), out_v.data_ptr(), out_i.data_ptr(), plan_c, dev.index, self._stream(dev))
        if marks is not None:
            if len(marks) != 5:
                raise ValueError("marks must hold 5 events")
            for ev in marks:
                if not ev.cuda_event:
                    ev.record()
            rc = self.lib.cvs_q8_topk_marked(*args, (ctypes.c_void_p * 5)(*[ev.cuda_event for ev in marks]))
        else:
            rc = self.lib.cvs_q8_topk(*args)
        if rc != 0:
            raise self._error(rc)
        return [out_v, out_i, plan]


def build(verbose: bool = False) -> Path:
    """Compile libcvs_hip.so in-tree (hipcc, gfx950) and record its source hash."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("_cvs_build", _PKG_ROOT / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.build(verbose=verbose)


def load(verbose: bool = False) -> Engine:
    """Load (building first if the library is missing or older than its sources)
    and return the engine."""
    global _mod
    if _mod is not None:
        return _mod
    with _lock:
        if _mod is not None:
            return _mod
        if not device_supported():
            raise RuntimeError("cuda-vector-search kernels need an AMD Instinct MI355X (gfx950) GPU")
        if not is_current():
            build(verbose)
        lib = open_library()
        import torch

        dev = torch.cuda.current_device()
        if not lib.cvs_device_supported(dev):
            raise RuntimeError(f"libcvs_hip does not support device {dev}: "
                               + lib.cvs_last_error().decode("utf-8", "replace"))
        _mod = Engine(lib)
        return _mod
