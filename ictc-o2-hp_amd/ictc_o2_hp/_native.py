"""ctypes binding of libictc_o2_hp_amd.so (C ABI in include/ictc_o2_hp_amd.h).

The library is built in-tree by ``build_native.py``.  torch must be imported
first so that the HIP runtime torch loads is the one the library binds to.
There is no fallback: on a GPU tensor, a missing or broken library raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library resolves against)

LIBRARY_NAME = "libictc_o2_hp_amd.so"
LIBRARY_PATH = Path(__file__).resolve().parent / LIBRARY_NAME

O2MI_OK = 0
PARITY = {"canonical": 0, "full": 1}
NORMALIZATION = {"component": 0, "norm": 1}

_lock = threading.Lock()
_lib = None


class NativeLibraryError(RuntimeError):
    """The HIP extension is missing, failed to load or reported an error."""


class UvuProblem(ctypes.Structure):
    """o2mi_uvu_problem of include/ictc_o2_hp_amd.h."""
    _fields_ = [("n_rows", ctypes.c_int64), ("channels", ctypes.c_int32),
                ("channels_in2", ctypes.c_int32), ("n_paths", ctypes.c_int32),
                ("n_out_entries", ctypes.c_int32), ("n_in2_entries", ctypes.c_int32),
                ("width1", ctypes.c_int32), ("width2", ctypes.c_int32),
                ("shared_weights", ctypes.c_int32), ("info", ctypes.c_void_p),
                ("coefficients", ctypes.c_void_p), ("first_order", ctypes.c_void_p),
                ("second_order", ctypes.c_void_p)]


def _declare(lib: ctypes.CDLL) -> None:
    c_int, c_i64, c_sz, vp = ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p
    fp = ctypes.c_void_p
    lib.o2mi_last_error.restype = ctypes.c_char_p
    lib.o2mi_last_error.argtypes = []
    lib.o2mi_version.restype = ctypes.c_char_p
    lib.o2mi_version.argtypes = []
    lib.o2mi_tp_plan_create.restype = c_int
    lib.o2mi_tp_plan_create.argtypes = [c_int, c_int, c_int, c_int, c_int, ctypes.POINTER(vp)]
    lib.o2mi_tp_plan_destroy.restype = c_int
    lib.o2mi_tp_plan_destroy.argtypes = [vp]
    lib.o2mi_tp_plan_compiled.restype = c_int
    lib.o2mi_tp_plan_compiled.argtypes = [vp]
    lib.o2mi_tp_forward_tables_f32.restype = c_int
    lib.o2mi_tp_forward_tables_f32.argtypes = [vp, fp, fp, fp, vp, fp, c_int, fp, c_i64, vp]
    lib.o2mi_tp_backward_tables_workspace_bytes.restype = c_sz
    lib.o2mi_tp_backward_tables_workspace_bytes.argtypes = [vp, c_i64]
    lib.o2mi_tp_backward_tables_f32.restype = c_int
    lib.o2mi_tp_backward_tables_f32.argtypes = [vp, fp, fp, fp, fp, vp, fp, c_int, fp, fp, fp, vp,
                                                c_sz, c_i64, c_int, vp]
    lib.o2mi_tp_width.restype = c_i64
    lib.o2mi_tp_width.argtypes = [vp]
    lib.o2mi_tp_weight_numel.restype = c_i64
    lib.o2mi_tp_weight_numel.argtypes = [vp]
    lib.o2mi_tp_table.restype = c_int
    lib.o2mi_tp_table.argtypes = [c_int, c_int, c_int, ctypes.POINTER(c_int), ctypes.POINTER(c_int),
                                  vp, vp, vp]
    lib.o2mi_tp_forward_f32.restype = c_int
    lib.o2mi_tp_forward_f32.argtypes = [vp, fp, fp, fp, fp, c_i64, vp]
    lib.o2mi_tp_backward_workspace_bytes.restype = c_sz
    lib.o2mi_tp_backward_workspace_bytes.argtypes = [vp, c_i64]
    lib.o2mi_tp_backward_f32.restype = c_int
    lib.o2mi_tp_backward_f32.argtypes = [vp, fp, fp, fp, fp, fp, fp, fp, vp, c_sz, c_i64, c_int, vp]
    lib.o2mi_tp_backward_noalloc_f32.restype = c_int
    lib.o2mi_tp_backward_noalloc_f32.argtypes = [vp, fp, fp, fp, fp, fp, fp, fp, c_i64, c_int, vp]
    prob = ctypes.POINTER(UvuProblem)
    lib.o2mi_uvu_forward_f32.restype = c_int
    lib.o2mi_uvu_forward_f32.argtypes = [prob, fp, fp, fp, fp, vp]
    lib.o2mi_uvu_backward_workspace_bytes.restype = c_sz
    lib.o2mi_uvu_backward_workspace_bytes.argtypes = [prob, c_int]
    lib.o2mi_uvu_backward_f32.restype = c_int
    lib.o2mi_uvu_backward_f32.argtypes = [prob, fp, fp, fp, fp, fp, fp, fp, c_int, vp, c_sz, vp]
    lib.o2mi_radial_plan_create.restype = c_int
    lib.o2mi_radial_plan_create.argtypes = [c_int, c_int, c_int, c_int, c_int, c_int,
                                            ctypes.POINTER(vp)]
    lib.o2mi_radial_plan_destroy.restype = c_int
    lib.o2mi_radial_plan_destroy.argtypes = [vp]
    lib.o2mi_radial_paths.restype = c_int
    lib.o2mi_radial_paths.argtypes = [vp]
    lib.o2mi_radial_forward_f32.restype = c_int
    lib.o2mi_radial_forward_f32.argtypes = [vp, fp, fp, fp, fp, fp, fp, fp, c_i64, vp]
    lib.o2mi_radial_backward_workspace_bytes.restype = c_sz
    lib.o2mi_radial_backward_workspace_bytes.argtypes = [vp, c_i64, c_int]
    lib.o2mi_radial_backward_f32.restype = c_int
    lib.o2mi_radial_backward_f32.argtypes = [vp, fp, fp, fp, fp, fp, fp, fp, fp, fp, fp, fp, fp,
                                             vp, c_sz, c_i64, c_int, vp]
    lib.o2mi_radial_forward_gather_f32.restype = c_int
    lib.o2mi_radial_forward_gather_f32.argtypes = [vp, fp, c_i64, vp, fp, fp, fp, fp, fp, fp,
                                                   c_i64, vp]
    lib.o2mi_radial_backward_gather_f32.restype = c_int
    lib.o2mi_radial_backward_gather_f32.argtypes = [vp, fp, c_i64, vp, fp, fp, fp, fp, fp, fp,
                                                    fp, fp, fp, fp, fp, vp, c_sz, c_i64, c_int,
                                                    vp]
    lib.o2mi_uvu_shared_plan_create.restype = c_int
    lib.o2mi_uvu_shared_plan_create.argtypes = [c_int, c_int, c_int, c_int, c_int, c_int,
                                                ctypes.POINTER(vp)]
    lib.o2mi_uvu_shared_forward_f32.restype = c_int
    lib.o2mi_uvu_shared_forward_f32.argtypes = [vp, fp, fp, fp, fp, fp, c_i64, vp]
    lib.o2mi_uvu_shared_backward_workspace_bytes.restype = c_sz
    lib.o2mi_uvu_shared_backward_workspace_bytes.argtypes = [vp, c_i64, c_int]
    lib.o2mi_uvu_shared_backward_f32.restype = c_int
    lib.o2mi_uvu_shared_backward_f32.argtypes = [vp, fp, fp, fp, fp, fp, fp, fp, fp, vp, c_sz,
                                                 c_i64, c_int, vp]
    lib.o2mi_uvu_rows_forward_f32.restype = c_int
    lib.o2mi_uvu_rows_forward_f32.argtypes = [vp, fp, fp, fp, fp, fp, c_i64, vp]
    lib.o2mi_uvu_rows_backward_workspace_bytes.restype = c_sz
    lib.o2mi_uvu_rows_backward_workspace_bytes.argtypes = [vp, c_i64, c_int]
    lib.o2mi_uvu_rows_backward_f32.restype = c_int
    lib.o2mi_uvu_rows_backward_f32.argtypes = [vp, fp, fp, fp, fp, fp, fp, fp, fp, vp, c_sz,
                                               c_i64, c_int, vp]
    lib.o2mi_rows_gather_f32.restype = c_int
    lib.o2mi_rows_gather_f32.argtypes = [fp, c_i64, vp, c_i64, c_i64, fp, vp]
    lib.o2mi_rows_segment_sum_f32.restype = c_int
    lib.o2mi_rows_segment_sum_f32.argtypes = [fp, c_i64, c_i64, vp, vp, c_i64, fp, vp]
    lib.o2mi_tp_launch_shape.restype = c_int
    lib.o2mi_tp_launch_shape.argtypes = [vp, c_i64, c_int] + [ctypes.POINTER(c_int)] * 4
    lib.o2mi_kernel_timing.restype = c_int
    lib.o2mi_kernel_timing.argtypes = [c_int]
    lib.o2mi_kernel_timing_read.restype = c_int
    lib.o2mi_kernel_timing_read.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(c_int),
                                            ctypes.POINTER(ctypes.c_double), ctypes.POINTER(c_int)]
    lib.o2mi_kernel_timing_read_kinds.restype = c_int
    lib.o2mi_kernel_timing_read_kinds.argtypes = [ctypes.POINTER(ctypes.c_double),
                                                  ctypes.POINTER(c_int), c_int]


def library() -> ctypes.CDLL:
    """The loaded library; raises NativeLibraryError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = os.environ.get("ICTC_O2_HP_AMD_LIBRARY", str(LIBRARY_PATH))
            if not Path(path).exists():
                raise NativeLibraryError(
                    f"{LIBRARY_NAME} is not built ({path}); run "
                    "`python ictc-o2-hp_amd/build_native.py` (or __graft_entry__.build())")
            try:
                lib = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
            except OSError as exc:
                raise NativeLibraryError(f"cannot load {path}: {exc}") from exc
            _declare(lib)
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != O2MI_OK:
        message = library().o2mi_last_error().decode(errors="replace")
        raise NativeLibraryError(f"{what} failed (status {status}): {message}")


class TPNativePlan:
    """Owns one o2mi_tp_plan handle."""

    def __init__(self, channels: int, m_max: int, parity: str, normalization: str, layout: int):
        lib = library()
        handle = ctypes.c_void_p()
        check(lib.o2mi_tp_plan_create(channels, m_max, PARITY[parity],
                                      NORMALIZATION[normalization], layout,
                                      ctypes.byref(handle)), "o2mi_tp_plan_create")
        self._lib = lib
        self.handle = handle
        self.width = int(lib.o2mi_tp_width(handle))
        self.weight_numel = int(lib.o2mi_tp_weight_numel(handle))
        # Plans beyond the compiled m_max run the table-driven kernels, which
        # read the op's path_info / path_coefficients device tables.
        self.compiled = lib.o2mi_tp_plan_compiled(handle) == 1

    def __del__(self):
        handle = getattr(self, "handle", None)
        if handle is not None and handle.value:
            try:
                self._lib.o2mi_tp_plan_destroy(handle)
            except Exception:  # interpreter shutdown
                pass
            self.handle = None

    def forward(self, x, y, w, out, n_rows: int, stream: int) -> None:
        check(self._lib.o2mi_tp_forward_f32(self.handle, x, y, w, out, n_rows, stream),
              "o2mi_tp_forward_f32")

    def launch_shape(self, n_rows: int, backward: bool) -> dict:
        """Grid, resident blocks per CU, rows per iteration, tiles (needs a GPU)."""
        vals = [ctypes.c_int() for _ in range(4)]
        check(self._lib.o2mi_tp_launch_shape(self.handle, n_rows, int(backward),
                                             *[ctypes.byref(v) for v in vals]),
              "o2mi_tp_launch_shape")
        return dict(zip(("grid", "blocks_per_cu", "rows_per_iter", "tiles"),
                        (v.value for v in vals)))

    def workspace_bytes(self, n_rows: int) -> int:
        return int(self._lib.o2mi_tp_backward_workspace_bytes(self.handle, n_rows))

    def backward(self, x, y, w, g, dx, dy, dw, workspace, workspace_bytes: int, n_rows: int,
                 needed: int, stream: int) -> None:
        check(self._lib.o2mi_tp_backward_f32(self.handle, x, y, w, g, dx, dy, dw, workspace,
                                             workspace_bytes, n_rows, needed, stream),
              "o2mi_tp_backward_f32")


class TablesCall:
    """Table-driven entry points of a plan (any m_max)."""

    def __init__(self, plan: TPNativePlan, path_info, path_coefficients, n_paths: int):
        self.plan, self.info, self.coef, self.n_paths = plan, path_info, path_coefficients, n_paths

    def forward(self, x, y, w, out, n_rows: int, stream: int) -> None:
        lib = self.plan._lib
        check(lib.o2mi_tp_forward_tables_f32(self.plan.handle, x, y, w, self.info, self.coef,
                                             self.n_paths, out, n_rows, stream),
              "o2mi_tp_forward_tables_f32")

    def workspace_bytes(self, n_rows: int) -> int:
        return int(self.plan._lib.o2mi_tp_backward_tables_workspace_bytes(self.plan.handle,
                                                                          n_rows))

    def backward(self, x, y, w, g, dx, dy, dw, workspace, workspace_bytes: int, n_rows: int,
                 needed: int, stream: int) -> None:
        lib = self.plan._lib
        check(lib.o2mi_tp_backward_tables_f32(self.plan.handle, x, y, w, g, self.info, self.coef,
                                              self.n_paths, dx, dy, dw, workspace,
                                              workspace_bytes, n_rows, needed, stream),
              "o2mi_tp_backward_tables_f32")


def compiled_table(m_max: int, parity: str, normalization: str):
    """(paths int32 [P, 7], magnitudes f32 [P], terms int32 [T, 4]) compiled
    into the library; host-only, needs no GPU."""
    import numpy as np
    lib = library()
    n_paths, n_terms = ctypes.c_int(), ctypes.c_int()
    check(lib.o2mi_tp_table(m_max, PARITY[parity], NORMALIZATION[normalization],
                            ctypes.byref(n_paths), ctypes.byref(n_terms), None, None, None),
          "o2mi_tp_table")
    paths = np.zeros((n_paths.value, 7), dtype=np.int32)
    mags = np.zeros(n_paths.value, dtype=np.float32)
    terms = np.zeros((n_terms.value, 4), dtype=np.int32)
    check(lib.o2mi_tp_table(m_max, PARITY[parity], NORMALIZATION[normalization],
                            ctypes.byref(n_paths), ctypes.byref(n_terms),
                            paths.ctypes.data, mags.ctypes.data, terms.ctypes.data),
          "o2mi_tp_table")
    return paths, mags, terms


def kernel_timing(enable: bool) -> None:
    """Record HIP events around every main forward/backward kernel."""
    check(library().o2mi_kernel_timing(1 if enable else 0), "o2mi_kernel_timing")


def kernel_timing_read():
    """(forward_ms_total, forward_count, backward_ms_total, backward_count)."""
    f_ms, b_ms = ctypes.c_double(), ctypes.c_double()
    f_n, b_n = ctypes.c_int(), ctypes.c_int()
    check(library().o2mi_kernel_timing_read(ctypes.byref(f_ms), ctypes.byref(f_n),
                                            ctypes.byref(b_ms), ctypes.byref(b_n)),
          "o2mi_kernel_timing_read")
    return f_ms.value, f_n.value, b_ms.value, b_n.value


TIMED_KINDS = ("tp_forward", "tp_backward", "radial_forward", "radial_backward", "radial_weight",
               "uvu_forward", "uvu_backward")


def kernel_timing_read_kinds() -> dict:
    """{kind: (total_ms, count)} of the launches timed since the previous read."""
    n = len(TIMED_KINDS)
    ms = (ctypes.c_double * n)()
    counts = (ctypes.c_int * n)()
    check(library().o2mi_kernel_timing_read_kinds(ms, counts, n), "o2mi_kernel_timing_read_kinds")
    return {kind: (ms[i], counts[i]) for i, kind in enumerate(TIMED_KINDS)}
