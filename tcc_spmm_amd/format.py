"""Host-side SW32 format API (Python mirror of include/format/csr.h and include/format/sw32.h).

Names follow the reference's C++ surface: make_canonical_csr <-> makeCanonicalCsr,
load_matrix_market <-> loadMatrixMarket, convert_csr_to_sw32 <-> convertCsrToSw32,
Sw32HostFormat.build_panel_tasks <-> buildPanelTasks. Errors raise ValueError
(std::invalid_argument), OverflowError (std::overflow_error) or RuntimeError (std::runtime_error),
the classes the reference throws. All work happens in libtcc_spmm.so.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import Sw32Arrays, Sw32Sizes, check, lib

# sw32BucketOrder and sw32TaskPanelLimit (reference include/format/sw32.h:9-12).
SW32_BUCKET_ORDER = (0, 1, 2, 4, 8, 3, 5, 6, 7, 9, 10, 11, 12, 13, 14, 15)
SW32_TASK_PANEL_LIMIT = 384
NO_PARTIAL = 0xFFFFFFFF

TASK_DTYPE = np.dtype([(n, "<u4") for n in ("sw", "begin", "end", "partial", "mask", "chunks",
                                            "reduceFirst")])
REDUCE_DTYPE = np.dtype([("begin", "<u4"), ("end", "<u4")])


def _view(ptr: int, count: int, dtype) -> np.ndarray:
    dtype = np.dtype(dtype)
    if count == 0 or not ptr:
        return np.zeros(0, dtype=dtype)
    buf = (C.c_char * (count * dtype.itemsize)).from_address(ptr)
    return np.frombuffer(buf, dtype=dtype, count=count)


class CsrMatrix:
    """Owns a canonical CSR (CsrMatrix, reference include/format/csr.h:7-10)."""

    def __init__(self, handle: C.c_void_p, rows: int, cols: int):
        self._h = handle
        self.rows = rows
        self.cols = cols

    def __del__(self):
        if getattr(self, "_h", None):
            lib().tcc_csr_free(self._h)
            self._h = None

    def _arrays(self):
        n_off, nnz = C.c_uint64(), C.c_uint64()
        check(lib().tcc_csr_info(self._h, C.byref(n_off), C.byref(nnz)))
        po, ps, pv = C.c_void_p(), C.c_void_p(), C.c_void_p()
        check(lib().tcc_csr_arrays(self._h, C.byref(po), C.byref(ps), C.byref(pv)))
        return (_view(po.value, n_off.value, np.uint32), _view(ps.value, nnz.value, np.uint32),
                _view(pv.value, nnz.value, np.float32))

    # Properties return copies; views() gives zero-copy arrays tied to this object's lifetime.
    def views(self):
        return self._arrays()

    @property
    def row_offsets(self) -> np.ndarray:
        return self._arrays()[0].copy()

    @property
    def source_ids(self) -> np.ndarray:
        return self._arrays()[1].copy()

    @property
    def values(self) -> np.ndarray:
        return self._arrays()[2].copy()

    @property
    def nnz(self) -> int:
        return int(self._arrays()[0][-1])


def make_canonical_csr(rows: int, cols: int, row_offsets, source_ids, values) -> CsrMatrix:
    """makeCanonicalCsr (reference src/format/csr.cpp:6-40)."""
    ro = np.ascontiguousarray(row_offsets, dtype=np.uint32)
    si = np.ascontiguousarray(source_ids, dtype=np.uint32)
    va = np.ascontiguousarray(values, dtype=np.float32)
    if ro.size != rows + 1 and rows > 0:
        raise ValueError("row_offsets must have rows + 1 entries")
    if si.size != va.size:
        raise ValueError("source_ids and values differ in length")
    nnz = int(ro[-1]) if ro.size else 0
    if nnz > si.size:
        raise ValueError("row_offsets point past the entry arrays")
    h = C.c_void_p()
    check(lib().tcc_make_canonical_csr(rows, cols, nnz, ro.ctypes.data, si.ctypes.data,
                                       va.ctypes.data, C.byref(h)))
    return CsrMatrix(h, rows, cols)


def csr_from_arrays(rows: int, cols: int, row_offsets, source_ids, values) -> CsrMatrix:
    """A CsrMatrix filled directly from arrays, without canonicalisation (the reference's CsrMatrix
    is a plain struct); convert_csr_to_sw32 validates it."""
    ro = np.ascontiguousarray(row_offsets, dtype=np.uint32)
    si = np.ascontiguousarray(source_ids, dtype=np.uint32)
    va = np.ascontiguousarray(values, dtype=np.float32)
    if si.size != va.size:
        raise ValueError("source_ids and values differ in length")
    h = C.c_void_p()
    check(lib().tcc_csr_from_arrays(ro.size, ro.ctypes.data, si.size, si.ctypes.data,
                                    va.ctypes.data, C.byref(h)))
    return CsrMatrix(h, rows, cols)


def load_matrix_market(path: str) -> CsrMatrix:
    """loadMatrixMarket (reference src/format/matrix_market.cpp:30-103)."""
    rows, cols, h = C.c_uint32(), C.c_uint32(), C.c_void_p()
    check(lib().tcc_load_matrix_market(str(path).encode(), C.byref(rows), C.byref(cols),
                                       C.byref(h)))
    return CsrMatrix(h, rows.value, cols.value)


def synth_csr(config: str) -> CsrMatrix:
    """Deterministic synthetic workload ("c1".."c5" or "t<rows>_<deg>_<seed>")."""
    rows, cols, h = C.c_uint32(), C.c_uint32(), C.c_void_p()
    check(lib().tcc_synth_csr(config.encode(), C.byref(rows), C.byref(cols), C.byref(h)))
    return CsrMatrix(h, rows.value, cols.value)


def synth_features(sources: int, features: int, seed: int, stddev: float = 1.0,
                   outlier_fraction: float = 0.0, outlier_scale: float = 1.0) -> np.ndarray:
    """N(0, stddev^2) FP32 features [sources, features] from the library's deterministic PRNG."""
    out = np.empty((sources, features), dtype=np.float32)
    check(lib().tcc_synth_features(sources, features, seed, stddev, outlier_fraction,
                                   outlier_scale, out.ctypes.data))
    return out


class Sw32HostFormat:
    """Owns a Sw32HostFormat (reference include/format/sw32.h:22-39); arrays are numpy views."""

    _ARRAYS = (("window_offsets", "windowOffsets", np.uint32),
               ("source_ids", "sourceIds", np.uint32),
               ("row_group_masks", "rowGroupMasks", np.uint32),
               ("source_metadata", "sourceMetadata", np.uint64),
               ("values", "values", np.float32),
               ("bucket_offsets", "bucketOffsets", np.uint32),
               ("tasks", "tasks", TASK_DTYPE),
               ("reductions", "reductions", REDUCE_DTYPE),
               ("partial_ids", "partialIds", np.uint32))

    def __init__(self, handle: C.c_void_p):
        self._h = handle

    def __del__(self):
        if getattr(self, "_h", None):
            lib().tcc_sw32_free(self._h)
            self._h = None

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def sizes(self) -> Sw32Sizes:
        s = Sw32Sizes()
        check(lib().tcc_sw32_get_sizes(self._h, C.byref(s)))
        return s

    def arrays(self, copy: bool = True) -> dict:
        """All arrays by name. copy=False returns views that are valid only while this object
        lives (and until build_panel_tasks re-plans)."""
        s = self.sizes()
        a = Sw32Arrays()
        check(lib().tcc_sw32_get_arrays(self._h, C.byref(a)))
        out = {py: _view(getattr(a, c), getattr(s, c), dt) for py, c, dt in self._ARRAYS}
        return {k: v.copy() for k, v in out.items()} if copy else out

    def __getattr__(self, name):
        for py, _, _ in self._ARRAYS:
            if name == py:
                return self.arrays(copy=True)[py]
        raise AttributeError(name)

    @property
    def rows(self) -> int:
        return self.sizes().rows

    @property
    def cols(self) -> int:
        return self.sizes().cols

    @property
    def partial_count(self) -> int:
        return self.sizes().partialCount

    @property
    def bucketed(self) -> bool:
        return bool(self.sizes().bucketed)

    def build_panel_tasks(self) -> None:
        """buildPanelTasks (reference src/format/sw32.cpp:25-65) — re-plan in place."""
        check(lib().tcc_build_panel_tasks(self._h))

    def stats(self) -> dict:
        s = self.sizes()
        tasks = self.tasks
        split = int(np.count_nonzero(tasks["partial"] != NO_PARTIAL)) if tasks.size else 0
        return {"rows": s.rows, "cols": s.cols, "nnz": int(s.values), "sw": int(s.windowOffsets - 1),
                "panels": int(s.rowGroupMasks), "slots": int(s.sourceIds), "tasks": int(s.tasks),
                "split_tasks": split, "split_sw": int(s.reductions // 4),
                "partial_count": int(s.partialCount)}


def convert_csr_to_sw32(rows: int, cols: int, csr: CsrMatrix,
                        bucket_by_rw_mask: bool = True) -> Sw32HostFormat:
    """convertCsrToSw32 (reference src/format/sw32.cpp:69-167)."""
    h = C.c_void_p()
    check(lib().tcc_convert_csr_to_sw32(rows, cols, csr._h, int(bool(bucket_by_rw_mask)),
                                        C.byref(h)))
    return Sw32HostFormat(h)
