"""ctypes access to the CPU checker — TEST INFRASTRUCTURE ONLY.

Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product.

  Oracle     the C restatement in tcc_oracle.c (oracle/_build/liboracle.so)
  RefFormat  the reference's own CPU format code compiled from /root/reference sources
             (oracle/_ref/libref_format.so), present only where it was built.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
# TCC_ORACLE_LIB selects another build of the checker (the sanitizer build: make -C oracle san).
ORACLE_SO = pathlib.Path(os.environ.get("TCC_ORACLE_LIB") or HERE / "_build" / "liboracle.so")
REF_SO = HERE / "_ref" / "libref_format.so"

TASK_DTYPE = np.dtype([(n, "<u4") for n in ("sw", "begin", "end", "partial", "mask", "chunks",
                                            "reduceFirst")])
REDUCE_DTYPE = np.dtype([("begin", "<u4"), ("end", "<u4")])
FORMAT_FIELDS = ("window_offsets", "source_ids", "row_group_masks", "source_metadata", "values",
                 "bucket_offsets", "tasks", "reductions", "partial_ids")


class _OrcSw32(C.Structure):
    _fields_ = [
        ("rows", C.c_uint32), ("cols", C.c_uint32),
        ("windowOffsets", C.c_void_p), ("nWindowOffsets", C.c_size_t),
        ("sourceIds", C.c_void_p), ("nSlots", C.c_size_t),
        ("sourceMetadata", C.c_void_p),
        ("rowGroupMasks", C.c_void_p), ("nPanels", C.c_size_t),
        ("values", C.c_void_p), ("nValues", C.c_size_t),
        ("bucketOffsets", C.c_void_p), ("nBucketOffsets", C.c_size_t),
        ("tasks", C.c_void_p), ("nTasks", C.c_size_t),
        ("reductions", C.c_void_p), ("nReductions", C.c_size_t),
        ("partialIds", C.c_void_p), ("nPartialIds", C.c_size_t),
        ("partialCount", C.c_uint32),
    ]


class _CheckStats(C.Structure):
    _fields_ = [
        ("checked", C.c_uint64), ("bad", C.c_uint64), ("relaxed", C.c_uint64),
        ("maxErr", C.c_double), ("firstBad", C.c_uint64),
        ("firstGot", C.c_double), ("firstWant", C.c_double), ("firstBound", C.c_double),
    ]


def _view(ptr, count, dtype):
    dtype = np.dtype(dtype)
    if not count or not ptr:
        return np.zeros(0, dtype=dtype)
    buf = (C.c_char * (count * dtype.itemsize)).from_address(ptr)
    return np.frombuffer(buf, dtype=dtype, count=count)


def _copy(ptr, count, dtype):
    return _view(ptr, count, dtype).copy()


def _sha256(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).view(np.uint8)).hexdigest()


def csr_digests(offsets, sources, values) -> dict:
    """SHA-256 of the three CsrMatrix arrays and the entry count."""
    return {"row_offsets": _sha256(np.asarray(offsets, np.uint32)),
            "source_ids": _sha256(np.asarray(sources, np.uint32)),
            "values": _sha256(np.asarray(values, np.float32)), "nnz": int(np.asarray(sources).size)}


def format_digests(arrays: dict, partial_count: int) -> dict:
    """SHA-256 of every Sw32HostFormat array (bytes as laid out in memory) plus the plan's counts:
    SWs, panels, slots, values, tasks, partial tiles (K) and split SWs (4 reductions each)."""
    d = {name: _sha256(arrays[name]) for name in FORMAT_FIELDS}
    d["counts"] = {"windows": int(len(arrays["window_offsets"])) - 1,
                   "panels": int(len(arrays["row_group_masks"])),
                   "slots": int(len(arrays["source_ids"])), "values": int(len(arrays["values"])),
                   "tasks": int(len(arrays["tasks"])), "partial_count": int(partial_count),
                   "split_sws": int(len(arrays["reductions"])) // 4}
    return d


def build() -> None:
    """make -C oracle (C restatement; reference format code when /root/reference exists)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


class OracleError(Exception):
    def __init__(self, code, message=""):
        super().__init__(f"oracle status {code}" + (f": {message}" if message else ""))
        self.code = code
        self.message = message


class Oracle:
    def __init__(self):
        if not ORACLE_SO.exists():
            build()
        self.so = C.CDLL(str(ORACLE_SO))
        so = self.so
        so.orc_tf32.restype = C.c_float
        so.orc_tf32.argtypes = [C.c_float]
        so.orc_sw32_convert.argtypes = [C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p,
                                        C.c_int, C.POINTER(_OrcSw32)]
        so.orc_sw32_free.argtypes = [C.POINTER(_OrcSw32)]
        so.orc_canonical_csr.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p,
                                         C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                         C.POINTER(C.c_uint32)]
        for name in ("orc_quantize", "orc_pack16", "orc_unpack16"):
            getattr(so, name).restype = None
        so.orc_spmm_csr_f64.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                        C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p]
        so.orc_spmm_sw32_f64.argtypes = [C.POINTER(_OrcSw32), C.c_void_p, C.c_void_p, C.c_uint32,
                                         C.c_void_p]
        so.orc_spmm_sw32_f64_windows.argtypes = [C.POINTER(_OrcSw32), C.c_void_p, C.c_void_p,
                                                 C.c_uint32, C.c_void_p, C.c_uint32, C.c_void_p,
                                                 C.c_void_p]
        so.orc_spmm_tasks_f32.argtypes = [C.POINTER(_OrcSw32), C.c_void_p, C.c_void_p, C.c_uint32,
                                          C.c_void_p, C.c_void_p]
        so.orc_spmm_sw32_f32_mt.argtypes = [C.POINTER(_OrcSw32), C.c_void_p, C.c_void_p,
                                            C.c_uint32, C.c_uint32, C.c_uint32, C.c_int, C.c_void_p]
        so.orc_spmm_sw32_f32_mt_path.argtypes = [C.POINTER(_OrcSw32), C.c_void_p, C.c_void_p,
                                                 C.c_uint32, C.c_uint32, C.c_uint32, C.c_int,
                                                 C.c_void_p, C.c_int]
        so.orc_cpu_has_avx2.restype = C.c_int
        so.orc_check_sw32_mt.argtypes = [C.POINTER(_OrcSw32), C.c_void_p, C.c_void_p, C.c_uint32,
                                         C.c_void_p, C.c_double, C.c_double, C.c_double, C.c_int,
                                         C.POINTER(_CheckStats), C.c_void_p]

    # ---- scalar helpers
    def tf32(self, v: float) -> float:
        return self.so.orc_tf32(v)

    def tf32_array(self, a: np.ndarray) -> np.ndarray:
        return np.array([self.so.orc_tf32(float(x)) for x in np.asarray(a, np.float32).ravel()],
                        dtype=np.float32).reshape(np.shape(a))

    # ---- CSR
    def canonical_csr(self, rows, cols, offsets, sources, values):
        off = np.ascontiguousarray(offsets, np.uint32)
        src = np.ascontiguousarray(sources, np.uint32)
        val = np.ascontiguousarray(values, np.float32)
        nnz = int(off[-1])
        oo = np.zeros(rows + 1, np.uint32)
        os_ = np.zeros(max(nnz, 1), np.uint32)
        ov = np.zeros(max(nnz, 1), np.float32)
        n = C.c_uint32()
        st = self.so.orc_canonical_csr(rows, cols, nnz, off.ctypes.data, src.ctypes.data,
                                       val.ctypes.data, oo.ctypes.data, os_.ctypes.data,
                                       ov.ctypes.data, C.byref(n))
        if st:
            raise OracleError(st)
        return oo, os_[:n.value].copy(), ov[:n.value].copy()

    # ---- SW32
    def sw32(self, rows, cols, offsets, sources, values, bucket=True) -> "OracleFormat":
        off = np.ascontiguousarray(offsets, np.uint32)
        src = np.ascontiguousarray(sources, np.uint32)
        val = np.ascontiguousarray(values, np.float32)
        f = _OrcSw32()
        st = self.so.orc_sw32_convert(rows, cols, off.ctypes.data, src.ctypes.data,
                                      val.ctypes.data, int(bucket), C.byref(f))
        if st:
            raise OracleError(st)
        return OracleFormat(self, f)

    # ---- features
    def quantize(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32)
        s, f = x.shape
        q = np.zeros((s, f), np.int8)
        sc = np.zeros(s, np.float32)
        self.so.orc_quantize(C.c_void_p(x.ctypes.data), C.c_void_p(q.ctypes.data),
                             C.c_void_p(sc.ctypes.data), C.c_uint32(s), C.c_uint32(f))
        return q, sc

    def pack16(self, q: np.ndarray) -> np.ndarray:
        q = np.ascontiguousarray(q, np.int8)
        out = np.zeros_like(q)
        self.so.orc_pack16(C.c_void_p(q.ctypes.data), C.c_void_p(out.ctypes.data),
                           C.c_uint32(q.shape[0]), C.c_uint32(q.shape[1]))
        return out

    def unpack16(self, p: np.ndarray) -> np.ndarray:
        p = np.ascontiguousarray(p, np.int8)
        out = np.zeros_like(p)
        self.so.orc_unpack16(C.c_void_p(p.ctypes.data), C.c_void_p(out.ctypes.data),
                             C.c_uint32(p.shape[0]), C.c_uint32(p.shape[1]))
        return out

    def spmm_csr_f64(self, rows, offsets, sources, values, packed, scales, cols):
        off = np.ascontiguousarray(offsets, np.uint32)
        src = np.ascontiguousarray(sources, np.uint32)
        val = np.ascontiguousarray(values, np.float32)
        packed = np.ascontiguousarray(packed, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        feats = packed.shape[1]
        y = np.zeros((rows, feats), np.float64)
        self.so.orc_spmm_csr_f64(rows, off.ctypes.data, src.ctypes.data, val.ctypes.data,
                                 packed.ctypes.data, scales.ctypes.data, cols, feats, y.ctypes.data)
        return y


class OracleFormat:
    """SW32 arrays produced by the C restatement."""

    def __init__(self, orc: Oracle, f: _OrcSw32):
        self._orc = orc
        self._f = f
        self.rows, self.cols, self.partial_count = f.rows, f.cols, f.partialCount

    def __del__(self):
        if getattr(self, "_f", None) is not None:
            self._orc.so.orc_sw32_free(C.byref(self._f))
            self._f = None

    def arrays(self, copy: bool = True) -> dict:
        """The nine arrays; copy=False gives views that live as long as this object."""
        f = self._f
        get = _copy if copy else _view
        return {
            "window_offsets": get(f.windowOffsets, f.nWindowOffsets, np.uint32),
            "source_ids": get(f.sourceIds, f.nSlots, np.uint32),
            "row_group_masks": get(f.rowGroupMasks, f.nPanels, np.uint32),
            "source_metadata": get(f.sourceMetadata, f.nSlots, np.uint64),
            "values": get(f.values, f.nValues, np.float32),
            "bucket_offsets": get(f.bucketOffsets, f.nBucketOffsets, np.uint32),
            "tasks": get(f.tasks, f.nTasks, TASK_DTYPE),
            "reductions": get(f.reductions, f.nReductions, REDUCE_DTYPE),
            "partial_ids": get(f.partialIds, f.nPartialIds, np.uint32),
        }

    def spmm_f64(self, packed, scales) -> np.ndarray:
        packed = np.ascontiguousarray(packed, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        y = np.zeros((self.rows, packed.shape[1]), np.float64)
        self._orc.so.orc_spmm_sw32_f64(C.byref(self._f), packed.ctypes.data, scales.ctypes.data,
                                       packed.shape[1], y.ctypes.data)
        return y

    def spmm_windows_f64(self, packed, scales, windows, with_abs=False):
        """Y rows of the listed SWs ([len(windows) * 32, F], rows past the end are 0); with_abs also
        returns sum |tf32(a) * xhat| per element."""
        packed = np.ascontiguousarray(packed, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        w = np.ascontiguousarray(windows, np.uint32)
        y = np.zeros((w.size * 32, packed.shape[1]), np.float64)
        ya = np.zeros_like(y) if with_abs else None
        self._orc.so.orc_spmm_sw32_f64_windows(C.byref(self._f), packed.ctypes.data,
                                               scales.ctypes.data, packed.shape[1], w.ctypes.data,
                                               w.size, y.ctypes.data,
                                               ya.ctypes.data if with_abs else None)
        return (y, ya) if with_abs else y

    def check_full(self, packed, scales, y, atol, rtol, cond=0.0, threads=8, with_ref=False):
        """Compare every element of y ([rows, F] float32) with the double reference, SW by SW on
        `threads` threads. Returns a dict of the counts (checked, bad, relaxed), max_err and the
        first bad element (index, got, want, bound); with_ref also returns the reference."""
        packed = np.ascontiguousarray(packed, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        y = np.ascontiguousarray(y, np.float32)
        feats = packed.shape[1]
        assert y.shape == (self.rows, feats)
        ref = np.empty((self.rows, feats), np.float64) if with_ref else None
        st = _CheckStats()
        rc = self._orc.so.orc_check_sw32_mt(C.byref(self._f), packed.ctypes.data,
                                            scales.ctypes.data, feats, y.ctypes.data, atol, rtol,
                                            cond, int(threads), C.byref(st),
                                            ref.ctypes.data if with_ref else None)
        if rc:
            raise OracleError(rc)
        out = {"checked": st.checked, "bad": st.bad, "relaxed": st.relaxed,
               "max_err": st.maxErr, "first_bad": None}
        if st.bad:
            out["first_bad"] = (divmod(int(st.firstBad), feats), st.firstGot, st.firstWant,
                                st.firstBound)
        return (out, ref) if with_ref else out

    def spmm_tasks_f32(self, packed, scales):
        packed = np.ascontiguousarray(packed, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        feats = packed.shape[1]
        y = np.full((self.rows, feats), np.nan, np.float32)
        part = np.full(max(self.partial_count, 1) * 8 * feats, np.nan, np.float32)
        self._orc.so.orc_spmm_tasks_f32(C.byref(self._f), packed.ctypes.data, scales.ctypes.data,
                                        feats, part.ctypes.data, y.ctypes.data)
        return y

    def spmm_f32_mt(self, packed, scales, sw_begin, sw_end, threads, y=None, vector=False):
        """FP32 SpMM of SWs [sw_begin, sw_end) on `threads` host threads; vector=True takes the
        AVX2 path (bitwise the same Y; RuntimeError when the CPU lacks AVX2 and FMA)."""
        packed = np.ascontiguousarray(packed, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        feats = packed.shape[1]
        if y is None:
            y = np.zeros((self.rows, feats), np.float32)
        used = self._orc.so.orc_spmm_sw32_f32_mt_path(C.byref(self._f), packed.ctypes.data,
                                                      scales.ctypes.data, feats, sw_begin, sw_end,
                                                      threads, y.ctypes.data, int(vector))
        if used < 0:
            raise RuntimeError("vector CPU path unavailable (needs AVX2 + FMA and features % 16 == 0)"
                               if used == -1 else "CPU SpMM worker out of memory")
        return y, used

    def has_vector_path(self) -> bool:
        return bool(self._orc.so.orc_cpu_has_avx2())


class RefFormat:
    """The reference's own makeCanonicalCsr / convertCsrToSw32 / loadMatrixMarket."""

    ARRAYS = ((0, "window_offsets", np.uint32), (1, "source_ids", np.uint32),
              (2, "row_group_masks", np.uint32), (3, "source_metadata", np.uint64),
              (4, "values", np.float32), (5, "bucket_offsets", np.uint32),
              (6, "tasks", TASK_DTYPE), (7, "reductions", REDUCE_DTYPE),
              (8, "partial_ids", np.uint32))

    @staticmethod
    def available() -> bool:
        return REF_SO.exists()

    def __init__(self):
        self.so = C.CDLL(str(REF_SO))
        so = self.so
        so.ref_last_error.restype = C.c_char_p
        so.ref_canonical_csr.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p,
                                         C.c_void_p, C.POINTER(C.c_void_p)]
        so.ref_load_matrix_market.argtypes = [C.c_char_p, C.POINTER(C.c_void_p)]
        so.ref_csr_info.argtypes = [C.c_void_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                                    C.POINTER(C.c_uint64)]
        so.ref_csr_copy.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        so.ref_csr_free.argtypes = [C.c_void_p]
        so.ref_convert.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p,
                                   C.c_void_p, C.c_int, C.POINTER(C.c_void_p)]
        so.ref_array.restype = C.c_uint64
        so.ref_array.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_void_p)]
        so.ref_partial_count.restype = C.c_uint32
        so.ref_partial_count.argtypes = [C.c_void_p]
        so.ref_free.argtypes = [C.c_void_p]

    def _csr_out(self, h):
        r, c, n = C.c_uint32(), C.c_uint32(), C.c_uint64()
        self.so.ref_csr_info(h, C.byref(r), C.byref(c), C.byref(n))
        off = np.zeros(r.value + 1, np.uint32)
        src = np.zeros(max(n.value, 1), np.uint32)
        val = np.zeros(max(n.value, 1), np.float32)
        self.so.ref_csr_copy(h, off.ctypes.data, src.ctypes.data, val.ctypes.data)
        self.so.ref_csr_free(h)
        return r.value, c.value, off, src[:n.value].copy(), val[:n.value].copy()

    def canonical_csr(self, rows, cols, offsets, sources, values):
        off = np.ascontiguousarray(offsets, np.uint32)
        src = np.ascontiguousarray(sources, np.uint32)
        val = np.ascontiguousarray(values, np.float32)
        h = C.c_void_p()
        st = self.so.ref_canonical_csr(rows, cols, int(off[-1]), off.ctypes.data, src.ctypes.data,
                                       val.ctypes.data, C.byref(h))
        if st:
            raise OracleError(st, self.so.ref_last_error().decode())
        return self._csr_out(h)[2:]

    def load_matrix_market(self, path):
        h = C.c_void_p()
        st = self.so.ref_load_matrix_market(str(path).encode(), C.byref(h))
        if st:
            raise OracleError(st, self.so.ref_last_error().decode())
        return self._csr_out(h)

    def convert(self, rows, cols, offsets, sources, values, bucket=True, digests=False) -> dict:
        """The reference's convertCsrToSw32 output: the nine arrays and partial_count, or with
        digests=True only format_digests() of them (no copies, for configuration-size inputs)."""
        off = np.ascontiguousarray(offsets, np.uint32)
        src = np.ascontiguousarray(sources, np.uint32)
        val = np.ascontiguousarray(values, np.float32)
        h = C.c_void_p()
        st = self.so.ref_convert(rows, cols, int(src.size), off.ctypes.data, src.ctypes.data,
                                 val.ctypes.data, int(bucket), C.byref(h))
        if st:
            raise OracleError(st, self.so.ref_last_error().decode())
        out = {}
        get = _view if digests else _copy
        for idx, name, dt in self.ARRAYS:
            p = C.c_void_p()
            nbytes = self.so.ref_array(h, idx, C.byref(p))
            out[name] = get(p.value, nbytes // np.dtype(dt).itemsize, dt)
        out["partial_count"] = int(self.so.ref_partial_count(h))
        if digests:
            out = format_digests(out, out["partial_count"])
        self.so.ref_free(h)
        return out
