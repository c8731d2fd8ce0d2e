"""ctypes binding of libtcc_spmm.so (declarations mirror include/tcc_spmm_c.h).

The library is built in-tree by ``python -m tcc_spmm_amd.build``. Importing this module loads it;
if it is missing, every entry point raises instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib

# TCC_SPMM_LIB selects another build of the library (the sanitizer build of tcc_spmm_amd.build).
LIB_PATH = pathlib.Path(os.environ.get("TCC_SPMM_LIB") or
                        pathlib.Path(__file__).resolve().parent / "libtcc_spmm.so")

u32p = C.POINTER(C.c_uint32)
u64p = C.POINTER(C.c_uint64)
f32p = C.POINTER(C.c_float)
i8p = C.POINTER(C.c_int8)


class DeviceView(C.Structure):
    """Layout of Sw32DeviceView / tcc_device_view (10 pointer-sized fields + taskCount)."""

    _fields_ = [
        ("windowOffsets", C.c_void_p),
        ("sourceIds", C.c_void_p),
        ("rowGroupMasks", C.c_void_p),
        ("sourceMetadata", C.c_void_p),
        ("values", C.c_void_p),
        ("bucketOffsets", C.c_void_p),
        ("tasks", C.c_void_p),
        ("reductions", C.c_void_p),
        ("partialIds", C.c_void_p),
        ("taskCount", C.c_uint32),
    ]


class Sw32Sizes(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("cols", C.c_uint32), ("partialCount", C.c_uint32),
                ("bucketed", C.c_uint32)] + [
        (n, C.c_uint64) for n in ("windowOffsets", "sourceIds", "rowGroupMasks", "sourceMetadata",
                                  "values", "bucketOffsets", "tasks", "reductions", "partialIds")]


class Sw32Arrays(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "windowOffsets", "sourceIds", "rowGroupMasks", "sourceMetadata", "values", "bucketOffsets",
        "tasks", "reductions", "partialIds")]


# Every exported symbol with (restype, argtypes). Tests check the library exports exactly these.
SIGNATURES = {
    "tcc_last_error": (C.c_char_p, []),
    "tcc_version": (C.c_char_p, []),
    "tcc_make_canonical_csr": (C.c_int, [C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p,
                                         C.c_void_p, C.POINTER(C.c_void_p)]),
    "tcc_load_matrix_market": (C.c_int, [C.c_char_p, u32p, u32p, C.POINTER(C.c_void_p)]),
    "tcc_csr_from_arrays": (C.c_int, [C.c_uint64, C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p,
                                      C.POINTER(C.c_void_p)]),
    "tcc_csr_info": (C.c_int, [C.c_void_p, u64p, u64p]),
    "tcc_csr_arrays": (C.c_int, [C.c_void_p, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p),
                                 C.POINTER(C.c_void_p)]),
    "tcc_csr_free": (None, [C.c_void_p]),
    "tcc_convert_csr_to_sw32": (C.c_int, [C.c_uint32, C.c_uint32, C.c_void_p, C.c_int,
                                          C.POINTER(C.c_void_p)]),
    "tcc_build_panel_tasks": (C.c_int, [C.c_void_p]),
    "tcc_sw32_get_sizes": (C.c_int, [C.c_void_p, C.POINTER(Sw32Sizes)]),
    "tcc_sw32_get_arrays": (C.c_int, [C.c_void_p, C.POINTER(Sw32Arrays)]),
    "tcc_sw32_free": (None, [C.c_void_p]),
    "tcc_launch_spmm_int8": (C.c_int, [C.POINTER(DeviceView), C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p,
                                       C.c_void_p]),
    "tcc_launch_spmm_int8_noalloc": (C.c_int, [C.POINTER(DeviceView), C.c_void_p, C.c_void_p,
                                               C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32,
                                               C.c_uint32, C.c_void_p]),
    "tcc_set_spmm_launch_overrides": (C.c_int, [C.c_uint32, C.c_int]),
    "tcc_quantize_features_int8": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32,
                                             C.c_uint32, C.c_void_p]),
    "tcc_pack_features_int8x16": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32,
                                            C.c_void_p]),
    "tcc_quantize_pack_features_int8": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32,
                                                  C.c_uint32, C.c_void_p]),
    "tcc_device_matrix_create": (C.c_int, [C.c_void_p, C.c_uint32, C.POINTER(C.c_void_p)]),
    "tcc_device_matrix_view": (C.c_int, [C.c_void_p, C.POINTER(DeviceView),
                                         C.POINTER(C.c_void_p), C.POINTER(C.c_void_p)]),
    "tcc_device_matrix_free": (None, [C.c_void_p]),
    "tcc_synth_csr": (C.c_int, [C.c_char_p, u32p, u32p, C.POINTER(C.c_void_p)]),
    "tcc_synth_features": (C.c_int, [C.c_uint32, C.c_uint32, C.c_uint64, C.c_float, C.c_float,
                                     C.c_float, C.c_void_p]),
}

_lib = None


def lib() -> C.CDLL:
    """Load libtcc_spmm.so once (raises OSError with a build hint when it is missing)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise OSError(f"{LIB_PATH} is missing: run `python -m tcc_spmm_amd.build` first")
        # One HIP runtime per process: PyTorch ships its own libamdhip64, and a library loaded
        # before it binds the system copy, after which the two runtimes do not share the device
        # (calls through the library then report "no ROCm-capable device"). Importing torch first
        # makes the library bind torch's runtime, the one torch tensors and streams belong to.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int) -> None:
    """Map a status code of the C ABI to the exception class the C++ API throws."""
    if status == 0:
        return
    message = lib().tcc_last_error().decode(errors="replace")
    if status == 1:
        raise ValueError(message)  # std::invalid_argument
    if status == 2:
        raise OverflowError(message)  # std::overflow_error
    raise RuntimeError(message)  # std::runtime_error and anything else
