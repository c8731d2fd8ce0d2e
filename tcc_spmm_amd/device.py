"""Device-side API on torch tensors (Python mirror of include/spmm.h and
include/format/int8_features.h).

PyTorch only provides device memory and the stream; every computation runs in the HIP kernels of
libtcc_spmm.so, reached through its C ABI. There is no fallback path: if the library or a GPU is
missing the calls raise.
"""
from __future__ import annotations

import contextlib
import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from ._lib import DeviceView, check, lib
from .format import Sw32HostFormat


def _stream_ptr(stream) -> int:
    if stream is None:
        stream = torch.cuda.current_stream()
    return int(stream.cuda_stream)


def _ptr(t) -> int:
    return 0 if t is None else int(t.data_ptr())


def _require_cuda(*tensors) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("device entry points take CUDA (HIP) tensors")


def _require_same_device(device, *tensors) -> None:
    for t in tensors:
        if t is not None and t.device != device:
            raise ValueError(f"tensor on {t.device}, expected {device}")


def _require_buffer(t, name: str, dtype, min_elements: int) -> None:
    """A kernel reads or writes `min_elements` elements of `t` from its first element: the tensor
    must have that dtype, be contiguous and hold at least that many elements. The kernels take
    their bounds from the sizes passed alongside (rows, cols, features), never from the allocation,
    so a short buffer would be read or written out of bounds."""
    if t is None:
        raise ValueError(f"{name} is required")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.numel() < min_elements:
        raise ValueError(f"{name} holds {t.numel()} elements, needs at least {min_elements}")


def quantize_features_int8(x: torch.Tensor, q: torch.Tensor | None = None,
                           scale: torch.Tensor | None = None, stream=None):
    """quantizeFeaturesInt8 (reference include/format/int8_features.cuh:9-10).

    x: float32 [sources, features] on the GPU. Returns (q int8 [sources, features], scale f32).
    """
    if x.dtype != torch.float32 or x.dim() != 2 or not x.is_contiguous():
        raise ValueError("x must be a contiguous float32 [sources, features] tensor")
    sources, features = x.shape
    if q is not None:
        _require_buffer(q, "q", torch.int8, sources * features)
    if scale is not None:
        _require_buffer(scale, "scale", torch.float32, sources)
    _require_cuda(x, q, scale)
    _require_same_device(x.device, q, scale)
    q = torch.empty((sources, features), dtype=torch.int8, device=x.device) if q is None else q
    scale = torch.empty(sources, dtype=torch.float32, device=x.device) if scale is None else scale
    check(lib().tcc_quantize_features_int8(_ptr(x), _ptr(q), _ptr(scale), sources, features,
                                           _stream_ptr(stream)))
    return q, scale


def pack_features_int8x16(q: torch.Tensor, packed: torch.Tensor | None = None, stream=None):
    """packFeaturesInt8x16 (reference include/format/int8_features.cuh:14-15)."""
    if q.dtype != torch.int8 or q.dim() != 2 or not q.is_contiguous():
        raise ValueError("q must be a contiguous int8 [sources, features] tensor")
    sources, features = q.shape
    if packed is not None:
        _require_buffer(packed, "packed", torch.int8, sources * features)
    _require_cuda(q, packed)
    _require_same_device(q.device, packed)
    packed = torch.empty_like(q) if packed is None else packed
    check(lib().tcc_pack_features_int8x16(_ptr(q), _ptr(packed), sources, features,
                                          _stream_ptr(stream)))
    return packed


def quantize_pack_features_int8(x: torch.Tensor, packed: torch.Tensor | None = None,
                                scale: torch.Tensor | None = None, stream=None):
    """quantizePackFeaturesInt8 (include/format/int8_features.h; no counterpart in the reference):
    quantize_features_int8 then pack_features_int8x16 in one pass, bit-identical to that pair.

    x: float32 [sources, features] on the GPU, features % 16 == 0. Returns (packed int8
    [sources, features], scale f32)."""
    if x.dtype != torch.float32 or x.dim() != 2 or not x.is_contiguous():
        raise ValueError("x must be a contiguous float32 [sources, features] tensor")
    sources, features = x.shape
    if packed is not None:
        _require_buffer(packed, "packed", torch.int8, sources * features)
    if scale is not None:
        _require_buffer(scale, "scale", torch.float32, sources)
    _require_cuda(x, packed, scale)
    _require_same_device(x.device, packed, scale)
    packed = (torch.empty((sources, features), dtype=torch.int8, device=x.device)
              if packed is None else packed)
    scale = torch.empty(sources, dtype=torch.float32, device=x.device) if scale is None else scale
    check(lib().tcc_quantize_pack_features_int8(_ptr(x), _ptr(packed), _ptr(scale), sources,
                                                features, _stream_ptr(stream)))
    return packed, scale


def _check_operands(packed_x, scales, output, rows: int, cols: int, features: int,
                    workspace=None) -> None:
    """Layout and size first, then the device, so that every rejection happens before a launch.

    Of the workspace contract (reference include/spmm.cuh:5-13) the view leaves these checkable:
    partials are contiguous float32; counters are contiguous int32 with ceil(rows/32) *
    features/128 elements. The partial count is the plan's, so sizing the partials is the caller's.
    """
    _require_buffer(packed_x, "packed_x", torch.int8, cols * features)
    _require_buffer(scales, "scales", torch.float32, cols)
    _require_buffer(output, "output", torch.float32, rows * features)
    partials = counters = None
    if workspace is not None:
        partials, counters = workspace.partials, workspace.counters
        if partials is not None and (partials.dtype != torch.float32 or
                                     not partials.is_contiguous()):
            raise ValueError("workspace partials must be a contiguous float32 tensor")
        if counters is not None:
            _require_buffer(counters, "workspace counters", torch.int32,
                            (rows + 31) // 32 * max(features // 128, 1))
    _require_cuda(packed_x, scales, output, partials, counters)
    _require_same_device(packed_x.device, scales, output, partials, counters)


@dataclass
class SpmmWorkspace:
    """SpmmWorkspace{partials, counters} (reference include/spmm.cuh:10-13) as torch tensors."""

    partials: torch.Tensor | None
    counters: torch.Tensor | None


def launch_spmm_int8(view: DeviceView, packed_x: torch.Tensor, scales: torch.Tensor,
                     output: torch.Tensor, rows: int, cols: int, features: int,
                     workspace: SpmmWorkspace | None = None, stream=None) -> None:
    """launchSpmmInt8 (reference include/spmm.cuh:21-23): asynchronous on `stream`.

    Raises ValueError before any launch unless packed_x (int8, >= cols * features elements),
    scales (float32, >= cols) and output (float32, >= rows * features) are contiguous tensors on
    one GPU, with a workspace (when given) of contiguous float32 partials and int32 counters of at
    least ceil(rows/32) * features/128 elements on that GPU; the feature count itself is checked by
    the library (128 or 256, invalid_argument).
    """
    ws = workspace or SpmmWorkspace(None, None)
    _check_operands(packed_x, scales, output, rows, cols, features, ws)
    check(lib().tcc_launch_spmm_int8(C.byref(view), _ptr(packed_x), _ptr(scales), _ptr(output),
                                     rows, cols, features, _ptr(ws.partials), _ptr(ws.counters),
                                     _stream_ptr(stream)))


def launch_spmm_int8_noalloc(view: DeviceView, packed_x: torch.Tensor, scales: torch.Tensor,
                             output: torch.Tensor, rows: int, cols: int, features: int,
                             partial_count: int, stream=None) -> None:
    """launchSpmmInt8NoAlloc (include/spmm.h; no counterpart in the reference): launchSpmmInt8
    with the split-SW workspace in the library's own per-GPU scratch, allocating nothing.
    partial_count is the plan's Sw32HostFormat.partial_count. Calls that overlap on one GPU race."""
    _check_operands(packed_x, scales, output, rows, cols, features)
    check(lib().tcc_launch_spmm_int8_noalloc(C.byref(view), _ptr(packed_x), _ptr(scales),
                                             _ptr(output), rows, cols, features, partial_count,
                                             _stream_ptr(stream)))


@contextlib.contextmanager
def launch_overrides(task_waves: int = 0, force_wide: bool = False):
    """setSpmmLaunchOverrides (include/spmm.h; no counterpart in the reference) for the body of a
    with-block, then back to automatic choices: task_waves 0 (automatic), 1 or 2 waves per task;
    force_wide selects the 64-bit-addressing kernel instance for any size. Process-wide; for tests
    and measurements."""
    check(lib().tcc_set_spmm_launch_overrides(task_waves, int(force_wide)))
    try:
        yield
    finally:
        check(lib().tcc_set_spmm_launch_overrides(0, 0))


class TorchDeviceMatrix:
    """Uploads every array of a bucketed Sw32HostFormat into torch tensors and builds the view.

    The workspace is allocated like the reference's DeviceMatrix (src/device_matrix.cuh:21-27):
    partials = partialCount * 8 * features floats, counters = nSW * features/128 zeroed uint32,
    both only when the plan has split SWs. Tests may poison or inspect them.
    """

    def __init__(self, fmt: Sw32HostFormat, features: int, device="cuda"):
        if not fmt.bucketed:
            raise ValueError("launchSpmmInt8 needs the RW-bucketed SW32 format")
        arrs = fmt.arrays(copy=False)
        self.rows, self.cols = fmt.rows, fmt.cols
        self.features = features
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.tensors = {}
        for name, arr in arrs.items():
            raw = np.ascontiguousarray(arr).view(np.uint8).copy()
            self.tensors[name] = torch.from_numpy(raw).to(device) if raw.size else None
        self.task_count = int(arrs["tasks"].shape[0])
        windows = int(arrs["window_offsets"].shape[0]) - 1
        k = self.partial_count = fmt.partial_count
        if k:
            self.partials = torch.empty(k * 8 * features, dtype=torch.float32, device=device)
            self.counters = torch.zeros(windows * (features // 128), dtype=torch.int32,
                                        device=device)
        else:
            self.partials = self.counters = None
        t = self.tensors
        self.view = DeviceView(
            _ptr(t["window_offsets"]), _ptr(t["source_ids"]), _ptr(t["row_group_masks"]),
            _ptr(t["source_metadata"]), _ptr(t["values"]), _ptr(t["bucket_offsets"]),
            _ptr(t["tasks"]), _ptr(t["reductions"]), _ptr(t["partial_ids"]), self.task_count)

    def workspace(self) -> SpmmWorkspace:
        return SpmmWorkspace(self.partials, self.counters)

    def spmm(self, packed_x: torch.Tensor, scales: torch.Tensor, output: torch.Tensor | None = None,
             stream=None) -> torch.Tensor:
        if output is None:
            output = torch.empty((self.rows, self.features), dtype=torch.float32,
                                 device=packed_x.device)
        _require_same_device(self.device, packed_x)
        launch_spmm_int8(self.view, packed_x, scales, output, self.rows, self.cols, self.features,
                         self.workspace(), stream)
        return output

    def spmm_noalloc(self, packed_x: torch.Tensor, scales: torch.Tensor,
                     output: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        """launch_spmm_int8_noalloc with the uploaded plan's own partial count (a wrong count is
        undefined behaviour in the free function, which cannot check it)."""
        if output is None:
            output = torch.empty((self.rows, self.features), dtype=torch.float32,
                                 device=packed_x.device)
        _require_same_device(self.device, packed_x)
        launch_spmm_int8_noalloc(self.view, packed_x, scales, output, self.rows, self.cols,
                                 self.features, self.partial_count, stream)
        return output


class NativeDeviceMatrix:
    """DeviceMatrix owned by the library (tcc_device_matrix_*): hipMalloc'd arrays + workspace."""

    def __init__(self, fmt: Sw32HostFormat, features: int):
        self._h = C.c_void_p()
        check(lib().tcc_device_matrix_create(fmt.handle, features, C.byref(self._h)))
        self.view = DeviceView()
        p, c = C.c_void_p(), C.c_void_p()
        check(lib().tcc_device_matrix_view(self._h, C.byref(self.view), C.byref(p), C.byref(c)))
        self.partials_ptr, self.counters_ptr = p.value or 0, c.value or 0
        self.rows, self.cols, self.features = fmt.rows, fmt.cols, features
        self.partial_count = fmt.partial_count
        # The library uploads to the device current at creation.
        self.device = torch.device("cuda", torch.cuda.current_device())

    def __del__(self):
        if getattr(self, "_h", None):
            lib().tcc_device_matrix_free(self._h)
            self._h = None

    def spmm(self, packed_x: torch.Tensor, scales: torch.Tensor, output: torch.Tensor,
             stream=None) -> torch.Tensor:
        _check_operands(packed_x, scales, output, self.rows, self.cols, self.features)
        _require_same_device(self.device, packed_x)
        check(lib().tcc_launch_spmm_int8(C.byref(self.view), _ptr(packed_x), _ptr(scales),
                                         _ptr(output), self.rows, self.cols, self.features,
                                         self.partials_ptr, self.counters_ptr,
                                         _stream_ptr(stream)))
        return output

    def spmm_noalloc(self, packed_x: torch.Tensor, scales: torch.Tensor, output: torch.Tensor,
                     stream=None) -> torch.Tensor:
        """launch_spmm_int8_noalloc with the uploaded plan's own partial count."""
        _require_same_device(self.device, packed_x)
        launch_spmm_int8_noalloc(self.view, packed_x, scales, output, self.rows, self.cols,
                                 self.features, self.partial_count, stream)
        return output
