"""Argument checks of the torch-facing device API (tcc_spmm_amd.device), on the CPU.

The kernels take their bounds from rows / cols / features, never from the allocations, so every
device entry point must reject a tensor of the wrong dtype, layout or size before it reaches the
library. These checks run before the device check, so CPU tensors exercise them without a GPU.
"""
import pytest
import torch

from tcc_spmm_amd._lib import DeviceView
from tcc_spmm_amd.device import (SpmmWorkspace, launch_spmm_int8, pack_features_int8x16,
                                 quantize_features_int8)

ROWS, COLS, F = 40, 48, 128


def _operands():
    return (torch.zeros((COLS, F), dtype=torch.int8), torch.ones(COLS, dtype=torch.float32),
            torch.zeros((ROWS, F), dtype=torch.float32))


def _launch(packed, scales, out, workspace=None):
    launch_spmm_int8(DeviceView(), packed, scales, out, ROWS, COLS, F, workspace)


@pytest.mark.parametrize("which,bad,match", [
    (0, torch.zeros((COLS, F), dtype=torch.uint8), "packed_x must be torch.int8"),
    (0, torch.zeros((F, COLS), dtype=torch.int8).t(), "packed_x must be contiguous"),
    (0, torch.zeros((COLS - 1, F), dtype=torch.int8), "packed_x holds"),
    (1, torch.ones(COLS, dtype=torch.float64), "scales must be torch.float32"),
    (1, torch.ones(COLS - 1, dtype=torch.float32), "scales holds"),
    (1, torch.ones(2 * COLS, dtype=torch.float32)[::2], "scales must be contiguous"),
    (2, torch.zeros((ROWS, F), dtype=torch.float16), "output must be torch.float32"),
    (2, torch.zeros((ROWS, F - 1), dtype=torch.float32), "output holds"),
    (2, None, "output is required"),
])
def test_launch_rejects_malformed_operands(which, bad, match):
    ops = list(_operands())
    ops[which] = bad
    with pytest.raises(ValueError, match=match):
        _launch(*ops)


def test_launch_rejects_host_tensors():
    with pytest.raises(ValueError, match="CUDA"):
        _launch(*_operands())


def test_launch_accepts_larger_buffers_before_the_device_check():
    packed = torch.zeros((COLS + 3, F), dtype=torch.int8)
    scales = torch.ones(COLS + 3, dtype=torch.float32)
    out = torch.zeros((ROWS + 1, F), dtype=torch.float32)
    with pytest.raises(ValueError, match="CUDA"):
        _launch(packed, scales, out, SpmmWorkspace(None, None))


@pytest.mark.parametrize("partials,counters,match", [
    (torch.zeros(8 * F, dtype=torch.float64), None, "partials must be a contiguous float32"),
    (torch.zeros((F, 8), dtype=torch.float32).t(), None, "partials must be a contiguous float32"),
    (None, torch.zeros(2, dtype=torch.int64), "counters must be torch.int32"),
    # ceil(40 / 32) = 2 SWs, one counter each at F = 128
    (None, torch.zeros(1, dtype=torch.int32), "counters holds 1 elements, needs at least 2"),
    (torch.zeros(8 * F, dtype=torch.float32), torch.zeros(2, dtype=torch.int32), "CUDA"),
])
def test_launch_rejects_malformed_workspace(partials, counters, match):
    with pytest.raises(ValueError, match=match):
        _launch(*_operands(), SpmmWorkspace(partials, counters))


@pytest.mark.parametrize("q,scale,match", [
    (torch.zeros((COLS, F), dtype=torch.uint8), None, "q must be torch.int8"),
    (torch.zeros((COLS, F - 1), dtype=torch.int8), None, "q holds"),
    (None, torch.ones(COLS - 1, dtype=torch.float32), "scale holds"),
    (None, torch.ones(COLS, dtype=torch.float64), "scale must be torch.float32"),
    (None, None, "CUDA"),
])
def test_quantize_rejects_malformed_outputs(q, scale, match):
    x = torch.zeros((COLS, F), dtype=torch.float32)
    with pytest.raises(ValueError, match=match):
        quantize_features_int8(x, q, scale)


def test_quantize_rejects_malformed_input():
    with pytest.raises(ValueError, match="contiguous float32"):
        quantize_features_int8(torch.zeros((COLS, F), dtype=torch.float64))
    with pytest.raises(ValueError, match="contiguous float32"):
        quantize_features_int8(torch.zeros((F, COLS), dtype=torch.float32).t())


@pytest.mark.parametrize("packed,match", [
    (torch.zeros((COLS, F - 16), dtype=torch.int8), "packed holds"),
    (torch.zeros((COLS, F), dtype=torch.float32), "packed must be torch.int8"),
    (None, "CUDA"),
])
def test_pack_rejects_malformed_output(packed, match):
    q = torch.zeros((COLS, F), dtype=torch.int8)
    with pytest.raises(ValueError, match=match):
        pack_features_int8x16(q, packed)
