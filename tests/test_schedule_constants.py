"""The kernel's dispatch-order constants and their restatements agree: the tail-window length and the
size-class thresholds of tcc_spmm_amd/csrc/kernel/spmm.hip (kTailWindow, sizeClass), the L2 model
(model/l2_model.c: TAIL_WINDOW, size_class) and the Python restatements in tests/. A change to the
kernel's order that left the model or the mapping tests behind would otherwise go unnoticed."""
import pathlib
import re

import test_l2_model
import test_task_mapping

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _body(text, start):
    i = text.index(start)
    return text[i:text.index("}", i)]


def test_tail_window_and_classes_agree():
    kernel = (ROOT / "tcc_spmm_amd" / "csrc" / "kernel" / "spmm.hip").read_text()
    model = (ROOT / "model" / "l2_model.c").read_text()
    window = int(re.search(r"constexpr unsigned kTailWindow = (\d+);", kernel).group(1))
    assert int(re.search(r"TAIL_WINDOW = (\d+)", model).group(1)) == window
    assert test_task_mapping.TAIL_WINDOW == window == test_l2_model.TAIL_WINDOW
    kernel_th = [int(v) for v in re.findall(r"p >= (\d+)", _body(kernel, "unsigned sizeClass("))]
    model_th = [int(v) for v in re.findall(r"p >= (\d+)", _body(model, "static uint32_t size_class("))]
    assert kernel_th == model_th == list(test_l2_model.CLASS_THRESHOLDS) == [96, 192, 288]
    import numpy as np
    probe = np.array([0, 95, 96, 191, 192, 287, 288, 384])
    assert test_task_mapping._size_class(probe).tolist() == [sum(int(p >= t) for t in kernel_th) for p in probe]
