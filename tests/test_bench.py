"""bench.py's accounting and argument handling (host only).

The roofline numerator is checked against the byte sizes of the uploaded format arrays (every array but
windowOffsets, each counted once), so a dropped or double-counted term in the formula fails here.
"""
import subprocess
import sys

import numpy as np

import bench
import tcc_spmm_amd as T
from conftest import ROOT


def _split_format():
    rng = np.random.default_rng(3)
    rows, cols = 150, 5000
    lists = [np.unique(rng.integers(0, cols, 12)) for _ in range(rows)]
    lists[9] = np.arange(0, cols, 2)      # 2,500 sources: 313 panels in SW 0's RW1 bucket
    lists[70] = np.arange(cols)           # 5,000 sources: a second split SW
    off = np.concatenate([[0], np.cumsum([len(c) for c in lists])]).astype(np.uint32)
    src = np.concatenate(lists).astype(np.uint32)
    val = rng.uniform(-1, 1, src.size).astype(np.float32)
    csr = T.make_canonical_csr(rows, cols, off, src, val)
    return csr, T.convert_csr_to_sw32(rows, cols, csr)


def test_algorithmic_bytes_equal_the_uploaded_arrays():
    csr, fmt = _split_format()
    a = fmt.arrays()
    assert fmt.partial_count > 0
    read_once = sum(a[k].nbytes for k in ("values", "source_ids", "source_metadata",
                                          "row_group_masks", "bucket_offsets", "tasks",
                                          "reductions", "partial_ids"))
    assert a["tasks"].itemsize == 28 and a["reductions"].itemsize == 8
    distinct = np.unique(csr.source_ids).size
    for feats in (128, 256):
        b = bench.algorithmic_bytes(fmt, csr.source_ids, feats)
        assert b["B_A"] == read_once
        assert b["B_X"] == distinct * feats + 4 * distinct          # int8 row + fp32 scale
        assert b["B_Y"] == csr.rows * feats * 4
        assert b["B_P"] == 2 * fmt.partial_count * 8 * feats * 4    # written once, read once
        assert b["B_alg"] == b["B_A"] + b["B_X"] + b["B_Y"] + b["B_P"]
        assert b["split_tasks"] == int(np.count_nonzero(a["tasks"]["partial"] != T.NO_PARTIAL))


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and not r.stdout.strip()
