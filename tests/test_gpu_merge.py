"""The split-SW merge against the oracle on SWs split into many chunks.

The last arriver of a split SW sums the SW's partial tiles in partialIds order, batching the loads of
several tiles and reading the tile ids 64 at a time. This plan makes every path of that loop run: an
SW split into more than 64 chunks (two batches of tile ids, an odd remainder), row groups of one SW
with different chunk counts, and a ragged last SW whose merge must not write rows past the end."""
import numpy as np
import pytest

import tcc_spmm_amd as T
from gpu_cases import assert_close_conditioned, features, gpu_prepare

pytestmark = pytest.mark.gpu


def _many_chunk_csr():
    rng = np.random.default_rng(7)
    rows, cols = 70, 240_000
    long_rows = {3: 220_000, 20: 30_000, 40: 30_000, 67: 140_000}
    offsets = np.zeros(rows + 1, np.uint32)
    sources, values = [], []
    for r in range(rows):
        d = long_rows.get(r, int(rng.integers(0, 12)))
        c = np.sort(rng.choice(cols, d, replace=False)).astype(np.uint32)
        v = rng.uniform(-1.0, 1.0, d).astype(np.float32)
        v[v == 0] = 0.5
        sources.append(c)
        values.append(v)
        offsets[r + 1] = offsets[r] + d
    return rows, cols, offsets, np.concatenate(sources), np.concatenate(values)


@pytest.mark.parametrize("waves", ["1", "2"])
@pytest.mark.parametrize("feats", [128, 256])
def test_merge_of_many_chunks(oracle, gpu, feats, waves, launch_overrides):
    launch_overrides(task_waves=int(waves))
    import torch
    from tcc_spmm_amd.device import TorchDeviceMatrix
    rows, cols, off, src, val = _many_chunk_csr()
    csr = T.make_canonical_csr(rows, cols, off, src, val)
    fmt = T.convert_csr_to_sw32(rows, cols, csr)
    tasks = fmt.tasks
    assert int(tasks["chunks"].max()) > 64 and int(tasks["chunks"].max()) % 2 == 1
    reductions = fmt.reductions
    items = reductions["end"].astype(np.int64) - reductions["begin"].astype(np.int64)
    assert items.max() > 64 and len(np.unique(items[items > 0])) > 2
    print(f"merge plan: {len(tasks)} tasks, chunks up to {int(tasks['chunks'].max())}, F{feats}, "
          f"waves {waves}", flush=True)
    x = features(cols, feats, seed=11, stddev=1.0, outlier_fraction=0.0, outlier_scale=1.0)
    packed, scale, _, sc, pk = gpu_prepare(x, gpu)
    dm = TorchDeviceMatrix(fmt, feats, device=gpu)
    dm.partials.fill_(float("nan"))
    y = torch.full((rows + 3, feats), float("nan"), device=gpu)  # 3 guard rows past the end
    dm.spmm(packed, scale, y[:rows])
    torch.cuda.synchronize()
    assert int(dm.counters.abs().sum()) == 0
    assert torch.isnan(y[rows:]).all(), "the merge wrote rows past the matrix"
    of = oracle.sw32(rows, cols, *csr.views())
    windows = np.arange(len(fmt.window_offsets) - 1, dtype=np.uint32)
    y_ref, y_abs = of.spmm_windows_f64(pk, sc, windows, with_abs=True)
    relaxed = assert_close_conditioned(y[:rows].cpu().numpy(), y_ref[:rows], y_abs[:rows],
                                       f"many-chunk merge F{feats} waves {waves}")
    assert relaxed <= rows * feats * 1e-3, f"{relaxed} elements needed the conditioning term"
