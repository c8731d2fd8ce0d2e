"""launchSpmmInt8NoAlloc (include/spmm.h) against launchSpmmInt8 with a caller workspace, through
the C ABI: two calls in a row on one GPU, the second on a smaller plan, so the second reuses the
scratch the first left behind (counters must be cleared, partial tiles overwritten)."""
import numpy as np
import pytest

import tcc_spmm_amd as T
from gpu_cases import assert_close, features, gpu_prepare

pytestmark = pytest.mark.gpu


def _split_heavy_csr():
    """t4000_40_9 with three rows referencing all 4,000 sources: two split SWs."""
    csr = T.synth_csr("t4000_40_9")
    rng = np.random.default_rng(4)
    off = csr.row_offsets.astype(np.int64)
    rows_cols = [csr.source_ids[off[r]:off[r + 1]] for r in range(csr.rows)]
    rows_vals = [csr.values[off[r]:off[r + 1]] for r in range(csr.rows)]
    for r in (5, 40, 41):
        rows_cols[r] = np.arange(0, csr.cols, dtype=np.uint32)
        rows_vals[r] = rng.uniform(0.1, 1.0, csr.cols).astype(np.float32)
    new_off = np.concatenate([[0], np.cumsum([len(c) for c in rows_cols])]).astype(np.uint32)
    return T.make_canonical_csr(csr.rows, csr.cols, new_off, np.concatenate(rows_cols),
                                np.concatenate(rows_vals))


def test_noalloc_matches_workspace_entry_on_two_calls(oracle, gpu):
    import torch
    from tcc_spmm_amd.device import TorchDeviceMatrix, launch_spmm_int8_noalloc
    cases = [("c2 F256", T.synth_csr("c2"), 256, 202), ("split-heavy F128", _split_heavy_csr(), 128, 78)]
    sizes = []
    for name, csr, feats, seed in cases:
        print(f"no-alloc case: {name}", flush=True)
        fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
        assert fmt.partial_count > 0
        sizes.append(fmt.partial_count * feats)
        packed, scale, _, sc, pk = gpu_prepare(features(csr.cols, feats, seed=seed), gpu)
        dm = TorchDeviceMatrix(fmt, feats, device=gpu)
        y_ws = torch.full((csr.rows, feats), float("nan"), device=gpu)
        dm.partials.fill_(float("nan"))
        dm.spmm(packed, scale, y_ws)
        outs = []
        for it in range(2):  # the repeat starts from the counters and tiles this call leaves
            y = torch.full((csr.rows, feats), float("nan"), device=gpu)
            if it == 0:
                launch_spmm_int8_noalloc(dm.view, packed, scale, y, csr.rows, csr.cols, feats,
                                         fmt.partial_count)
            else:  # the matrix object passes its own plan's partial count
                dm.spmm_noalloc(packed, scale, y)
            outs.append(y)
        torch.cuda.synchronize()
        want = y_ws.cpu().numpy()
        for y in outs:
            assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32)), name
        y_ref = oracle.spmm_csr_f64(csr.rows, csr.row_offsets, csr.source_ids, csr.values, pk, sc,
                                    csr.cols)
        assert_close(outs[0].cpu().numpy(), y_ref, name)
    assert sizes[1] < sizes[0]  # the second plan is the smaller one
