"""GPU parity: the HIP path (through the C ABI) against the C oracle on the same seeded inputs.

Features: quantized scales and INT8 values and the packed16 bytes must be bit-identical.
SpMM: |Y - Y_ref| <= 1e-3 + 1e-4 |Y_ref| against the oracle's TF32-operand sum accumulated in
double. Protocol invariants: every Y element overwritten, counters back to zero, partials content
irrelevant, repeated launches bitwise identical.
"""
import os

import numpy as np
import pytest

import tcc_spmm_amd as T
from gpu_cases import (ATOL, RTOL, assert_close, assert_close_conditioned, check_features,
                       features, gpu_prepare)

pytestmark = pytest.mark.gpu

# Host threads of the full-size checks (a one-GPU box gets a 16-core share of its host).
CHECK_THREADS = max(1, min(16, os.cpu_count() or 1))
# Summation-conditioning factor of the checks with cancelling hub rows (assert_close_conditioned).
COND = 16.0


def _run(fmt, packed, scale, feats, device, poison=True):
    import torch
    from tcc_spmm_amd.device import TorchDeviceMatrix
    dm = TorchDeviceMatrix(fmt, feats, device=device)
    y = torch.full((dm.rows, feats), float("nan"), device=device)
    if dm.partials is not None and poison:
        dm.partials.fill_(float("nan"))
    dm.spmm(packed, scale, y)
    torch.cuda.synchronize()
    if dm.counters is not None:
        assert int(dm.counters.abs().sum()) == 0, "completion counters must return to zero"
    return dm, y.cpu().numpy()


def _golden_names(golden):
    return [str(x) for x in golden["index/format_cases"]]


@pytest.mark.parametrize("shape", [(1, 16), (37, 48), (1000, 128), (513, 256), (64, 1024)])
def test_quantize_and_pack_bit_exact(oracle, gpu, shape):
    s, f = shape
    x = features(s, f, seed=11 + s, stddev=3.0, outlier_fraction=0.05, outlier_scale=100.0)
    x[0] = 0.0  # all-zero row -> scale 1, q = 0
    if s > 2:
        x[1, :] = np.float32(0.5) * np.arange(f, dtype=np.float32)  # many exact .5 quotients
    packed, scale, q, sc, pk = gpu_prepare(x, gpu)
    check_features(oracle, x, q, sc, pk)
    assert sc[0] == 1.0 and not q[0].any()


@pytest.mark.parametrize("feats", [128, 256])
def test_spmm_golden_format_cases(oracle, golden, gpu, feats):
    for name in _golden_names(golden):
        rows, cols = (int(x) for x in golden[f"{name}/dims"])
        off, src, val = (golden[f"{name}/csr_offsets"], golden[f"{name}/csr_sources"],
                         golden[f"{name}/csr_values"])
        fmt = T.convert_csr_to_sw32(rows, cols, T.make_canonical_csr(rows, cols, off, src, val))
        x = features(cols, feats, seed=rows * 7 + cols, stddev=2.0)
        packed, scale, _, sc, pk = gpu_prepare(x, gpu)
        _, y = _run(fmt, packed, scale, feats, gpu)
        y_ref = oracle.sw32(rows, cols, off, src, val).spmm_f64(pk, sc)
        assert_close(y, y_ref, f"{name} F{feats}")


def test_spmm_c1(oracle, gpu):
    csr = T.synth_csr("c1")
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    x = features(csr.cols, 128, seed=0)
    packed, scale, q, sc, pk = gpu_prepare(x, gpu)
    check_features(oracle, x, q, sc, pk)
    _, y = _run(fmt, packed, scale, 128, gpu)
    off, src, val = csr.row_offsets, csr.source_ids, csr.values
    y_ref = oracle.spmm_csr_f64(csr.rows, off, src, val, pk, sc, csr.cols)
    assert_close(y, y_ref, "c1")


@pytest.mark.parametrize("feats", [128, 256])
def test_spmm_c2_full(oracle, gpu, feats):
    """Every output row of c2 (8.4M nnz, split SWs included); F256 runs both slices in one wave."""
    csr = T.synth_csr("c2")
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    assert fmt.partial_count > 0
    x = features(csr.cols, feats, seed=102 if feats == 128 else 202)
    packed, scale, _, sc, pk = gpu_prepare(x, gpu)
    _, y = _run(fmt, packed, scale, feats, gpu)
    y_ref = oracle.spmm_csr_f64(csr.rows, csr.row_offsets, csr.source_ids, csr.values, pk, sc,
                                csr.cols)
    assert_close(y, y_ref, f"c2 F{feats}")


@pytest.mark.parametrize("waves", ["1", "2"])
@pytest.mark.parametrize("feats", [128, 256])
def test_spmm_both_task_forms(oracle, golden, gpu, feats, waves, launch_overrides):
    """Each task form whatever the launch would pick (forced through setSpmmLaunchOverrides): one wave per task, or
    the task's panels shared by two waves whose accumulators wave 0 adds in wave order. On the
    split and bucket-edge golden cases and on c2: Y within tolerance of the oracle, counters back to
    zero (checked by _run), and a repeated launch bitwise identical."""
    launch_overrides(task_waves=int(waves))
    for case in ("empty_all", "single", "tail_33", "long_shared", "panels_384", "panels_385",
                 "split_mixed", "split_two"):
        rows, cols = (int(x) for x in golden[f"{case}/dims"])
        off, src, val = (golden[f"{case}/csr_offsets"], golden[f"{case}/csr_sources"],
                         golden[f"{case}/csr_values"])
        fmt = T.convert_csr_to_sw32(rows, cols, T.make_canonical_csr(rows, cols, off, src, val))
        x = features(cols, feats, seed=rows + 7 * cols, stddev=2.0)
        packed, scale, _, sc, pk = gpu_prepare(x, gpu)
        _, y = _run(fmt, packed, scale, feats, gpu)
        _, y_again = _run(fmt, packed, scale, feats, gpu)
        assert np.array_equal(y.view(np.uint32), y_again.view(np.uint32)), case
        y_ref = oracle.sw32(rows, cols, off, src, val).spmm_f64(pk, sc)
        assert_close(y, y_ref, f"{case} F{feats} waves {waves}")
    csr = T.synth_csr("c2")
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    x = features(csr.cols, feats, seed=302)
    packed, scale, _, sc, pk = gpu_prepare(x, gpu)
    _, y = _run(fmt, packed, scale, feats, gpu)
    y_ref = oracle.spmm_csr_f64(csr.rows, csr.row_offsets, csr.source_ids, csr.values, pk, sc,
                                csr.cols)
    assert_close(y, y_ref, f"c2 F{feats} waves {waves}")


def _check_windows(oracle, csr, fmt, y, pk, sc, windows, what, conditioned=False):
    of = oracle.sw32(csr.rows, csr.cols, *csr.views())
    y_ref, y_abs = of.spmm_windows_f64(pk, sc, windows, with_abs=True)
    relaxed = 0
    for i, w in enumerate(windows):
        r0, r1 = int(w) * 32, min(csr.rows, int(w) * 32 + 32)
        sl = slice(i * 32, i * 32 + (r1 - r0))
        if conditioned:
            relaxed += assert_close_conditioned(y[r0:r1], y_ref[sl], y_abs[sl],
                                                f"{what} SW {int(w)}")
        else:
            assert_close(y[r0:r1], y_ref[sl], f"{what} SW {int(w)}")
    return relaxed


def _check_full(oracle_fmt, y, pk, sc, what, cond=0.0):
    """Every element of y against the oracle's double reference (SW by SW on the host's cores)."""
    st = oracle_fmt.check_full(pk, sc, y, ATOL, RTOL, cond=cond, threads=CHECK_THREADS)
    assert st["checked"] == y.size
    assert st["bad"] == 0, (f"{what}: {st['bad']} elements out of tolerance, max err "
                            f"{st['max_err']}, first (row, feature), got, want, bound: "
                            f"{st['first_bad']}")
    return st


def test_spmm_c5_stress_f256(oracle, gpu):
    """Every element of c5 (hub SWs split 49 ways, empty rows, tail SW, x100 outlier rows)."""
    csr = T.synth_csr("c5")
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    x = features(csr.cols, 256, seed=105, stddev=2.0, outlier_fraction=0.01, outlier_scale=100.0)
    packed, scale, q, sc, pk = gpu_prepare(x, gpu)
    check_features(oracle, x, q, sc, pk)
    _, y = _run(fmt, packed, scale, 256, gpu)
    st = _check_full(oracle.sw32(csr.rows, csr.cols, *csr.views()), y, pk, sc, "c5",
                     cond=COND)
    print(f"c5: {st['relaxed']} of {st['checked']} elements needed the conditioning term, "
          f"max err {st['max_err']:.3g}")
    assert st["relaxed"] <= st["checked"] * 1e-3


@pytest.fixture(scope="module")
def c3_case(oracle):
    """c3's CSR, this build's format and the oracle's own format (built once for both widths)."""
    csr = T.synth_csr("c3")
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    return csr, fmt, oracle.sw32(csr.rows, csr.cols, *csr.views())


@pytest.mark.parametrize("feats", [128, 256])
def test_spmm_c3_full(oracle, gpu, c3_case, feats):
    """Every element of the north-star workload (2,449,029 x F, 126,167,053 nnz, ~2,000 split
    SWs) against the oracle."""
    csr, fmt, ofmt = c3_case
    x = features(csr.cols, feats, seed=103 if feats == 128 else 104)
    packed, scale, _, sc, pk = gpu_prepare(x, gpu)
    _, y = _run(fmt, packed, scale, feats, gpu)
    st = _check_full(ofmt, y, pk, sc, f"c3 F{feats}")
    print(f"c3 F{feats}: {st['checked']} elements, max err {st['max_err']:.3g}")


def _split_heavy_csr():
    """t4000_40_9 with rows 5, 40 and 41 referencing all 4,000 sources: two split SWs (500 panels
    each) among ordinary ones."""
    csr = T.synth_csr("t4000_40_9")
    rng = np.random.default_rng(4)
    off = csr.row_offsets.astype(np.int64)
    src, val = csr.source_ids, csr.values
    heavy = np.arange(0, csr.cols, dtype=np.uint32)
    rows_cols = [src[off[r]:off[r + 1]] for r in range(csr.rows)]
    rows_vals = [val[off[r]:off[r + 1]] for r in range(csr.rows)]
    for r in (5, 40, 41):
        rows_cols[r] = heavy
        rows_vals[r] = rng.uniform(0.1, 1.0, heavy.size).astype(np.float32)
    new_off = np.concatenate([[0], np.cumsum([len(c) for c in rows_cols])]).astype(np.uint32)
    return T.make_canonical_csr(csr.rows, csr.cols, new_off, np.concatenate(rows_cols),
                                np.concatenate(rows_vals))


def test_stream_reuse_and_overwrite(oracle, gpu):
    import torch
    from tcc_spmm_amd.device import TorchDeviceMatrix
    c2 = _split_heavy_csr()
    fmt = T.convert_csr_to_sw32(c2.rows, c2.cols, c2)
    assert fmt.partial_count > 0
    x = features(c2.cols, 256, seed=77)
    packed, scale, _, sc, pk = gpu_prepare(x, gpu)
    dm = TorchDeviceMatrix(fmt, 256, device=gpu)
    stream = torch.cuda.Stream()
    outs = []
    with torch.cuda.stream(stream):
        for it in range(3):
            y = torch.full((c2.rows, 256), float("nan"), device=gpu)
            dm.partials.fill_(float("nan") if it % 2 == 0 else 1e30)
            dm.spmm(packed, scale, y, stream=stream)
            outs.append(y)
    stream.synchronize()
    assert int(dm.counters.abs().sum()) == 0
    y0 = outs[0].cpu().numpy()
    for y in outs[1:]:
        assert np.array_equal(y.cpu().numpy().view(np.uint32), y0.view(np.uint32))
    y_ref = oracle.sw32(c2.rows, c2.cols, *c2.views()).spmm_f64(pk, sc)
    assert_close(y0, y_ref, "stream reuse")


@pytest.mark.parametrize("feats", [128, 256])
def test_concurrent_launches_with_separate_workspaces(oracle, gpu, feats):
    """Launches on two streams at once, each with its own workspace (the reference's contract for
    concurrent use, include/spmm.cuh:8-9), four back to back per stream with no host wait: every
    output matches the serial result bitwise and both counter arrays end at zero."""
    import torch
    from tcc_spmm_amd.device import TorchDeviceMatrix
    c2 = _split_heavy_csr()
    fmt = T.convert_csr_to_sw32(c2.rows, c2.cols, c2)
    x = features(c2.cols, feats, seed=78)
    packed, scale, _, sc, pk = gpu_prepare(x, gpu)
    _, y_serial = _run(fmt, packed, scale, feats, gpu)
    dms = [TorchDeviceMatrix(fmt, feats, device=gpu) for _ in range(2)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[torch.full((c2.rows, feats), float("nan"), device=gpu) for _ in range(4)]
            for _ in range(2)]
    torch.cuda.synchronize()
    for it in range(4):
        for k in range(2):
            with torch.cuda.stream(streams[k]):
                dms[k].spmm(packed, scale, outs[k][it], stream=streams[k])
    torch.cuda.synchronize()
    for k in range(2):
        assert int(dms[k].counters.abs().sum()) == 0
        for y in outs[k]:
            assert np.array_equal(y.cpu().numpy().view(np.uint32), y_serial.view(np.uint32))
    y_ref = oracle.sw32(c2.rows, c2.cols, *c2.views()).spmm_f64(pk, sc)
    assert_close(y_serial, y_ref, f"concurrent F{feats}")


@pytest.mark.parametrize("form", ["one wave", "two waves", "64-bit", "u16 packed X"])
@pytest.mark.parametrize("feats", [128, 256])
def test_spmm_float_aligned_output_and_partials(oracle, gpu, feats, form, launch_overrides):
    """Y and the workspace partials need only be float-aligned, as in the reference (it stores single
    floats, src/kernel/spmm_kernel.cuh:236-245): bases 4, 8 and 12 bytes past a 16-byte boundary, for
    either buffer or both, on a plan with split SWs, give Y bitwise equal to the aligned launch, leave
    the floats around Y untouched and the counters at zero; the allocation-free entry point takes
    such a Y as well. Every kernel instance compiles its own float-wise path: one and two waves per
    task, the 64-bit instance, and the u16 instance (packed X 2 bytes past a 16-byte boundary)."""
    import torch
    from tcc_spmm_amd.device import SpmmWorkspace, launch_spmm_int8, launch_spmm_int8_noalloc
    launch_overrides(task_waves=2 if form == "two waves" else 1, force_wide=form == "64-bit")
    c2 = _split_heavy_csr()
    fmt = T.convert_csr_to_sw32(c2.rows, c2.cols, c2)
    assert fmt.partial_count > 0
    x = features(c2.cols, feats, seed=79)
    packed, scale, _, sc, pk = gpu_prepare(x, gpu)
    if form == "u16 packed X":
        buf = torch.zeros(packed.numel() + 32, dtype=torch.int8, device=gpu)
        base = (16 - buf.data_ptr() % 16) % 16
        view = buf[base + 2: base + 2 + packed.numel()].view(packed.shape)
        view.copy_(packed)
        assert view.data_ptr() % 16 == 2
        packed = view
    dm, y_aligned = _run(fmt, packed, scale, feats, gpu)
    ny, npart = c2.rows * feats, dm.partials.numel()
    for oy, op in ((1, 1), (2, 2), (3, 3), (0, 1), (2, 0), (3, 2)):
        ybuf = torch.full((ny + 8,), float("nan"), device=gpu)
        pbuf = torch.full((npart + 8,), float("nan"), device=gpu)
        assert ybuf.data_ptr() % 16 == 0 and pbuf.data_ptr() % 16 == 0
        y, part = ybuf[oy:oy + ny], pbuf[op:op + npart]
        launch_spmm_int8(dm.view, packed, scale, y, c2.rows, c2.cols, feats,
                         SpmmWorkspace(part, dm.counters))
        torch.cuda.synchronize()
        assert int(dm.counters.abs().sum()) == 0, (oy, op)
        got = ybuf.cpu().numpy()
        assert np.array_equal(got[oy:oy + ny].view(np.uint32),
                              y_aligned.ravel().view(np.uint32)), (feats, form, oy, op)
        assert np.isnan(got[:oy]).all() and np.isnan(got[oy + ny:]).all(), (oy, op)
    ybuf = torch.full((ny + 8,), float("nan"), device=gpu)
    launch_spmm_int8_noalloc(dm.view, packed, scale, ybuf[1:1 + ny], c2.rows, c2.cols, feats,
                             fmt.partial_count)
    torch.cuda.synchronize()
    assert np.array_equal(ybuf[1:1 + ny].cpu().numpy().view(np.uint32),
                          y_aligned.ravel().view(np.uint32))
    y_ref = oracle.sw32(c2.rows, c2.cols, *c2.views()).spmm_f64(pk, sc)
    assert_close(y_aligned, y_ref, f"float-aligned F{feats} {form}")


@pytest.mark.parametrize("feats", [128, 256])
def test_spmm_view_over_a_later_part_of_the_task_list(gpu, feats, launch_overrides):
    """A view whose task list starts at a later SW (valid input: the reference maps blockIdx to a
    task directly) computes exactly those SWs' rows, bitwise as the whole launch does, and leaves
    the earlier rows untouched. On c2 the XCD ranges are panel-balanced, measured from the first
    task's begin."""
    import torch
    from tcc_spmm_amd._lib import DeviceView
    from tcc_spmm_amd.device import TorchDeviceMatrix, launch_spmm_int8
    launch_overrides(task_waves=1)
    csr = T.synth_csr("c2")
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    tasks = fmt.tasks
    # The first task of an SW a third of the way in (every chunk of a split SW stays in the view).
    first_of_sw = np.flatnonzero(np.diff(tasks["sw"].astype(np.int64), prepend=-1) != 0)
    cut = int(first_of_sw[first_of_sw.size // 3])
    sw0 = int(tasks["sw"][cut])
    packed, scale, *_ = gpu_prepare(features(csr.cols, feats, seed=81), gpu)
    dm, y_full = _run(fmt, packed, scale, feats, gpu)
    view = DeviceView.from_buffer_copy(dm.view)
    view.tasks = dm.view.tasks + cut * tasks.dtype.itemsize
    view.taskCount = tasks.size - cut
    y = torch.full((csr.rows, feats), float("nan"), device=gpu)
    launch_spmm_int8(view, packed, scale, y, csr.rows, csr.cols, feats, dm.workspace())
    torch.cuda.synchronize()
    assert int(dm.counters.abs().sum()) == 0
    got = y.cpu().numpy()
    assert np.isnan(got[:sw0 * 32]).all()
    assert np.array_equal(got[sw0 * 32:].view(np.uint32), y_full[sw0 * 32:].view(np.uint32))


@pytest.mark.parametrize("feats", [128, 256])
def test_launches_from_several_host_threads(gpu, feats):
    """launchSpmmInt8 keeps no per-call host state beyond read-only launch choices (the reference's
    free functions are callable from several host threads with distinct workspaces and streams): four
    host threads, each with its own stream and workspace, launching three times at once (the ctypes
    calls release the interpreter lock), give Y bitwise equal to a serial launch, and every counter
    array ends at zero."""
    import threading
    import torch
    from tcc_spmm_amd.device import TorchDeviceMatrix
    c2 = _split_heavy_csr()
    fmt = T.convert_csr_to_sw32(c2.rows, c2.cols, c2)
    packed, scale, *_ = gpu_prepare(features(c2.cols, feats, seed=83), gpu)
    _, y_serial = _run(fmt, packed, scale, feats, gpu)
    dms = [TorchDeviceMatrix(fmt, feats, device=gpu) for _ in range(4)]
    outs = [[torch.full((c2.rows, feats), float("nan"), device=gpu) for _ in range(3)] for _ in range(4)]
    torch.cuda.synchronize()
    errors = []

    def worker(i):
        try:
            torch.cuda.set_device(gpu)
            stream = torch.cuda.Stream(device=gpu)
            with torch.cuda.stream(stream):
                for y in outs[i]:
                    dms[i].spmm(packed, scale, y, stream=stream)
            stream.synchronize()
        except Exception as e:  # reported below, in the test's thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for i in range(4):
        assert int(dms[i].counters.abs().sum()) == 0
        for y in outs[i]:
            assert np.array_equal(y.cpu().numpy().view(np.uint32), y_serial.view(np.uint32)), i


def test_native_device_matrix_matches_torch_upload(gpu):
    import torch
    from tcc_spmm_amd.device import NativeDeviceMatrix
    csr = T.synth_csr("c1")
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    x = features(csr.cols, 128, seed=1)
    packed, scale, _, _, _ = gpu_prepare(x, gpu)
    _, y_torch = _run(fmt, packed, scale, 128, gpu)
    nm = NativeDeviceMatrix(fmt, 128)
    y = torch.empty((csr.rows, 128), device=gpu)
    nm.spmm(packed, scale, y)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), y_torch.view(np.uint32))


def test_bad_feature_count_raises_before_launch(gpu):
    import torch
    from tcc_spmm_amd.device import TorchDeviceMatrix, launch_spmm_int8
    csr = T.synth_csr("t64_4_1")
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    dm = TorchDeviceMatrix(fmt, 128, device=gpu)
    y = torch.zeros((64, 64), device=gpu)
    with pytest.raises(ValueError):
        launch_spmm_int8(dm.view, torch.zeros((64, 64), dtype=torch.int8, device=gpu),
                         torch.ones(64, device=gpu), y, 64, 64, 64)


def _fallback_entries(csr, scales):
    """Entries whose scaled f16 A operand tf32(a) * 2^(e + 10) (e: binary exponent of the source's
    scale, scale = m * 2^e with m in [0.5, 1)) leaves f16's normal range, or whose scale is
    subnormal: the panels holding them take the kernel's FP32 path."""
    from test_oracle import tf32_exact
    a = np.array([tf32_exact(float(v)) for v in csr.values])
    _, e = np.frexp(scales.astype(np.float64)[csr.source_ids])
    scaled = np.abs(np.ldexp(a, e + 10))
    return ((scaled < 2.0 ** -14) | (scaled >= 2.0 ** 16)
            | (scales[csr.source_ids] < np.float32(2.0 ** -126)))


@pytest.mark.parametrize("waves", ["1", "2"])
@pytest.mark.parametrize("feats", [128, 256])
def test_spmm_fp32_path_for_extreme_magnitudes(oracle, gpu, feats, waves, launch_overrides):
    """A values of 1e4, 1e-7 and 1e-30 and X rows scaled by 1e6, 1e-6 and into the subnormal range
    push some panels onto the FP32 path; Y must still match the oracle (summation-conditioned
    bound: the rows mix terms across 40 orders of magnitude). At F256 panels go in pairs through
    one MFMA, so flagged panels sit in either place of a pair and beside unflagged ones, and walks
    of every length modulo six end with and without an unpaired panel."""
    launch_overrides(task_waves=int(waves))
    base = T.synth_csr("t3000_24_11")
    rng = np.random.default_rng(12)
    val = base.values.copy()
    pick = rng.random(val.size)
    val[pick < 0.04] *= np.float32(1e4)
    val[(pick >= 0.04) & (pick < 0.08)] *= np.float32(1e-7)
    val[(pick >= 0.08) & (pick < 0.085)] *= np.float32(1e-30)
    csr = T.make_canonical_csr(base.rows, base.cols, base.row_offsets, base.source_ids, val)
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    x = features(csr.cols, feats, seed=21, stddev=1.0)
    rows = rng.permutation(csr.cols)
    x[rows[:60]] *= np.float32(1e6)
    x[rows[60:120]] *= np.float32(1e-6)
    x[rows[120:125]] *= np.float32(1e-39)   # subnormal features -> subnormal scales
    x[rows[125]] = 0.0
    packed, scale, q, sc, pk = gpu_prepare(x, gpu)
    check_features(oracle, x, q, sc, pk)
    flagged = _fallback_entries(csr, sc)
    assert 0.01 < flagged.mean() < 0.5, flagged.mean()
    _, y = _run(fmt, packed, scale, feats, gpu)
    assert np.isfinite(y).all()
    windows = np.arange(len(fmt.window_offsets) - 1, dtype=np.uint32)
    _check_windows(oracle, csr, fmt, y, pk, sc, windows, "extreme", conditioned=True)


def _walk_length_csr():
    """14 SWs: SW i has i + 1 panels in the exclusive bucket of row group i % 4 (its last panel short of
    a slot when i % 3 != 0) and (5 i) % 7 panels in the shared bucket of row groups {0, 1}; in SWs 4 to 7
    one entry in 16 is 1e6 times larger, so some panels, in either place of an F256 pair, take the FP32
    path."""
    rng = np.random.default_rng(7)
    nsw, cols = 14, 4096
    rows = 32 * nsw
    row_cols = [[] for _ in range(rows)]
    row_vals = [[] for _ in range(rows)]
    nxt = 0

    def add(r, c, big):
        v = float(rng.uniform(0.1, 1.0)) * float(rng.choice([-1.0, 1.0]))
        row_cols[r].append(c)
        row_vals[r].append(v * (1e6 if big and rng.random() < 1 / 16 else 1.0))

    for i in range(nsw):
        g, big = i % 4, 4 <= i < 8
        for c in range(nxt, nxt + 8 * (i + 1) - i % 3):
            add(32 * i + 8 * g + int(rng.integers(0, 8)), c, big)
        nxt += 8 * (i + 1) - i % 3
        for c in range(nxt, nxt + 8 * ((5 * i) % 7)):
            add(32 * i + int(rng.integers(0, 8)), c, big)
            add(32 * i + 8 + int(rng.integers(0, 8)), c, big)
        nxt += 8 * ((5 * i) % 7)
    off = np.zeros(rows + 1, np.uint32)
    src, val = [], []
    for r in range(rows):
        order = np.argsort(row_cols[r], kind="stable")
        src += [row_cols[r][j] for j in order]
        val += [row_vals[r][j] for j in order]
        off[r + 1] = len(src)
    return T.make_canonical_csr(rows, cols, off, np.array(src, np.uint32), np.array(val, np.float32))


@pytest.mark.parametrize("waves", ["1", "2"])
@pytest.mark.parametrize("feats", [128, 256])
def test_spmm_every_walk_length(oracle, gpu, feats, waves, launch_overrides):
    """Exclusive walks of 1 to 14 panels in every row group and shared walks of 0 to 6: every length
    modulo six of the F256 loop (panels in pairs, a loop of six, a last panel alone) and of the F128
    loop (pairs of panels), in both task forms (the two-wave form halves each walk)."""
    launch_overrides(task_waves=int(waves))
    csr = _walk_length_csr()
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    per = np.diff(fmt.bucket_offsets.reshape(-1, 17).astype(np.int64)[:, 1:17], axis=1)
    assert sorted(per[:, :4].max(axis=1).tolist()) == list(range(1, 15))
    assert sorted(set(per[:, 4:].sum(axis=1).tolist())) == list(range(7))
    x = features(csr.cols, feats, seed=31)
    packed, scale, q, sc, pk = gpu_prepare(x, gpu)
    assert _fallback_entries(csr, sc).any()
    _, y = _run(fmt, packed, scale, feats, gpu)
    windows = np.arange(len(fmt.window_offsets) - 1, dtype=np.uint32)
    _check_windows(oracle, csr, fmt, y, pk, sc, windows, "walk lengths")


@pytest.mark.parametrize("waves", ["1", "2"])
@pytest.mark.parametrize("feats", [128, 256])
def test_spmm_non_finite_scales(oracle, gpu, feats, waves, launch_overrides):
    """Scales of +inf, -inf and NaN (a caller may pass any scales). Such a slot's panel takes the FP32
    path, whose MFMA also multiplies the SW's absent entries (zeros) by the slot's non-finite
    features, so NaN may spread over rows of that SW that do not reference the source; the
    reference's tensor-core tiles do the same over their rows. Tiling-independent checks: every
    element the oracle makes non-finite is non-finite here, every finite element here matches the
    oracle, and SWs without such a source are all finite."""
    launch_overrides(task_waves=int(waves))
    csr = T.synth_csr("t2000_16_5")
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    x = features(csr.cols, feats, seed=9)
    packed, scale, _, sc, pk = gpu_prepare(x, gpu)
    bad = {3: float("inf"), 10: float("nan"), 20: float("-inf")}
    for c, v in bad.items():
        scale[c] = v
        sc[c] = v
    _, y = _run(fmt, packed, scale, feats, gpu)
    y_ref = oracle.spmm_csr_f64(csr.rows, csr.row_offsets, csr.source_ids, csr.values, pk, sc, csr.cols)
    assert np.isnan(y_ref).any() and np.isinf(y_ref).any()
    assert not np.isfinite(y[~np.isfinite(y_ref)]).any()
    fin = np.isfinite(y)
    assert np.isfinite(y_ref[fin]).all()
    assert_close(np.where(fin, y, 0.0), np.where(fin, y_ref, 0.0), "finite elements")
    off = csr.row_offsets.astype(np.int64)
    touched = np.zeros(csr.rows, bool)
    for r in range(csr.rows):
        touched[r] = np.isin(csr.source_ids[off[r]:off[r + 1]], list(bad)).any()
    sw = np.arange(csr.rows) // 32
    sw_has = np.zeros(sw[-1] + 1, bool)
    np.logical_or.at(sw_has, sw, touched)
    assert np.isfinite(y[~sw_has[sw]]).all()


@pytest.mark.parametrize("feats", [128, 256])
def test_spmm_huge_a_values_stay_finite(oracle, gpu, feats):
    """A values at and above 2^118 (where tf32(a) * 2^10 would overflow FP32) up to 3e38 and 2^127,
    one per row, with features in [-1, 1] so that every product the reference forms is finite.
    The sources of the huge entries have zero features (q = 0: a product inf * 0 would be NaN) and
    one of them is an all-zero row (scale 1, every q = 0). Y must be finite and match the oracle on
    every element with the plain bound."""
    base = T.synth_csr("t2000_20_13")
    rng = np.random.default_rng(14)
    off = base.row_offsets.astype(np.int64)
    val = base.values.copy()
    huge = np.array([2.0 ** 118, -(2.0 ** 118), 1.0e36, -1.0e36, 3.0e38, -3.0e38, 2.0 ** 127,
                     np.nextafter(np.float32(2.0 ** 118), np.float32(0))], np.float32)
    rows = rng.choice(base.rows, 240, replace=False)
    picked = []
    for i, r in enumerate(rows):
        if off[r + 1] > off[r]:
            e = int(rng.integers(off[r], off[r + 1]))
            val[e] = huge[i % huge.size]
            picked.append(e)
    csr = T.make_canonical_csr(base.rows, base.cols, base.row_offsets, base.source_ids, val)
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    x = rng.uniform(-1.0, 1.0, (csr.cols, feats)).astype(np.float32)
    huge_sources = np.unique(base.source_ids[np.array(picked)])
    x[huge_sources, ::3] = 0.0                      # q = 0 next to the huge A values
    x[huge_sources[0]] = 0.0                        # an all-zero row: scale 1, every q = 0
    packed, scale, q, sc, pk = gpu_prepare(x, gpu)
    check_features(oracle, x, q, sc, pk)
    assert (q[huge_sources][:, ::3] == 0).all()
    _, y = _run(fmt, packed, scale, feats, gpu)
    assert np.isfinite(y).all(), f"{int((~np.isfinite(y)).sum())} non-finite outputs"
    y_ref = oracle.sw32(csr.rows, csr.cols, *csr.views()).spmm_f64(pk, sc)
    assert np.isfinite(y_ref).all()
    assert np.abs(y_ref).max() > 1e37
    assert_close(y, y_ref, f"huge A F{feats}")


@pytest.mark.parametrize("feats", [128, 256])
def test_spmm_u16_aligned_packed_x(oracle, golden, gpu, feats, launch_overrides):
    """packedX need only be u16-aligned, as in the reference (include/format/int8_features.cuh:11-13):
    packed features placed 2, 6 and 14 bytes past a 16-byte boundary give Y bitwise equal to the
    aligned launch; an odd address raises invalid_argument before any launch. (The u16 instance
    runs one wave per task, so the aligned launch is held to one wave as well.)"""
    import torch
    from tcc_spmm_amd.device import TorchDeviceMatrix
    launch_overrides(task_waves=1)
    for case in ("tail_33", "all_masks", "split_mixed", "random_3"):
        rows, cols = (int(v) for v in golden[f"{case}/dims"])
        off, src, val = (golden[f"{case}/csr_offsets"], golden[f"{case}/csr_sources"],
                         golden[f"{case}/csr_values"])
        fmt = T.convert_csr_to_sw32(rows, cols, T.make_canonical_csr(rows, cols, off, src, val))
        x = features(cols, feats, seed=rows + 5 * cols, stddev=2.0)
        packed, scale, _, sc, pk = gpu_prepare(x, gpu)
        _, y_aligned = _run(fmt, packed, scale, feats, gpu)
        for shift in (2, 6, 14):
            buf = torch.zeros(cols * feats + 32, dtype=torch.int8, device=gpu)
            base = (16 - buf.data_ptr() % 16) % 16
            view = buf[base + shift: base + shift + cols * feats].view(cols, feats)
            view.copy_(packed)
            assert view.data_ptr() % 16 == shift
            _, y = _run(fmt, view, scale, feats, gpu)
            assert np.array_equal(y.view(np.uint32), y_aligned.view(np.uint32)), (case, shift)
        y_ref = oracle.sw32(rows, cols, off, src, val).spmm_f64(pk, sc)
        assert_close(y_aligned, y_ref, f"{case} F{feats}")
    dm = TorchDeviceMatrix(fmt, feats, device=gpu)
    odd = torch.zeros(cols * feats + 2, dtype=torch.int8, device=gpu)[1:1 + cols * feats]
    with pytest.raises(ValueError, match="u16-aligned"):
        dm.spmm(odd.view(cols, feats), scale, torch.empty((rows, feats), device=gpu))


def test_quantize_subnormal_and_huge_rows_bit_exact(oracle, gpu):
    """Subnormal features (down to a scale of a few hundred denormal quanta) and features near the
    top of the FP32 range quantize bit-exactly. Rows whose absmax / 127 underflows to zero
    (absmax < 127 * 2^-150) are outside the contract: the reference then rounds +-inf or NaN with
    lrintf, whose result C leaves unspecified."""
    x = features(64, 128, seed=31, stddev=1.0)
    x[1] *= np.float32(1e-39)      # subnormal inputs, subnormal scale
    x[2] *= np.float32(1e-41)      # scale of about a hundred denormal quanta
    x[3] *= np.float32(1e37)       # near the top of the FP32 range
    x[4, :] = np.float32(3.0e38)
    x[4, 1::2] = -np.float32(3.0e38)
    packed, scale, q, sc, pk = gpu_prepare(x, gpu)
    q_ref, s_ref = oracle.quantize(x)
    assert (s_ref > 0).all()
    bad = [r for r in range(x.shape[0])
           if sc[r].view(np.uint32) != s_ref[r].view(np.uint32) or not np.array_equal(q[r], q_ref[r])]
    assert not bad, f"rows differing from the oracle: {bad}"
    check_features(oracle, x, q, sc, pk)


@pytest.mark.parametrize("feats", [128, 256])
def test_spmm_wide_addressing_instance(oracle, golden, gpu, feats, launch_overrides):
    """The 64-bit-addressing kernel instance (taken when packed X exceeds 32-bit byte offsets) gives
    the same Y as the buffer-addressed one (both at one wave per task, the wide instance's only
    form)."""
    launch_overrides(task_waves=1)
    for case in ("single", "tail_33", "all_masks", "long_shared", "panels_385", "split_mixed",
                 "split_two", "random_3"):
        rows, cols = (int(x) for x in golden[f"{case}/dims"])
        off, src, val = (golden[f"{case}/csr_offsets"], golden[f"{case}/csr_sources"],
                         golden[f"{case}/csr_values"])
        fmt = T.convert_csr_to_sw32(rows, cols, T.make_canonical_csr(rows, cols, off, src, val))
        x = features(cols, feats, seed=rows + 3 * cols, stddev=2.0)
        packed, scale, _, sc, pk = gpu_prepare(x, gpu)
        _, y_narrow = _run(fmt, packed, scale, feats, gpu)
        launch_overrides(task_waves=1, force_wide=True)
        _, y_wide = _run(fmt, packed, scale, feats, gpu)
        launch_overrides(task_waves=1)
        assert np.array_equal(y_wide.view(np.uint32), y_narrow.view(np.uint32)), case
        y_ref = oracle.sw32(rows, cols, off, src, val).spmm_f64(pk, sc)
        assert_close(y_wide, y_ref, f"{case} F{feats} wide")


@pytest.mark.parametrize("feats", [128, 256])
def test_spmm_wide_addressing_at_real_size(oracle, gpu, feats):
    """Packed X of more than 4 GiB (cols * F > 2^32 - 256): the launch takes the 64-bit-addressing
    instance on its own. Sources are drawn so that many byte offsets exceed 2^32, two rows make
    split SWs, and X is generated on the GPU (17 GB of FP32 features). Quantize and pack are
    checked bit-exactly on every referenced row, Y on every element (the oracle runs on the
    referenced rows only, renumbered in order, which leaves every sum unchanged)."""
    import torch
    from tcc_spmm_amd.device import pack_features_int8x16, quantize_features_int8
    cols = (1 << 32) // feats + 65_537
    assert cols * feats > 0xFFFFFF00
    rows, rng = 2_053, np.random.default_rng(feats)
    top = (1 << 32) // feats                                  # first source past 32-bit offsets
    lists = []
    for r in range(rows):
        if r in (7, 1_900):                                   # > 384 panels: split SWs
            picks = np.concatenate([rng.choice(top, 1_600, replace=False),
                                    top + rng.choice(cols - top, 1_600, replace=False)])
        else:
            picks = np.concatenate([rng.integers(0, cols, 8), rng.integers(top, cols, 8),
                                    [cols - 1]])
        lists.append(np.unique(picks).astype(np.uint32))
    off = np.concatenate([[0], np.cumsum([len(c) for c in lists])]).astype(np.uint32)
    src = np.concatenate(lists)
    val = rng.uniform(-1, 1, src.size).astype(np.float32)
    csr = T.make_canonical_csr(rows, cols, off, src, val)
    fmt = T.convert_csr_to_sw32(rows, cols, csr)
    assert fmt.partial_count > 0

    gen = torch.Generator(device=gpu)
    gen.manual_seed(1000 + feats)
    x = torch.randn((cols, feats), generator=gen, device=gpu)
    q, scale = quantize_features_int8(x)
    packed = pack_features_int8x16(q)
    used = np.unique(csr.source_ids)
    assert int(used.max()) * feats >= 1 << 32
    idx = torch.from_numpy(used.astype(np.int64)).to(gpu)
    x_u = x.index_select(0, idx).cpu().numpy()
    q_u = q.index_select(0, idx).cpu().numpy()
    sc_u = scale.index_select(0, idx).cpu().numpy()
    pk_u = packed.index_select(0, idx).cpu().numpy()
    del x, q
    torch.cuda.empty_cache()
    check_features(oracle, x_u, q_u, sc_u, pk_u)

    _, y = _run(fmt, packed, scale, feats, gpu)
    renumbered = np.searchsorted(used, csr.source_ids).astype(np.uint32)
    ofmt = oracle.sw32(rows, used.size, csr.row_offsets, renumbered, csr.values)
    _check_full(ofmt, y, pk_u, sc_u, f"wide F{feats}")


@pytest.mark.parametrize("shape,x_offset,out_offset", [
    ((40, 64), 1, 0), ((9, 32), 0, 2), ((5, 16), 0, 1),    # scalar kernel: x or packed misaligned
    ((3, 2048), 0, 0), ((70, 272), 0, 0),                   # long-row kernel: > 64 groups per row
    ((1, 16), 0, 0), ((1029, 16), 0, 0), ((515, 48), 0, 0),  # fit kernel, 4 and 16 lanes (12 live)
    ((257, 112), 0, 0), ((131, 128), 0, 0), ((67, 256), 0, 0),  # 32 and 64 lanes, ragged tail
])
def test_quantize_pack_fused_bit_exact(oracle, gpu, shape, x_offset, out_offset):
    """quantizePackFeaturesInt8 writes exactly the scales and packed16 bytes of quantizeFeaturesInt8
    followed by packFeaturesInt8x16, on every kernel path (scalar for misaligned x or output, long
    rows, the register kernel with idle lanes and a partial last block), and the oracle's."""
    import torch
    from tcc_spmm_amd.device import quantize_pack_features_int8
    s, f = shape
    x = features(s, f, seed=s * 37 + f, stddev=2.0, outlier_fraction=0.1, outlier_scale=50.0)
    x[0] = 0.0
    flat = torch.zeros(s * f + x_offset, dtype=torch.float32, device=gpu)
    flat[x_offset:] = torch.from_numpy(x.ravel()).to(gpu)
    xs = flat[x_offset:].view(s, f)
    out = torch.full((s * f + out_offset,), 0x5A, dtype=torch.int8, device=gpu)
    packed, scale = quantize_pack_features_int8(xs, out[out_offset:].view(s, f))
    torch.cuda.synchronize()
    assert packed.data_ptr() % 4 == out_offset % 4
    p2, s2, q2, sc2, pk2 = gpu_prepare(x, gpu)
    assert np.array_equal(scale.cpu().numpy().view(np.uint32), sc2.view(np.uint32))
    assert np.array_equal(packed.cpu().numpy(), pk2)
    q_ref, s_ref = oracle.quantize(x)
    assert np.array_equal(packed.cpu().numpy(), oracle.pack16(q_ref))
    assert np.array_equal(scale.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


def test_quantize_pack_fused_rejects_bad_widths(gpu):
    import torch
    from tcc_spmm_amd.device import quantize_pack_features_int8
    with pytest.raises(ValueError, match="features % 16"):
        quantize_pack_features_int8(torch.zeros((4, 24), dtype=torch.float32, device=gpu))


@pytest.mark.parametrize("shape,offset", [
    ((33, 18), 0), ((20, 5), 0), ((40, 64), 1),            # scalar kernel: F % 4 != 0, misaligned
    ((3, 2052), 0), ((70, 260), 0),                         # long-row kernel: > 64 groups per row
    ((1, 4), 0), ((1029, 4), 0), ((515, 12), 0),            # fit kernel, 1 and 4 lanes (3 live)
    ((257, 100), 0), ((131, 128), 0), ((67, 256), 0),       # fit kernel, 32 and 64 lanes, ragged tail
])
def test_quantize_scalar_and_vector_paths_bit_exact(oracle, gpu, shape, offset):
    """Widths that are not a multiple of 4 and inputs that are not 16-byte aligned take the one-wave-
    per-row kernel; rows of more than 64 4-feature groups take the long-row kernel; the rest take the
    register kernel (power-of-two lanes per row, idle lanes when F/4 is not a power of two, row
    counts that leave a partial last block)."""
    import torch
    from tcc_spmm_amd.device import quantize_features_int8
    s, f = shape
    x = features(s, f, seed=s * 31 + f, stddev=2.0, outlier_fraction=0.1, outlier_scale=50.0)
    x[0] = 0.0
    flat = torch.zeros(s * f + offset, dtype=torch.float32, device=gpu)
    flat[offset:] = torch.from_numpy(x.ravel()).to(gpu)
    xs = flat[offset:].view(s, f)
    q, scale = quantize_features_int8(xs)
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.quantize(x)
    assert np.array_equal(scale.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_ref)
