"""Host format parity: product builder and C oracle against the reference's own bytes.

Fixtures (tests/golden/format_reference.npz) hold inputs and the outputs of the reference's
makeCanonicalCsr / convertCsrToSw32 / loadMatrixMarket compiled from its sources
(tests/golden/make_fixtures.py). Bit-exact comparison of every array.
"""
import numpy as np
import pytest

import tcc_spmm_amd as T
from oracle import OracleError

FIELDS = ("window_offsets", "source_ids", "row_group_masks", "source_metadata", "values",
          "bucket_offsets", "tasks", "reductions", "partial_ids")


def _cases(golden, key):
    return [str(x) for x in golden[f"index/{key}"]]


def _same_bytes(a, b):
    a = np.ascontiguousarray(a).view(np.uint8)
    b = np.ascontiguousarray(b).view(np.uint8)
    return a.shape == b.shape and bool((a == b).all())


def test_fixture_inventory(golden):
    assert len(_cases(golden, "format_cases")) >= 20
    assert len(_cases(golden, "error_cases")) >= 6
    assert len(_cases(golden, "mtx_cases")) >= 6


@pytest.mark.parametrize("bucket", [1, 0])
def test_product_builder_matches_reference_bytes(golden, bucket):
    for name in _cases(golden, "format_cases"):
        rows, cols = (int(x) for x in golden[f"{name}/dims"])
        csr = T.make_canonical_csr(rows, cols, golden[f"{name}/in_offsets"],
                                   golden[f"{name}/in_sources"], golden[f"{name}/in_values"])
        assert _same_bytes(csr.row_offsets, golden[f"{name}/csr_offsets"]), name
        assert _same_bytes(csr.source_ids, golden[f"{name}/csr_sources"]), name
        assert _same_bytes(csr.values, golden[f"{name}/csr_values"]), name
        fmt = T.convert_csr_to_sw32(rows, cols, csr, bool(bucket))
        arrs = fmt.arrays()
        for f in FIELDS:
            assert _same_bytes(arrs[f], golden[f"{name}/b{bucket}/{f}"]), (name, f)
        assert fmt.partial_count == int(golden[f"{name}/b{bucket}/partial_count"][0]), name


@pytest.mark.parametrize("bucket", [1, 0])
def test_oracle_matches_reference_bytes(golden, oracle, bucket):
    for name in _cases(golden, "format_cases"):
        rows, cols = (int(x) for x in golden[f"{name}/dims"])
        off, src, val = oracle.canonical_csr(rows, cols, golden[f"{name}/in_offsets"],
                                             golden[f"{name}/in_sources"],
                                             golden[f"{name}/in_values"])
        assert _same_bytes(off, golden[f"{name}/csr_offsets"]), name
        assert _same_bytes(src, golden[f"{name}/csr_sources"]), name
        assert _same_bytes(val, golden[f"{name}/csr_values"]), name
        fmt = oracle.sw32(rows, cols, off, src, val, bool(bucket))
        arrs = fmt.arrays()
        for f in FIELDS:
            assert _same_bytes(arrs[f], golden[f"{name}/b{bucket}/{f}"]), (name, f)
        assert fmt.partial_count == int(golden[f"{name}/b{bucket}/partial_count"][0]), name


def test_build_panel_tasks_replans_identically(golden):
    for name in _cases(golden, "format_cases"):
        rows, cols = (int(x) for x in golden[f"{name}/dims"])
        csr = T.make_canonical_csr(rows, cols, golden[f"{name}/csr_offsets"],
                                   golden[f"{name}/csr_sources"], golden[f"{name}/csr_values"])
        fmt = T.convert_csr_to_sw32(rows, cols, csr)
        fmt.build_panel_tasks()
        fmt.build_panel_tasks()
        arrs = fmt.arrays()
        for f in ("tasks", "reductions", "partial_ids"):
            assert _same_bytes(arrs[f], golden[f"{name}/b1/{f}"]), (name, f)


def test_build_panel_tasks_needs_bucketed_format(golden):
    name = _cases(golden, "format_cases")[-1]
    rows, cols = (int(x) for x in golden[f"{name}/dims"])
    csr = T.make_canonical_csr(rows, cols, golden[f"{name}/csr_offsets"],
                               golden[f"{name}/csr_sources"], golden[f"{name}/csr_values"])
    fmt = T.convert_csr_to_sw32(rows, cols, csr, bucket_by_rw_mask=False)
    with pytest.raises(ValueError):
        fmt.build_panel_tasks()


STATUS_TO_EXC = {1: ValueError, 2: OverflowError, 3: RuntimeError}


def test_canonical_csr_errors_match_reference_classes(golden, oracle):
    for name in _cases(golden, "error_cases"):
        rows, cols = (int(x) for x in golden[f"{name}/dims"])
        status = int(golden[f"{name}/status"][0])
        assert status != 0, name
        args = (golden[f"{name}/in_offsets"], golden[f"{name}/in_sources"],
                golden[f"{name}/in_values"])
        with pytest.raises(STATUS_TO_EXC[status]):
            T.make_canonical_csr(rows, cols, *args)
        if rows and golden[f"{name}/in_offsets"].size == rows + 1:
            from oracle import OracleError
            with pytest.raises(OracleError) as e:
                oracle.canonical_csr(rows, cols, *args)
            assert e.value.code == status, name


def test_conversion_errors_match_reference_classes(golden, oracle):
    from oracle import OracleError
    for name in _cases(golden, "conv_error_cases"):
        rows, cols = (int(x) for x in golden[f"{name}/dims"])
        status = int(golden[f"{name}/status"][0])
        assert status == 1, name
        off, src, val = (golden[f"{name}/in_offsets"], golden[f"{name}/in_sources"],
                         golden[f"{name}/in_values"])
        raw = T.csr_from_arrays(rows, cols, off, src, val)
        with pytest.raises(STATUS_TO_EXC[status]):
            T.convert_csr_to_sw32(rows, cols, raw)
        with pytest.raises(OracleError) as e:
            oracle.sw32(rows, cols, off, src, val)
        assert e.value.code == status, name


def test_conversion_rejects_malformed_csr_struct():
    # Offsets that disagree with the entry arrays (reference src/format/sw32.cpp:71-77).
    with pytest.raises(ValueError):
        T.convert_csr_to_sw32(2, 4, T.csr_from_arrays(2, 4, [0, 1], [0], [1.0]))
    with pytest.raises(ValueError):
        T.convert_csr_to_sw32(2, 4, T.csr_from_arrays(2, 4, [0, 2, 1], [0, 1], [1.0, 1.0]))
    with pytest.raises(ValueError):
        T.convert_csr_to_sw32(0, 4, T.csr_from_arrays(0, 4, [0], [], []))


def test_matrix_market_matches_reference(golden, tmp_path):
    for name in _cases(golden, "mtx_cases"):
        p = tmp_path / f"{name}.mtx"
        p.write_bytes(golden[f"{name}/text"].tobytes())
        status = int(golden[f"{name}/status"][0])
        if status:
            with pytest.raises(STATUS_TO_EXC[status]):
                T.load_matrix_market(p)
            continue
        csr = T.load_matrix_market(p)
        rows, cols = (int(x) for x in golden[f"{name}/dims"])
        assert (csr.rows, csr.cols) == (rows, cols)
        assert _same_bytes(csr.row_offsets, golden[f"{name}/csr_offsets"]), name
        assert _same_bytes(csr.source_ids, golden[f"{name}/csr_sources"]), name
        assert _same_bytes(csr.values, golden[f"{name}/csr_values"]), name


def _rows_csr(rows, per_row, cols, rng):
    src = np.concatenate([np.sort(rng.choice(cols, per_row, replace=False)) for _ in range(rows)])
    off = np.arange(0, rows * per_row + 1, per_row, dtype=np.uint32)
    return off, src.astype(np.uint32), rng.uniform(0.5, 1.0, src.size).astype(np.float32)


@pytest.mark.parametrize("first,second", [("overflow", "column"), ("column", "overflow"),
                                          ("nan", "overflow")])
def test_canonical_csr_reports_first_defect_in_row_order(ref_format, first, second):
    """Two defects in rows thousands apart (different parallel blocks): the message is the first
    row's, as in the reference's row-by-row scan (src/format/csr.cpp:15-36)."""
    rows, cols, per = 6000, 500, 6
    off, src, val = _rows_csr(rows, per, cols, np.random.default_rng(8))
    for row, kind in ((150, first), (4700, second)):
        e = row * per
        if kind == "overflow":      # a duplicate pair whose FP32 sum overflows
            src[e + 1] = src[e]
            val[e:e + 2] = np.float32(3e38)
        elif kind == "column":
            src[e + 2] = cols
        else:
            val[e + 3] = np.nan
    with pytest.raises(OracleError) as ref:
        ref_format.canonical_csr(rows, cols, off, src, val)
    with pytest.raises(ValueError) as got:
        T.make_canonical_csr(rows, cols, off, src, val)
    want = {"overflow": "nonfinite coalesced weight",
            "column": "invalid CSR column or nonfinite value",
            "nan": "invalid CSR column or nonfinite value"}[first]
    assert want in str(got.value)
    assert ref.value.code == 1  # invalid_argument


def test_conversion_reports_first_defective_sw(ref_format):
    """A zero value in SW 3 and a repeated source in SW 150 (different SW blocks of the parallel
    builder): the reported message is SW 3's."""
    rows, cols, per = 6400, 700, 5
    off, src, val = _rows_csr(rows, per, cols, np.random.default_rng(9))
    val[3 * 32 * per + 7] = 0.0
    e = 150 * 32 * per + 11
    src[e + 1] = src[e]
    raw = T.csr_from_arrays(rows, cols, off, src, val)
    with pytest.raises(ValueError, match="finite nonzero"):
        T.convert_csr_to_sw32(rows, cols, raw)
    with pytest.raises(OracleError):
        ref_format.convert(rows, cols, off, src, val)


def _defect_cases():
    import json
    import pathlib
    path = pathlib.Path(__file__).resolve().parent / "golden" / "sw32_defects.json"
    return json.loads(path.read_text())


@pytest.mark.parametrize("case", _defect_cases(), ids=lambda c: c["name"])
def test_conversion_reports_reference_first_defect_within_sw(case, request):
    """Several entry defects in one SW (tests/golden/sw32_defects.json, written from the reference's
    compiled converter): the product raises the reference's exception class and message. The
    reference meets entries in ascending (source, row) order (src/format/sw32.cpp:96-120), so a
    row-order scan would report a different defect for most of these."""
    rows, cols = case["rows"], case["cols"]
    off = np.array(case["offsets"], np.uint32)
    src = np.array(case["sources"], np.uint32)
    val = np.array([float(v) for v in case["values"]], np.float32)
    assert case["status"] == 1 and case["message"]
    raw = T.csr_from_arrays(rows, cols, off, src, val)
    with pytest.raises(ValueError) as got:
        T.convert_csr_to_sw32(rows, cols, raw)
    assert str(got.value) == case["message"]
    from oracle import RefFormat
    if RefFormat.available():  # the live reference agrees with the committed fixture
        with pytest.raises(OracleError) as ref:
            RefFormat().convert(rows, cols, off, src, val)
        assert (ref.value.code, ref.value.message) == (1, case["message"])


def test_host_builders_run_concurrently_from_several_threads():
    """The format builders keep no state between calls (reference include/format/sw32.h, csr.h:
    free functions): several host threads canonicalising and converting different matrices at once
    (the ctypes calls release the interpreter lock) get exactly the arrays of serial calls."""
    import concurrent.futures as cf
    cases = []
    for seed in range(6):
        rng = np.random.default_rng(100 + seed)
        rows, cols = 3000 + 97 * seed, 5000
        per_row = [rng.integers(0, cols, int(rng.integers(0, 40))) for _ in range(rows)]
        off = np.concatenate([[0], np.cumsum([len(c) for c in per_row])]).astype(np.uint32)
        src = np.concatenate(per_row).astype(np.uint32)
        val = rng.uniform(0.1, 1.0, src.size).astype(np.float32)
        cases.append((rows, cols, off, src, val))

    def build(case):
        rows, cols, off, src, val = case
        csr = T.make_canonical_csr(rows, cols, off, src, val)
        fmt = T.convert_csr_to_sw32(rows, cols, csr)
        return {k: np.array(v, copy=True) for k, v in fmt.arrays(copy=False).items()}

    serial = [build(c) for c in cases]
    with cf.ThreadPoolExecutor(max_workers=6) as pool:
        for _ in range(2):
            for want, got in zip(serial, pool.map(build, cases)):
                for name in FIELDS:
                    assert _same_bytes(got[name], want[name]), name
