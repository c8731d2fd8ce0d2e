"""Write tests/golden/*.npz from the REFERENCE's own CPU format code.

Inputs are small synthetic CSR matrices built here (seeded numpy); expected outputs come from the
reference's makeCanonicalCsr / convertCsrToSw32 (with its internal buildPanelTasks) /
loadMatrixMarket, compiled from /root/reference/src/format/*.cpp into oracle/_ref/libref_format.so
by oracle/Makefile. Only data is committed: inputs and the reference's outputs.

It also writes tests/golden/config_digests.json: SHA-256 digests and counts of the reference's
convertCsrToSw32 output (all nine arrays, partialCount) for the synthetic configurations c1, c2, c3
and c5 (c4 shares c3's matrix), and of its makeCanonicalCsr output for a non-canonical input of c2's
size (noncanonical_from below). The matrices come from this repository's deterministic generator.

It also writes tests/golden/sw32_defects.json: small CSRs with several entry defects in one SW and
the exception the reference's convertCsrToSw32 raises for each (class and message).

Run from the repository root:  python tests/golden/make_fixtures.py  (add --defects-only to write
only sw32_defects.json)
"""
from __future__ import annotations

import json
import pathlib
import sys
import tempfile

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import OracleError, RefFormat, build, csr_digests  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent
FIELDS = ("window_offsets", "source_ids", "row_group_masks", "source_metadata", "values",
          "bucket_offsets", "tasks", "reductions", "partial_ids")


def csr_from_rows(rows_cols, rows_vals=None, rng=None):
    off = [0]
    src, val = [], []
    for i, cols in enumerate(rows_cols):
        cols = list(cols)
        src += cols
        if rows_vals is not None:
            val += list(rows_vals[i])
        else:
            v = rng.uniform(-1, 1, len(cols)).astype(np.float32)
            v[v == 0] = 0.25
            val += list(v)
        off.append(len(src))
    return (np.array(off, np.uint32), np.array(src, np.uint32), np.array(val, np.float32))


def random_rows(rng, rows, cols, max_deg, distinct=True):
    out = []
    for _ in range(rows):
        d = int(rng.integers(0, max_deg + 1))
        c = rng.integers(0, cols, d)
        out.append(np.unique(c) if distinct else c)
    return out


def format_cases(rng):
    """(name, rows, cols, raw CSR) — raw CSR may be non-canonical; it is canonicalised first."""
    cases = []
    cases.append(("empty_all", 5, 7, csr_from_rows([[]] * 5, rng=rng)))
    cases.append(("single", 1, 1, csr_from_rows([[0]], rng=rng)))
    for rows in (31, 32, 33, 63, 65, 95, 97):
        cases.append((f"tail_{rows}", rows, 120, csr_from_rows(random_rows(rng, rows, 120, 9), rng=rng)))
    # All 15 RW masks in SW 0: column 100+m in one row of every RW of m.
    rowsets = [[] for _ in range(32)]
    for m in range(1, 16):
        for g in range(4):
            if m >> g & 1:
                rowsets[8 * g + (m % 8)].append(100 + m)
    cases.append(("all_masks", 32, 200, csr_from_rows([sorted(r) for r in rowsets], rng=rng)))
    # Long exclusive bucket, long shared bucket.
    cases.append(("long_exclusive", 32, 300,
                  csr_from_rows([list(range(0, 300, 3)) if r == 5 else [] for r in range(32)], rng=rng)))
    cases.append(("long_shared", 40, 500,
                  csr_from_rows([list(range(0, 500, 2)) if r in (1, 9, 17, 25) else [r]
                                 for r in range(40)], rng=rng)))
    # Exactly 384 panels (no split) and 385 panels (split), in one exclusive bucket.
    cases.append(("panels_384", 32, 4000,
                  csr_from_rows([list(range(384 * 8)) if r == 0 else [] for r in range(32)], rng=rng)))
    cases.append(("panels_385", 32, 4000,
                  csr_from_rows([list(range(384 * 8 + 1)) if r == 0 else [] for r in range(32)], rng=rng)))
    # Split SW whose chunks straddle exclusive and shared buckets, plus a tail SW.
    rows = []
    for r in range(70):
        if r == 3:
            rows.append(list(range(0, 3500)))
        elif r == 12:
            rows.append(list(range(1000, 4200)))
        elif r == 20:
            rows.append(list(range(0, 6000, 2)))
        else:
            rows.append(sorted(set(rng.integers(0, 6000, 20).tolist())))
    cases.append(("split_mixed", 70, 6000, csr_from_rows(rows, rng=rng)))
    # Two split SWs and a heavy SW with all four RWs.
    rows = []
    for r in range(96):
        if r in (0, 8, 16, 24):
            rows.append(sorted(set(rng.integers(0, 9000, 1500).tolist())))
        elif r == 70:
            rows.append(list(range(0, 9000, 1)))
        else:
            rows.append(sorted(set(rng.integers(0, 9000, 10).tolist())))
    cases.append(("split_two", 96, 9000, csr_from_rows(rows, rng=rng)))
    # Non-canonical input: unsorted, duplicates, zero sums.
    rows_c, rows_v = [], []
    for r in range(40):
        c = rng.integers(0, 30, 12)
        v = rng.choice(np.array([-1.0, -0.5, 0.5, 1.0, 0.75], np.float32), 12)
        rows_c.append(c)
        rows_v.append(v)
    cases.append(("noncanonical", 40, 30, csr_from_rows(rows_c, rows_v)))
    for i, (rows, cols, deg) in enumerate([(64, 64, 20), (100, 1000, 50), (257, 300, 30),
                                           (500, 500, 8), (128, 40, 40), (1000, 5000, 12),
                                           (33, 2000, 700), (320, 320, 64)]):
        cases.append((f"random_{i}", rows, cols, csr_from_rows(random_rows(rng, rows, cols, deg),
                                                               rng=rng)))
    return cases


def error_cases():
    """(name, rows, cols, offsets, sources, values) raw inputs the reference rejects."""
    nan = np.float32(np.nan)
    return [
        ("err_rows0", 0, 4, [0], [], []),
        ("err_cols0", 2, 0, [0, 0, 0], [], []),
        ("err_offsets_first", 2, 4, [1, 1, 2], [0, 1], [1.0, 1.0]),
        ("err_offsets_decreasing", 3, 4, [0, 2, 1, 2], [0, 1], [1.0, 1.0]),
        ("err_column_range", 2, 4, [0, 1, 2], [0, 4], [1.0, 1.0]),
        ("err_nonfinite", 2, 4, [0, 1, 2], [0, 1], [1.0, nan]),
        ("err_inf", 2, 4, [0, 1, 2], [0, 1], [np.inf, 1.0]),
        ("err_overflow_sum", 1, 4, [0, 2], [1, 1], [3e38, 3e38]),
    ]


def mtx_cases():
    return {
        "mtx_general_real": "%%MatrixMarket matrix coordinate real general\n% comment\n\n"
                            "3 4 5\n1 1 1.5\n2 4 -2\n3 2 0.25\n1 1 0.5\n3 3 1e-3\n",
        "mtx_symmetric_pattern": "%%MatrixMarket matrix coordinate pattern symmetric\n"
                                 "4 4 4\n1 1\n2 1\n4 3\n3 2\n",
        "mtx_integer_upper": "%%MATRIXMARKET MATRIX COORDINATE INTEGER GENERAL\n"
                             "2 2 3\n1 2 3\n2 1 -3\n2 2 7\n",
        "mtx_zero_sum": "%%MatrixMarket matrix coordinate real general\n"
                        "2 2 3\n1 1 1\n1 1 -1\n2 2 5\n",
        "err_mtx_banner": "%%MatrixMarket matrix array real general\n2 2\n1\n2\n3\n4\n",
        "err_mtx_truncated": "%%MatrixMarket matrix coordinate real general\n2 2 3\n1 1 1\n",
        "err_mtx_range": "%%MatrixMarket matrix coordinate real general\n2 2 1\n3 1 1\n",
        "err_mtx_symmetric_rect": "%%MatrixMarket matrix coordinate real symmetric\n2 3 1\n1 1 1\n",
    }


def defect_cases():
    """(name, rows, cols, rows_entries) canonical-shaped CSRs with several entry defects in ONE SW,
    each row a list of (source, value). The reference's converter meets them in ascending
    (source, row) order, not in row order, so these pin which message it reports."""
    nan, inf = float("nan"), float("inf")
    return [
        ("defect_range_then_zero", 2, 4, [[(5, 1.0)], [(0, 0.0)]]),
        ("defect_order_then_nan", 2, 4, [[(0, 1.0), (2, 1.0), (1, 1.0)], [(1, nan)]]),
        ("defect_zero_then_duplicate", 6, 8, [[(3, 0.0)], [], [], [], [], [(1, 1.0), (1, 1.0)]]),
        ("defect_range_rows_then_inf", 32, 6,
         [[(0, 1.0), (7, 1.0)]] + [[]] * 2 + [[(2, 1.0), (9, 1.0), (8, 1.0)]] + [[]] * 27 +
         [[(1, inf)]]),
        ("defect_late_row_small_source", 21, 16,
         [[(10, 1.0), (11, 0.0)]] + [[]] * 19 + [[(5, 1.0), (4, 1.0)]]),
        ("defect_same_source_rows", 3, 8, [[(2, 1.0)], [(3, 1.0), (2, 1.0)], [(3, 0.0)]]),
        ("defect_range_vs_value", 3, 8, [[(9, 1.0)], [(8, 1.0)], [(7, 0.0)]]),
    ]


def write_defects(ref):
    """tests/golden/sw32_defects.json: each defect case's input and the reference's exception."""
    out = []
    for name, rows, cols, entries in defect_cases():
        off = np.concatenate([[0], np.cumsum([len(r) for r in entries])]).astype(np.uint32)
        src = np.array([s for r in entries for s, _ in r], np.uint32)
        val = np.array([v for r in entries for _, v in r], np.float32)
        try:
            ref.convert(rows, cols, off, src, val, True)
            code, message = 0, ""
        except OracleError as e:
            code, message = e.code, e.message
        out.append({"name": name, "rows": rows, "cols": cols, "offsets": off.tolist(),
                    "sources": src.tolist(), "values": [repr(float(v)) for v in val],
                    "status": code, "message": message})
    path = OUT / "sw32_defects.json"
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path}: {len(out)} cases")


DIGEST_CONFIGS = ("c1", "c2", "c5", "c3")


def noncanonical_from(offsets, sources, values, seed):
    """A raw CSR with the same row sums as (offsets, sources, values) that exercises every rule of
    canonicalisation at scale: entries of each row in random order, one entry in ten split into two
    halves (duplicates to coalesce in input order) and one in fifty joined by a +w / -w pair on a
    random column (zero sums to drop, or extra terms on an existing column)."""
    rng = np.random.default_rng(seed)
    off = np.asarray(offsets, np.int64)
    src = np.asarray(sources, np.uint32)
    val = np.asarray(values, np.float32)
    rows = np.repeat(np.arange(off.size - 1, dtype=np.int64), np.diff(off))
    cols = int(src.max()) + 1 if src.size else 1
    half = rng.random(src.size) < 0.1
    val = val.copy()
    val[half] *= np.float32(0.5)
    pair = np.flatnonzero(rng.random(src.size) < 0.02)
    pcol = rng.integers(0, cols, pair.size).astype(np.uint32)
    pw = rng.uniform(-1, 1, pair.size).astype(np.float32)
    all_rows = np.concatenate([rows, rows[half], rows[pair], rows[pair]])
    all_src = np.concatenate([src, src[half], pcol, pcol])
    all_val = np.concatenate([val, val[half], pw, -pw])
    order = np.lexsort((rng.random(all_rows.size), all_rows))
    new_off = np.concatenate([[0], np.cumsum(np.bincount(all_rows, minlength=off.size - 1))])
    return new_off.astype(np.uint32), all_src[order], all_val[order]


def config_digests(ref):
    """Digests of the reference's format for each configuration and of its canonical CSR of a
    non-canonical c2-sized input."""
    import tcc_spmm_amd as T
    out = {"configs": {}, "canonical": {}}
    for cfg in DIGEST_CONFIGS:
        csr = T.synth_csr(cfg)
        off, src, val = csr.views()
        out["configs"][cfg] = {"dims": [csr.rows, csr.cols], "csr": csr_digests(off, src, val),
                               "format": ref.convert(csr.rows, csr.cols, off, src, val, True,
                                                     digests=True)}
        print(f"{cfg}: {out['configs'][cfg]['format']['counts']}", flush=True)
        if cfg == "c2":
            raw = noncanonical_from(off, src, val, seed=2026)
            canon = ref.canonical_csr(csr.rows, csr.cols, *raw)
            out["canonical"]["c2_noncanonical"] = {
                "dims": [csr.rows, csr.cols], "seed": 2026, "raw": csr_digests(*raw),
                "canonical": csr_digests(*canon)}
        del csr
    return out


def main():
    build()
    if not RefFormat.available():
        raise SystemExit("oracle/_ref/libref_format.so was not built (is /root/reference present?)")
    ref = RefFormat()
    write_defects(ref)
    if "--defects-only" in sys.argv:
        return
    rng = np.random.default_rng(20261201)
    store = {}
    names = []
    for name, rows, cols, (off, src, val) in format_cases(rng):
        c_off, c_src, c_val = ref.canonical_csr(rows, cols, off, src, val)
        store[f"{name}/in_offsets"] = off
        store[f"{name}/in_sources"] = src
        store[f"{name}/in_values"] = val
        store[f"{name}/dims"] = np.array([rows, cols], np.uint32)
        store[f"{name}/csr_offsets"] = c_off
        store[f"{name}/csr_sources"] = c_src
        store[f"{name}/csr_values"] = c_val
        for bucket in (1, 0):
            out = ref.convert(rows, cols, c_off, c_src, c_val, bool(bucket))
            for f in FIELDS:
                store[f"{name}/b{bucket}/{f}"] = out[f]
            store[f"{name}/b{bucket}/partial_count"] = np.array([out["partial_count"]], np.uint32)
        names.append(name)
    errs = []
    for name, rows, cols, off, src, val in error_cases():
        o = np.array(off, np.uint32)
        s = np.array(src, np.uint32)
        v = np.array(val, np.float32)
        try:
            ref.canonical_csr(rows, cols, o, s, v)
            code = 0
        except OracleError as e:
            code = e.code
        store[f"{name}/dims"] = np.array([rows, cols], np.uint32)
        store[f"{name}/in_offsets"] = o
        store[f"{name}/in_sources"] = s
        store[f"{name}/in_values"] = v
        store[f"{name}/status"] = np.array([code], np.int32)
        errs.append(name)
    # Conversion-level rejections (canonical shape, but values the SW32 builder refuses).
    conv_errs = {"conv_zero_value": (2, 4, [0, 1, 2], [0, 1], [0.0, 1.0]),
                 "conv_unsorted": (1, 4, [0, 2], [2, 1], [1.0, 1.0]),
                 "conv_duplicate": (1, 4, [0, 2], [1, 1], [1.0, 1.0]),
                 "conv_column_range": (1, 4, [0, 1], [4], [1.0])}
    for name, (rows, cols, off, src, val) in conv_errs.items():
        o = np.array(off, np.uint32)
        s = np.array(src, np.uint32)
        v = np.array(val, np.float32)
        try:
            ref.convert(rows, cols, o, s, v, True)
            code = 0
        except OracleError as e:
            code = e.code
        store[f"{name}/dims"] = np.array([rows, cols], np.uint32)
        store[f"{name}/in_offsets"] = o
        store[f"{name}/in_sources"] = s
        store[f"{name}/in_values"] = v
        store[f"{name}/status"] = np.array([code], np.int32)
    mtx = []
    with tempfile.TemporaryDirectory() as td:
        for name, text in mtx_cases().items():
            p = pathlib.Path(td) / f"{name}.mtx"
            p.write_text(text)
            store[f"{name}/text"] = np.frombuffer(text.encode(), np.uint8)
            try:
                rows, cols, off, src, val = ref.load_matrix_market(p)
                store[f"{name}/dims"] = np.array([rows, cols], np.uint32)
                store[f"{name}/csr_offsets"] = off
                store[f"{name}/csr_sources"] = src
                store[f"{name}/csr_values"] = val
                store[f"{name}/status"] = np.array([0], np.int32)
            except OracleError as e:
                store[f"{name}/status"] = np.array([e.code], np.int32)
            mtx.append(name)
    store["index/format_cases"] = np.array(names)
    store["index/error_cases"] = np.array(errs)
    store["index/conv_error_cases"] = np.array(list(conv_errs))
    store["index/mtx_cases"] = np.array(mtx)
    np.savez_compressed(OUT / "format_reference.npz", **store)
    print(f"wrote {OUT / 'format_reference.npz'}: {len(names)} format cases, {len(errs)} + "
          f"{len(conv_errs)} error cases, {len(mtx)} Matrix Market cases")
    digests = config_digests(ref)
    (OUT / "config_digests.json").write_text(json.dumps(digests, indent=1, sort_keys=True) + "\n")
    print(f"wrote {OUT / 'config_digests.json'}: {', '.join(digests['configs'])}")


if __name__ == "__main__":
    main()
