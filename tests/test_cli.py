"""tcc_spmm_run, the command-line harness (reference src/main.cu:1-114).

CPU tests: argument handling and exit status (everything that fails before the first HIP call), and
the feature stream the GPU tests restate. GPU tests: the harness's Y (saved with --save-y) against
the oracle on the same inputs, for a Matrix Market file with a split SW and for a synthetic config,
and the JSON record against the saved Y.
"""
import json
import pathlib
import subprocess

import numpy as np
import pytest

import tcc_spmm_amd as T
from gpu_cases import assert_close

CLI = pathlib.Path(__file__).resolve().parents[1] / "tcc_spmm_amd" / "tcc_spmm_run"


def _run(*args, timeout=300):
    return subprocess.run([str(CLI), *map(str, args)], capture_output=True, text=True, timeout=timeout)


def reference_features(sources, features):
    """The harness's X (reference src/main.cu:11-17): each output of std::mt19937 seeded 20261025,
    shifted right by 8 and scaled by 2^-23, minus 1, row-major. numpy's legacy RandomState with an
    integer seed runs the same MT19937 initialisation and, for 32-bit draws over the full range,
    returns the raw outputs (pinned by test_feature_stream_is_std_mt19937)."""
    raw = np.random.RandomState(20261025).randint(0, 2**32, size=sources * features, dtype=np.uint32)
    x = (raw >> np.uint32(8)).astype(np.float32) * np.float32(2.0**-23) - np.float32(1.0)
    return x.reshape(sources, features)


def test_feature_stream_is_std_mt19937():
    # C++ [rand.predef]: the 10000th output of a default-constructed std::mt19937 (seed 5489) is
    # 4123659995.
    raw = np.random.RandomState(5489).randint(0, 2**32, size=10000, dtype=np.uint32)
    assert int(raw[-1]) == 4123659995
    x = reference_features(4, 16)
    assert x.dtype == np.float32 and x.min() >= -1.0 and x.max() < 1.0
    # on the 2^-23 grid: x + 1 is an integer multiple of 2^-23 below 2
    k = (x.astype(np.float64) + 1.0) * 2.0**23
    assert np.array_equal(k, np.round(k))


def test_usage_and_argument_errors():
    r = _run()
    assert r.returncode == 1 and r.stderr.startswith("Usage: ")
    r = _run("a.mtx", "128")
    assert r.returncode == 1 and "Usage: " in r.stderr
    r = _run("--config", "c1", "a.mtx", "128", "0")
    assert r.returncode == 1 and "Usage: " in r.stderr
    r = _run("--bogus", "a.mtx", "128", "0")
    assert r.returncode == 1 and "Usage: " in r.stderr
    for feats in ("100", "64", "512"):
        r = _run("a.mtx", feats, "0")
        assert r.returncode == 1
        assert r.stderr == "Error: feature dimension must be 128 or 256\n"
    r = _run("--warmup", "x", "a.mtx", "128", "0")
    assert r.returncode == 1 and r.stderr.startswith("Error: ")
    r = _run("a.mtx", "abc", "0")
    assert r.returncode == 1 and r.stderr.startswith("Error: ")


def _write_mtx(path, rows, cols, offsets, sources, values):
    lines = ["%%MatrixMarket matrix coordinate real general", "% written by test_cli.py",
             f"{rows} {cols} {len(sources)}"]
    for r in range(rows):
        for e in range(int(offsets[r]), int(offsets[r + 1])):
            lines.append(f"{r + 1} {int(sources[e]) + 1} {float(values[e])!r}")
    path.write_text("\n".join(lines) + "\n")


def _split_case(seed=21):
    """A 70 x 3500 matrix whose row 9 holds 3,200 distinct sources (400 panels: one split SW), plus
    uniform rows and an empty row."""
    rng = np.random.default_rng(seed)
    rows, cols = 70, 3500
    per_row = [np.sort(rng.choice(cols, rng.integers(1, 40), replace=False)) for _ in range(rows)]
    per_row[9] = np.sort(rng.choice(cols, 3200, replace=False))
    per_row[33] = np.zeros(0, np.int64)
    offsets = np.concatenate([[0], np.cumsum([len(p) for p in per_row])]).astype(np.uint32)
    sources = np.concatenate(per_row).astype(np.uint32)
    values = rng.uniform(-1.0, 1.0, sources.size).astype(np.float32)
    values[values == 0] = 0.5
    return rows, cols, offsets, sources, values


@pytest.mark.gpu
@pytest.mark.parametrize("feats", [128, 256])
def test_mtx_run_matches_oracle(oracle, tmp_path, feats):
    rows, cols, off, src, val = _split_case()
    fmt = T.convert_csr_to_sw32(rows, cols, T.make_canonical_csr(rows, cols, off, src, val))
    assert fmt.partial_count > 0
    mtx, js, ybin = tmp_path / "a.mtx", tmp_path / "r.json", tmp_path / "y.bin"
    _write_mtx(mtx, rows, cols, off, src, val)
    print(f"tcc_spmm_run {mtx.name} F{feats}", flush=True)
    r = _run("--json", js, "--save-y", ybin, "--warmup", 2, "--iterations", 3, mtx, feats, 0)
    assert r.returncode == 0, r.stderr
    assert "SpMM kernel average: " in r.stdout and "Output Y[0,0:8]:" in r.stdout
    y = np.fromfile(ybin, np.float32).reshape(rows, feats)
    x = reference_features(cols, feats)
    q, sc = oracle.quantize(x)
    pk = oracle.pack16(q)
    y_ref = oracle.spmm_csr_f64(rows, off, src, val, pk, sc, cols)
    assert_close(y, y_ref, f"tcc_spmm_run mtx F{feats}")
    rec = json.loads(js.read_text())
    assert (rec["rows"], rec["cols"], rec["nnz"], rec["features"]) == (rows, cols, src.size, feats)
    assert rec["partial_count"] == fmt.partial_count and rec["tasks"] == len(fmt.tasks)
    assert rec["iterations"] == 3 and rec["ms"] > 0 and rec["achieved_gbps"] > 0
    assert np.array_equal(np.float32(rec["y0"]), y[0, :8])


@pytest.mark.gpu
def test_config_run_with_normal_features_matches_oracle(oracle, tmp_path):
    js, ybin = tmp_path / "r.json", tmp_path / "y.bin"
    print("tcc_spmm_run --config c1 --normal-seed 7 F128", flush=True)
    r = _run("--config", "c1", "--normal-seed", 7, "--json", js, "--save-y", ybin, 128, 0)
    assert r.returncode == 0, r.stderr
    csr = T.synth_csr("c1")
    y = np.fromfile(ybin, np.float32).reshape(csr.rows, 128)
    q, sc = oracle.quantize(T.synth_features(csr.cols, 128, 7))
    pk = oracle.pack16(q)
    y_ref = oracle.spmm_csr_f64(csr.rows, csr.row_offsets, csr.source_ids, csr.values, pk, sc,
                                csr.cols)
    assert_close(y, y_ref, "tcc_spmm_run c1")
    rec = json.loads(js.read_text())
    assert rec["source"] == "config:c1" and rec["x"] == "normal:7" and rec["nnz"] == 65536
    assert rec["warmup"] == 10 and rec["iterations"] == 10
    # The harness's GB/s uses the same byte count as bench.py.
    import bench
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    assert rec["algorithmic_bytes"] == bench.algorithmic_bytes(fmt, csr.source_ids, 128)["B_alg"]


@pytest.mark.gpu
def test_missing_file_reports_error(tmp_path):
    r = _run(tmp_path / "absent.mtx", 128, 0)
    assert r.returncode == 1 and r.stderr.startswith("Error: ")
