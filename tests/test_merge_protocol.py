"""CPU model of the split-SW ticket and merge protocol (oracle/merge_model.cpp), on real plans.

The kernel's end of a split task (tcc_spmm_amd/csrc/kernel/spmm.hip, runTask and mergeSlice;
reference src/kernel/spmm_kernel.cuh:228-282) is restated for host threads: partial-tile writes, an
acquire-release wrapping ticket per slice, and the last arriver's merge with the kernel's lane
layout, 64-id chunks and batches of four tiles. Checked here, without a GPU:
  - lane map: every element of a row group's 8 x 128 block is summed by exactly one lane, from every
    tile of its reduction range exactly once, in partialIds order, and written once (ranges of 1 to
    130 tiles, and every split SW of c5 and of a plan with an SW split 73 ways);
  - protocol: under shuffled task orders and random delays on 8 threads, two workspaces at once and
    repeated launches on the same counters, each (SW, slice) has exactly one merger per launch, the
    counters are back at zero after every launch, and every merged element is bitwise the serial sum
    of the tile values in partialIds order;
  - ordering: the same runs under ThreadSanitizer report no data race, while a planted mistake
    (relaxed tickets and no acquire fence) is reported as one. The GPU's agent-scope acquire-release
    RMW and C++'s acq_rel RMW give the same guarantee here: the last RMW of the release sequence
    makes every earlier ticket-taker's tile writes visible to the merger.
"""
import pathlib
import subprocess

import numpy as np
import pytest

import tcc_spmm_amd as T

ROOT = pathlib.Path(__file__).resolve().parents[1]
MODEL = ROOT / "oracle" / "_build" / "merge_model"
MODEL_TSAN = ROOT / "oracle" / "_build" / "merge_model_tsan"


def _write_plan(path, fmt, features):
    tasks = np.ascontiguousarray(fmt.tasks)
    red = np.ascontiguousarray(fmt.reductions)
    ids = np.ascontiguousarray(fmt.partial_ids, np.uint32)
    head = np.array([0x50434354, 1, features, fmt.rows, tasks.size, red.size, ids.size,
                     fmt.partial_count], np.uint32)
    with open(path, "wb") as f:
        for arr in (head, tasks, red, ids):
            f.write(arr.tobytes())


def _many_chunk_fmt():
    """An SW split 73 ways whose row groups have 73, 3, 11 and 1 chunks, and a ragged last SW
    (the plan of tests/test_gpu_merge.py)."""
    rng = np.random.default_rng(7)
    rows, cols = 70, 240_000
    long_rows = {3: 220_000, 20: 30_000, 40: 30_000, 67: 140_000}
    per_row, vals = [], []
    for r in range(rows):
        d = long_rows.get(r, int(rng.integers(0, 12)))
        per_row.append(np.sort(rng.choice(cols, d, replace=False)).astype(np.uint32))
        v = rng.uniform(-1.0, 1.0, d).astype(np.float32)
        v[v == 0] = 0.5
        vals.append(v)
    off = np.concatenate([[0], np.cumsum([len(c) for c in per_row])]).astype(np.uint32)
    csr = T.make_canonical_csr(rows, cols, off, np.concatenate(per_row), np.concatenate(vals))
    return T.convert_csr_to_sw32(rows, cols, csr)


@pytest.fixture(scope="module")
def plans(tmp_path_factory):
    d = tmp_path_factory.mktemp("plans")
    out = {}
    many = _many_chunk_fmt()
    c5 = T.synth_csr("c5")
    c5fmt = T.convert_csr_to_sw32(c5.rows, c5.cols, c5)
    del c5
    for name, fmt in (("many", many), ("c5", c5fmt)):
        assert fmt.partial_count > 0
        for feats in (128, 256):
            path = d / f"{name}_f{feats}.plan"
            _write_plan(path, fmt, feats)
            out[(name, feats)] = path
    counts = np.bincount(many.tasks["sw"][many.tasks["partial"] != T.NO_PARTIAL])
    assert counts.max() == 73  # the 73-chunk SW is there
    return out


def _run(binary, *args, env=None):
    return subprocess.run([str(binary), *map(str, args)], capture_output=True, text=True,
                          timeout=600, env=env)


def _ok(res):
    assert res.returncode == 0, (res.returncode, res.stdout, res.stderr[-2000:])
    assert '"ok": true' in res.stdout, res.stdout
    return res.stdout


@pytest.mark.parametrize("feats", [128, 256])
def test_lane_map_on_range_lengths(feats):
    _ok(_run(MODEL, "map-lengths", feats, 1, 2, 3, 4, 5, 7, 8, 63, 64, 65, 66, 67, 68, 127, 128,
             129, 130, 131))


@pytest.mark.parametrize("name", ["many", "c5"])
def test_lane_map_on_plans(plans, name):
    out = _ok(_run(MODEL, "map", plans[(name, 256)]))
    if name == "many":
        assert '"max_tiles": 73' in out


@pytest.mark.parametrize("name,feats", [("many", 128), ("many", 256), ("c5", 256)])
def test_protocol_on_threads(plans, name, feats):
    out = _ok(_run(MODEL, "run", plans[(name, feats)], 8, 4, 2, 11))
    assert '"launches": 4' in out and '"workspaces": 2' in out


def _tsan_env():
    import os
    env = dict(os.environ)
    env["TSAN_OPTIONS"] = "exitcode=66 halt_on_error=0 report_signal_unsafe=0 history_size=7"
    return env


def _tsan(*args):
    import os
    if os.environ.get("TCC_SANITIZER_RUN"):
        # The AddressSanitizer run of this suite preloads ASan's runtime into every child process;
        # a ThreadSanitizer binary cannot run beside it (and is a sanitizer run of its own).
        pytest.skip("ThreadSanitizer binaries do not run inside the AddressSanitizer run")
    res = _run(MODEL_TSAN, *args, env=_tsan_env())
    if res.returncode != 0 and "unexpected memory mapping" in res.stderr:
        # Some kernels place mappings where this TSan runtime does not expect them; without
        # address-space randomisation it runs.
        res = subprocess.run(["setarch", "-R", str(MODEL_TSAN), *map(str, args)],
                             capture_output=True, text=True, timeout=600, env=_tsan_env())
    return res


@pytest.mark.parametrize("name,feats", [("many", 256), ("c5", 128)])
def test_protocol_is_race_free_under_tsan(plans, name, feats):
    res = _tsan("run", plans[(name, feats)], 8, 2, 2, 5)
    assert "ThreadSanitizer" not in res.stderr, res.stderr[-3000:]
    _ok(res)


def test_tsan_reports_a_planted_relaxed_ticket(plans):
    """The planted mistake: relaxed tickets and no acquire fence leave the mergers' tile reads
    unordered after the other tasks' writes. The values still come out right on this host (its
    stores are ordered anyway), so only the race detector can tell; it must."""
    res = _tsan("--plant", "relaxed", "run", plans[("many", 128)], 8, 1, 1, 5)
    assert res.returncode == 66, (res.returncode, res.stdout, res.stderr[-2000:])
    assert "WARNING: ThreadSanitizer: data race" in res.stderr


@pytest.mark.parametrize("mistake,mode,want", [
    ("batch-order", "map", "tiles not added in partialIds order"),
    ("batch-order", "run", "merged value differs from the serial sum"),
    ("ticket-limit", "run", "counter not back at zero"),
])
def test_checks_catch_planted_mistakes(plans, mistake, mode, want):
    """Mistakes planted in the model (tiles of a batch added last to first; a ticket that wraps at
    chunks instead of chunks - 1) fail the lane-map and protocol checks with the expected message."""
    args = ("map", plans[("many", 256)]) if mode == "map" else ("run", plans[("many", 128)], 4, 1, 1, 3)
    res = _run(MODEL, "--plant", mistake, *args)
    assert res.returncode == 1 and want in res.stdout, (res.returncode, res.stdout, res.stderr[-500:])
