"""Descriptor identity at the benchmark configurations.

tests/golden/config_digests.json holds SHA-256 digests of the reference's own convertCsrToSw32
output (reference src/format/sw32.cpp:25-65,69-167, compiled from its sources into oracle/_ref by
tests/golden/make_fixtures.py) for c1, c2, c3 and c5 (c4 shares c3's matrix): all nine arrays plus
the counts (SWs, panels, slots, tasks, partial tiles, split SWs). The product's parallel builder
only takes its full shape at this scale (thousands of nnz-balanced SW blocks stitched together,
hub SWs split 49 ways), so each configuration is rebuilt here by the product and by the oracle
and compared digest for digest. A non-canonical input of c2's size pins makeCanonicalCsr
(reference src/format/csr.cpp:6-40) the same way.
"""
import json
import pathlib
import sys

import pytest

import tcc_spmm_amd as T
from oracle import csr_digests, format_digests

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
CONFIGS = ("c1", "c2", "c5", "c3")


def _digests():
    return json.loads((GOLDEN / "config_digests.json").read_text())


def _diff(got: dict, want: dict) -> list:
    return [k for k in sorted(set(got) | set(want)) if got.get(k) != want.get(k)]


@pytest.mark.parametrize("cfg", CONFIGS)
def test_product_and_oracle_formats_match_reference_digests(oracle, cfg):
    want = _digests()["configs"][cfg]
    csr = T.synth_csr(cfg)
    assert [csr.rows, csr.cols] == want["dims"]
    off, src, val = csr.views()
    assert not _diff(csr_digests(off, src, val), want["csr"]), "generator output changed"
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    got = format_digests(fmt.arrays(copy=False), fmt.partial_count)
    assert not _diff(got, want["format"]), (cfg, "product", _diff(got, want["format"]))
    del fmt
    ofmt = oracle.sw32(csr.rows, csr.cols, off, src, val)
    got = format_digests(ofmt.arrays(copy=False), ofmt.partial_count)
    assert not _diff(got, want["format"]), (cfg, "oracle", _diff(got, want["format"]))


def _noncanonical(case):
    sys.path.insert(0, str(GOLDEN))
    try:
        from make_fixtures import noncanonical_from
    finally:
        sys.path.remove(str(GOLDEN))
    csr = T.synth_csr("c2")
    return csr, noncanonical_from(*csr.views(), seed=case["seed"])


def test_canonical_csr_at_scale_matches_reference_digests(oracle):
    case = _digests()["canonical"]["c2_noncanonical"]
    csr, raw = _noncanonical(case)
    assert not _diff(csr_digests(*raw), case["raw"]), "raw input changed"
    rows, cols = case["dims"]
    got = T.make_canonical_csr(rows, cols, *raw)
    assert not _diff(csr_digests(*got.views()), case["canonical"])
    assert not _diff(csr_digests(*oracle.canonical_csr(rows, cols, *raw)), case["canonical"])


@pytest.mark.parametrize("cfg", ("c1", "c2", "c5"))
def test_committed_digests_are_the_reference_output(ref_format, cfg):
    """Where the reference's format code is built (oracle/_ref), recompute its digests live: the
    committed fixture is what the reference produces today."""
    want = _digests()["configs"][cfg]
    csr = T.synth_csr(cfg)
    got = ref_format.convert(csr.rows, csr.cols, *csr.views(), True, digests=True)
    assert not _diff(got, want["format"]), _diff(got, want["format"])
