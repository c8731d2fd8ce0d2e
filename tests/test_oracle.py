"""Pins the C oracle's feature and SpMM functions (the format functions are pinned byte-for-byte
against the reference's own compiled code in test_format_golden.py).

Every check here comes from outside the oracle's own formulas: known answers at rounding ties,
closed-form special cases (power-of-two scales, permutation matrices), an independent rational-
arithmetic TF32 rounding, and a dense brute-force product.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

import tcc_spmm_amd as T
from gpu_cases import ATOL, RTOL, assert_close


def f32_bits(v):
    return int(np.array(v, np.float32).view(np.uint32))


def from_bits(b):
    return float(np.array(b, np.uint32).view(np.float32))


def tf32_exact(x: float) -> float:
    """Round a normal float32 to 11 significant bits, ties away from zero, in rational arithmetic."""
    if x == 0.0:
        return x
    m, e = math.frexp(abs(x))          # |x| = m * 2^e, m in [0.5, 1)
    scaled = Fraction(m) * 2 ** 11     # [1024, 2048)
    whole = math.floor(scaled)
    r = whole + 1 if scaled - whole >= Fraction(1, 2) else whole
    return math.copysign(math.ldexp(r, e - 11), x)


# ---------------------------------------------------------------------------------------------
# TF32 rounding (reference src/kernel/spmm_kernel.cuh:7-11: cvt.rna.tf32.f32)

@pytest.mark.parametrize("src,want", [
    (0x3F801000, 0x3F802000),  # exact tie, even below: away from zero (RNE would keep 0x3F800000)
    (0xBF801000, 0xBF802000),  # negative tie: away from zero, not toward +inf
    (0x3F803000, 0x3F804000),  # tie from an odd kept bit
    (0x3F800FFF, 0x3F800000),  # just below half: down
    (0x3F801001, 0x3F802000),  # just above half: up
    (0x3FFFF000, 0x40000000),  # carry into the exponent
    (0x00000000, 0x00000000),
    (0x80000000, 0x80000000),
    (0x00001000, 0x00002000),  # subnormal tie at the same bit position
])
def test_tf32_known_answers(oracle, src, want):
    assert f32_bits(oracle.tf32(from_bits(src))) == want


def test_tf32_matches_rational_rounding(oracle):
    rng = np.random.default_rng(7)
    bits = rng.integers(0x00800000, 0x7F000000, 4000, dtype=np.uint32)  # positive normals
    bits[::2] |= np.uint32(0x80000000)
    bits[::7] = (bits[::7] & np.uint32(0xFFFFE000)) | np.uint32(0x1000)  # force exact ties
    xs = bits.view(np.float32)
    got = oracle.tf32_array(xs)
    want = np.array([tf32_exact(float(x)) for x in xs], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------------------------------------
# Quantization (reference src/format/int8_quantize.cu:4-31)

def test_quantize_zero_row_and_power_of_two_ties(oracle):
    # absmax 127/8 -> scale exactly 1/8, so x / s lands on the listed halves exactly.
    row = np.array([127, 2.5, 3.5, -2.5, 0.5, -0.5, 1.5, 126.5, -126.5, 0, 64, -127],
                   np.float32) / np.float32(8)
    x = np.zeros((2, 16), np.float32)
    x[1, :row.size] = row
    q, s = oracle.quantize(x)
    assert s[0] == 1.0 and not q[0].any()                    # all-zero row: scale 1, q = 0
    assert s[1] == np.float32(0.125)
    # round half to even (lrintf), not half away from zero
    assert q[1, :row.size].tolist() == [127, 2, 4, -2, 0, 0, 2, 126, -126, 0, 64, -127]


def test_quantize_scale_is_an_ieee_divide(oracle):
    # absmax / 127 and absmax * (1 / 127) differ in float32 for this absmax: the reference divides.
    a = None
    rng = np.random.default_rng(3)
    for v in rng.uniform(1, 100, 20000).astype(np.float32):
        if np.float32(v) / np.float32(127) != np.float32(v) * (np.float32(1) / np.float32(127)):
            a = np.float32(v)
            break
    assert a is not None
    q, s = oracle.quantize(np.array([[a] + [0] * 15], np.float32))
    assert s[0] == np.float32(a) / np.float32(127) and q[0, 0] == 127


def test_quantize_invariants(oracle):
    rng = np.random.default_rng(5)
    x = rng.normal(0, 3, (300, 64)).astype(np.float32)
    x[::17] *= 1000
    q, s = oracle.quantize(x)
    absmax = np.abs(x).max(axis=1)
    assert (np.abs(q.astype(np.int32)) <= 127).all()
    arg = np.abs(x).argmax(axis=1)
    assert (np.abs(q[np.arange(300), arg]) == 127).all()
    err = np.abs(q.astype(np.float64) * s[:, None] - x)
    assert (err <= s[:, None] * 0.5 * (1 + 1e-6)).all()
    assert np.allclose(s, absmax / 127, rtol=1e-7)


# ---------------------------------------------------------------------------------------------
# Packing (reference src/format/pack_int8.cu:6-25)

def test_pack16_known_answer(oracle):
    q = np.arange(32, dtype=np.int8).reshape(1, 32)
    want = [0, 8, 1, 9, 2, 10, 3, 11, 4, 12, 5, 13, 6, 14, 7, 15,
            16, 24, 17, 25, 18, 26, 19, 27, 20, 28, 21, 29, 22, 30, 23, 31]
    assert oracle.pack16(q)[0].tolist() == want


def test_pack16_round_trip(oracle):
    q = np.random.default_rng(1).integers(-127, 128, (33, 256)).astype(np.int8)
    assert np.array_equal(oracle.unpack16(oracle.pack16(q)), q)


# ---------------------------------------------------------------------------------------------
# SpMM (reference src/kernel/spmm_kernel.cuh: Y = sum tf32(a) * tf32(fp32(q * scale)))

def _xhat_independent(q, s):
    """Dequantized features from the definition, with the rational TF32 rounding."""
    prod = q.astype(np.float32) * s[:, None].astype(np.float32)   # one IEEE multiply
    return np.vectorize(tf32_exact, otypes=[np.float64])(prod.astype(np.float64))


def _random_csr(rng, rows, cols, density):
    dense = np.where(rng.random((rows, cols)) < density,
                     rng.uniform(-1, 1, (rows, cols)), 0.0).astype(np.float32)
    dense[rows // 3] = 0.0                                   # an empty row
    off = np.concatenate([[0], np.cumsum((dense != 0).sum(axis=1))]).astype(np.uint32)
    r, c = np.nonzero(dense)
    return dense, off, c.astype(np.uint32), dense[r, c]


@pytest.mark.parametrize("rows,cols,feats,density", [(70, 50, 16, 0.2), (97, 300, 32, 0.05)])
def test_spmm_matches_dense_brute_force(oracle, rows, cols, feats, density):
    rng = np.random.default_rng(rows)
    dense, off, src, val = _random_csr(rng, rows, cols, density)
    x = rng.normal(0, 2, (cols, feats)).astype(np.float32)
    q, s = oracle.quantize(x)
    pk = oracle.pack16(q)
    a_t = np.vectorize(tf32_exact, otypes=[np.float64])(dense.astype(np.float64))
    want = a_t @ _xhat_independent(q, s)
    got_csr = oracle.spmm_csr_f64(rows, off, src, val, pk, s, cols)
    fmt = oracle.sw32(rows, cols, off, src, val)
    assert np.allclose(got_csr, want, rtol=1e-12, atol=1e-12)
    assert np.allclose(fmt.spmm_f64(pk, s), want, rtol=1e-12, atol=1e-12)
    assert_close(fmt.spmm_tasks_f32(pk, s), want, "tasks f32")
    y, _ = fmt.spmm_f32_mt(pk, s, 0, (rows + 31) // 32, 2)
    assert_close(y, want, "mt f32")
    if fmt.has_vector_path():  # the CPU baseline's AVX2 path: bitwise the scalar path's Y
        yv, _ = fmt.spmm_f32_mt(pk, s, 0, (rows + 31) // 32, 2, vector=True)
        assert np.array_equal(yv.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("feats", [128, 256])
def test_cpu_baseline_vector_path_is_bitwise_the_scalar_path(oracle, feats):
    """The AVX2 path of the CPU baseline (per slot: byte-shuffle unpack, eight conversions, scale and
    TF32 rounding per instruction, fused multiply-adds of exact products) gives Y bitwise equal to
    the portable scalar path, on c1 with both widths and 1 or 3 threads; the scalar path is pinned
    by the brute-force test above."""
    of = None
    csr = T.synth_csr("c1")
    of = oracle.sw32(csr.rows, csr.cols, *csr.views())
    if not of.has_vector_path():
        pytest.skip("this CPU has no AVX2 + FMA")
    x = T.synth_features(csr.cols, feats, 5)
    q, s = oracle.quantize(x)
    pk = oracle.pack16(q)
    n_sw = (csr.rows + 31) // 32
    y0, _ = of.spmm_f32_mt(pk, s, 0, n_sw, 3)
    for threads in (1, 3):
        y1, _ = of.spmm_f32_mt(pk, s, 0, n_sw, threads, vector=True)
        assert np.array_equal(y1.view(np.uint32), y0.view(np.uint32))
    with pytest.raises(RuntimeError):
        of.spmm_f32_mt(pk[:, :8].copy(), s, 0, n_sw, 1, vector=True)  # features % 16 != 0


def test_spmm_permutation_picks_rows_exactly(oracle):
    n, feats = 96, 16
    perm = np.random.default_rng(2).permutation(n).astype(np.uint32)
    off = np.arange(n + 1, dtype=np.uint32)
    x = np.random.default_rng(4).normal(0, 1, (n, feats)).astype(np.float32)
    q, s = oracle.quantize(x)
    pk = oracle.pack16(q)
    want = _xhat_independent(q, s)[perm]
    y = oracle.sw32(n, n, off, perm, np.ones(n, np.float32)).spmm_f64(pk, s)
    assert np.array_equal(y, want)


def test_spmm_split_tasks_merge_to_the_unsplit_sum(oracle):
    # Row 3 references 4000 distinct sources: its SW needs more than 384 panels, so the plan
    # splits it into several tasks whose partial tiles the last one merges.
    rows, cols, feats = 64, 4000, 16
    rng = np.random.default_rng(9)
    lists = [rng.choice(cols, 5, replace=False) for _ in range(rows)]
    lists[3] = np.arange(cols)
    off = np.concatenate([[0], np.cumsum([len(c) for c in lists])]).astype(np.uint32)
    src = np.concatenate([np.sort(c) for c in lists]).astype(np.uint32)
    val = rng.uniform(-1, 1, src.size).astype(np.float32)
    csr = T.make_canonical_csr(rows, cols, off, src, val)
    fmt = oracle.sw32(rows, cols, csr.row_offsets, csr.source_ids, csr.values)
    assert fmt.partial_count > 0
    x = rng.normal(0, 1, (cols, feats)).astype(np.float32)
    q, s = oracle.quantize(x)
    pk = oracle.pack16(q)
    y = fmt.spmm_tasks_f32(pk, s)
    assert np.isfinite(y).all()
    want = oracle.spmm_csr_f64(rows, csr.row_offsets, csr.source_ids, csr.values, pk, s, cols)
    err = np.abs(y - want)
    assert (err <= ATOL + RTOL * np.abs(want)).all()


def test_full_checker_reference_and_verdicts(oracle):
    """check_full recomputes the reference SW by SW on several threads: its reference must equal
    the window oracle bitwise and the dense brute force, and its verdicts must flag exactly the
    planted errors (the first one by index), NaN included."""
    rows, cols, feats = 203, 300, 32                         # 7 SWs, the last with 11 rows
    rng = np.random.default_rng(21)
    dense, off, src, val = _random_csr(rng, rows, cols, 0.05)
    x = rng.normal(0, 1, (cols, feats)).astype(np.float32)
    q, s = oracle.quantize(x)
    pk = oracle.pack16(q)
    fmt = oracle.sw32(rows, cols, off, src, val)
    a_t = np.vectorize(tf32_exact, otypes=[np.float64])(dense.astype(np.float64))
    want = a_t @ _xhat_independent(q, s)
    windows = np.arange((rows + 31) // 32, dtype=np.uint32)
    win, mag = fmt.spmm_windows_f64(pk, s, windows, with_abs=True)
    win, mag = win[:rows], mag[:rows]

    y = want.astype(np.float32)
    st, ref = fmt.check_full(pk, s, y, ATOL, RTOL, threads=3, with_ref=True)
    assert np.array_equal(ref.view(np.uint64), win.view(np.uint64))
    assert np.allclose(ref, want, rtol=1e-12, atol=1e-12)
    assert (st["checked"], st["bad"], st["relaxed"], st["first_bad"]) == (rows * feats, 0, 0, None)

    plain = ATOL + RTOL * np.abs(ref)
    bad = y.copy()
    bad[150, 7] = np.float32(ref[150, 7] + 2 * plain[150, 7])   # SW 4 (third thread)
    bad[40, 3] = np.float32(ref[40, 3] - 3 * plain[40, 3])      # SW 1 (first thread): the first
    bad[200, 31] = np.nan                                       # tail SW
    bad[90, 0] = np.float32(ref[90, 0] + 0.5 * plain[90, 0])    # within the bound
    st = fmt.check_full(pk, s, bad, ATOL, RTOL, threads=3)
    assert st["bad"] == 3 and st["max_err"] == np.inf
    (r, f), got, wnt, bound = st["first_bad"]
    assert (r, f) == (40, 3) and got == float(bad[40, 3]) and wnt == ref[40, 3]
    assert bound == plain[40, 3]

    # The conditioning term: an error beyond the plain bound but within cond * 2^-24 * sum|terms|.
    cond = 1e-2 * 2.0 ** 24
    r, f = np.unravel_index(np.argmax(mag), mag.shape)
    loose = y.copy()
    loose[r, f] = np.float32(ref[r, f] + plain[r, f] + 0.5 * 1e-2 * mag[r, f])
    assert fmt.check_full(pk, s, loose, ATOL, RTOL, threads=2)["bad"] == 1
    st = fmt.check_full(pk, s, loose, ATOL, RTOL, cond=cond, threads=2)
    assert (st["bad"], st["relaxed"]) == (0, 1)
