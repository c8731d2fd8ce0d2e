"""The kernel's workgroup -> task rule (xcdTask in tcc_spmm_amd/csrc/kernel/spmm.hip), restated, covers
every task exactly once for any task list.

Workgroups are dispatched to the 8 XCDs round-robin; XCD x walks one contiguous range of tasks. The
ranges hold equal task counts unless some XCD would get more than 3% above the mean panel count;
then they hold equal panel counts, each boundary clamped to half the spare share from its equal-count
place, and the grid adds ceil(T / 16) spare workgroups per XCD. Checked on the synthetic configs and
on adversarial lists (all tasks empty, one task holding every panel, heavy skew, random sizes), for
task counts 1..39 and a few larger ones."""
import numpy as np
import pytest

import tcc_spmm_amd as T


def _spare(count):
    return (count + 15) // 16


def _equal(count, x):
    q, r = count >> 3, count & 7
    return x * q + min(x, r)


def _bounds(begin, panels_total):
    count = len(begin)
    first = [int(begin[t]) if t < count else panels_total for t in (_equal(count, k) for k in range(9))]
    panels = first[8]
    balanced = max(first[k + 1] - first[k] for k in range(8)) * 8 * 100 > panels * 103
    reach = _spare(count) // 2

    def bound(k):
        if k in (0, 8) or not balanced:
            return _equal(count, k)
        lower = int(np.searchsorted(begin, panels * k // 8, side="left"))
        eq = _equal(count, k)
        return min(max(lower, eq - reach if eq > reach else 0), eq + reach)

    return balanced, [bound(k) for k in range(9)]


def _covered_once(begin, panels_total):
    count = len(begin)
    balanced, b = _bounds(begin, panels_total)
    seen = np.zeros(count, np.int64)
    for bid in range(count + 8 * _spare(count)):
        x, j = bid & 7, bid >> 3
        t = b[x] + j
        if t < b[x + 1]:
            seen[t] += 1
    return balanced, bool((seen == 1).all())


@pytest.mark.parametrize("cfg,expect_balanced", [("c1", False), ("c2", True), ("c3", False),
                                                 ("c5", True)])
def test_configs(cfg, expect_balanced):
    csr = T.synth_csr(cfg)
    tasks = T.convert_csr_to_sw32(csr.rows, csr.cols, csr).tasks
    balanced, ok = _covered_once(tasks["begin"].astype(np.int64), int(tasks["end"][-1]))
    assert ok and balanced == expect_balanced


def test_adversarial_lists():
    rng = np.random.default_rng(0)
    for n in list(range(1, 40)) + [100, 1000, 4097]:
        for kind in ("random", "empty", "onebig", "skew"):
            if kind == "random":
                sizes = rng.integers(0, 385, n)
            elif kind == "empty":
                sizes = np.zeros(n, np.int64)
            elif kind == "onebig":
                sizes = np.zeros(n, np.int64)
                sizes[rng.integers(0, n)] = 384
            else:
                sizes = np.where(rng.random(n) < 0.05, 384, rng.integers(0, 3, n))
            begin = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
            assert _covered_once(begin, int(sizes.sum()))[1], (kind, n)
