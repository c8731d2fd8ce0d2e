"""The kernel's workgroup -> task rule (xcdTask in tcc_spmm_amd/csrc/kernel/spmm.hip), restated, covers
every task exactly once for any task list.

Workgroups are dispatched to the 8 XCDs round-robin; XCD x walks one contiguous range of tasks. The
ranges hold equal task counts unless some XCD would get more than 3% above the mean panel count;
then they hold equal panel counts, each boundary clamped to half the spare share from its equal-count
place, and the grid adds ceil(T / 16) spare workgroups per XCD. The last TAIL_WINDOW tasks of a
range run longest size class first (tailTask: per 64-lane chunk a ballot count of each class, then
the k-th member of the chosen class by its rank among the chunk's members). Checked on the synthetic
configs and on adversarial lists (all tasks empty, one task holding every panel, heavy skew, random
sizes), for task counts 1..39 and a few larger ones; the window's order is checked against a stable
sort by descending class."""
import numpy as np
import pytest

import tcc_spmm_amd as T


TAIL_WINDOW = 512
WAVE = 64


def _size_class(panels):
    return (panels >= 96).astype(np.int64) + (panels >= 192) + (panels >= 288)


def _tail_order(cls, w0):
    """tailTask for every position r of the window [w0, w0 + cls.size); cls holds its classes."""
    chunks = [cls[base:base + WAVE] for base in range(0, cls.size, WAVE)]
    counts = [sum(int(np.count_nonzero(ch == c)) for ch in chunks) for c in range(4)]
    # Per chunk and class, the member lanes by rank: the lane whose mbcnt (members in lower lanes)
    # equals k is the k-th member.
    lanes = [[np.flatnonzero(ch == c) for c in range(4)] for ch in chunks]
    order = []
    for r in range(cls.size):
        c, k = 3, r
        while c > 0 and k >= counts[c]:
            k -= counts[c]
            c -= 1
        for i, per_class in enumerate(lanes):
            member = per_class[c]
            if k < member.size:
                order.append(w0 + i * WAVE + int(member[k]))
                break
            k -= member.size
        else:
            raise AssertionError("the window holds every position")
    return order


def _panel_bound(begin, count, target):
    """panelBound for one half: 32 probes per step over [l, r], task r known to qualify."""
    l, r = 0, count
    while l < r:
        stride = (r - l + 31) // 32
        at = [l + j * stride >= r or begin[min(l + j * stride, count - 1)] >= target
              for j in range(32)]
        first = at.index(True) if True in at else 32
        nl = l if first == 0 else l + (first - 1) * stride + 1
        r = min(l + first * stride, r) if first < 32 else r
        l = nl
    return l


def _spare(count):
    return (count + 15) // 16


def _equal(count, x):
    q, r = count >> 3, count & 7
    return x * q + min(x, r)


def _bounds(begin, panels_total):
    count = len(begin)
    first = [int(begin[t]) if t < count else panels_total for t in (_equal(count, k) for k in range(9))]
    panels = first[8] - first[0]
    balanced = max(first[k + 1] - first[k] for k in range(8)) * 8 * 100 > panels * 103
    reach = _spare(count) // 2

    def bound(k):
        if k in (0, 8) or not balanced:
            return _equal(count, k)
        lower = int(np.searchsorted(begin, first[0] + panels * k // 8, side="left"))
        eq = _equal(count, k)
        return min(max(lower, eq - reach if eq > reach else 0), eq + reach)

    return balanced, [bound(k) for k in range(9)]


def _covered_once(begin, panels_total):
    count = len(begin)
    balanced, b = _bounds(begin, panels_total)
    cls = _size_class(np.diff(np.append(begin, panels_total)))
    windows = {}
    for x in range(8):
        lo, hi = b[x], b[x + 1]
        w0 = hi - min(hi - lo, TAIL_WINDOW)
        order = _tail_order(cls[w0:hi], w0)
        assert order == [w0 + i for i in np.argsort(-cls[w0:hi], kind="stable")]
        windows[x] = (w0, order)
    seen = np.zeros(count, np.int64)
    for bid in range(count + 8 * _spare(count)):
        x, j = bid & 7, bid >> 3
        t = b[x] + j
        if t < b[x + 1]:
            w0, order = windows[x]
            seen[order[t - w0] if t >= w0 else t] += 1
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


def test_probe_search_is_a_lower_bound():
    """The kernel's 32-probe boundary search finds the first task at or past the target, as a
    binary search does: non-decreasing begins with runs of equal values (empty tasks), targets
    before, between, on and past the begins."""
    rng = np.random.default_rng(5)
    for n in list(range(1, 70)) + [1000, 38281, 79199]:
        for kind in ("random", "runs", "empty"):
            if kind == "random":
                sizes = rng.integers(0, 385, n)
            elif kind == "runs":
                sizes = np.where(rng.random(n) < 0.7, 0, rng.integers(1, 385, n))
            else:
                sizes = np.zeros(n, np.int64)
            begin = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
            total = int(sizes.sum())
            targets = {0, total, total + 1} | {total * k // 8 for k in range(9)}
            targets |= set(int(v) for v in rng.integers(0, total + 2, 8))
            for target in targets:
                want = int(np.searchsorted(begin, target, side="left"))
                assert _panel_bound(begin, n, target) == want, (kind, n, target)


@pytest.mark.parametrize("cfg", ["c2", "c5"])
def test_offset_task_list_maps_like_the_whole(cfg):
    """A view over a later part of a plan's task list (valid input: the reference maps blockIdx to a
    task directly) starts past panel 0. The ranges are measured from its first task's begin, so the
    boundaries of a shifted list are those of the same list starting at 0, and every task is still
    covered once."""
    csr = T.synth_csr(cfg)
    tasks = T.convert_csr_to_sw32(csr.rows, csr.cols, csr).tasks
    begin = tasks["begin"].astype(np.int64)
    end = int(tasks["end"][-1])
    cut = int(np.searchsorted(begin, begin[begin.size // 3], side="left"))
    sub = begin[cut:]
    base = _bounds(sub - sub[0], end - int(sub[0]))
    assert base[0]  # skewed enough to take the panel-balanced ranges
    for shift in (int(sub[0]), int(sub[0]) + 12345):
        assert _bounds(sub - sub[0] + shift, end - int(sub[0]) + shift) == base
        assert _covered_once(sub - sub[0] + shift, end - int(sub[0]) + shift) == (True, True)
