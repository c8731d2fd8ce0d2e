"""The L2 traffic model (model/l2_model.c) against an independent Python replay of the same
specification on small formats, and the ordering its policies must satisfy."""
import numpy as np
import pytest

import model
import tcc_spmm_amd as T

LINE = 128
TAIL_WINDOW = 512
CLASS_THRESHOLDS = (96, 192, 288)  # the kernel's size classes (sizeClass in spmm.hip)


def _format(cfg="t300_24_5"):
    csr = T.synth_csr(cfg)
    return T.convert_csr_to_sw32(csr.rows, csr.cols, csr)


def _ranges(begins, total, xcds):
    """The kernel's XCD ranges (xcdTask in spmm.hip), restated for any XCD count: equal task counts
    unless an XCD would get more than 3% above the mean panel count; then each boundary is the first
    task at or past k/xcds of the panels, clamped to half the spare share from its equal place."""
    n = len(begins)
    eq = [k * (n // xcds) + min(k, n % xcds) for k in range(xcds + 1)]
    begin_of = lambda t: begins[t] if t < n else total
    per = [begin_of(eq[k + 1]) - begin_of(eq[k]) for k in range(xcds)]
    if max(per) * xcds * 100 <= total * 103:
        return eq
    reach = ((n + 2 * xcds - 1) // (2 * xcds)) // 2
    out = [0]
    for k in range(1, xcds):
        lo = next((t for t in range(n) if begins[t] >= total * k // xcds), n)
        out.append(min(max(lo, eq[k] - reach if eq[k] > reach else 0), eq[k] + reach))
    return out + [n]


def _sequence(fmt, features, xcd, xcds, waves):
    """The model's access order, restated: the kernel's contiguous task range of this XCD (its last
    TAIL_WINDOW tasks longest size class first, a stable sort), `waves` resident tasks taking one
    panel each in turn; per panel the sourceIds, metadata and values
    lines, then per real slot its X lines and scale line. Keys are (array, line)."""
    a = fmt.arrays(copy=False)
    tasks = [tuple(int(v) for v in t) for t in a["tasks"][["sw", "begin", "end"]]]
    ids = np.asarray(a["source_ids"])
    base = (np.asarray(a["source_metadata"])[::8] >> np.uint64(32)).astype(np.int64)
    n_panels, n_values = base.size, int(a["values"].size)
    b = _ranges([t[1] for t in tasks], tasks[-1][2], xcds)
    lo, hi = b[xcd], b[xcd + 1]
    w0 = hi - min(hi - lo, TAIL_WINDOW)
    size_class = lambda t: sum(t[2] - t[1] >= v for v in CLASS_THRESHOLDS)
    order = list(range(lo, w0)) + sorted(range(w0, hi), key=lambda i: -size_class(tasks[i]))
    queue = [tasks[i] for i in order if tasks[i][2] > tasks[i][1]]
    slots = [None] * waves
    for w in range(waves):
        slots[w] = list(queue.pop(0)[1:]) if queue else None
    seq = []
    while any(s is not None for s in slots):
        for w in range(waves):
            s = slots[w]
            if s is None:
                continue
            p = s[0]
            s[0] += 1
            seq.append((("ids", p * 32 // LINE), "source_ids"))
            seq.append((("meta", p * 64 // LINE), "metadata"))
            v0 = int(base[p])
            v1 = int(base[p + 1]) if p + 1 < n_panels else n_values
            if v1 > v0:
                for line in range(v0 * 4 // LINE, (v1 * 4 - 1) // LINE + 1):
                    seq.append((("val", line), "values"))
            for k in range(8):
                src = int(ids[p * 8 + k])
                if src == 0xFFFFFFFF:
                    continue
                for j in range(features // 128):
                    seq.append((("x", src * (features // 128) + j), "x"))
                seq.append((("scale", src // 32), "scale"))
            if s[0] == s[1]:
                slots[w] = list(queue.pop(0)[1:]) if queue else None
    return seq


def _replay(seq, lines, policy):
    """Fully associative LRU / optimal (with bypass) / unbounded replay; misses per stream."""
    misses = {}
    if policy == "cold":
        seen = set()
        for key, st in seq:
            if key not in seen:
                seen.add(key)
                misses[st] = misses.get(st, 0) + 1
        return misses
    nxt = [0] * len(seq)
    last = {}
    for i in range(len(seq) - 1, -1, -1):
        nxt[i] = last.get(seq[i][0], 1 << 62)
        last[seq[i][0]] = i
    cache = {}  # key -> stamp (LRU: last use; optimal: next use)
    for i, (key, st) in enumerate(seq):
        mark = nxt[i] if policy == "opt" else i
        if key in cache:
            cache[key] = mark
            continue
        misses[st] = misses.get(st, 0) + 1
        if len(cache) < lines:
            cache[key] = mark
            continue
        if policy == "opt":
            victim = max(cache, key=cache.get)
            if mark >= cache[victim]:
                continue
        else:
            victim = min(cache, key=cache.get)
        del cache[victim]
        cache[key] = mark
    return misses


@pytest.mark.parametrize("policy", ["lru", "opt", "cold"])
@pytest.mark.parametrize("features", [128, 256])
def test_model_matches_an_independent_replay(policy, features):
    """One set of `lines` ways (fully associative), so the set hash plays no part."""
    fmt = _format()
    lines, waves = 64, 6
    got = model.traffic(fmt, features, policy, waves=waves, l2_bytes=lines * LINE, ways=lines)
    want = {s: 0 for s in model.STREAMS}
    for xcd in range(model.XCDS):
        for st, n in _replay(_sequence(fmt, features, xcd, model.XCDS, waves), lines, policy).items():
            want[st] += n
    assert got["misses"] == want


def test_ranges_follow_the_kernel_rule():
    """t300_24_5's equal split is within 3% (kept); t2000_30_7's is not (balanced, boundaries moved)."""
    for cfg, balanced in (("t300_24_5", False), ("t2000_30_7", True)):
        tasks = _format(cfg).arrays(copy=False)["tasks"]
        begins = [int(v) for v in tasks["begin"]]
        n = len(begins)
        b = _ranges(begins, int(tasks["end"][-1]), model.XCDS)
        equal = [k * (n // 8) + min(k, n % 8) for k in range(9)]
        assert b[0] == 0 and b[-1] == n and all(x <= y for x, y in zip(b, b[1:]))
        assert (b != equal) == balanced, cfg


def test_model_follows_balanced_ranges():
    """The replay comparison on a format whose XCD ranges are panel-balanced (LRU only)."""
    fmt = _format("t2000_30_7")
    lines, waves = 64, 6
    got = model.traffic(fmt, 128, "lru", waves=waves, l2_bytes=lines * LINE, ways=lines)
    want = {s: 0 for s in model.STREAMS}
    for xcd in range(model.XCDS):
        for st, n in _replay(_sequence(fmt, 128, xcd, model.XCDS, waves), lines, "lru").items():
            want[st] += n
    assert got["misses"] == want


def _mixed_format():
    """48 SWs whose tasks fall in every size class (panel counts from 8 to about 340), in an
    order where the tail window's class order differs from list order."""
    rng = np.random.default_rng(3)
    sws, cols = 48, 6000
    degree = rng.choice([2, 40, 75, 110], sws)
    offsets, ids = [0], []
    for s in range(sws):
        for _ in range(32):
            ids.extend(np.sort(rng.choice(cols, degree[s], replace=False)))
            offsets.append(len(ids))
    ids = np.asarray(ids, np.uint32)
    csr = T.csr_from_arrays(sws * 32, cols, np.asarray(offsets, np.uint32), ids,
                            np.ones(ids.size, np.float32))
    return T.convert_csr_to_sw32(csr.rows, csr.cols, csr)


def test_model_follows_the_tail_order():
    """The replay comparison on a format whose ranges lie inside the tail window and mix size
    classes, so the dispatch order is not list order (LRU only)."""
    fmt = _mixed_format()
    tasks = fmt.arrays(copy=False)["tasks"]
    p = (tasks["end"] - tasks["begin"]).astype(np.int64)
    classes = (p >= 96).astype(int) + (p >= 192) + (p >= 288)
    assert np.bincount(classes, minlength=4).min() > 0
    assert any(np.any(np.diff(classes[b:e]) > 0) for b, e in zip(range(0, 48, 6), range(6, 54, 6)))
    lines, waves = 64, 3
    for features in (128, 256):
        got = model.traffic(fmt, features, "lru", waves=waves, l2_bytes=lines * LINE, ways=lines)
        want = {s: 0 for s in model.STREAMS}
        for xcd in range(model.XCDS):
            for st, n in _replay(_sequence(fmt, features, xcd, model.XCDS, waves), lines,
                                 "lru").items():
                want[st] += n
        assert got["misses"] == want, features


def test_policies_are_ordered_and_bytes_add_up():
    fmt = _format("t2000_30_7")
    r = {p: model.traffic(fmt, 128, p) for p in ("cold", "opt", "lru")}
    total = lambda d: sum(d["misses"].values())
    assert total(r["cold"]) <= total(r["opt"]) <= total(r["lru"])
    for d in r.values():
        assert d["bytes"] == LINE * total(d) + 4 * fmt.rows * 128 + 64 * 128 * fmt.partial_count
        assert d["accesses"] == r["lru"]["accesses"]
    # every slot of a real source reads one X line and one scale line at F=128
    ids = np.asarray(fmt.arrays(copy=False)["source_ids"])
    assert r["lru"]["accesses"]["x"] == int(np.count_nonzero(ids != 0xFFFFFFFF))
    assert r["lru"]["accesses"]["scale"] == r["lru"]["accesses"]["x"]


def test_cold_misses_are_distinct_lines_per_xcd():
    fmt = _format("t2000_30_7")
    a = fmt.arrays(copy=False)
    tasks, ids = a["tasks"], np.asarray(a["source_ids"])
    b = _ranges([int(v) for v in tasks["begin"]], int(tasks["end"][-1]), model.XCDS)
    want = 0
    for x in range(model.XCDS):
        part = tasks[b[x]:b[x + 1]]
        if not len(part):
            continue
        src = ids[int(part["begin"][0]) * 8:int(part["end"][-1]) * 8]
        want += np.unique(src[src != 0xFFFFFFFF]).size
    got = model.traffic(fmt, 128, "cold")
    assert got["misses"]["x"] == want
