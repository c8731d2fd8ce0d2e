"""L2 traffic model of the SpMM kernel (measurement infrastructure for bench.py; l2_model.c).

traffic(fmt, features, policy) replays every XCD's share of the kernel's line accesses through one
XCD's L2 (4 MiB, 16-way, 128-byte lines on MI355X) and returns the misses per stream, summed over
the 8 XCDs, plus the bytes the launch must move beyond L2 under that policy:

    lines missed x 128 B  +  Y written (4 R F)  +  partial tiles written and read (2 x 32 F K)

Policies: "lru" (what the hardware approximates), "opt" (optimal replacement: the fewest misses any
policy could reach on the kernel's access order and this capacity), "cold" (unbounded L2 per XCD:
every line an XCD touches is fetched once, whatever the schedule within that XCD).

    python -m model c3          # all three policies at F = 128 and 256, as JSON

The time side comes from a random-gather probe measured on MI355X (profiles/gather_probe_rates.md):
the memory system serves a fixed number of random requests per second beyond L2 (about 50-55 G/s),
whether they are 32, 64 or 128 bytes long, so a launch's beyond-L2 request count divided by that rate
bounds its time.
"""
from __future__ import annotations

import concurrent.futures as cf
import ctypes as C
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
SO = HERE / "_build" / "libl2model.so"
STREAMS = ("x", "scale", "source_ids", "metadata", "values")
POLICIES = {"lru": 0, "opt": 1, "cold": 2}
XCDS = 8
L2_BYTES = 4 << 20
L2_WAYS = 16
LINE = 128


class _Input(C.Structure):
    _fields_ = [("taskCount", C.c_uint32), ("tasks", C.c_void_p), ("sourceIds", C.c_void_p),
                ("panelBase", C.c_void_p), ("panels", C.c_uint64), ("values", C.c_uint64),
                ("cols", C.c_uint32), ("features", C.c_uint32), ("xcds", C.c_uint32),
                ("xcd", C.c_uint32), ("waves", C.c_uint32), ("lines", C.c_uint32),
                ("ways", C.c_uint32), ("policy", C.c_uint32), ("bypassStreams", C.c_uint32),
                ("farRows", C.c_uint32), ("farStreams", C.c_uint32)]


class _Result(C.Structure):
    _fields_ = [("accesses", C.c_uint64 * 5), ("misses", C.c_uint64 * 5)]


def build() -> None:
    res = subprocess.run(["make", "-s", "-C", str(HERE)], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"model build failed:\n{res.stdout}\n{res.stderr}")


def _lib():
    if not SO.exists() or SO.stat().st_mtime < (HERE / "l2_model.c").stat().st_mtime:
        build()
    so = C.CDLL(str(SO))
    so.l2m_replay.argtypes = [C.POINTER(_Input), C.POINTER(_Result)]
    so.l2m_replay.restype = C.c_int
    return so


def waves_per_xcd(features: int) -> int:
    """Resident tasks per XCD: 32 CUs x 4 SIMDs x the kernel's waves per SIMD (4 at F=128, 2 at
    F=256)."""
    return 32 * 4 * (4 if features == 128 else 2)


def traffic(fmt, features: int, policy: str, threads: int = 8, waves: int | None = None,
            l2_bytes: int = L2_BYTES, ways: int = L2_WAYS, bypass=(), far_rows: int = 0,
            far_streams=()) -> dict:
    """Misses per stream summed over the XCDs, and the bytes beyond L2 of one launch.

    bypass: streams whose accesses never allocate in L2 (a load that misses leaves no line behind);
    far_rows / far_streams: the same for accesses of those streams (x, scale) whose source lies more
    than far_rows rows away from the SW's rows. These model cache hints a kernel could give."""
    def mask(names):
        return sum(1 << STREAMS.index(n) for n in names)
    arrs = fmt.arrays(copy=False)
    tasks = np.ascontiguousarray(arrs["tasks"]).view(np.uint32)
    ids = np.ascontiguousarray(arrs["source_ids"], np.uint32)
    md = np.asarray(arrs["source_metadata"])
    panel_base = np.ascontiguousarray((md[::8] >> np.uint64(32)).astype(np.uint32))
    n_values = int(arrs["values"].shape[0])
    so = _lib()

    def one(xcd: int) -> _Result:
        inp = _Input(int(len(arrs["tasks"])), tasks.ctypes.data, ids.ctypes.data,
                     panel_base.ctypes.data, int(panel_base.size), n_values, fmt.cols, features,
                     XCDS, xcd, waves or waves_per_xcd(features), l2_bytes // LINE, ways,
                     POLICIES[policy], mask(bypass), far_rows, mask(far_streams))
        out = _Result()
        rc = so.l2m_replay(C.byref(inp), C.byref(out))
        if rc:
            raise RuntimeError(f"l2m_replay failed ({rc})")
        return out

    with cf.ThreadPoolExecutor(max_workers=max(1, min(threads, XCDS))) as pool:
        parts = list(pool.map(one, range(XCDS)))
    misses = {s: int(sum(p.misses[i] for p in parts)) for i, s in enumerate(STREAMS)}
    accesses = {s: int(sum(p.accesses[i] for p in parts)) for i, s in enumerate(STREAMS)}
    writes = 4 * fmt.rows * features + 2 * 32 * features * fmt.partial_count
    read_bytes = LINE * sum(misses.values())
    return {"policy": policy, "misses": misses, "accesses": accesses, "read_bytes": read_bytes,
            "write_bytes": writes, "bytes": read_bytes + writes,
            "requests": sum(misses.values()) + writes // LINE}
