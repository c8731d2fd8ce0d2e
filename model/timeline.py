"""Per-task timeline of the SpMM kernel on a synthetic configuration (measurement infrastructure).

    python -m model.timeline c5 [c3 ...]      # on a GPU box; prints a report per config and width

The measurement build compiles tcc_spmm_amd/csrc/kernel/spmm.hip with TCC_SPMM_TIMELINE, which makes
lane 0 of every workgroup store its task's start, the time the task was found, its end
(s_memrealtime, 100 MHz) and its XCC id (TaskClock in the kernel). It links that object with the
library's other objects into model/_build/libtcc_spmm_timeline.so; the library build itself is not
changed. This process loads that library instead of tcc_spmm_amd/libtcc_spmm.so, so run it on its
own, not next to the library in one process. The measurement build is not held to the library's
assembly check (its u16-aligned and 64-bit F128 instances spill 3 registers; the buffer-addressed
instances that c2, c3 and c5 use do not), its Y is not checked, and its stamps add a few registers
and instructions per task, so its times are close to, not equal to, the library's.

Per configuration and width it reports, after 40 warm-up launches, from one launch:
- the span, and per XCC its wave-slot utilisation (task time over peak concurrent tasks x the XCC's
  busy time), its tail (its end minus its last task start) and its end;
- the time a workgroup takes to find its task (range search and tail window), inside and outside
  the tail window;
- the panel throughput per 100 us of the launch (each task's panels spread evenly over its duration);
- the time per panel by task size, and the tasks furthest above (panels x the median time per
  panel of unsplit tasks of 288 panels or more), with their SW's chunk count: a split SW's merging
  task shows up there.
"""
from __future__ import annotations

import os
import pathlib
import shlex
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent
LIB = HERE / "_build" / "libtcc_spmm_timeline.so"


def build() -> pathlib.Path:
    """The timeline library: the kernel with TCC_SPMM_TIMELINE, every other object as built."""
    sys.path.insert(0, str(ROOT))
    from tcc_spmm_amd import build as B
    kernel = B.CSRC / "kernel" / "spmm.hip"
    others = [B.BUILD / (str(s.relative_to(B.CSRC)).replace(os.sep, "__") + ".o")
              for s in B._sources() if s != kernel]
    if not all(o.exists() for o in others):
        B.build()
    (HERE / "_build").mkdir(exist_ok=True)
    obj = HERE / "_build" / "spmm_timeline.o"
    for cmd in ([str(B.ROCM / "bin" / "hipcc"), *B.HIP_FLAGS, "-DTCC_SPMM_TIMELINE", "-c",
                 str(kernel), "-o", str(obj)],
                [str(B.ROCM / "bin" / "hipcc"), "-shared", f"--offload-arch={B.ARCH}", "-fPIC",
                 "-o", str(LIB), str(obj), *map(str, others), "-lpthread"]):
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"timeline build failed: {shlex.join(cmd)}\n{res.stderr}")
    return LIB


def _report(cfg: str) -> None:
    import ctypes as C

    import numpy as np
    import torch

    import tcc_spmm_amd as T
    from tcc_spmm_amd import _lib
    from tcc_spmm_amd.device import (TorchDeviceMatrix, pack_features_int8x16,
                                     quantize_features_int8)
    lib = _lib.lib()
    lib.tcc_timeline_stamps.argtypes = [C.c_void_p, C.c_uint32]
    csr = T.synth_csr(cfg)
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    a = fmt.arrays(copy=True)
    tasks = a["tasks"]
    n = len(tasks)
    begin, end = tasks["begin"].astype(np.int64), tasks["end"].astype(np.int64)
    panels = end - begin
    chunks = tasks["chunks"].astype(np.int64)
    print(f"== {cfg}: {csr.rows} rows, {n} tasks, {int(panels.sum())} panels, "
          f"{int((chunks > 1).sum())} split tasks", flush=True)
    dev = torch.device("cuda:0")
    for feats, seed in ((128, 103), (256, 104)):
        x = torch.from_numpy(T.synth_features(csr.cols, feats, seed)).to(dev)
        q, scale = quantize_features_int8(x)
        packed = pack_features_int8x16(q)
        del x, q
        dm = TorchDeviceMatrix(fmt, feats, device=dev)
        y = torch.empty((csr.rows, feats), dtype=torch.float32, device=dev)
        for _ in range(40):
            dm.spmm(packed, scale, y)
        torch.cuda.synchronize()
        dm.spmm(packed, scale, y)
        torch.cuda.synchronize()
        st = np.zeros((n, 4), np.uint64)
        if lib.tcc_timeline_stamps(st.ctypes.data, n) != 0:
            raise RuntimeError("no timeline stamps: is this the timeline library?")
        st = st.astype(np.int64)
        t0 = (st[:, 0] - st[:, 0].min()) / 100.0  # us
        tm = (st[:, 1] - st[:, 0].min()) / 100.0
        t1 = (st[:, 2] - st[:, 0].min()) / 100.0
        xcc = st[:, 3] >> 32
        dur = t1 - t0
        print(f" F{feats}: span {t1.max() / 1e3:.3f} ms", flush=True)
        for x_ in range(8):
            m = xcc == x_
            s0, s1 = t0[m], t1[m]
            ev = np.concatenate([np.stack([s0, np.ones_like(s0)], 1), np.stack([s1, -np.ones_like(s1)], 1)])
            ev = ev[np.lexsort((ev[:, 1], ev[:, 0]))]
            peak = int(np.cumsum(ev[:, 1]).max())
            util = (s1 - s0).sum() / (peak * (s1.max() - s0.min()))
            print(f"   XCC {x_}: {int(m.sum())} tasks, peak {peak} at once, slot utilisation {util:.3f}, "
                  f"tail {(s1.max() - s0.max()) / 1e3:.3f} ms, end {s1.max() / 1e3:.3f} ms", flush=True)
        # the kernel's tail windows: the last 512 tasks of each XCC's range (ranges from the stamps)
        window = np.zeros(n, bool)
        for x_ in range(8):
            ids = np.flatnonzero(xcc == x_)
            if ids.size:
                window[ids[-min(ids.size, 512):]] = True
        find = tm - t0
        print(f"   finding the task: median {np.median(find):.2f} us, in the tail window "
              f"{np.median(find[window]):.2f} us, outside {np.median(find[~window]) if (~window).any() else 0:.2f} us",
              flush=True)
        for name, m in (("< 32 panels", panels < 32), ("32-95", (panels >= 32) & (panels < 96)),
                        ("96-287", (panels >= 96) & (panels < 288)), (">= 288", panels >= 288)):
            if m.any():
                print(f"   tasks {name:>11}: {int(m.sum()):6d}, {dur[m].sum() / panels[m].sum() * 1e3:7.1f} ns "
                      f"per panel", flush=True)
        # Panel throughput over the launch, each task's panels spread evenly over its duration.
        edges = np.arange(0.0, t1.max() + 100.0, 100.0)
        rate_bins = np.zeros(len(edges) - 1)
        for lo, hi, p in zip(t0, t1, panels):
            if p == 0 or hi <= lo:
                continue
            a, b = np.searchsorted(edges, lo, "right") - 1, np.searchsorted(edges, hi, "right") - 1
            for k in range(a, min(b, len(rate_bins) - 1) + 1):
                rate_bins[k] += p * (min(hi, edges[k + 1]) - max(lo, edges[k])) / (hi - lo)
        print("   panels per us, per 100 us of the launch: " +
              " ".join(f"{v / 100.0:.0f}" for v in rate_bins), flush=True)
        big = (panels >= 288) & (chunks == 1)
        rate = np.median(dur[big] / panels[big]) if big.any() else np.median(dur / np.maximum(panels, 1))
        excess = dur - rate * panels
        print(f"   largest excess over {rate * 1e3:.0f} ns per panel:", flush=True)
        for t in np.argsort(-excess)[:6]:
            print(f"     task {t}: {panels[t]} panels, SW of {chunks[t]} chunks, {dur[t]:.0f} us "
                  f"(+{excess[t]:.0f}), from {t0[t] / 1e3:.3f} to {t1[t] / 1e3:.3f} ms", flush=True)
        del dm, y, packed
        torch.cuda.empty_cache()


def main(argv: list[str]) -> int:
    # Read when tcc_spmm_amd._lib is first imported (build() below imports the package); the library
    # itself is loaded lazily, after the build.
    os.environ["TCC_SPMM_LIB"] = str(LIB)
    sys.path.insert(0, str(ROOT))
    if not LIB.exists() or LIB.stat().st_mtime < (ROOT / "tcc_spmm_amd" / "libtcc_spmm.so").stat().st_mtime:
        build()
    for cfg in argv or ["c5"]:
        _report(cfg)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
