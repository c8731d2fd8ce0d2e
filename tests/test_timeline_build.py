"""The measurement build of model/timeline.py compiles (hipcc cross-compiles for gfx950 here) and
exports its stamp read-back, which the library build does not."""
import subprocess
import sys

import pytest

import model.timeline as tl
from tcc_spmm_amd import build as B


def _exports(path):
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    return out.stdout


@pytest.mark.skipif(sys.platform != "linux", reason="hipcc and nm on Linux")
def test_timeline_library_builds_and_exports_stamps():
    lib = tl.build()
    assert "tcc_timeline_stamps" in _exports(lib)
    assert "launchSpmmInt8" in _exports(lib)
    assert "tcc_timeline_stamps" not in _exports(B.LIB)
