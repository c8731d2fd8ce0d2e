import os
import pathlib
import subprocess
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: large synthetic configurations")


def _ensure_built():
    lib = ROOT / "tcc_spmm_amd" / "libtcc_spmm.so"
    cli = ROOT / "tcc_spmm_amd" / "tcc_spmm_run"
    if not lib.exists() or not cli.exists():
        subprocess.run([sys.executable, "-m", "tcc_spmm_amd.build"], cwd=ROOT, check=True)
    orc = ROOT / "oracle" / "_build" / "liboracle.so"
    if not orc.exists():
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)


_ensure_built()


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref_format():
    from oracle import RefFormat
    if not RefFormat.available():
        pytest.skip("reference format library (oracle/_ref) not built here")
    return RefFormat()


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN / "format_reference.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture
def launch_overrides():
    """setSpmmLaunchOverrides for one test (task form, 64-bit instance); automatic choices again
    afterwards. Calling it needs no GPU."""
    from tcc_spmm_amd._lib import check, lib

    def set_overrides(task_waves=0, force_wide=False):
        check(lib().tcc_set_spmm_launch_overrides(int(task_waves), int(bool(force_wide))))

    yield set_overrides
    set_overrides(0, False)
