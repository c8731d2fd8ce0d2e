"""The C-ABI library loads on a CPU-only host and exports every symbol include/*.h declares."""
import ctypes
import re

import pytest

from conftest import ROOT


def declared_functions():
    text = (ROOT / "include" / "tcc_spmm_c.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tcc_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    for required in ("tcc_launch_spmm_int8", "tcc_quantize_features_int8",
                     "tcc_pack_features_int8x16", "tcc_convert_csr_to_sw32",
                     "tcc_build_panel_tasks", "tcc_make_canonical_csr"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from tcc_spmm_amd._lib import LIB_PATH, SIGNATURES
    lib = ctypes.CDLL(str(LIB_PATH))
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in tcc_spmm_c.h but not exported"
    assert set(declared_functions()) == set(SIGNATURES), "ctypes table out of sync with header"


CXX_HEADERS = ("format/csr.h", "format/sw32.h", "format/int8_features.h", "spmm.h")


def declared_cxx_functions():
    """Names of the non-inline functions the C++ headers declare (the reference's surface)."""
    names = set()
    for h in CXX_HEADERS:
        text = (ROOT / "include" / h).read_text()
        text = re.sub(r"//[^\n]*", "", text)
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^(?!\s*(?:static_assert|inline|return|#|struct|constexpr))[A-Za-z_][\w:<>]*\s+"
                             r"([A-Za-z_]\w*)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return sorted(names)


def test_library_exports_the_cxx_surface():
    import shutil
    import subprocess
    from tcc_spmm_amd._lib import LIB_PATH
    names = declared_cxx_functions()
    assert {"makeCanonicalCsr", "loadMatrixMarket", "convertCsrToSw32", "buildPanelTasks",
            "quantizeFeaturesInt8", "packFeaturesInt8x16", "launchSpmmInt8"} <= set(names), names
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm is not installed")
    out = subprocess.run([nm, "-DC", "--defined-only", str(LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {m.group(1) for m in re.finditer(r"\s[TW]\s+([A-Za-z_]\w*)\(", out)}
    missing = [n for n in names if n not in exported]
    assert not missing, f"declared in include/ but not exported: {missing}"


def test_version_and_error_reporting():
    from tcc_spmm_amd._lib import check, lib
    assert b"gfx950" in lib().tcc_version()
    h = ctypes.c_void_p()
    st = lib().tcc_synth_csr(b"no-such-config", ctypes.byref(ctypes.c_uint32()),
                             ctypes.byref(ctypes.c_uint32()), ctypes.byref(h))
    assert st == 1
    assert b"unknown synthetic config" in lib().tcc_last_error()
    with pytest.raises(ValueError):
        check(st)


def test_device_entry_points_reject_bad_features_before_any_launch():
    # std::invalid_argument for F not in {128, 256} is raised before touching the GPU, so this
    # runs on a CPU-only host (reference src/kernel/spmm.cu:20-29).
    from tcc_spmm_amd._lib import DeviceView, lib
    view = DeviceView()
    view.taskCount = 1
    st = lib().tcc_launch_spmm_int8(ctypes.byref(view), None, None, None, 32, 32, 64, None, None,
                                    None)
    assert st == 1
    assert b"128 or 256" in lib().tcc_last_error()
    st = lib().tcc_pack_features_int8x16(None, None, 4, 24, None)
    assert st == 1  # features % 16 != 0


def test_header_structs_match_cpp_layouts():
    from tcc_spmm_amd._lib import DeviceView
    assert ctypes.sizeof(DeviceView) == 10 * 8  # 9 pointers + uint32 padded to 8
    header = (ROOT / "include" / "format" / "sw32.h").read_text()
    assert "static_assert(sizeof(Sw32Task) == 28" in header


def test_noalloc_entry_point_rejects_before_any_launch():
    """launchSpmmInt8NoAlloc checks the feature count and the size of the plan's workspace against
    its fixed scratch before touching the GPU, so both rejections run on a CPU-only host."""
    from tcc_spmm_amd._lib import DeviceView, lib
    view = DeviceView()
    view.taskCount = 1
    st = lib().tcc_launch_spmm_int8_noalloc(ctypes.byref(view), None, None, None, 32, 32, 64, 1,
                                            None)
    assert st == 1 and b"128 or 256" in lib().tcc_last_error()
    # c3 at F=256: 14,731 partial tiles of 8 KiB need 120.7 MB, more than the 64 MiB scratch.
    st = lib().tcc_launch_spmm_int8_noalloc(ctypes.byref(view), None, None, None, 2449029,
                                            2449029, 256, 14731, None)
    assert st == 1 and b"scratch" in lib().tcc_last_error()
    # The largest plan that fits at F=128 for 4096 rows: 128 counters (one 256-byte block) plus
    # K tiles of 4 KiB in 64 MiB.
    k_max = ((64 << 20) - 256) // (8 * 128 * 4)
    st = lib().tcc_launch_spmm_int8_noalloc(ctypes.byref(view), None, None, None, 4096, 4096, 128,
                                            k_max + 1, None)
    assert st == 1 and b"scratch" in lib().tcc_last_error()
    assert b"noalloc" in (ROOT / "include" / "tcc_spmm_c.h").read_bytes()
