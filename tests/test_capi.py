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


# A non-null address the host never dereferences: the checks that see it reject the call before
# any launch or copy.
PLACEHOLDER = 0x1000


def _placeholder_view():
    from tcc_spmm_amd._lib import DeviceView
    view = DeviceView()
    for name, _ in DeviceView._fields_:
        if name != "taskCount":
            setattr(view, name, PLACEHOLDER)
    view.taskCount = 1
    return view


def test_device_entry_points_reject_null_buffers_before_any_launch():
    """A null device buffer would fault the GPU: the launch, quantize and pack entry points reject
    it with TCC_INVALID_ARGUMENT first, so this runs on a CPU-only host."""
    from tcc_spmm_amd._lib import DeviceView, lib
    L, P = lib(), PLACEHOLDER
    view = _placeholder_view()
    for args in ((None, P, P), (P, None, P), (P, P, None)):
        st = L.tcc_launch_spmm_int8(ctypes.byref(view), *args, 32, 32, 128, None, None, None)
        assert st == 1 and b"null" in L.tcc_last_error()
        st = L.tcc_launch_spmm_int8_noalloc(ctypes.byref(view), *args, 32, 32, 128, 0, None)
        assert st == 1 and b"null" in L.tcc_last_error()
    bad = _placeholder_view()
    bad.tasks = None
    st = L.tcc_launch_spmm_int8(ctypes.byref(bad), P, P, P, 32, 32, 256, None, None, None)
    assert st == 1 and b"null tasks" in L.tcc_last_error()
    for args in ((None, P, P), (P, None, P), (P, P, None)):
        st = L.tcc_quantize_features_int8(*args, 4, 128, None)
        assert st == 1 and b"null" in L.tcc_last_error()
    for args in ((None, P), (P, None)):
        st = L.tcc_pack_features_int8x16(*args, 4, 128, None)
        assert st == 1 and b"null" in L.tcc_last_error()
    for args in ((None, P, P), (P, None, P), (P, P, None)):
        st = L.tcc_quantize_pack_features_int8(*args, 4, 128, None)
        assert st == 1 and b"null" in L.tcc_last_error()
    # the fused entry applies pack's width rule and quantize's size rule before anything else
    st = L.tcc_quantize_pack_features_int8(P, P, P, 4, 24, None)
    assert st == 1 and b"features % 16" in L.tcc_last_error()
    st = L.tcc_quantize_pack_features_int8(P, P, P, 0, 128, None)
    assert st == 3


def test_output_and_partials_must_be_float_aligned():
    """Y and the partial tiles are written as floats, so any float-aligned base is accepted, as in
    the reference (src/kernel/spmm_kernel.cuh:236-245; the GPU test
    test_spmm_float_aligned_output_and_partials runs +4/+8/+12-byte bases). A base that is not
    float-aligned is refused with TCC_INVALID_ARGUMENT before any launch (placeholders, so this
    runs without a GPU; only offsets that must be refused are passed here)."""
    from tcc_spmm_amd._lib import lib
    L, P = lib(), PLACEHOLDER
    view = _placeholder_view()
    for off in (1, 2, 3, 6, 13):
        st = L.tcc_launch_spmm_int8(ctypes.byref(view), P, P, P + off, 32, 32, 128, None, None, None)
        assert st == 1 and b"output must be float-aligned" in L.tcc_last_error()
        st = L.tcc_launch_spmm_int8_noalloc(ctypes.byref(view), P, P, P + off, 32, 32, 128, 0, None)
        assert st == 1 and b"output must be float-aligned" in L.tcc_last_error()
        st = L.tcc_launch_spmm_int8(ctypes.byref(view), P + 2, P, P + 4, 32, 32, 256, P + off, P, None)
        assert st == 1 and b"partials must be float-aligned" in L.tcc_last_error()


def test_noalloc_entry_point_rejects_before_any_launch():
    """launchSpmmInt8NoAlloc checks the feature count and the size of the plan's workspace against
    its fixed scratch before touching the GPU, so both rejections run on a CPU-only host."""
    from tcc_spmm_amd._lib import DeviceView, lib
    view = _placeholder_view()
    st = lib().tcc_launch_spmm_int8_noalloc(ctypes.byref(view), None, None, None, 32, 32, 64, 1,
                                            None)
    assert st == 1 and b"128 or 256" in lib().tcc_last_error()
    # Placeholder addresses pass the null checks; the size check rejects before anything reads them.
    x, sc, y = PLACEHOLDER, PLACEHOLDER, PLACEHOLDER
    # c3 at F=256: 14,731 partial tiles of 8 KiB need 120.7 MB, more than the 64 MiB scratch.
    st = lib().tcc_launch_spmm_int8_noalloc(ctypes.byref(view), x, sc, y, 2449029, 2449029, 256,
                                            14731, None)
    assert st == 1 and b"scratch" in lib().tcc_last_error()
    # The largest plan that fits at F=128 for 4096 rows: 128 counters (one 256-byte block) plus
    # K tiles of 4 KiB in 64 MiB.
    k_max = ((64 << 20) - 256) // (8 * 128 * 4)
    st = lib().tcc_launch_spmm_int8_noalloc(ctypes.byref(view), x, sc, y, 4096, 4096, 128,
                                            k_max + 1, None)
    assert st == 1 and b"scratch" in lib().tcc_last_error()
    assert b"noalloc" in (ROOT / "include" / "tcc_spmm_c.h").read_bytes()


def test_null_outputs_and_arrays_are_rejected():
    """A null output pointer, handle or input array returns TCC_INVALID_ARGUMENT (1) instead of
    crashing the caller; these are host-only entry points, so this runs on a CPU-only host."""
    import numpy as np
    from tcc_spmm_amd._lib import Sw32Sizes, lib
    L = lib()
    offsets = np.array([0, 1, 2], np.uint32)
    ids = np.array([0, 1], np.uint32)
    vals = np.array([1.0, 2.0], np.float32)
    h = ctypes.c_void_p()
    u32 = ctypes.c_uint32()

    def rejected(status, what):
        assert status == 1, what
        assert b"null" in L.tcc_last_error(), what

    rejected(L.tcc_make_canonical_csr(2, 2, 2, offsets.ctypes.data, ids.ctypes.data,
                                      vals.ctypes.data, None), "make_canonical_csr out")
    rejected(L.tcc_make_canonical_csr(2, 2, 2, None, ids.ctypes.data, vals.ctypes.data,
                                      ctypes.byref(h)), "make_canonical_csr rowOffsets")
    rejected(L.tcc_make_canonical_csr(2, 2, 2, offsets.ctypes.data, None, vals.ctypes.data,
                                      ctypes.byref(h)), "make_canonical_csr sourceIds")
    rejected(L.tcc_csr_from_arrays(3, offsets.ctypes.data, 2, None, vals.ctypes.data,
                                   ctypes.byref(h)), "csr_from_arrays sourceIds")
    rejected(L.tcc_load_matrix_market(b"x.mtx", None, ctypes.byref(u32), ctypes.byref(h)),
             "load_matrix_market rows")
    assert L.tcc_make_canonical_csr(2, 2, 2, offsets.ctypes.data, ids.ctypes.data,
                                    vals.ctypes.data, ctypes.byref(h)) == 0
    try:
        rejected(L.tcc_csr_info(h, None, None), "csr_info")
        rejected(L.tcc_convert_csr_to_sw32(2, 2, h, 1, None), "convert out")
        fmt = ctypes.c_void_p()
        assert L.tcc_convert_csr_to_sw32(2, 2, h, 1, ctypes.byref(fmt)) == 0
        try:
            rejected(L.tcc_sw32_get_sizes(fmt, None), "sw32_get_sizes")
            rejected(L.tcc_sw32_get_arrays(fmt, None), "sw32_get_arrays")
            sizes = Sw32Sizes()
            assert L.tcc_sw32_get_sizes(fmt, ctypes.byref(sizes)) == 0 and sizes.rows == 2
        finally:
            L.tcc_sw32_free(fmt)
    finally:
        L.tcc_csr_free(h)


def test_launch_overrides_hook(launch_overrides):
    """setSpmmLaunchOverrides takes 0 (automatic), 1 or 2 waves per task and rejects other counts;
    it touches no GPU."""
    from tcc_spmm_amd._lib import lib
    for waves in (0, 1, 2):
        assert lib().tcc_set_spmm_launch_overrides(waves, 0) == 0
    assert lib().tcc_set_spmm_launch_overrides(1, 1) == 0
    assert lib().tcc_set_spmm_launch_overrides(3, 0) == 1
    assert b"taskWaves" in lib().tcc_last_error()
