"""The build's assembly check (tcc_spmm_amd/asm_check.py) on small hand-written listings, and on
the kernel source as built here."""
import pathlib

from tcc_spmm_amd import asm_check, build

HEAD = "_ZN4test10TestKernelEv:\n"
TAIL = "\ts_endpgm\n.Lfunc_end0:\n"


def _listing(body: str) -> str:
    return HEAD + body + TAIL


def test_early_read_is_flagged():
    problems = asm_check.check(_listing(
        "\tv_mfma_f32_32x32x8_f16 v[0:15], v[16:17], v[18:19], v[0:15]\n"
        "\ts_nop 3\n"
        "\tv_mov_b32_e32 v20, v3\n"))
    assert len(problems) == 1 and "4 wait states" in problems[0]  # s_nop 3 = 4


def test_padded_read_and_accumulator_chain_pass():
    assert asm_check.check(_listing(
        "\tv_mfma_f32_32x32x8_f16 v[0:15], v[16:17], v[18:19], v[0:15]\n"
        "\tv_mfma_f32_32x32x8_f16 v[0:15], v[20:21], v[18:19], v[0:15]\n"
        "\ts_nop 7\n\ts_nop 7\n\ts_nop 1\n"
        "\tv_mov_b32_e32 v20, v3\n")) == []


def test_read_on_a_branch_path_is_flagged():
    problems = asm_check.check(_listing(
        "\tv_mfma_f32_32x32x8_f16 v[0:15], v[16:17], v[18:19], v[0:15]\n"
        "\ts_cbranch_scc1 .LBB0_2\n"
        "\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n"
        ".LBB0_2:\n"
        "\tglobal_store_dwordx4 v[30:31], v[0:3], off\n"))
    assert len(problems) == 1 and "global_store_dwordx4" in problems[0]


def test_overwritten_register_is_not_a_read_of_the_result():
    assert asm_check.check(_listing(
        "\tv_mfma_f32_32x32x8_f16 v[0:15], v[16:17], v[18:19], v[0:15]\n"
        "\tv_mov_b32_e32 v20, v40\n")) == []


def test_spill_is_flagged():
    problems = asm_check.check(_listing("\tscratch_store_dwordx4 off, v[4:7], off offset:16\n"))
    assert any("spills" in p for p in problems)


def test_kernel_source_passes(tmp_path):
    """The shipped SpMM kernels compile to clean assembly (this is also part of every build)."""
    build.check_kernel_asm()
    listing = build.BUILD / "spmm-gfx950.s"
    assert listing.exists()
    assert asm_check.check(listing.read_text()) == []
    assert pathlib.Path(build.CSRC / "kernel" / "spmm.hip").exists()
