"""Build libtcc_spmm.so in-tree for gfx950.

HIP sources (*.hip) go through hipcc for gfx950 with packed-FP32 instructions disabled; host-only
C++ sources (*.cpp) go through g++ against the ROCm headers. Objects land in tcc_spmm_amd/_build/,
the library in tcc_spmm_amd/libtcc_spmm.so. The command-line harness (cli/tcc_spmm_run.cpp) is linked
against it as tcc_spmm_amd/tcc_spmm_run. Run ``python -m tcc_spmm_amd.build``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shlex
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libtcc_spmm.so"
CLI_SRC = PKG / "cli" / "tcc_spmm_run.cpp"
CLI = PKG / "tcc_spmm_run"
ROCM = pathlib.Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = os.environ.get("TCC_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]
CXX_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-pthread", "-D__HIP_PLATFORM_AMD__",
    f"-I{ROOT / 'include'}", f"-I{CSRC}", f"-I{ROCM / 'include'}",
]


def _sources():
    return sorted(p for p in CSRC.rglob("*") if p.suffix in (".hip", ".cpp"))


def _compile(src: pathlib.Path) -> pathlib.Path:
    rel = src.relative_to(CSRC)
    obj = BUILD / (str(rel).replace(os.sep, "__") + ".o")
    if src.suffix == ".hip":
        cmd = [str(ROCM / "bin" / "hipcc"), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [os.environ.get("CXX", "g++"), *CXX_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {shlex.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def check_kernel_asm(src: pathlib.Path = CSRC / "kernel" / "spmm.hip") -> None:
    """Assemble the SpMM kernels for gfx950 and refuse them if they spill to scratch or read an
    MFMA result too early (tcc_spmm_amd/asm_check.py explains why the build checks this)."""
    from . import asm_check
    out = BUILD / "spmm-gfx950.s"
    cmd = [str(ROCM / "bin" / "hipcc"), *HIP_FLAGS, "--cuda-device-only", "-S", str(src), "-o",
           str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"assembly listing failed: {shlex.join(cmd)}\n{res.stderr}")
    problems = asm_check.check(out.read_text())
    if problems:
        raise RuntimeError("SpMM kernel assembly check failed:\n  " + "\n  ".join(problems))


def build(verbose: bool = False) -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    srcs = _sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        asm = pool.submit(check_kernel_asm)
        objs = list(pool.map(_compile, srcs))
        asm.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [str(ROCM / "bin" / "hipcc"), "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", str(tmp),
           *map(str, objs), "-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {shlex.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    build_cli()
    if verbose:
        print(f"built {LIB} and {CLI}")
    return LIB


def build_cli() -> pathlib.Path:
    """Link the command-line harness against the in-tree library (found at run time via $ORIGIN)."""
    tmp = CLI.with_suffix(".tmp")
    cmd = [os.environ.get("CXX", "g++"), *CXX_FLAGS, "-o", str(tmp), str(CLI_SRC), f"-L{PKG}", "-ltcc_spmm",
           "-Wl,-rpath,$ORIGIN", f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"CLI build failed: {shlex.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, CLI)
    return CLI


def build_oracle(verbose: bool = False) -> None:
    """Compile oracle/ (C restatement, and the reference's own CPU format code when present)."""
    res = subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    if verbose:
        print("built oracle")


SAN_DIR = PKG / "_san"
SAN_FLAGS = ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
             "-fno-sanitize-recover=undefined"]


def build_sanitized(verbose: bool = False) -> pathlib.Path:
    """AddressSanitizer + UBSan build of the host code, for CPU test runs only.

    The host C++ sources (format builders, Matrix Market reader, C ABI, synthetic generators) are
    compiled by clang with the sanitizers; the HIP sources keep their ordinary build, since the
    sanitizers here cover host code only. The result goes to tcc_spmm_amd/_san/libtcc_spmm.so and
    oracle/_san/liboracle.so; run the CPU suite against them with clang's ASan runtime preloaded:

        python -m tcc_spmm_amd.build --sanitize
        TCC_SPMM_LIB=tcc_spmm_amd/_san/libtcc_spmm.so TCC_ORACLE_LIB=oracle/_san/liboracle.so \
        TCC_SANITIZER_RUN=1 \
        LD_PRELOAD=$(/opt/rocm/llvm/bin/clang -print-file-name=libclang_rt.asan-x86_64.so) \
        ASAN_OPTIONS=detect_leaks=0 python -m pytest tests -m "not gpu"

    (TCC_SANITIZER_RUN makes the ThreadSanitizer tests of the merge model skip: their binaries cannot
    run with ASan's runtime preloaded.)
    """
    SAN_DIR.mkdir(exist_ok=True)
    build()  # the ordinary objects, HIP ones included
    clang = str(ROCM / "llvm" / "bin" / "clang++")
    objs = []
    for src in _sources():
        if src.suffix == ".hip":
            objs.append(BUILD / (str(src.relative_to(CSRC)).replace(os.sep, "__") + ".o"))
            continue
        obj = SAN_DIR / (str(src.relative_to(CSRC)).replace(os.sep, "__") + ".o")
        cmd = [clang, *SAN_FLAGS, *[f for f in CXX_FLAGS if f != "-O3"], "-c", str(src), "-o",
               str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"compile failed: {shlex.join(cmd)}\n{res.stderr}")
        objs.append(obj)
    out = SAN_DIR / "libtcc_spmm.so"
    cmd = [str(ROCM / "bin" / "hipcc"), "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", str(out),
           *map(str, objs), "-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {shlex.join(cmd)}\n{res.stderr}")
    res = subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "san"], capture_output=True,
                         text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle sanitizer build failed:\n{res.stdout}\n{res.stderr}")
    if verbose:
        print(f"built {out} and oracle/_san/liboracle.so")
    return out


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        build_sanitized(verbose=True)
    else:
        build(verbose=True)
    if "--with-oracle" in sys.argv:
        build_oracle(verbose=True)
