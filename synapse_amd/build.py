"""Builds the gfx950 attention library (and, for tests, the CPU oracle and the
C++ host tests) in-tree.

    python -m synapse_amd.build            # library + oracle + host tests
    python -m synapse_amd.build --lib      # library only
    python -m synapse_amd.build --stamps   # the decode phase-stamp timing build

Outputs (git-ignored, but shipped to the GPU box with the tree):
    synapse_amd/libsynapse_hip.so          the C ABI of include/synapse_hip.h
    synapse_amd/libsynapse_hip_stamps.so   the same with decode phase stamps
                                           (synapse_amd/decode_phases.py reads them)
    oracle/liboracle.so                    CPU oracle (test infrastructure)
    oracle/_ref/libref_half.so             the reference's own binary16 code
    tests/cpp/_bin/*                       C++ host tests
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parent.parent
PKG = ROOT / "synapse_amd"
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libsynapse_hip.so"
STAMPS_LIB = PKG / "libsynapse_hip_stamps.so"
HOST_INC = PKG / "host"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Werror",
    # Packed-FP32 instructions stay off on this pool (wrong results seen).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# Per-source additions: the int8 GEMM's products feed vector work directly,
# so their results go to VGPRs (no accumulator-register moves). The same for
# the decode kernel measured no change.
SOURCE_FLAGS = {"quant_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
HIP_SOURCES = ["kv_append.hip", "decode.hip", "prefill.hip", "flash.hip", "generic.hip", "rope.hip", "ops.hip",
               "quant.hip", "quant_gemm.hip", "capi.hip"]


def _run(cmd: list[str], cwd: pathlib.Path | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build failed ({' '.join(cmd)}):\n{out}")


def build_library(stamps: bool = False) -> pathlib.Path:
    """The library; with stamps, the timing build whose decode kernels record
    phase timestamps (SYN_DECODE_STAMPS), to its own file."""
    build = BUILD / "stamps" if stamps else BUILD
    lib = STAMPS_LIB if stamps else LIB
    build.mkdir(parents=True, exist_ok=True)
    objs = []

    def compile_one(src: str) -> pathlib.Path:
        obj = build / (pathlib.Path(src).stem + ".o")
        extra = ["-DSYN_DECODE_STAMPS"] if stamps else []
        _run([HIPCC, *HIP_FLAGS, *SOURCE_FLAGS.get(src, []), *extra, "-c", str(CSRC / src), "-o", str(obj)])
        return obj

    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(HIP_SOURCES))) as ex:
        objs = list(ex.map(compile_one, HIP_SOURCES))
    tmp = lib.with_suffix(".so.tmp")
    # -z defs: an unresolved symbol fails the link (a kernel whose host stub
    # the compiler silently dropped would otherwise surface only at load time).
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, lib)
    return lib


def build_oracle() -> None:
    _run(["make", "-s", "-C", str(ROOT / "oracle")])


CPP_TESTS = {
    # name: (source, links the CPU oracle)
    "test_graph": ("tests/cpp/test_graph.cpp", False),
    "test_session": ("tests/cpp/test_session.cpp", True),
    "test_model_session": ("tests/cpp/test_model_session.cpp", False),
}
# Host builds of device-side math (no library, no HIP).
CPP_MATH_TESTS = {"test_rope_math": "tests/cpp/test_rope_math.cpp"}
# Host tests linked against tests/cpp/stub_abi.cpp (a C ABI that launches
# nothing) instead of the library: they run on the CPU.
CPP_STUB_TESTS = {"test_no_alloc": "tests/cpp/test_no_alloc.cpp"}


def build_host_tests() -> None:
    """The C++20 host tests: both link libsynapse_hip.so (the builder sizes
    attention scratch through it); the session test also links the oracle."""
    out = ROOT / "tests" / "cpp" / "_bin"
    out.mkdir(parents=True, exist_ok=True)
    for name, (src, oracle) in CPP_TESTS.items():
        cmd = ["g++", "-std=c++20", "-O2", "-Wall", "-Wextra", "-Werror", "-ffp-contract=off", f"-I{HOST_INC}",
               f"-I{ROOT / 'include'}", f"-I{ROOT / 'tests' / 'cpp'}", str(ROOT / src), "-o", str(out / name),
               f"-L{PKG}", "-lsynapse_hip", f"-Wl,-rpath,{PKG}", "-pthread"]
        if oracle:
            cmd += [f"-I{ROOT / 'oracle'}", f"-L{ROOT / 'oracle'}", "-loracle", f"-Wl,-rpath,{ROOT / 'oracle'}"]
        _run(cmd)
    for name, src in CPP_MATH_TESTS.items():
        _run(["g++", "-std=c++20", "-O2", "-Wall", "-Wextra", "-Werror", "-Wno-unknown-pragmas", "-ffp-contract=off", f"-I{CSRC}",
              f"-I{ROOT / 'tests' / 'cpp'}", str(ROOT / src), "-o", str(out / name)])
    for name, src in CPP_STUB_TESTS.items():
        _run(["g++", "-std=c++20", "-O2", "-Wall", "-Wextra", "-Werror", "-ffp-contract=off", f"-I{HOST_INC}",
              f"-I{ROOT / 'include'}", f"-I{ROOT / 'tests' / 'cpp'}", str(ROOT / src),
              str(ROOT / "tests" / "cpp" / "stub_abi.cpp"), "-o", str(out / name)])


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--lib", action="store_true", help="build the HIP library only")
    ap.add_argument("--stamps", action="store_true", help="build the decode phase-stamp timing library only")
    args = ap.parse_args(argv)
    if not shutil.which(HIPCC) and not pathlib.Path(HIPCC).exists():
        print(f"hipcc not found at {HIPCC}", file=sys.stderr)
        return 1
    if args.stamps:
        build_library(stamps=True)
        print(f"built {STAMPS_LIB.relative_to(ROOT)}")
        return 0
    build_library()
    print(f"built {LIB.relative_to(ROOT)}")
    if not args.lib:
        build_oracle()
        print("built oracle/liboracle.so")
        build_host_tests()
        print("built tests/cpp/_bin")
    return 0


if __name__ == "__main__":
    sys.exit(main())
