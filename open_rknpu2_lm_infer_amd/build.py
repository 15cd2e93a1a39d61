"""Builds libqlinear.so and libqlinear.a (the HIP kernels, the C ABI and the C++ npu
mirror) in-tree for gfx950, libqlcalib.so (the calibration kernels of bench.py --mode
calib, not part of the library), and the native test binaries under tests/cpp/_build:
the npu mirror's test and a C program linked against the static archive.

    python -m open_rknpu2_lm_infer_amd.build

Every .hip / .cpp file under csrc/ is compiled to an object in parallel with hipcc,
then linked into open_rknpu2_lm_infer_amd/libqlinear.so next to this file and archived
into libqlinear.a (the form a Rust build.rs links: the archive whole, plus -lamdhip64
and the C++ runtime).  Device code
is compiled with single-rounding IEEE semantics: no FP contraction, correctly
rounded f32 divide and sqrt, denormals kept, packed-FP32 instructions disabled.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libqlinear.so")
STATIC_LIB = os.path.join(HERE, "libqlinear.a")
ARCH = os.environ.get("QLIN_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


# Per-file additions.  The GEMM keeps its MFMA accumulators in VGPRs: with the
# compiler's AGPR heuristics the two-tile unrolled k loop re-shuffled the accumulator
# registers on every iteration.
FILE_FLAGS = {"qlin_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}

ROOT = os.path.dirname(HERE)
TEST_SRC = os.path.join(ROOT, "tests", "cpp", "npu_backend_test.cpp")
TEST_BUILD = os.path.join(ROOT, "tests", "cpp", "_build")
TEST_BIN = os.path.join(TEST_BUILD, "npu_backend_test")
STATIC_TEST_SRC = os.path.join(ROOT, "tests", "cpp", "static_link_test.c")
STATIC_TEST_BIN = os.path.join(TEST_BUILD, "static_link_test")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    objs, procs = [], []
    for src in sources():
        obj = os.path.join(BUILD, os.path.splitext(os.path.basename(src))[0] + ".o")
        objs.append(obj)
        cmd = [HIPCC, *COMMON, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        text = out.decode(errors="replace")
        lines = [l for l in text.splitlines() if "packed-fp32-ops" not in l]
        if lines and (verbose or p.returncode):
            print("\n".join(lines), file=sys.stderr)
        if p.returncode:
            failed.append(src)
    if failed:
        raise RuntimeError(f"hipcc failed for {failed}")
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           "-Wl,-rpath,/opt/rocm/lib"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    tmp = STATIC_LIB + ".tmp"
    if os.path.exists(tmp):
        os.remove(tmp)
    subprocess.run(["ar", "rcs", tmp, *objs], check=True)
    os.replace(tmp, STATIC_LIB)
    build_calib()
    build_tests()
    return LIB


CALIB_SRC = os.path.join(HERE, "calib", "qlin_calib.hip")
CALIB_LIB = os.path.join(HERE, "libqlcalib.so")


def build_calib() -> str:
    """Calibration kernels of the roofline figures (bench.py --mode calib); not part of
    libqlinear.so."""
    tmp = CALIB_LIB + ".tmp"
    subprocess.run([HIPCC, *COMMON, "-shared", CALIB_SRC, "-o", tmp, "-Wl,-rpath,/opt/rocm/lib"], check=True,
                   stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    os.replace(tmp, CALIB_LIB)
    return CALIB_LIB


def build_tests() -> str:
    """Native test of the npu mirror; its checker (the CPU oracle) is compiled in."""
    os.makedirs(TEST_BUILD, exist_ok=True)
    oracle_obj = os.path.join(TEST_BUILD, "qlin_oracle.o")
    subprocess.run(["gcc", "-O2", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-std=c11", "-c",
                    os.path.join(ROOT, "oracle", "qlin_oracle.c"), "-o", oracle_obj], check=True)
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", TEST_SRC, oracle_obj, "-o", TEST_BIN,
                    f"-L{HERE}", "-lqlinear", "-Wl,-rpath,$ORIGIN/../../../open_rknpu2_lm_infer_amd", "-lm"], check=True)
    # a C caller of the static archive, linked as a Rust build.rs would link it (its GPU
    # mode checks the kernels against the oracle, compiled in as the checker)
    static_obj = os.path.join(TEST_BUILD, "static_link_test.o")
    subprocess.run(["gcc", "-O2", "-std=c11", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-c",
                    STATIC_TEST_SRC, "-o", static_obj], check=True)
    subprocess.run(["g++", static_obj, oracle_obj, "-o", STATIC_TEST_BIN, "-Wl,--whole-archive", STATIC_LIB,
                    "-Wl,--no-whole-archive", "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib", "-lm"],
                   check=True)
    return TEST_BIN


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
