"""Builds libllmcp_q8.so in place with hipcc for gfx950.

All HIP code is compiled with packed-fp32 instruction selection disabled and
without floating-point contraction, so the scalar epilogue keeps separate
multiply and add roundings.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libllmcp_q8.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["q8_kernels.hip", "q8_gemv_fma.hip", "q8_gemm.hip", "q8_microbench.hip",
           "q8_runtime.cpp"]

ROOT = os.path.dirname(HERE)
CONSUMER_SRC = os.path.join(ROOT, "tests", "c_consumer", "q8_consumer.cpp")
CONSUMER = os.path.join(ROOT, "tests", "c_consumer", "q8_consumer")

COMMON = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def build(verbose=False):
    # the sources compile independently: run the compilers side by side
    objs, procs = [], []
    for src in SOURCES:
        path = os.path.join(CSRC, src)
        if not os.path.exists(path):
            continue
        obj = os.path.join(CSRC, os.path.splitext(src)[0] + ".o")
        cmd = [HIPCC] + COMMON + ["-c", path, "-o", obj]
        if src.endswith(".cpp"):
            cmd = [HIPCC] + COMMON + ["-fopenmp", "-x", "hip", "-c", path, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd)))
        objs.append(obj)
    failed = [src for src, p in procs if p.wait() != 0]
    if failed:
        raise subprocess.CalledProcessError(1, "hipcc " + " ".join(failed))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fopenmp", "-o", tmp] + objs
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


def build_consumer(verbose=False):
    """Links the C++17 test host of the C ABI against the built library with
    the plain host compiler, as an AOT runtime would: only include/ and
    -lllmcp_q8, no HIP headers."""
    tmp = CONSUMER + ".tmp"
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra",
           "-I", os.path.join(ROOT, "include"), CONSUMER_SRC,
           "-L", HERE, "-lllmcp_q8",
           "-Wl,-rpath,$ORIGIN/../../llmcp_amd",
           "-Wl,-rpath-link,/opt/rocm/lib", "-Wl,-rpath-link,/opt/rocm/llvm/lib",
           "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, CONSUMER)
    return CONSUMER


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    build_consumer(verbose="-v" in sys.argv)
    print(LIB)
