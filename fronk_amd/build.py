"""Build the MI355X libraries in-tree (no JIT cache, no site-packages).

libfronk_hip.so      HIP kernels + C ABI (include/fronk_hip.h), gfx950 only.
libfr_hip.so         the "hip" fr_backend vtable (host/hip.c, plain C11),
                     compiled against the reference's own src/ headers where
                     they lie (hidden size fixed there at 2560) and linked
                     against libfronk_hip.so. Its remaining symbols (hw_probe,
                     fr_vectors_check, ...) come from the reference program it
                     is loaded into. Built only when the reference is present.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HIP_SRC = os.path.join(HERE, "csrc", "fronk_hip.hip")
HIP_LIB = os.path.join(HERE, "libfronk_hip.so")
VTABLE_SRC = os.path.join(HERE, "host", "hip.c")
VTABLE_LIB = os.path.join(HERE, "libfr_hip.so")
REFERENCE_SRC = os.path.join(os.environ.get("FRONK_REFERENCE", "/root/reference"), "src")

# Packed-FP32 instructions are disabled for every HIP translation unit.
HIPCC_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-I" + os.path.join(ROOT, "include")]


def build_hip(verbose=False):
    cmd = ["hipcc", *HIPCC_FLAGS, HIP_SRC, "-o", HIP_LIB + ".tmp"]
    subprocess.run(cmd, check=True, capture_output=not verbose)
    os.replace(HIP_LIB + ".tmp", HIP_LIB)
    return HIP_LIB


def build_vtable(verbose=False):
    cmd = ["gcc", "-std=c11", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", "-Werror",
           "-D_POSIX_C_SOURCE=200809L", "-D_DEFAULT_SOURCE", "-DFR_BENCH_RUNTIME=1", "-DFR_HIP_MODULE=1", "-I" + REFERENCE_SRC, "-I" + os.path.join(ROOT, "include"),
           VTABLE_SRC, "-o", VTABLE_LIB + ".tmp", "-L" + HERE, "-lfronk_hip", "-Wl,-rpath,$ORIGIN", "-lm"]
    subprocess.run(cmd, check=True, capture_output=not verbose)
    os.replace(VTABLE_LIB + ".tmp", VTABLE_LIB)
    return VTABLE_LIB


def build_all(verbose=False):
    build_hip(verbose)
    if os.path.isdir(REFERENCE_SRC):
        build_vtable(verbose)


if __name__ == "__main__":
    build_all(verbose=True)
