"""Build the MI355X libraries in-tree (no JIT cache, no site-packages).

libfronk_hip.so      HIP kernels + C ABI (include/fronk_hip.h), gfx950 only.
libfr_hip_<H>.so     the fr_backend vtable (host/hip.c, plain C) for hidden H,
                     linked against libfronk_hip.so.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HIP_SRC = os.path.join(HERE, "csrc", "fronk_hip.hip")
HIP_LIB = os.path.join(HERE, "libfronk_hip.so")
VTABLE_SRC = os.path.join(HERE, "host", "hip.c")
HIDDEN_SIZES = (2560, 4096)

# Packed-FP32 instructions are disabled for every HIP translation unit.
HIPCC_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-I" + os.path.join(ROOT, "include")]


def vtable_lib(hidden):
    return os.path.join(HERE, f"libfr_hip_{hidden}.so")


def build_hip(verbose=False):
    cmd = ["hipcc", *HIPCC_FLAGS, HIP_SRC, "-o", HIP_LIB + ".tmp"]
    subprocess.run(cmd, check=True, capture_output=not verbose)
    os.replace(HIP_LIB + ".tmp", HIP_LIB)
    return HIP_LIB


def build_vtable(hidden, verbose=False):
    out = vtable_lib(hidden)
    cmd = ["gcc", "-std=c11", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", "-Werror",
           f"-DFR_HIDDEN={hidden}", "-I" + os.path.join(HERE, "host"), "-I" + os.path.join(ROOT, "include"),
           VTABLE_SRC, "-o", out + ".tmp", "-L" + HERE, "-lfronk_hip", "-Wl,-rpath,$ORIGIN", "-lm"]
    subprocess.run(cmd, check=True, capture_output=not verbose)
    os.replace(out + ".tmp", out)
    return out


def build_all(verbose=False):
    build_hip(verbose)
    if os.path.exists(VTABLE_SRC):
        for h in HIDDEN_SIZES:
            build_vtable(h, verbose)


if __name__ == "__main__":
    build_all(verbose=True)
