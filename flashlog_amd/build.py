"""Build recipe for libflashlog_hip.so (gfx950).  Run as a script or through
``__graft_entry__.build()``; always recompiles."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libflashlog_hip.so")
HIP_SOURCES = ["fl_dense.hip", "fl_ranks.hip", "fl_scan.hip", "fl_sparse.hip", "fl_rules.hip", "fl_grounding.hip"]
HOST_SOURCES = ["fl_host.cpp"]

# -ffp-contract=off: the bit-exact paths must not fuse a*b+c.
# -packed-fp32-ops disabled: packed FP32 forms are avoided on this platform.
HIP_FLAGS = ["-O3", "-std=c++17", "--offload-arch=gfx950", "-fPIC", "-ffp-contract=off",
             "-fno-fast-math", "-fno-gpu-flush-denormals-to-zero",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wno-unused-command-line-argument"]


def build(verbose=False):
    build_dir = os.path.join(HERE, "_build")
    os.makedirs(build_dir, exist_ok=True)
    objs = []
    for src in HIP_SOURCES + HOST_SOURCES:
        obj = os.path.join(build_dir, os.path.splitext(src)[0] + ".o")
        cmd = ["hipcc", "-c", os.path.join(CSRC, src), "-o", obj] + HIP_FLAGS
        if src.endswith(".cpp"):
            cmd = ["hipcc", "-c", "-x", "c++", os.path.join(CSRC, src), "-o", obj, "-O3", "-std=c++17",
                   "-fPIC", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include"]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.check_call(cmd)
        objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = ["hipcc", "-shared", "--offload-arch=gfx950", "-o", tmp] + objs
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.check_call(cmd)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
