"""Build recipe for libflashlog_hip.so (gfx950).  Run as a script or through
``__graft_entry__.build()``; always recompiles."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libflashlog_hip.so")
HIP_SOURCES = ["fl_dense.hip", "fl_ranks.hip", "fl_scan.hip", "fl_sparse.hip", "fl_rules.hip", "fl_grounding.hip",
               "fl_csr.hip", "fl_extract.hip"]
HOST_SOURCES = ["fl_host.cpp"]

# -ffp-contract=off: the bit-exact paths must not fuse a*b+c.
# -packed-fp32-ops disabled: packed FP32 forms are avoided on this platform.
HIP_FLAGS = ["-O3", "-std=c++17", "--offload-arch=gfx950", "-fPIC", "-ffp-contract=off",
             "-fno-fast-math", "-fno-gpu-flush-denormals-to-zero",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wno-unused-command-line-argument"]


def _compile(src, build_dir, verbose):
    obj = os.path.join(build_dir, os.path.splitext(src)[0] + ".o")
    if src.endswith(".cpp"):
        cmd = ["hipcc", "-c", "-x", "c++", os.path.join(CSRC, src), "-o", obj, "-O3", "-std=c++17",
               "-fPIC", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include"]
    else:
        cmd = ["hipcc", "-c", os.path.join(CSRC, src), "-o", obj] + HIP_FLAGS
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.check_call(cmd)
    return obj


def build(verbose=False, jobs=None):
    """Compiles every source (in parallel, one hipcc per file) and links the
    library; returns its path."""
    from concurrent.futures import ThreadPoolExecutor
    build_dir = os.path.join(HERE, "_build")
    os.makedirs(build_dir, exist_ok=True)
    srcs = HIP_SOURCES + HOST_SOURCES
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, build_dir, verbose), srcs))
    tmp = LIB + ".tmp"
    cmd = ["hipcc", "-shared", "--offload-arch=gfx950", "-o", tmp] + objs
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.check_call(cmd)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
