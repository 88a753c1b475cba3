"""Ahead-of-time build of librda_gfx950.so from csrc/*.hip for gfx950 (MI355X).

Run as ``python build.py`` from this directory, or call ``build()``. The reference JIT-compiles
its kernels on first use (hip_attention.py:19-25); here the library is built once, in the tree,
so that it ships with the package and loads with no compiler at run time.

The library links against the HIP runtime inside torch (torch/lib/libamdhip64.so): the package
is always loaded after ``import torch``, and one process must not carry two HIP runtimes.
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_NAME = "librda_gfx950.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = "gfx950"

# -ffp-contract=off: every fused multiply-add in the kernels is an explicit __builtin_fmaf, so the
# rounding points are the ones the code shows. Packed fp32 instructions are disabled.
HIPFLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-ffp-contract=off", "-Wall", "-Wno-unused-function",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# Per-source flags. attention.hip: MFMA results in VGPRs (the scores feed VALU softmax directly; with AGPR results
# the compiler copies them out and spills the Q fragments).
FILE_FLAGS = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def torch_lib_dir():
    import torch
    return os.path.join(os.path.dirname(torch.__file__), "lib")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src, hipcc):
    obj = os.path.join(BUILD_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc, *HIPFLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in (r.stderr or "").splitlines() if noise not in line)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    return obj, err


def build(verbose=False, jobs=None):
    hipcc = os.environ.get("HIPCC", "hipcc")
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        results = list(pool.map(lambda s: _compile(s, hipcc), srcs))
    for obj, err in results:
        if verbose and err.strip():
            print(err, file=sys.stderr)
    tl = torch_lib_dir()
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *[o for o, _ in results], "-o", tmp, f"-L{tl}", f"-Wl,-rpath,{tl}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
