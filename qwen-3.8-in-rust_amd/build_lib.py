"""Build libaq.so (the HIP kernels and the C-ABI of include/aq.h) for gfx950 with hipcc, in-tree.

Flags: -ffp-contract=off keeps the reference's no-FMA arithmetic where the kernels reproduce its order;
`-Xclang -target-feature -Xclang -packed-fp32-ops` keeps the compiler from emitting packed FP32 ops.
"""
import hashlib
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "aqueduct")
LIB = os.path.join(OUT_DIR, "libaq.so")
OBJ_DIR = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = ["-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-mllvm", "-amdgpu-mfma-vgpr-form",  # matrix-core results in VGPRs: no accumulator-register copies
          # the leading scalar / pointer kernel arguments arrive in SGPRs at wave launch instead of by a scalar load
          # from the kernel-argument segment (the small kernels' first loads no longer wait on it)
          "-mllvm", "-amdgpu-kernarg-preload-count=16",
          "-Wall", "-Wno-unused-function",
          "-Wno-unused-variable", "-Wno-unused-but-set-variable"]


INCLUDE = os.path.join(os.path.dirname(HERE), "include", "aq.h")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def source_hash() -> str:
    """sha256 of every csrc/ source and header, include/aq.h and the compiler flags: the stamp libaq.so carries
    (aq_build_hash) and aqueduct.lib() checks, so a library built from other sources is never loaded."""
    h = hashlib.sha256()
    files = sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".h")))
    for f in files:
        h.update(f.encode() + b"\0")
        h.update(open(os.path.join(CSRC, f), "rb").read())
    h.update(open(INCLUDE, "rb").read())
    h.update(" ".join(COMMON + [ARCH]).encode())
    return h.hexdigest()[:32]


def build(verbose: bool = False, jobs: int = 8) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    stamp = [f'-DAQ_BUILD_HASH="{source_hash()}"']

    def compile_one(src):
        obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
        cmd = [HIPCC] + COMMON + stamp + ["-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", LIB + ".tmp"] + objs
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
