"""Build recipe for the CPU oracle (test infrastructure only): compiles oracle/*.c into oracle/liboracle.so.

-ffp-contract=off keeps every multiply-add a rounded multiply then a rounded add, as the reference's kernels
require; -mavx2 lets gcc vectorise the independent-lane loops without changing their order (no -ffast-math), and
-mfma makes the explicit fused multiply-adds of aq_math.h single instructions (with contraction still off).
exp / log1p are the platform libm's expf / log1pf, as in the reference; aq_math.h (the device's restatement of them)
is compiled in only for or_math_sweep and or_eval_math(restated=1), which compare the two.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCES = ["oracle_kernels.c", "oracle_model.c", "oracle_sample.c", "oracle_simd.c"]
LIB = os.path.join(HERE, "liboracle.so")

MATH_DIR = os.path.join(os.path.dirname(HERE), "qwen-3.8-in-rust_amd", "csrc")  # aq_math.h, shared with the device


def build(verbose: bool = False) -> str:
    out = LIB
    cmd = ["gcc", "-O3", "-std=gnu11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
           "-mavx2", "-mfma", "-Wall", "-Wno-unknown-pragmas", "-I", MATH_DIR, "-o", out + ".tmp"]
    cmd += [os.path.join(HERE, s) for s in SOURCES] + ["-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(out + ".tmp", out)
    stale = os.path.join(HERE, "liboracle_libm.so")
    if os.path.exists(stale):
        os.remove(stale)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
