"""Build recipe for the CPU oracle (test infrastructure only): compiles oracle/*.c into oracle/liboracle.so.

-ffp-contract=off keeps every multiply-add a rounded multiply then a rounded add, as the reference's kernels
require; -mavx2 lets gcc vectorise the independent-lane loops without changing their order (no -ffast-math), and
-mfma makes the explicit fused multiply-adds of aq_math.h single instructions (with contraction still off).
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCES = ["oracle_kernels.c", "oracle_model.c"]
LIB = os.path.join(HERE, "liboracle.so")


LIB_LIBM = os.path.join(HERE, "liboracle_libm.so")
MATH_DIR = os.path.join(os.path.dirname(HERE), "qwen-3.8-in-rust_amd", "csrc")  # aq_math.h, shared with the device


def build(verbose: bool = False) -> str:
    """liboracle.so (exp / log1p from aq_math.h) and liboracle_libm.so (the platform libm's expf / log1pf)."""
    for out, libm in ((LIB, 0), (LIB_LIBM, 1)):
        cmd = ["gcc", "-O3", "-std=gnu11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
               "-mavx2", "-mfma", "-Wall", "-Wno-unknown-pragmas", f"-DOR_LIBM={libm}", "-I", MATH_DIR, "-o", out + ".tmp"]
        cmd += [os.path.join(HERE, s) for s in SOURCES] + ["-lm"]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        os.replace(out + ".tmp", out)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
