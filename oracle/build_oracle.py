"""Build recipe for the CPU oracle (test infrastructure only): compiles oracle/*.c into oracle/liboracle.so.

-ffp-contract=off keeps every multiply-add a rounded multiply then a rounded add, as the reference's kernels
require; -mavx2 lets gcc vectorise the independent-lane loops without changing their order (no -ffast-math).
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCES = ["oracle_kernels.c", "oracle_model.c"]
LIB = os.path.join(HERE, "liboracle.so")


def build(verbose: bool = False) -> str:
    cmd = ["gcc", "-O3", "-std=gnu11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
           "-mavx2", "-Wall", "-Wno-unknown-pragmas", "-o", LIB + ".tmp"]
    cmd += [os.path.join(HERE, s) for s in SOURCES] + ["-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
