"""Build recipe for the CPU oracle (test infrastructure only).

Compiles oracle/lia_oracle.c into oracle/liblia_oracle.so with gcc.  Floating-point
contraction is disabled so that every multiply and add rounds exactly where the
reference's Rust source rounds (Rust never contracts a*b+c into an FMA).
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "lia_oracle.c")
OUT = os.path.join(HERE, "liblia_oracle.so")


# The CPU baseline is built on the machine that times it (-march=native must target that
# host's cores): same source and FP semantics, optimised at -O3.
BASELINE_FLAGS = ["-O3", "-march=native", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
                  "-fno-fast-math", "-std=c11", "-Wall", "-Wno-unused-function"]


def build_baseline(out: str, verbose: bool = False) -> str:
    """Compile the oracle at -O3 -march=native into `out` (the bench's CPU baseline)."""
    cmd = ["gcc", *BASELINE_FLAGS, SRC, "-o", out, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return out


def build(verbose: bool = False) -> str:
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
           "-fno-fast-math", "-std=c11", "-Wall", "-Wno-unused-function",
           SRC, "-o", OUT, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return OUT


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
