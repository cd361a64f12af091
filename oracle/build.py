"""Build the CPU oracle (test infrastructure only) into oracle/_build/libjit_oracle.so.

The reference's implementation of this path is Python + MLX Metal kernels (no C or C++ sources to
compile), so there is no oracle/_ref build: the oracle is the C restatement in jit_oracle.c.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "libjit_oracle.so")


def build(verbose: bool = False) -> str:
    """Compile jit_oracle.c with gcc (OpenMP, no FP contraction) and return the library path."""
    os.makedirs(OUT_DIR, exist_ok=True)
    src = os.path.join(HERE, "jit_oracle.c")
    tmp = LIB + ".tmp"
    cmd = [
        "gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
        "-fno-fast-math", "-Wall", "-o", tmp, src, "-lm",
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
