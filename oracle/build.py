"""Build the C restatement (``delta_ref.c``) into ``oracle/libdelta_oracle.so``.

Test infrastructure: the library is the CPU baseline ``bench.py`` times and
a second checker for ``tests/``; it is never linked into the product.
The reference (teddytennant/prometheus) is Python/JAX for this path, so
there is no reference C/C++ source to compile into ``oracle/_ref``.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "delta_ref.c")
LIB = os.path.join(HERE, "libdelta_oracle.so")


def build(verbose: bool = False) -> str:
    cmd = ["gcc", "-O3", "-march=native", "-fopenmp", "-shared", "-fPIC", "-std=c11",
           SRC, "-o", LIB + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
