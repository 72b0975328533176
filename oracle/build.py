"""Build recipe for the CPU oracle (test infrastructure only).

Compiles ``oracle/nsmlp_oracle.c`` into ``oracle/libnsmlp_oracle.so`` with gcc.
The reference repository is pure Python (no C/C++ sources on this path), so
there is no ``oracle/_ref`` build: the oracle is a restatement, pinned by the
checks under ``tests/``.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "nsmlp_oracle.c")
OUT = os.path.join(HERE, "libnsmlp_oracle.so")


def build(verbose: bool = False) -> str:
    cmd = [
        "gcc", "-O2", "-fPIC", "-shared", "-fopenmp", "-std=gnu11",
        "-ffp-contract=off", "-o", OUT + ".tmp", SRC, "-lm",
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(OUT)
