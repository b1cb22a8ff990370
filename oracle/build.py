"""Build recipe for the C oracle (test infrastructure only).

``python oracle/build.py`` compiles ``oracle/mxfp4_oracle.c`` with gcc into
``oracle/_build/libmxfp4_oracle.so``.  The reference repository is pure
Python/Triton, so there is no reference C source to build into
``oracle/_ref``; this file builds only our own restatement.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "mxfp4_oracle.c")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "libmxfp4_oracle.so")


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    # -ffp-contract=off / no fast-math: the quantizer's float steps must
    # round exactly as written.
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off",
           "-Wall", "-Wextra", SRC, "-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
