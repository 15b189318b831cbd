"""Builds the C oracle (moe_oracle.c) into oracle/_build/libmoe_oracle.so.

TEST INFRASTRUCTURE ONLY: the checker, never the product path.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "moe_oracle.c")
OUT_DIR = os.path.join(HERE, "_build")
OUT = os.path.join(OUT_DIR, "libmoe_oracle.so")

# -ffp-contract=off: every a*b+c in the restatement rounds twice, exactly as
# written; the only fused operations are the explicit fmaf() calls.
CFLAGS = ["-O2", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
          "-mfma", "-fno-fast-math"]


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    cmd = ["gcc", *CFLAGS, SRC, "-o", OUT, "-lm"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    return OUT


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(OUT)
