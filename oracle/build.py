"""Builds oracle/liboracle.so from vqk_oracle.c (TEST INFRASTRUCTURE ONLY).

gcc, -O2, OpenMP, no floating-point contraction (the oracle's float32 operations must be
exactly the IEEE operations written in the source)."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "vqk_oracle.c")
OUT = os.path.join(HERE, "liboracle.so")


def build(out=OUT):
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
           "-std=gnu11", "-Wall", "-o", out + ".tmp", SRC, "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + r.stderr)
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    print(build())
    sys.exit(0)
