"""Builds oracle/liboracle.so from ress_oracle.c with gcc (test infrastructure).

The reference repository has no C/C++/CUDA sources for this path (its native kernels
come from the un-vendored SpargeAttn package), so there is no oracle/_ref build.
"""

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")


def build_oracle():
    src = os.path.join(HERE, "ress_oracle.c")
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O2", "-std=c11", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared", "-o", tmp, src,
           "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build_oracle())
