"""Builds libress_hip.so (every kernel under csrc/) for gfx950 with hipcc.

    python -m ress_amd.build            # or ress_amd.build.build_library()

Objects go to ress_amd/_build/, the library to ress_amd/libress_hip.so (in-tree, so it
travels with the source tree to the GPU host). bench.py's measured-peak kernels
(csrc_bench/peak.hip) build into ress_amd/libress_peak.so. Always recompiles.
"""

import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
# bench support (measured MFMA peak), a library of its own: libress_peak.so
BENCH_SRC = os.path.join(HERE, "csrc_bench", "peak.hip")
PEAK_LIB = os.path.join(HERE, "libress_peak.so")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libress_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # No contraction of a*b+c unless written as fmaf(): the block-map numerics are
    # defined operation by operation.
    "-ffp-contract=off",
    # Packed-fp32 VALU forms stay off.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# Per-file additions. attn.hip: its scores are finite (or -inf for masked keys), never
# NaN, so NaN semantics are dropped there and the row max over MFMA results compiles to
# v_max3_f32 without a NaN-quieting self-max per operand.
FILE_FLAGS = {"attn.hip": ["-fno-honor-nans"]}


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build_library(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    cmd = [HIPCC, *FLAGS, "-shared", "-o", PEAK_LIB + ".tmp", BENCH_SRC]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {BENCH_SRC}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(PEAK_LIB + ".tmp", PEAK_LIB)
    if verbose:
        print(f"built {PEAK_LIB}")
    return LIB


if __name__ == "__main__":
    build_library(verbose=True)
    sys.exit(0)
