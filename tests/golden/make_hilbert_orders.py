"""Writes tests/golden/hilbert_orders.json: the generalized Hilbert curve of the reference
(src/ress/models/hilbert.py: gilbert2d and make_hilbert_gather_idx, the forward and the
inverse gather tables) on the 37x37 VGGT patch grid and two odd rectangles (13x11, 23x7),
as vectors only.

Run in a container that holds the reference checkout (its module is loaded by file path;
it needs only math, functools, torch and einops):

    python tests/golden/make_hilbert_orders.py /root/reference

The fixture is data (grid sizes, cell lists, gather tables); nothing of the reference's
source is kept. tests/test_oracle.py checks ress_amd.synth against it."""

import importlib.util
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
GRIDS = [(37, 37), (13, 11), (23, 7)]


def main(ref_root):
    path = os.path.join(ref_root, "src", "ress", "models", "hilbert.py")
    spec = importlib.util.spec_from_file_location("_ref_hilbert", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    out = []
    for w, h in GRIDS:
        out.append({
            "width": w,
            "height": h,
            "cells": [list(map(int, p)) for p in mod.gilbert2d(w, h)],
            "gather": [int(i) for i in mod.make_hilbert_gather_idx(w, h)],
            "gather_inverse": [int(i) for i in mod.make_hilbert_gather_idx(w, h, inverse=True)],
        })
    dst = os.path.join(HERE, "hilbert_orders.json")
    with open(dst, "w") as f:
        json.dump({"source": "src/ress/models/hilbert.py (gilbert2d, make_hilbert_gather_idx)", "grids": out}, f)
    print(f"wrote {dst}: {[(g['width'], g['height']) for g in out]}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
