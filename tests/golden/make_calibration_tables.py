"""Writes the package's calibration tables, ress_amd/calibration/fisher_scores_<backbone>_<pcd|cam_pos>.pt,
from the six tables the reference ships (src/ress/calibration/*.pt).

Each source file is read with torch.load(weights_only=True) -- a plain float32 tensor of
shape (3, n_global_blocks, n_heads), nothing executed from the file -- checked, and saved
again with torch.save as a plain tensor. These are data: HessBudget reads slice [0]
(W_Q) of each (src/ress/budget/hess.py:66-90). Run in the build container, where the
reference is mounted:

    python tests/golden/make_calibration_tables.py [/root/reference]
"""

import os
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
OUT = os.path.join(ROOT, "ress_amd", "calibration")
SHAPES = {"vggt": (3, 24, 16), "pi3": (3, 18, 16), "da3": (3, 14, 24)}


def main(ref_root="/root/reference"):
    src_dir = os.path.join(ref_root, "src", "ress", "calibration")
    os.makedirs(OUT, exist_ok=True)
    for name, shape in SHAPES.items():
        for kind in ("pcd", "cam_pos"):
            fname = f"fisher_scores_{name}_{kind}.pt"
            t = torch.load(os.path.join(src_dir, fname), map_location="cpu", weights_only=True)
            if not (torch.is_tensor(t) and tuple(t.shape) == shape and t.dtype == torch.float32):
                raise ValueError(f"{fname}: expected a float32 tensor of shape {shape}")
            if not bool(torch.isfinite(t).all()) or bool((t <= 0).any()):
                raise ValueError(f"{fname}: expected finite positive scores")
            torch.save(t.clone().contiguous(), os.path.join(OUT, fname))
            print(f"{fname}: {tuple(t.shape)} min {t.min().item():.3e} max {t.max().item():.3e}")


if __name__ == "__main__":
    main(*sys.argv[1:])
