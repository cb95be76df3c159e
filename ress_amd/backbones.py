"""The backbones ReSS/HeSS are wired into and the constants each needs
(reference src/ress/backbones.py:23-200).

Loading published checkpoints needs network access to the Hugging Face hub and the
third-party model trees; this package does not fetch them. Build or load a model
yourself, wire its global blocks with `wire_ress_attention`, and tag it with
`model._ress_backbone = "vggt"` (or pass `backbone=` to the apply_* functions).

Calibration tables are read from `RESS_CALIBRATION_DIR` (default: the `calibration/`
directory next to this file) as `fisher_scores_<name>_{pcd,cam_pos}.pt`, or taken from
`model._ress_calibration_tables = (pcd, cam_pos)` when a model carries them.
"""

import os
from dataclasses import dataclass

CALIBRATION_DIR = os.environ.get(
    "RESS_CALIBRATION_DIR", os.path.join(os.path.dirname(os.path.abspath(__file__)), "calibration"))


def _no_download(name, repo):
    def load(device="cuda", **kwargs):
        raise RuntimeError(
            f"loading the published {name} checkpoint ({repo}) needs the Hugging Face hub and the {name} "
            "model tree, which this package does not fetch; construct the model yourself, wire it with "
            "ress_amd.wiring.wire_ress_attention and set model._ress_backbone")
    return load


@dataclass(frozen=True)
class Backbone:
    name: str
    n_global_blocks: int
    n_heads: int
    hess_lam: float
    load: object

    def calibration_paths(self):
        """(pcd, cam_pos) Fisher tables, each (3, n_global_blocks, n_heads)."""
        return (os.path.join(CALIBRATION_DIR, f"fisher_scores_{self.name}_pcd.pt"),
                os.path.join(CALIBRATION_DIR, f"fisher_scores_{self.name}_cam_pos.pt"))


BACKBONES = {
    "vggt": Backbone("vggt", 24, 16, 0.5, _no_download("VGGT", "facebook/VGGT-1B")),
    "pi3": Backbone("pi3", 18, 16, 0.0, _no_download("Pi3", "yyfz233/Pi3")),
    "da3": Backbone("da3", 14, 24, 1.0, _no_download("Depth-Anything-3", "depth-anything/DA3-GIANT-1.1")),
}


def get_backbone(name):
    try:
        return BACKBONES[name]
    except KeyError:
        raise ValueError(f"unknown backbone {name!r} -- known: {', '.join(sorted(BACKBONES))}") from None


def infer_backbone(model):
    name = getattr(model, "_ress_backbone", None)
    if name is None:
        raise ValueError(
            "cannot tell which backbone this model is -- pass backbone=\"vggt\"/\"pi3\"/"
            "\"da3\" explicitly, or tag the model with model._ress_backbone")
    return get_backbone(name)
