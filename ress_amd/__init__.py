"""MI355X-native block-sparse global attention for ReSS / HeSS / SparseVGGT.

    import ress_amd as ress
    ress.apply_hess(model, sparse_ratio=0.7)     # model wired with wire_ress_attention
    out = model(images)

The hot path runs on hand-written HIP kernels for gfx950 (libress_hip.so, built by
`python -m ress_amd.build`); see ress_amd.attention for the per-layer pipeline.
"""

from ress_amd.api import apply_dense, apply_hess, apply_ress, apply_sparse_vggt, load_backbone
from ress_amd.attention import check_layers
from ress_amd.backbones import BACKBONES, get_backbone
from ress_amd.qkv import declare_rope

__all__ = [
    "BACKBONES",
    "apply_dense",
    "apply_hess",
    "apply_ress",
    "apply_sparse_vggt",
    "check_layers",
    "declare_rope",
    "get_backbone",
    "load_backbone",
]
