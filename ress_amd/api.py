"""Public entry points (reference src/ress/api.py): one loaded model, four modes.

    mode           budget                    block order
    dense          -- (sparse_ratio 0)       --
    sparse_vggt    uniform across heads      attention probability
    hess           calibrated per head       attention probability
    ress           calibrated per head       residual-drift restore-swap

Every apply_* resets the previous mode (set_static_budget).
"""

from ress_amd.backbones import get_backbone, infer_backbone
from ress_amd.budget import HessBudget, UniformBudget
from ress_amd.projected import bake_and_attach_M
from ress_amd.static import set_static_budget

RESS_CRITERION = "restore_swap_iter{n_iters}_bf16_trackbest"


def load_backbone(name, device="cuda", **kwargs):
    """Load a published backbone (reference api.py:47-57). Needs the HF hub; see backbones."""
    backbone = get_backbone(name)
    model = backbone.load(device=device, **kwargs)
    model._ress_backbone = backbone.name
    return model


def _budgets(model, backbone, lam=None):
    """(uniform, hess) budgets, built once and cached on the model; bakes M on first use
    (reference api.py:60-87)."""
    key = ("_ress_budgets", lam)
    cached = getattr(model, "_ress_budget_cache", None)
    if cached is not None and cached[0] == key:
        return cached[1]
    if not getattr(model, "_ress_M_baked", False):
        bake_and_attach_M(model)
        model._ress_M_baked = True
    uniform = UniformBudget(n_blocks=backbone.n_global_blocks, n_heads=backbone.n_heads)
    tables = getattr(model, "_ress_calibration_tables", None)
    score_pcd, score_cam_pos = tables if tables is not None else backbone.calibration_paths()
    hess = HessBudget(score_cam_pos, score_pcd, lam=backbone.hess_lam if lam is None else lam, qkv_idx=0)
    model._ress_budget_cache = (key, (uniform, hess))
    return uniform, hess


def _resolve(model, backbone):
    return get_backbone(backbone) if backbone is not None else infer_backbone(model)


def apply_dense(model, backbone=None):
    """All candidate blocks kept (sparse_ratio 0), reference api.py:95-100."""
    spec = _resolve(model, backbone)
    uniform, _ = _budgets(model, spec)
    set_static_budget(model, uniform, 0.0, None, beta=1.0)
    return model


def apply_sparse_vggt(model, sparse_ratio, cdf_threshold=None, backbone=None):
    """SparseVGGT: one budget for all heads, blocks by probability (reference api.py:103-114)."""
    spec = _resolve(model, backbone)
    uniform, _ = _budgets(model, spec)
    set_static_budget(model, uniform, sparse_ratio, cdf_threshold, beta=1.0)
    return model


def apply_hess(model, sparse_ratio, cdf_threshold=None, lam=None, backbone=None):
    """HeSS: calibrated per-head budget, blocks by probability (reference api.py:117-127)."""
    spec = _resolve(model, backbone)
    _, hess = _budgets(model, spec, lam=lam)
    set_static_budget(model, hess, sparse_ratio, cdf_threshold, beta=1.0)
    return model


def apply_ress(model, sparse_ratio, n_iters=5, lam=None, backbone=None):
    """ReSS: HeSS budget, blocks by residual-drift restore-swap (reference api.py:130-144)."""
    spec = _resolve(model, backbone)
    _, hess = _budgets(model, spec, lam=lam)
    set_static_budget(model, hess, sparse_ratio, None, beta=1.0,
                      block_criterion=RESS_CRITERION.format(n_iters=n_iters))
    return model
