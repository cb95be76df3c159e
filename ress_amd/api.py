"""Public entry points: one loaded model, four modes (reference src/ress/api.py:95-144).

    apply_dense(model)                         every candidate block kept (sparse_ratio 0)
    apply_sparse_vggt(model, sr, cdf)          one budget for all heads, blocks by probability
    apply_hess(model, sr, cdf, lam)            calibrated per-head budget, blocks by probability
    apply_ress(model, sr, n_iters, lam)        calibrated per-head budget, blocks by residual drift

Each call switches the mode in place (set_static_budget resets every per-call knob) and
returns the model. What a mode needs from the model is built lazily and kept on it in one
`_ModelState`: the per-head metrics M_h (baked from W_O once) and the budget objects, one
HeSS budget per lambda asked for.
"""

from dataclasses import dataclass, field

from ress_amd.backbones import get_backbone, infer_backbone
from ress_amd.budget import HessBudget, UniformBudget
from ress_amd.projected import bake_and_attach_M
from ress_amd.static import set_static_budget

# The published ReSS recipe as a criterion name (reference api.py:44): n_iters rounds,
# bf16 k-wide tensors, best state kept across rounds.
RESS_CRITERION = "restore_swap_iter{n_iters}_bf16_trackbest"

_STATE_ATTR = "_ress_state"


@dataclass
class _ModelState:
    backbone: str
    metrics_baked: bool = False
    uniform: UniformBudget = None
    hess: dict = field(default_factory=dict)  # lambda -> HessBudget


def load_backbone(name, device="cuda", **kwargs):
    """A published backbone with the block-sparse forward wired in (reference api.py:47-57).
    The checkpoints come from the Hugging Face hub, which this build cannot reach; the
    loaders in ress_amd.backbones raise a clear error instead of downloading."""
    spec = get_backbone(name)
    model = spec.load(device=device, **kwargs)
    model._ress_backbone = spec.name
    return model


def _state(model, spec):
    st = getattr(model, _STATE_ATTR, None)
    if st is None or st.backbone != spec.name:
        st = _ModelState(backbone=spec.name)
        setattr(model, _STATE_ATTR, st)
    if not st.metrics_baked:  # M_h depends on the weights only: once per model
        bake_and_attach_M(model)
        st.metrics_baked = True
    return st


def _uniform_budget(model, spec):
    st = _state(model, spec)
    if st.uniform is None:
        st.uniform = UniformBudget(n_blocks=spec.n_global_blocks, n_heads=spec.n_heads)
    return st.uniform


def _hess_budget(model, spec, lam):
    """The HeSS budget at mixing weight `lam` (the backbone's tuned value when None). The
    tables are the model's `_ress_calibration_tables` = (point cloud, camera) when set, else
    the backbone's shipped files; HessBudget takes them as (camera, point cloud)."""
    st = _state(model, spec)
    lam = spec.hess_lam if lam is None else lam
    bud = st.hess.get(lam)
    if bud is None:
        tables = getattr(model, "_ress_calibration_tables", None)
        pcd, cam = tables if tables is not None else spec.calibration_paths()
        bud = HessBudget(cam, pcd, lam=lam, qkv_idx=0)
        st.hess[lam] = bud
    return bud


def _backbone_of(model, backbone):
    return infer_backbone(model) if backbone is None else get_backbone(backbone)


def apply_dense(model, backbone=None):
    """No block dropped: the uniform budget at sparse_ratio 0 (reference api.py:95-100)."""
    spec = _backbone_of(model, backbone)
    set_static_budget(model, _uniform_budget(model, spec), 0.0, None, beta=1.0)
    return model


def apply_sparse_vggt(model, sparse_ratio, cdf_threshold=None, backbone=None):
    """SparseVGGT: one budget for every head (sparse_ratio and, if given, the CDF cut; the
    larger count wins), blocks ranked by pooled probability (reference api.py:103-114)."""
    spec = _backbone_of(model, backbone)
    set_static_budget(model, _uniform_budget(model, spec), sparse_ratio, cdf_threshold, beta=1.0)
    return model


def apply_hess(model, sparse_ratio, cdf_threshold=None, lam=None, backbone=None):
    """HeSS: the baseline budget reallocated across heads by the calibrated importance table,
    blocks ranked by probability (reference api.py:117-127)."""
    spec = _backbone_of(model, backbone)
    set_static_budget(model, _hess_budget(model, spec, lam), sparse_ratio, cdf_threshold, beta=1.0)
    return model


def apply_ress(model, sparse_ratio, n_iters=5, lam=None, backbone=None):
    """ReSS: the HeSS budget, blocks chosen by residual-drift restore-swap over n_iters rounds;
    no CDF cut (reference api.py:130-144)."""
    spec = _backbone_of(model, backbone)
    set_static_budget(model, _hess_budget(model, spec, lam), sparse_ratio, None, beta=1.0,
                      block_criterion=RESS_CRITERION.format(n_iters=n_iters))
    return model
