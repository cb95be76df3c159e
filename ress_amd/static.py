"""Switching a mode on (reference src/ress/runtime/static.py:20-77): every global block's
attention module gets a budget callback and a fresh set of per-call knobs, so a previous
mode can never leak into the next forward."""

from ress_amd.wiring import global_blocks

# knob -> value every mode starts from (set_static_budget then sets its own)
_RESET = (
    ("dense", False),
    ("num_to_select", None),
    ("retain_output_grad", False),
    ("joint_select_fn", None),
    ("perhead_budget_fn", None),
    ("budget_fn", None),
)


def _budget_callback(budget, layer, sparse_ratio, cdf_threshold, beta, with_v_bar):
    if with_v_bar:
        def perhead(attn_pooled, v_bar):
            return budget.num_to_select(layer, attn_pooled, sparse_ratio, cdf_threshold, beta, v_bar=v_bar)
        return "perhead_budget_fn", perhead

    def per_layer(attn_pooled):
        return budget.num_to_select(layer, attn_pooled, sparse_ratio, cdf_threshold, beta)
    return "budget_fn", per_layer


def set_static_budget(model, budget, sparse_ratio=None, cdf_threshold=None, beta=1.0,
                      block_criterion="probability", pooled_fallback=False, protect_own_frame=False,
                      attention_sink=0):
    """`budget` has `.num_to_select(layer_idx, attn_pooled, sparse_ratio, cdf_threshold,
    beta)`; one whose `needs_v_bar` is true is installed as `perhead_budget_fn(attn_pooled,
    v_bar)` instead of `budget_fn(attn_pooled)` (reference static.py:38,68-77).
    attention_sink (not a reference argument; 0 keeps the reference's behaviour): leading
    tokens whose key blocks every row keeps (see sparse_global_attention)."""
    with_v_bar = bool(getattr(budget, "needs_v_bar", False))
    for layer, block in enumerate(global_blocks(model)):
        attn = block.attn
        for knob, value in _RESET:
            setattr(attn, knob, value)
        attn.block_criterion = block_criterion
        attn.pooled_fallback = pooled_fallback
        attn.protect_own_frame = protect_own_frame
        attn.attention_sink = attention_sink
        name, fn = _budget_callback(budget, layer, sparse_ratio, cdf_threshold, beta, with_v_bar)
        setattr(attn, name, fn)
