"""Switching a mode on: install a budget callback on every global block and reset every
per-call knob (reference src/ress/runtime/static.py)."""

from ress_amd.wiring import global_blocks


def set_static_budget(model, budget, sparse_ratio=None, cdf_threshold=None, beta=1.0,
                      block_criterion="probability", pooled_fallback=False, protect_own_frame=False):
    """`budget` has `.num_to_select(layer_idx, attn_pooled, sparse_ratio, cdf_threshold,
    beta)`; a budget with `needs_v_bar` true is wired through `perhead_budget_fn(attn_pooled,
    v_bar)` instead (reference static.py:20-77). Every knob a previous mode may have set is
    cleared first, so modes never leak into each other."""
    needs_v_bar = getattr(budget, "needs_v_bar", False)
    for i, block in enumerate(global_blocks(model)):
        attn = block.attn
        attn.dense = False
        attn.num_to_select = None
        attn.retain_output_grad = False
        attn.block_criterion = block_criterion
        attn.pooled_fallback = pooled_fallback
        attn.protect_own_frame = protect_own_frame
        attn.joint_select_fn = None
        attn.perhead_budget_fn = None
        attn.budget_fn = None
        if needs_v_bar:
            def _perhead(attn_pooled, v_bar, _layer=i):
                return budget.num_to_select(_layer, attn_pooled, sparse_ratio, cdf_threshold, beta, v_bar=v_bar)

            attn.perhead_budget_fn = _perhead
        else:
            def _budget(attn_pooled, _layer=i):
                return budget.num_to_select(_layer, attn_pooled, sparse_ratio, cdf_threshold, beta)

            attn.budget_fn = _budget
