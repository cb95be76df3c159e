"""Installing the block-sparse forward on a model's global-attention blocks
(reference src/ress/models/wiring.py)."""

from types import MethodType

from ress_amd.attention import ress_attention_forward


def global_blocks(model):
    """The blocks whose `.attn` is sparsified, in layer order: the list recorded by
    wire_ress_attention, else VGGT's `model.aggregator.global_blocks`
    (reference wiring.py:33-40)."""
    blocks = getattr(model, "ress_global_blocks", None)
    if blocks is not None:
        return blocks
    return model.aggregator.global_blocks


def global_attns(model):
    return [block.attn for block in global_blocks(model)]


def wire_ress_attention(model, blocks, aux_output_store=None, aux_full=True, num_special_tokens=5):
    """Replace each block's `attn.forward` with the block-sparse forward and record the
    block list on the model (reference wiring.py:49-109). Per-call configuration is read
    from attributes of each attn module at forward time (set by set_static_budget). The
    positional encoding is accepted as `pos=` (VGGT) or `xpos=` (Pi3); `attn_bias` and
    `attn_mask` must be None."""
    blocks = list(blocks)
    for i, block in enumerate(blocks):
        store_i = aux_output_store[i] if aux_output_store is not None else None

        def _fwd(self, x, pos=None, xpos=None, attn_bias=None, attn_mask=None, _store=store_i, _attn=block.attn):
            assert attn_bias is None and attn_mask is None, (
                "ress_attention_forward builds its own block mask and cannot honor an "
                "externally supplied attn_bias/attn_mask")
            return ress_attention_forward(
                _attn, x, pos if pos is not None else xpos,
                num_to_select=getattr(_attn, "num_to_select", None),
                budget_fn=getattr(_attn, "budget_fn", None),
                perhead_budget_fn=getattr(_attn, "perhead_budget_fn", None),
                joint_select_fn=getattr(_attn, "joint_select_fn", None),
                block_criterion=getattr(_attn, "block_criterion", "probability"),
                num_special_tokens=num_special_tokens,
                num_heads=_attn.num_heads,
                shape=getattr(_attn, "ress_shape", None),
                aux_store=_store,
                aux_full=aux_full,
                dense=getattr(_attn, "dense", False),
                retain_output_grad=getattr(_attn, "retain_output_grad", False),
                pooled_fallback=getattr(_attn, "pooled_fallback", False),
                protect_own_frame=getattr(_attn, "protect_own_frame", False),
            )

        block.attn.forward = MethodType(_fwd, block.attn)
    model.ress_global_blocks = blocks
    return blocks
