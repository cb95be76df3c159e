"""Installing the block-sparse forward on a model's global-attention blocks
(the interface of the reference's src/ress/models/wiring.py:33-109).

`wire_ress_attention(model, blocks)` gives each block's attention module a
`SparseAttentionForward` as its `forward`. The object reads the module's per-call
configuration attributes (set by set_static_budget) at every call, from one table,
`CALL_ATTRIBUTES`, and hands them to `ress_attention_forward`. The block list is recorded
on the model for `global_blocks`.
"""

from ress_amd.attention import ress_attention_forward

# Module attribute read at call time -> its value when the attribute is absent. Each is
# passed to ress_attention_forward under the same name.
CALL_ATTRIBUTES = (
    ("num_to_select", None),
    ("budget_fn", None),
    ("perhead_budget_fn", None),
    ("joint_select_fn", None),
    ("block_criterion", "probability"),
    ("dense", False),
    ("retain_output_grad", False),
    ("pooled_fallback", False),
    ("protect_own_frame", False),
    ("attention_sink", 0),
    ("patch_order", None),
    ("eager_check", False),
    ("sink_mass", False),
    ("sink_protect", True),
)


def global_blocks(model):
    """The blocks whose `.attn` is sparsified, in layer order: the list recorded by
    wire_ress_attention, else VGGT's `model.aggregator.global_blocks`
    (reference wiring.py:33-40)."""
    recorded = getattr(model, "ress_global_blocks", None)
    return recorded if recorded is not None else model.aggregator.global_blocks


def global_attns(model):
    """The attention modules of global_blocks(model) (reference wiring.py:43-46)."""
    return [b.attn for b in global_blocks(model)]


class SparseAttentionForward:
    """Callable installed as `attn.forward`: (x, pos=None, xpos=None, attn_bias=None,
    attn_mask=None) -> (B, N*P, dim). The positional encoding is accepted under VGGT's name
    (`pos`) or Pi3's (`xpos`); a mask or bias cannot be honoured by a forward that builds its
    own block mask, so a non-None one is refused (reference wiring.py:76-81)."""

    def __init__(self, attn, aux_store=None, aux_full=True, num_special_tokens=5):
        self.attn = attn
        self.aux_store = aux_store
        self.aux_full = aux_full
        self.num_special_tokens = num_special_tokens

    def config(self):
        """The call-time configuration read off the module."""
        return {name: getattr(self.attn, name, default) for name, default in CALL_ATTRIBUTES}

    def __call__(self, x, pos=None, xpos=None, attn_bias=None, attn_mask=None):
        if attn_bias is not None or attn_mask is not None:
            raise AssertionError("the block-sparse attention forward builds its own block mask; attn_bias and "
                                 "attn_mask must be None")
        return ress_attention_forward(
            self.attn, x, xpos if pos is None else pos, num_special_tokens=self.num_special_tokens,
            num_heads=self.attn.num_heads, shape=getattr(self.attn, "ress_shape", None), aux_store=self.aux_store,
            aux_full=self.aux_full, **self.config())


def wire_ress_attention(model, blocks, aux_output_store=None, aux_full=True, num_special_tokens=5):
    """Install SparseAttentionForward on every block's attention module and record the block
    list as `model.ress_global_blocks` (reference wiring.py:49-109). aux_output_store: one
    dict per block (or None) that receives the layer's AttentionAux."""
    blocks = list(blocks)
    for i, block in enumerate(blocks):
        store = None if aux_output_store is None else aux_output_store[i]
        block.attn.forward = SparseAttentionForward(block.attn, store, aux_full, num_special_tokens)
    model.ress_global_blocks = blocks
    return blocks
