"""Q/K/V projection, qk-norm and RoPE for a VGGT-family attention module, and the
output projection (reference src/ress/models/qkv.py:25-87, tokens.py:8-52).

Unlike the reference, Q/K/V stay in storage order (B, nh, frames*P, hd): the patch /
special split happens inside the GPU preparation pass (no `.contiguous()` copies), and
the attention kernel writes its output back in storage order.
"""

import torch

from ress_amd import _lib


def grid_shape(x, pos, num_special_tokens=5, num_heads=16, shape=None):
    """(B, N frames, P tokens/frame, H, W, S, hd) of one global-attention input
    (reference qkv.py:44-58: H/W from the +1-shifted positions, or an explicit
    {"N","H","W"} override)."""
    B, NP, dim = x.shape
    S = num_special_tokens
    if shape is not None:
        H, W, N = shape["H"], shape["W"], shape["N"]
    else:
        H = int(pos[0].max(0).values[0])
        W = int(pos[0].max(0).values[1])
        N = NP // (H * W + S)
    P = H * W + S
    if N * P != NP:
        raise AssertionError(f"token split mismatch: N={N} x P={P} (= H*W+S = {H}*{W}+{S}) != {NP} tokens")
    return {"B": B, "N": N, "P": P, "head_dim": dim // num_heads, "num_heads": num_heads, "H": H, "W": W, "S": S}


# The rotation the fused kernel implements: the head dim split in two halves, the first
# rotated by the row position pos[..., 0] and the second by the column pos[..., 1]; in each
# half of width d, element i < d/2 pairs with i + d/2 (rotate-half: x*cos + (-x2, x1)*sin)
# at angle pos * base^(-2i/d), angles in fp32.
ROPE_LAYOUT = "rotate_half_2d"


def declare_rope(rope, base, layout=ROPE_LAYOUT):
    """Declare a backbone's own RoPE module (the `self.rope` the reference forward calls,
    src/ress/models/qkv.py:56-58) to be the rotation the fused q/k-norm + RoPE kernel
    implements, with the given base frequency, so that its attention takes the fused path.
    The declaration is the caller's statement about the module's arithmetic: the fused
    kernel does not run the module. Returns the module."""
    if layout != ROPE_LAYOUT:
        raise ValueError(f"RoPE layout {layout!r} is not implemented by the fused kernel (only {ROPE_LAYOUT!r})")
    base = float(base)
    if not base > 1.0:
        raise ValueError(f"RoPE base must be > 1, got {base}")
    rope.ress_rope = (layout, base)
    return rope


def rope_base(rope):
    """Base frequency of a rotation the fused kernel implements (this package's RoPE2D, or
    a module passed to declare_rope), else None."""
    from ress_amd.aggregator import RoPE2D
    if isinstance(rope, RoPE2D):
        return float(rope.base)
    decl = getattr(rope, "ress_rope", None)
    if isinstance(decl, tuple) and len(decl) == 2 and decl[0] == ROPE_LAYOUT:
        return float(decl[1])
    return None


def _fusable(self, x, hd):
    """True when the module's q/k normalisation and rotary embedding are the ones the
    fused kernel implements: bf16 on the GPU, LayerNorm(64) with affine weights, and a
    RoPE with a known base (rope_base) or no rotation."""
    rope = getattr(self, "rope", None)
    qn, kn = getattr(self, "q_norm", None), getattr(self, "k_norm", None)
    return (x.is_cuda and x.dtype == torch.bfloat16 and hd == 64
            and all(isinstance(n, torch.nn.LayerNorm) and n.normalized_shape == (64,) and n.weight is not None
                    and n.bias is not None and n.weight.dtype == torch.bfloat16 for n in (qn, kn))
            and (rope is None or rope_base(rope) is not None))


def fused_qk_norm_rope(self, qkv_out, pos, nh):
    """q_norm / k_norm and the 2D RoPE of a qkv Linear output (B, T, 3*nh*64) bf16 in one
    kernel (ress_qk_norm_rope) -> q, k, v (B, nh, T, 64) bf16 contiguous."""
    B, T, _ = qkv_out.shape
    dev = qkv_out.device
    src = qkv_out.contiguous()
    q = torch.empty(B, nh, T, 64, dtype=torch.bfloat16, device=dev)
    k, v = torch.empty_like(q), torch.empty_like(q)
    rope = getattr(self, "rope", None)
    p = None if rope is None or pos is None else pos.to(device=dev, dtype=torch.int64).reshape(B, T, 2).contiguous()
    qn, kn = self.q_norm, self.k_norm
    _lib.call("ress_qk_norm_rope", _lib.ptr(src), B, T, nh, _lib.ptr(qn.weight), _lib.ptr(qn.bias),
              _lib.ptr(kn.weight), _lib.ptr(kn.bias), float(qn.eps), _lib.ptr(p),
              rope_base(rope) if rope is not None else 0.0, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v),
              _lib.stream_handle(dev))
    return q, k, v


def compute_qkv(self, x, pos, num_special_tokens=5, num_heads=16, shape=None):
    """(q, k, v, shape): each (B, nh, N*P, hd) in storage order, after q_norm/k_norm and
    RoPE -- reference qkv.py:60-68 without the split. Modules with LayerNorm q/k norms and
    a RoPE the fused kernel implements (rope_base: this package's RoPE2D or a declared one)
    take the fused kernel; others run the torch modules."""
    shp = grid_shape(x, pos, num_special_tokens, num_heads, shape)
    B, NP, _ = x.shape
    nh, hd = shp["num_heads"], shp["head_dim"]
    if _fusable(self, x, hd) and self.q_norm.eps == self.k_norm.eps:
        q, k, v = fused_qk_norm_rope(self, self.qkv(x), pos, nh)
        return q, k, v, shp
    qkv = self.qkv(x).reshape(B, NP, 3, nh, hd).permute(2, 0, 3, 1, 4)
    q, k, v = qkv.unbind(0)
    q, k = self.q_norm(q), self.k_norm(k)
    if getattr(self, "rope", None) is not None:
        q = self.rope(q, pos)
        k = self.rope(k, pos)
    return q, k, v, shp


def get_patch_tokens(x, N, P, S):
    """(..., N*P, C) -> (..., N*(P-S), C) patch tokens, frame-major (reference tokens.py:8-30)."""
    assert x.shape[-2] == N * P
    lead, C = x.shape[:-2], x.shape[-1]
    return x.view(*lead, N, P, C)[..., S:, :].reshape(*lead, N * (P - S), C)


def get_special_tokens(x, N, P, S):
    """(..., N*P, C) -> (..., N*S, C) special tokens or None (reference tokens.py:33-52)."""
    assert x.shape[-2] == N * P
    if S == 0:
        return None
    lead, C = x.shape[:-2], x.shape[-1]
    return x.view(*lead, N, P, C)[..., :S, :].reshape(*lead, N * S, C)


def combine_special_and_patch(x_special, x_patch, shape):
    """Inverse split (reference qkv.py:71-81): (B,nh,N*S,hd) + (B,nh,N*(P-S),hd) ->
    (B,nh,N*P,hd)."""
    B, N, P, hd, nh, S = (shape[k] for k in ("B", "N", "P", "head_dim", "num_heads", "S"))
    xp = x_patch.reshape(B, nh, N, P - S, hd)
    x = xp if x_special is None else torch.cat([x_special.reshape(B, nh, N, S, hd), xp], dim=-2)
    return x.reshape(B, nh, N * P, hd)


def project_out(self, x, B, N, P, nh, hd):
    """W_O projection (reference qkv.py:84-87)."""
    x = x.transpose(1, 2).reshape(B, N * P, nh * hd)
    x = self.proj(x)
    return self.proj_drop(x)
