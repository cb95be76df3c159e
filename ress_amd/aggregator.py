"""A VGGT-1B-style aggregator with random weights, for end-to-end runs of the
block-sparse global attention (64 frames of 518x518, ReSS on every global layer).

Structure of the aggregator the reference wires (VGGT, `model.aggregator.global_blocks`,
reference src/ress/models/wiring.py:33-40; the attention module shape read by
src/ress/models/qkv.py:25-87): a 14x14 patch embedding, one camera and four register
tokens per frame (the first frame's own pair, the others share the second), then
`depth` pairs of ViT blocks: a frame block attends within each frame, a global block
over every token of every frame. Blocks are pre-norm with LayerScale; attention has
qk-norm and a 2D rotary embedding of the patch grid (special tokens at position 0,
patches at their (row, column) + 1). The checkpoints need the network, so the weights
are random; `build_vggt_aggregator` wires the global blocks to the block-sparse forward
and tags the model as the "vggt" backbone for the apply_* functions.
"""

import torch
import torch.nn as nn
import torch.nn.functional as F

from ress_amd.synth import hilbert_permutation
from ress_amd.wiring import wire_ress_attention

_IMAGENET_MEAN = (0.485, 0.456, 0.406)
_IMAGENET_STD = (0.229, 0.224, 0.225)


class RoPE2D(nn.Module):
    """Rotary embedding over (row, column): the first half of the head dim rotates with
    the row position, the second half with the column, each as rotate-half pairs at
    frequencies base^(-2i/d_half)."""

    def __init__(self, base=100.0):
        super().__init__()
        self.base = base

    def _rotate(self, x, p):
        d = x.shape[-1]
        inv = 1.0 / (self.base ** (torch.arange(0, d, 2, device=x.device, dtype=torch.float32) / d))
        ang = p.float()[:, None, :, None] * inv  # (B, 1, T, d/2)
        cos = torch.cat([ang.cos(), ang.cos()], dim=-1)
        sin = torch.cat([ang.sin(), ang.sin()], dim=-1)
        x1, x2 = x[..., : d // 2], x[..., d // 2:]
        rot = torch.cat([-x2, x1], dim=-1)
        return x.float() * cos + rot.float() * sin

    def forward(self, t, pos):
        """t (B, nh, T, hd), pos (B, T, 2) -> t rotated, same dtype."""
        half = t.shape[-1] // 2
        out = torch.cat([self._rotate(t[..., :half], pos[..., 0]), self._rotate(t[..., half:], pos[..., 1])], dim=-1)
        return out.to(t.dtype)


class Attention(nn.Module):
    """qkv Linear, per-head LayerNorm on q and k, 2D RoPE, SDPA, output projection: the
    module layout the block-sparse forward reads (qkv, q_norm, k_norm, rope, proj,
    proj_drop, num_heads). On the GPU in bf16 the norms and the rotation run as one fused
    kernel (ress_qk_norm_rope); `fused = False` keeps the torch modules."""

    def __init__(self, dim, num_heads, rope):
        super().__init__()
        self.num_heads = num_heads
        hd = dim // num_heads
        self.qkv = nn.Linear(dim, 3 * dim, bias=True)
        self.q_norm = nn.LayerNorm(hd)
        self.k_norm = nn.LayerNorm(hd)
        self.rope = rope
        self.proj = nn.Linear(dim, dim, bias=True)
        self.proj_drop = nn.Identity()
        self.fused = True  # q/k norm + RoPE through the fused kernel when on the GPU in bf16

    def forward(self, x, pos=None):
        from ress_amd.qkv import _fusable, fused_qk_norm_rope
        B, T, C = x.shape
        nh = self.num_heads
        if self.fused and _fusable(self, x, C // nh):
            q, k, v = fused_qk_norm_rope(self, self.qkv(x), pos, nh)
        else:
            q, k, v = self.qkv(x).reshape(B, T, 3, nh, C // nh).permute(2, 0, 3, 1, 4).unbind(0)
            q, k = self.q_norm(q), self.k_norm(k)
            if pos is not None:
                q, k = self.rope(q, pos), self.rope(k, pos)
        o = F.scaled_dot_product_attention(q, k, v)
        return self.proj_drop(self.proj(o.transpose(1, 2).reshape(B, T, C)))


class Mlp(nn.Module):
    def __init__(self, dim, hidden):
        super().__init__()
        self.fc1 = nn.Linear(dim, hidden)
        self.act = nn.GELU()
        self.fc2 = nn.Linear(hidden, dim)

    def forward(self, x):
        return self.fc2(self.act(self.fc1(x)))


class LayerScale(nn.Module):
    def __init__(self, dim, init=0.01):
        super().__init__()
        self.gamma = nn.Parameter(torch.full((dim,), init))

    def forward(self, x):
        return x * self.gamma


class Block(nn.Module):
    def __init__(self, dim, num_heads, mlp_ratio, rope):
        super().__init__()
        self.norm1 = nn.LayerNorm(dim)
        self.attn = Attention(dim, num_heads, rope)
        self.ls1 = LayerScale(dim)
        self.norm2 = nn.LayerNorm(dim)
        self.mlp = Mlp(dim, int(dim * mlp_ratio))
        self.ls2 = LayerScale(dim)

    def forward(self, x, pos=None):
        x = x + self.ls1(self.attn(self.norm1(x), pos=pos))
        return x + self.ls2(self.mlp(self.norm2(x)))


class Aggregator(nn.Module):
    """images (B, S, 3, H, W) in [0, 1] -> tokens (B, S*P, dim) after `depth` frame/global
    block pairs, P = (H/14)(W/14) + 5."""

    def __init__(self, depth=24, dim=1024, num_heads=16, mlp_ratio=4.0, patch=14, n_register=4):
        super().__init__()
        self.patch = patch
        self.n_special = 1 + n_register
        self.patch_embed = nn.Conv2d(3, dim, kernel_size=patch, stride=patch)
        self.camera_token = nn.Parameter(torch.randn(1, 2, 1, dim) * 1e-2)
        self.register_token = nn.Parameter(torch.randn(1, 2, n_register, dim) * 1e-2)
        rope = RoPE2D()
        self.frame_blocks = nn.ModuleList(Block(dim, num_heads, mlp_ratio, rope) for _ in range(depth))
        self.global_blocks = nn.ModuleList(Block(dim, num_heads, mlp_ratio, rope) for _ in range(depth))
        self.register_buffer("mean", torch.tensor(_IMAGENET_MEAN).view(1, 1, 3, 1, 1), persistent=False)
        self.register_buffer("std", torch.tensor(_IMAGENET_STD).view(1, 1, 3, 1, 1), persistent=False)
        self._hilbert = {}  # (w, h) -> the patch grid's Hilbert gather table

    def _special(self, B, S):
        def pick(tok):  # frame 0 takes index 0, the other frames index 1
            first = tok[:, :1].expand(B, 1, *tok.shape[2:])
            rest = tok[:, 1:].expand(B, S - 1, *tok.shape[2:])
            return torch.cat([first, rest], dim=1).reshape(B * S, *tok.shape[2:])
        return torch.cat([pick(self.camera_token), pick(self.register_token)], dim=1)

    def _embed_patches(self, x):
        """(N, 3, H, W) -> (N, h*w, dim): the stride-`patch` convolution (kernel = stride, no
        padding) as one GEMM over the flattened patches, in the conv weight's (channel, row,
        column) order. ROCm's convolution picks a direct kernel for this shape that takes
        ~50 ms on 64 frames of 518x518; the GEMM takes well under a millisecond."""
        N, cin, Hi, Wi = x.shape
        p = self.patch
        h, w = Hi // p, Wi // p
        x = x[:, :, :h * p, :w * p].reshape(N, cin, h, p, w, p).permute(0, 2, 4, 1, 3, 5).reshape(N, h * w, cin * p * p)
        weight = self.patch_embed.weight.reshape(self.patch_embed.out_channels, cin * p * p)
        return F.linear(x, weight, self.patch_embed.bias), h, w

    def forward(self, images, use_hilbert=False):
        """use_hilbert: the reference aggregator's flag (src/ress/models/vggt.py:32, 62-64):
        the global layers form their blocks along the per-frame Hilbert curve of the patch
        grid. The tokens stay in raster order: each global attention reads them through the
        curve's gather table (its patch_order) instead of the reference's permuted copy, and
        frame attention, being per-frame dense, is unaffected by the order."""
        B, S, _, Hi, Wi = images.shape
        x = ((images - self.mean) / self.std).to(self.patch_embed.weight.dtype)
        x, h, w = self._embed_patches(x.reshape(B * S, 3, Hi, Wi))  # (B*S, h*w, dim)
        order = None
        if use_hilbert:
            order = self._hilbert.get((w, h))
            if order is None:
                order = self._hilbert[(w, h)] = torch.from_numpy(hilbert_permutation(w, h))
        for gb in self.global_blocks:
            gb.attn.patch_order = order
        x = torch.cat([self._special(B, S).to(x.dtype), x], dim=1)
        P, C = x.shape[1], x.shape[2]
        yy, xx = torch.meshgrid(torch.arange(h, device=x.device), torch.arange(w, device=x.device), indexing="ij")
        grid = torch.stack([yy.flatten(), xx.flatten()], dim=-1) + 1
        pos = torch.cat([torch.zeros(self.n_special, 2, dtype=grid.dtype, device=x.device), grid], dim=0)
        pos_f = pos[None].expand(B * S, P, 2)
        pos_g = pos[None].expand(B, S, P, 2).reshape(B, S * P, 2)
        for fb, gb in zip(self.frame_blocks, self.global_blocks):
            x = fb(x.reshape(B * S, P, C), pos=pos_f)
            x = gb(x.reshape(B, S * P, C), pos=pos_g)
        return x.reshape(B, S * P, C)


class VGGTLike(nn.Module):
    def __init__(self, **kw):
        super().__init__()
        self.aggregator = Aggregator(**kw)

    def forward(self, images, use_hilbert=False):
        return self.aggregator(images, use_hilbert=use_hilbert)


def build_vggt_aggregator(depth=24, dim=1024, num_heads=16, device="cuda", dtype=torch.bfloat16, seed=0,
                          tables=None, wire=True):
    """A random-init VGGT-style model (seeded), its global blocks wired to the block-sparse
    forward and tagged as the "vggt" backbone; `tables` = (pcd, cam_pos) HeSS tables of
    shape (3, depth, num_heads) for apply_hess / apply_ress."""
    torch.manual_seed(seed)
    model = VGGTLike(depth=depth, dim=dim, num_heads=num_heads).to(device=device, dtype=dtype).eval()
    if wire:
        wire_ress_attention(model, model.aggregator.global_blocks)
    model._ress_backbone = "vggt"
    if tables is not None:
        model._ress_calibration_tables = tables
    return model


def synthetic_frames(S, size=518, B=1, seed=0, device="cuda"):
    """(B, S, 3, size, size) pixels: uniform [0,1] noise plus a shared low-frequency
    pattern (a smooth sinusoidal field common to every frame), clamped to [0,1]."""
    g = torch.Generator().manual_seed(seed)
    noise = torch.rand(B, S, 3, size, size, generator=g)
    yy, xx = torch.meshgrid(torch.linspace(0, 1, size), torch.linspace(0, 1, size), indexing="ij")
    phase = torch.rand(3, generator=g) * 6.2832
    pattern = torch.stack([torch.sin(6.2832 * (1.5 * xx + 0.7 * yy) + ph) for ph in phase])  # (3, size, size)
    img = (0.5 * noise + 0.25 * (1 + pattern)[None, None]).clamp(0, 1)
    return img.to(device)
