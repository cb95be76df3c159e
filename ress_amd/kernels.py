"""Thin tensor-level wrappers over the libress_hip C ABI, plus the layer geometry.

Every function here takes device tensors, allocates its outputs with torch (the
caching allocator, so steady-state calls do not reach hipMalloc) and enqueues the
kernels on torch's current stream. Nothing here synchronises with the host.
"""

import math
from dataclasses import dataclass

import torch

from ress_amd import _lib

KS_Q = 128  # query block (reference src/ress/models/attention.py:37)
KS_K = 64   # key block (attention.py:38-39)
HEAD_DIM = 64


def _cdiv(a, b):
    return -(-a // b)


@dataclass(frozen=True)
class LayerGrid:
    """Block geometry of one global-attention layer (reference attention.py:446-491).

    Storage order per (batch, head): `frames` frames of `P` tokens, the first `S` of
    each special. Kernel key order is cat(patch, special); query blocks are the patch
    blocks followed by the special blocks (dense rows)."""

    B: int
    H: int
    frames: int
    P: int
    S: int
    sink_protect: bool = True
    # pool the map over every key (kernel order cat(patch, special)) instead of the patch
    # keys alone: the reference's RESS_SINK_MASS (attention.py:78, 451-452), default off
    sink_mass: bool = False

    @property
    def BH(self):
        return self.B * self.H

    @property
    def T_p(self):
        return self.frames * (self.P - self.S)

    @property
    def T_s(self):
        return self.frames * self.S

    @property
    def Tk(self):
        return self.frames * self.P

    @property
    def q_blk_p(self):
        return _cdiv(self.T_p, KS_Q)

    @property
    def q_blk_s(self):
        return _cdiv(self.T_s, KS_Q)

    @property
    def q_blk_total(self):
        return self.q_blk_p + self.q_blk_s

    @property
    def kb_p(self):
        """Width of the pooled map: the patch key blocks (ceil), or with sink_mass every key
        block of the kernel grid."""
        return self.kb_tot if self.sink_mass else _cdiv(self.T_p, KS_K)

    @property
    def kb_tot(self):
        """Kernel key-block grid over cat(patch, special)."""
        return _cdiv(self.Tk, KS_K)

    @property
    def n_cand(self):
        """Droppable candidate blocks: only blocks holding patch keys exclusively
        when special tokens exist (attention.py:453-456)."""
        if self.S > 0 and self.sink_protect:
            return self.T_p // KS_K
        return _cdiv(self.T_p, KS_K)

    @property
    def sink_blocks(self):
        return self.kb_tot - self.n_cand


QK_MODES = ("f16", "i8x2", "i8")


@dataclass
class Blocks:
    """Output of the preparation pass (see ress_prep_qkv). `mode` names the QK^T
    operands the attention kernel will use:
      "f16"   16-bit operands: the bf16 queries (converted to fp16 per row by the kernel),
              k_pack (fp16 K blocks) and k_scale = each key block's largest key norm
              (with |q'| the row's logit bound, which picks the kernel's softmax path); no codes are written
      "i8x2"  two-term INT8 codes (q_i8 + q_lo, k_i8 + k_lo) with per-block scales
      "i8"    the reference's single-term per-block INT8 codes (q_i8, k_i8)"""

    grid: LayerGrid
    mode: str
    q: torch.Tensor  # the bf16 queries (storage order), read directly in "f16" mode
    q_i8: torch.Tensor
    q_lo: torch.Tensor
    q_scale: torch.Tensor
    pooled_q: torch.Tensor
    k_i8: torch.Tensor
    k_lo: torch.Tensor
    k_scale: torch.Tensor
    pooled_k: torch.Tensor
    pooled_v: torch.Tensor
    v_pack: torch.Tensor
    k_pack: torch.Tensor
    ksum: torch.Tensor
    km: torch.Tensor
    patch_order: torch.Tensor = None  # device int32 (P-S,) or None: the frame's patch order


def patch_order_table(order, grid, device):
    """Validate a per-frame patch order (a permutation of the P-S patch positions: block
    position j holds the frame's patch token order[j], the gather of the reference's
    hilbert_permute, src/ress/models/hilbert.py:128-162) on the host and return it as the
    device int32 table the kernels read, or None for storage order."""
    if order is None:
        return None
    o = torch.as_tensor(order).detach().to("cpu", torch.int64).reshape(-1)
    hw = grid.P - grid.S
    if o.numel() != hw or not torch.equal(torch.sort(o).values, torch.arange(hw)):
        raise ValueError(f"patch_order must be a permutation of the {hw} patch positions of a frame")
    return o.to(device=device, dtype=torch.int32)


def _check_qkv(t, name, grid):
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a device tensor (the block-sparse path runs only on the GPU)")
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {t.dtype}")
    if t.dim() != 4 or t.shape[0] != grid.B or t.shape[1] != grid.H or t.shape[2] != grid.Tk or t.shape[3] != HEAD_DIM:
        raise ValueError(f"{name} must be (B,H,frames*P,64) = ({grid.B},{grid.H},{grid.Tk},64), got {tuple(t.shape)}")
    if t.stride(3) != 1:
        raise ValueError(f"{name} must have a unit-stride head dim")


def prepare_blocks(q, k, v, grid, mode="f16", split=None, patch_order=None):
    """Pool and pack one layer's Q/K/V (bf16, storage order) for the attention mode
    `mode` (see Blocks). `split` is the older spelling: True = "i8x2", False = "i8".
    patch_order: None, or a per-frame permutation of the patch positions (a device int32
    table from patch_order_table, or anything it accepts): blocks are formed in that order
    with the tokens read in place, and sparse_attention writes each row back to its
    tokens' storage positions."""
    if split is not None:
        mode = "i8x2" if split else "i8"
    if mode not in QK_MODES:
        raise ValueError(f"mode must be one of {QK_MODES}, got {mode!r}")
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _check_qkv(t, n, grid)
    dev = q.device
    if patch_order is not None and not (torch.is_tensor(patch_order) and patch_order.is_cuda
                                        and patch_order.dtype == torch.int32):
        patch_order = patch_order_table(patch_order, grid, dev)
    BH = grid.BH
    quant = mode != "f16"
    e = lambda *s, dt=torch.float32: torch.empty(*s, dtype=dt, device=dev)  # noqa: E731
    b = Blocks(
        grid=grid,
        mode=mode,
        q=q,
        q_i8=e(BH, grid.q_blk_total, KS_Q, HEAD_DIM, dt=torch.int8) if quant else None,
        q_lo=e(BH, grid.q_blk_total, KS_Q, HEAD_DIM, dt=torch.int8) if mode == "i8x2" else None,
        q_scale=e(BH, grid.q_blk_total) if quant else None,
        pooled_q=e(BH, grid.q_blk_p, HEAD_DIM),
        k_i8=e(BH, grid.kb_tot, KS_K, HEAD_DIM, dt=torch.int8) if quant else None,
        k_lo=e(BH, grid.kb_tot, KS_K, HEAD_DIM, dt=torch.int8) if mode == "i8x2" else None,
        k_scale=e(BH, grid.kb_tot),
        pooled_k=e(BH, grid.kb_p, HEAD_DIM),
        pooled_v=e(BH, grid.kb_p, HEAD_DIM),
        v_pack=e(BH, grid.kb_tot, 4096, dt=torch.bfloat16),
        k_pack=None if quant else e(BH, grid.kb_tot, KS_K, HEAD_DIM, dt=torch.float16),
        ksum=e(BH, grid.kb_tot, HEAD_DIM) if quant else None,
        km=e(BH, HEAD_DIM) if quant else None,
        patch_order=patch_order,
    )
    P = _lib.ptr
    _lib.call(
        "ress_prep_qkv", P(q), P(k), P(v), grid.B, grid.H, grid.frames, grid.P, grid.S, P(patch_order),
        *q.stride()[:3], *k.stride()[:3], *v.stride()[:3],
        P(b.q_i8), P(b.q_lo), P(b.q_scale), P(b.pooled_q), P(b.k_i8), P(b.k_lo), P(b.k_scale), P(b.pooled_k),
        P(b.pooled_v), P(b.v_pack), P(b.k_pack), P(b.ksum), P(b.km), 1 if grid.sink_mass else 0,
        _lib.stream_handle(dev))
    return b


def pooled_scores(blocks):
    """(attn_full, attn_cond): the pooled softmax over the kb_p key blocks of the map and its
    renormalisation over the n_cand candidates, both (B,H,q_blk_p,*) fp32."""
    g = blocks.grid
    dev = blocks.pooled_q.device
    full = torch.empty(g.B, g.H, g.q_blk_p, g.kb_p, dtype=torch.float32, device=dev)
    cond = torch.empty(g.B, g.H, g.q_blk_p, g.n_cand, dtype=torch.float32, device=dev)
    _lib.call("ress_pooled_scores", _lib.ptr(blocks.pooled_q), _lib.ptr(blocks.pooled_k), g.BH, g.q_blk_p, g.kb_p,
              g.n_cand, 1.0 / math.sqrt(HEAD_DIM), _lib.ptr(full), _lib.ptr(cond), _lib.stream_handle(dev))
    return full, cond


def topk_from_ratio(k_blk, sparse_ratio):
    """int(k_blk * (1 - sparse_ratio)) in Python double arithmetic (attention.py:287)."""
    return int(k_blk * (1 - sparse_ratio))


def baseline_budget(attn_pooled, sparse_ratio=None, cdf_threshold=None):
    """compute_baseline_num_to_select (attention.py:268-293) on the GPU. Returns int32
    counts shaped attn_pooled.shape[:-1]."""
    if sparse_ratio is None and cdf_threshold is None:
        raise AssertionError("at least one of sparse_ratio/cdf_threshold required")
    if not attn_pooled.is_cuda or attn_pooled.dtype != torch.float32:
        raise RuntimeError("baseline_budget takes an fp32 device tensor")
    ap = attn_pooled.contiguous()
    k_blk = ap.shape[-1]
    rows = ap.numel() // k_blk if k_blk else 0
    out = torch.empty(ap.shape[:-1], dtype=torch.int32, device=ap.device)
    topk = topk_from_ratio(k_blk, sparse_ratio) if sparse_ratio is not None else -1
    cdf = float(cdf_threshold) if cdf_threshold is not None else -1.0
    _lib.call("ress_baseline_budget", _lib.ptr(ap), rows, k_blk, cdf, topk, _lib.ptr(out),
              _lib.stream_handle(ap.device))
    return out


def head_budget(baseline, scores_norm, beta, max_val, max_iters=1000, min_select=0, iters_out=None):
    """adjust_attention_selection (src/ress/budget/_proportional.py:49-115) on the GPU.
    baseline (B,H,q_blk) int32; scores_norm (H,) fp32 device tensor or None."""
    if baseline.dtype != torch.int32:
        baseline = baseline.to(torch.int32)
    baseline = baseline.contiguous()
    B, H, q_blk = baseline.shape
    out = torch.empty_like(baseline)
    _lib.call("ress_head_budget", _lib.ptr(baseline), B, H, q_blk, _lib.ptr(scores_norm), float(beta), int(max_val),
              int(max_iters), int(min_select), _lib.ptr(out), _lib.ptr(iters_out), _lib.stream_handle(baseline.device))
    return out


def select_blocks(rank_key, counts, grid, min_select, sink_lead=0, want_map=True):
    """Top-n selection + sinks + LUT. rank_key (B,H,q_blk_p,n_cand) fp32, counts
    (B,H,q_blk_p) int. Returns (final_map uint8 (B,H,q_blk_p,kb_tot) or None, lut, nvalid)."""
    dev = rank_key.device
    rk = rank_key.contiguous()
    if rk.dtype != torch.float32:
        rk = rk.float()
    cn = counts.to(torch.int32).contiguous()
    fmap = (torch.empty(grid.B, grid.H, grid.q_blk_p, grid.kb_tot, dtype=torch.uint8, device=dev)
            if want_map else None)
    lut = torch.empty(grid.BH, grid.q_blk_total, grid.kb_tot, dtype=torch.int32, device=dev)
    nvalid = torch.empty(grid.BH, grid.q_blk_total, dtype=torch.int32, device=dev)
    _lib.call("ress_select_blocks", _lib.ptr(rk), _lib.ptr(cn), grid.BH, grid.q_blk_p, grid.q_blk_total, grid.n_cand,
              grid.kb_tot, int(sink_lead), int(min_select), _lib.ptr(fmap), _lib.ptr(lut), _lib.ptr(nvalid),
              _lib.stream_handle(dev))
    return fmap, lut, nvalid


def lut_from_map(final_map, grid):
    """LUT of an externally built final_map (B,H,q_blk_p,kb_tot) bool, plus the dense
    special rows (block_map_lut_triton, attention.py:224)."""
    dev = final_map.device
    m = final_map.to(torch.uint8).contiguous()
    lut = torch.empty(grid.BH, grid.q_blk_total, grid.kb_tot, dtype=torch.int32, device=dev)
    nvalid = torch.empty(grid.BH, grid.q_blk_total, dtype=torch.int32, device=dev)
    # dense rows first via an empty selection, then the map rows
    _lib.call("ress_select_blocks", None, None, grid.BH, 0, grid.q_blk_total, grid.n_cand, grid.kb_tot, 0, 0, None,
              _lib.ptr(lut), _lib.ptr(nvalid), _lib.stream_handle(dev))
    if grid.q_blk_p:
        lut_p = torch.empty(grid.BH, grid.q_blk_p, grid.kb_tot, dtype=torch.int32, device=dev)
        nv_p = torch.empty(grid.BH, grid.q_blk_p, dtype=torch.int32, device=dev)
        _lib.call("ress_block_map_lut", _lib.ptr(m), grid.BH * grid.q_blk_p, grid.kb_tot, _lib.ptr(lut_p),
                  _lib.ptr(nv_p), _lib.stream_handle(dev))
        lut[:, :grid.q_blk_p] = lut_p
        nvalid[:, :grid.q_blk_p] = nv_p
    return lut, nvalid


def sparse_attention(blocks, lut, nvalid, out=None, out_dtype=torch.float32):
    """Block-sparse attention over the prepared blocks; returns (B,H,frames*P,64) in
    storage order (patch rows sparse, special rows dense). In the "f16" mode the returned
    tensor carries `ress_attn_status`, a device int32 (1,) that the kernel sets to 1 (a key)
    or 2 (a query) or both when an operand element was outside fp16's range (|x| >= 65520):
    read it at the next synchronisation (LayerResult.check does)."""
    g = blocks.grid
    dev = blocks.pooled_q.device
    if out is None:
        out = torch.empty(g.B, g.H, g.Tk, HEAD_DIM, dtype=out_dtype, device=dev)
    code = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[out.dtype]
    sched = torch.empty(_lib.lib().ress_attn_sched_bytes(g.B, g.H, g.Tk), dtype=torch.uint8, device=dev)
    P = _lib.ptr
    sm = 1.0 / math.sqrt(HEAD_DIM)
    if blocks.mode == "f16":
        _lib.call("ress_sparse_attn_fwd_f16", P(blocks.q), *blocks.q.stride()[:3], P(blocks.k_pack), P(blocks.k_scale),
                  P(blocks.v_pack), P(lut), P(nvalid), g.B, g.H, g.frames, g.P, g.S, P(blocks.patch_order), sm,
                  P(out), code, *out.stride()[:3], P(sched), _lib.stream_handle(dev))
        out.ress_attn_status = sched[96:100].view(torch.int32)  # word 24 of the schedule header
    else:
        _lib.call("ress_sparse_attn_fwd", P(blocks.q_i8), P(blocks.q_lo), P(blocks.q_scale), P(blocks.k_i8),
                  P(blocks.k_lo), P(blocks.k_scale), P(blocks.v_pack), 0, P(lut), P(nvalid), g.B, g.H,
                  g.frames, g.P, g.S, P(blocks.patch_order), sm, P(out), code, *out.stride()[:3], P(sched),
                  _lib.stream_handle(dev))
    return out
