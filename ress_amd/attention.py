"""The block-sparse global-attention forward (reference src/ress/models/attention.py).

`ress_attention_forward` is the drop-in replacement of a global block's attention
forward. Its hot path, `sparse_global_attention`, runs on the GPU kernels only:

    prepare_blocks     pool Q/K/V, packed K/V + key norms (f16 mode) or key mean +
                       per-block INT8 Q/K codes (INT8 modes)                 (prep.hip)
    pooled_scores      pooled softmax attn_full, renormalised attn_cond      (scores.hip)
    budget_fn          per-(head, q-block) counts                            (budget.hip)
    rank key           attn_cond, or ReSS restore-swap / projected / random
    select_blocks      top-n + sinks -> final_map, LUT                       (select.hip)
    sparse_attention   QK^T (bf16 or INT8), online softmax, bf16 PV over the
                       LUT, special rows dense                               (attn.hip)

No step falls back to the CPU or to a dense PyTorch path.
"""

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from ress_amd import _lib, kernels, trace
from ress_amd import criterion as _criterion
from ress_amd.kernels import KS_K, KS_Q, LayerGrid
from ress_amd.qkv import combine_special_and_patch, compute_qkv, get_patch_tokens, get_special_tokens, project_out

KBLK = 64
MIN_NUM_TO_SELECT = 2  # floor on real key blocks per query row (reference attention.py:40-42)

# QK^T operands of the attention kernel. "f16" (fp16 K blocks, queries converted to fp16
# per row) is the fastest and within the tolerance; the INT8 modes reproduce the
# reference's SpargeAttn quantiser ("i8") or refine it with a second code per element
# ("i8x2").
DEFAULT_QK_MODE = "f16"

_RANDOM_SEED = 20260826  # block_criterion="random" (reference attention.py:177-196)
_random_gens = {}


def _random_gen(device):
    gen = _random_gens.get(device)
    if gen is None:
        gen = torch.Generator(device=device).manual_seed(_RANDOM_SEED)
        _random_gens[device] = gen
    return gen


@dataclass
class AttentionAux:
    """Per-layer auxiliary values (reference attention.py:246-265)."""

    attn_pooled: torch.Tensor = None
    v_bar: torch.Tensor = None
    attn_full: torch.Tensor = None
    v_bar_full: torch.Tensor = None
    n_cand: int = None
    q_patch: torch.Tensor = None
    shape: dict = None
    sparsity: float = None
    output: torch.Tensor = None


@dataclass
class LayerResult:
    out: torch.Tensor              # (B, H, frames*P, 64) storage order
    attn_full: torch.Tensor = None
    attn_cond: torch.Tensor = None
    v_bar_full: torch.Tensor = None
    final_map: torch.Tensor = None
    counts: torch.Tensor = None
    lut: torch.Tensor = None
    nvalid: torch.Tensor = None
    blocks: kernels.Blocks = None
    # device-side budget status: the number of HeSS columns that did not converge (0-dim
    # int32), or the per-column iteration counts it is taken from (negative = not converged;
    # counted at the sync, so the layer step launches no reduction for it)
    unconverged: torch.Tensor = None
    budget_iters: torch.Tensor = None
    max_iters: int = None
    # device-side 16-bit operand status (kernels.sparse_attention's ress_attn_status), or None
    attn_status: torch.Tensor = None

    def _raise_unconverged(self, n):
        if n:
            raise RuntimeError(f"adjust_attention_selection did not converge in {self.max_iters} iterations "
                               f"({int(n)} query-block columns)")

    @staticmethod
    def _raise_range(st):
        st = int(st)
        if st:
            what = " and ".join(n for bit, n in ((1, "key"), (2, "query")) if st & bit)
            raise ValueError(f"a {what} element lies outside the fp16 range (|x| >= 65520), which the 16-bit "
                             f"attention mode cannot represent; run the layer with qk_mode='i8x2'")

    def _status_values(self):
        vals = []
        if self.unconverged is not None:
            vals.append(self.unconverged.float().reshape(()))
        if self.budget_iters is not None:
            vals.append((self.budget_iters < 0).sum().float())
        if self.attn_status is not None:
            vals.append(self.attn_status[0].float())
        return vals

    def _raise_status(self, got):
        i = 0
        if self.unconverged is not None:
            self._raise_unconverged(got[i])
            i += 1
        if self.budget_iters is not None:
            self._raise_unconverged(got[i])
            i += 1
        if self.attn_status is not None:
            self._raise_range(got[i])

    def check(self):
        """Raise RuntimeError if the layer's HeSS budget did not converge (reference
        _proportional.py:112-113), or ValueError if the 16-bit attention met an operand
        outside fp16's range. Synchronises with the device once."""
        vals = self._status_values()
        if vals:
            self._raise_status(torch.stack(vals).tolist())

    def sparsity(self):
        """Realized sparsity 1 - mean(final_map), sinks included (reference
        attention.py:242). Synchronises with the device once, and raises there on what
        check() reports."""
        if self.final_map is None:
            self.check()
            return 0.0
        got = torch.stack([1.0 - self.final_map.float().mean()] + self._status_values()).tolist()
        self._raise_status(got[1:])
        return got[0]


def _rank_key(block_criterion, attn_cond, attn_full, v_bar_full, counts, grid, M, hd):
    if block_criterion == "probability":
        return attn_cond
    if block_criterion == "random":
        return torch.rand(attn_cond.shape, device=attn_cond.device, dtype=torch.float32,
                          generator=_random_gen(attn_cond.device))
    from ress_amd import projected as _projected
    if block_criterion == "projected":
        if M is None:
            raise AssertionError("block_criterion='projected' requires bake_and_attach_M(model) first (self.M)")
        return _projected.projected_score(attn_full, v_bar_full, M, n_cand=grid.n_cand)
    if _criterion.is_restore_swap(block_criterion):
        spec = _criterion.parse_restore_swap(block_criterion)
        if spec.use_wo:
            if M is None:
                raise AssertionError(f"block_criterion={block_criterion!r} requires bake_and_attach_M(model) first")
        else:
            M = torch.eye(hd, device=attn_full.device, dtype=torch.float32).expand(grid.H, hd, hd)
        # the keep set as a 1/0 key: top-counts of it is the set the reference's rank_by
        # (where(drop, s, s + max|s| + 1)) yields through build_block_mask
        return _projected.restore_swap_keep(
            attn_full, v_bar_full, M, counts, n_cand=grid.n_cand, n_iters=spec.n_iters, track_best=spec.track_best,
            big_dtype=spec.big_dtype, restore_frac=spec.restore_frac, decay=spec.decay, maximize=spec.maximize,
            invert_cut=spec.invert_cut)
    raise ValueError(block_criterion)


def same_frame_block_mask(q_blk, k_blk, N, H, W, device):
    """(q_blk, k_blk) bool: True where query block q (128 patch tokens) and key block k
    (64 patch tokens) touch a common frame of the frame-major N*(H*W) patch sequence, as
    interval overlap of the frames each block spans (a block can straddle a frame
    boundary) -- reference attention.py:112-144."""
    HW = H * W
    T = N * HW
    q0 = torch.arange(q_blk, device=device) * KS_Q
    q1 = (q0 + KS_Q - 1).clamp(max=T - 1)
    k0 = torch.arange(k_blk, device=device) * KS_K
    k1 = (k0 + KS_K - 1).clamp(max=T - 1)
    qf0, qf1, kf0, kf1 = q0 // HW, q1 // HW, k0 // HW, k1 // HW
    return ~((qf1[:, None] < kf0[None, :]) | (kf1[None, :] < qf0[:, None]))


def protect_own_frame_swap(final_map, attn_pooled, grid):
    """Budget-neutral own-frame protection (reference attention.py:583-618): per (head,
    query-block) row, every own-frame candidate block that is not kept replaces a kept
    block of another frame, one for one -- the lowest-attn_pooled swappable blocks go out,
    the highest-attn_pooled missing ones come in, n_swap = min(#missing, #swappable) of
    each -- so the kept count per row is unchanged. final_map (B,H,q_blk_p,kb_tot) bool or
    uint8, attn_pooled (B,H,q_blk_p,n_cand). Ties of attn_pooled go to the lower block
    index (the reference's CUDA argsort leaves them unspecified). Returns a bool map."""
    n = grid.n_cand
    fm = final_map.bool()
    same = same_frame_block_mask(grid.q_blk_p, n, grid.frames, grid.P - grid.S, 1, fm.device)
    same = same.expand_as(fm[..., :n])
    kept = fm[..., :n]
    missing = same & ~kept
    swappable = kept & ~same
    n_swap = torch.minimum(missing.sum(-1), swappable.sum(-1)).unsqueeze(-1)
    out_pri = attn_pooled.float().masked_fill(~swappable, float("inf"))
    rank_out = torch.argsort(torch.argsort(out_pri, dim=-1, stable=True), dim=-1, stable=True)
    in_pri = attn_pooled.float().masked_fill(~missing, float("-inf"))
    rank_in = torch.argsort(torch.argsort(in_pri, dim=-1, descending=True, stable=True), dim=-1, stable=True)
    new_kept = (kept & ~(rank_out < n_swap)) | (rank_in < n_swap)
    return torch.cat([new_kept, fm[..., n:]], dim=-1)


def sink_lead_blocks(attention_sink, grid):
    """Leading key blocks forced on by an attention sink of `attention_sink` leading
    tokens: ceil(attention_sink / 64) (SpargeAttn get_block_map_meansim_fuse_quant as
    patched, external/patches/spargeattn.patch:61-65), at most the candidate count. On the
    kernel's cat(patch, special) key grid the leading blocks hold the first frame's patch
    keys; its special keys are already in the always-kept trailing blocks."""
    n = int(attention_sink or 0)
    if n < 0:
        raise ValueError(f"attention_sink must be a token count >= 0, got {attention_sink!r}")
    return min(-(-n // KBLK), grid.n_cand)


def sparse_global_attention(q, k, v, grid, *, num_to_select=None, budget_fn=None, perhead_budget_fn=None,
                            joint_select_fn=None, block_criterion="probability", M=None, out=None,
                            out_dtype=torch.float32, keep_intermediates=False, qk_mode=None,
                            protect_own_frame=False, attention_sink=0, patch_order=None):
    """One layer's block-sparse global attention on the GPU.

    q, k, v: bf16 (B, H, frames*P, 64) in storage order (per frame S special then P-S
    patch tokens). Patch queries attend to the selected key blocks plus the trailing
    special blocks; special queries attend densely (reference attention.py:404-412,
    446-491, 510-581, 625). qk_mode: the QK^T operands, "f16" (default), "i8x2" or
    "i8" (see kernels.Blocks); the block map does not depend on it. protect_own_frame:
    the budget-neutral own-frame swap on the selected map (protect_own_frame_swap).
    attention_sink: leading tokens whose key blocks every row keeps on top of its budget
    (sink_lead_blocks; 0 = none, the reference's ReSS default). patch_order: None, or a
    per-frame permutation of the P-S patch positions (kernels.patch_order_table): blocks are
    formed in that order, as if the tokens had gone through the reference's hilbert_permute
    (src/ress/models/hilbert.py:128-162), but read and written in place.
    Returns a LayerResult whose `out` is (B, H, frames*P, 64) in storage order."""
    sink_lead = sink_lead_blocks(attention_sink, grid)
    with trace.stage("ress.prepare_blocks"):
        blocks = kernels.prepare_blocks(q, k, v, grid, mode=qk_mode or DEFAULT_QK_MODE, patch_order=patch_order)
    with trace.stage("ress.pooled_scores"):
        attn_full, attn_cond = kernels.pooled_scores(blocks)
    v_bar_full = blocks.pooled_v.view(grid.B, grid.H, grid.kb_p, 64)
    counts = None
    final_map = None
    budget_iters, max_iters = None, None
    if joint_select_fn is not None:
        with trace.stage("ress.joint_select"):
            final_map = joint_select_fn(attn_cond, v_bar_full[..., :grid.n_cand, :], grid.sink_blocks)
        if sink_lead and not protect_own_frame:
            final_map = final_map.clone()
            final_map[..., :sink_lead] = True
        lut, nvalid = kernels.lut_from_map(final_map, grid)
    else:
        with trace.stage("ress.budget"):
            if perhead_budget_fn is not None:
                counts = perhead_budget_fn(attn_cond, v_bar_full[..., :grid.n_cand, :])
            elif budget_fn is not None:
                counts = budget_fn(attn_cond)
            else:
                counts = num_to_select
        if counts is None:
            raise AssertionError("num_to_select (or budget_fn/perhead_budget_fn) required unless dense=True "
                                 "or joint_select_fn is given")
        budget_iters = getattr(counts, "ress_iters", None)
        max_iters = getattr(counts, "ress_max_iters", None)
        if not torch.is_tensor(counts):
            counts = torch.full((grid.B, grid.H, grid.q_blk_p), int(counts), dtype=torch.int32, device=q.device)
        counts = counts.reshape(grid.B, grid.H, grid.q_blk_p)
        with trace.stage("ress.select"):
            rank = _rank_key(block_criterion, attn_cond, attn_full, v_bar_full,
                             counts.clamp(min=min(MIN_NUM_TO_SELECT, grid.n_cand))
                             if block_criterion != "probability" else counts, grid, M, 64)
            final_map, lut, nvalid = kernels.select_blocks(rank, counts, grid, min(MIN_NUM_TO_SELECT, grid.n_cand),
                                                           sink_lead=0 if protect_own_frame else sink_lead)
    if protect_own_frame and grid.q_blk_p:  # after either selection path, as the reference does
        final_map = protect_own_frame_swap(final_map, attn_full[..., :grid.n_cand], grid)
        if sink_lead:  # forced blocks go on last, so the swap never trades one away
            final_map[..., :sink_lead] = True
        lut, nvalid = kernels.lut_from_map(final_map, grid)
    if M is not None:  # after every step that can move the map, as the reference records it
        from ress_amd import projected as _projected
        _projected.record_layer_drift(M, attn_full, v_bar_full, final_map, grid.n_cand)
    with trace.stage("ress.sparse_attention"):
        o = kernels.sparse_attention(blocks, lut, nvalid, out=out, out_dtype=out_dtype)
    res = LayerResult(out=o, final_map=final_map, budget_iters=budget_iters, max_iters=max_iters,
                      attn_status=getattr(o, "ress_attn_status", None))
    if keep_intermediates:
        res.attn_full, res.attn_cond, res.v_bar_full = attn_full, attn_cond, v_bar_full
        res.counts, res.lut, res.nvalid, res.blocks = counts, lut, nvalid, blocks
    return res


def _dense_storage(q, k, v, shp):
    """Exact SDPA of every query over cat(patch, special) keys (reference attention.py:404-412,
    484-486), written back in storage order."""
    N, P, S = shp["N"], shp["P"], shp["S"]
    kp, ks = get_patch_tokens(k, N, P, S), get_special_tokens(k, N, P, S)
    vp, vs = get_patch_tokens(v, N, P, S), get_special_tokens(v, N, P, S)
    key = kp if ks is None else torch.cat([kp, ks], dim=-2)
    value = vp if vs is None else torch.cat([vp, vs], dim=-2)
    xp = F.scaled_dot_product_attention(get_patch_tokens(q, N, P, S), key, value)
    qs = get_special_tokens(q, N, P, S)
    xs = None if qs is None else F.scaled_dot_product_attention(qs, key, value)
    return combine_special_and_patch(xs, xp, shp)


def ress_attention_forward(self, x, pos, num_to_select=None, budget_fn=None, perhead_budget_fn=None,
                           joint_select_fn=None, block_criterion="probability", pool_mode="avg",
                           num_special_tokens=5, num_heads=16, shape=None, aux_store=None, aux_full=True,
                           dense=False, retain_output_grad=False, pooled_fallback=False, protect_own_frame=False,
                           attention_sink=0, patch_order=None, eager_check=False, sink_mass=False,
                           sink_protect=True):
    """Replacement forward of a global-attention block (reference attention.py:296-659),
    same arguments and return value: (B, N*P, dim) after the W_O projection.
    sink_mass / sink_protect: the reference's RESS_SINK_MASS / RESS_SINK_PROTECT process
    flags (attention.py:50-79) as per-call arguments with the same defaults: pool the map
    over every key instead of the patch keys, and keep the block that straddles the patch
    tail and the special keys out of the candidates (kernels.LayerGrid).
    attention_sink (not a reference argument; default 0 = the reference's behaviour):
    leading tokens whose key blocks every row keeps, as sparse_global_attention.
    patch_order (not a reference argument; the module attribute set by the aggregator's
    use_hilbert): the per-frame patch order the blocks are formed in, read in place (the
    reference permutes the token tensor itself, hilbert.py:128-162). When
    aux_store is given the forward synchronises once for the realized sparsity and raises
    there if the HeSS budget did not converge; without it the forward does not synchronise
    (check_layers / LayerResult.check is the deferred check). eager_check (not a reference
    argument; the module attribute of the same name): synchronise at the end of the forward
    and raise there, as the reference raises a non-converged HeSS budget at once
    (_proportional.py:112-113)."""
    if pool_mode != "avg":
        raise NotImplementedError("only avg pooling (the reference default) is implemented")
    q, k, v, shp = compute_qkv(self, x, pos, num_special_tokens=num_special_tokens, num_heads=num_heads,
                               shape=shape)
    B, N, P, hd, nh, S = shp["B"], shp["N"], shp["P"], shp["head_dim"], shp["num_heads"], shp["S"]
    if hd != 64:
        raise ValueError(f"head_dim {hd} unsupported (the kernels are written for 64)")
    grid = LayerGrid(B=B, H=nh, frames=N, P=P, S=S, sink_protect=bool(sink_protect), sink_mass=bool(sink_mass))
    res = None
    if dense:
        x_out = _dense_storage(q, k, v, shp).float()
        sparsity = 0.0
        self._ress_status = None   # a dense forward leaves nothing to report
    else:
        qb, kbf, vbf = (t.to(torch.bfloat16) for t in (q, k, v))
        order = _device_patch_order(self, patch_order, grid, q.device)
        res = sparse_global_attention(
            qb, kbf, vbf, grid, num_to_select=num_to_select, budget_fn=budget_fn, perhead_budget_fn=perhead_budget_fn,
            joint_select_fn=joint_select_fn, block_criterion=block_criterion, M=getattr(self, "M", None),
            keep_intermediates=aux_store is not None and aux_full, protect_own_frame=protect_own_frame,
            attention_sink=attention_sink, patch_order=order)
        x_out = res.out
        # the forward does not synchronise: the layer's device-side status (HeSS convergence,
        # 16-bit operand range) stays on the module for check_layers
        self._ress_status = LayerResult(out=None, unconverged=res.unconverged, budget_iters=res.budget_iters,
                                        max_iters=res.max_iters, attn_status=res.attn_status)
        sparsity = res.sparsity() if aux_store is not None else None
        if eager_check and aux_store is None:
            res.check()
    if aux_store is not None:
        if aux_full and res is not None:
            aux_store["value"] = AttentionAux(
                attn_pooled=res.attn_full[..., :grid.n_cand], v_bar=res.v_bar_full[..., :grid.n_cand, :],
                attn_full=res.attn_full, v_bar_full=res.v_bar_full, n_cand=grid.n_cand,
                q_patch=_in_block_order(get_patch_tokens(q, N, P, S), order, N), shape=shp, sparsity=sparsity)
        else:
            aux_store["value"] = AttentionAux(shape=shp, sparsity=sparsity)
    if retain_output_grad and x_out.requires_grad:
        x_out.retain_grad()
    if aux_store is not None and aux_full:
        aux_store["value"].output = x_out
    return project_out(self, x_out.to(x.dtype) if x.dtype != x_out.dtype else x_out, B, N, P, nh, hd)


def check_layers(model_or_modules):
    """Synchronise once and raise what the last forward of each block-sparse attention
    module left unreported: RuntimeError if a HeSS budget did not converge (reference
    _proportional.py:112-113), ValueError if the 16-bit attention met an operand outside
    fp16's range. Takes a model (every submodule) or an iterable of modules."""
    mods = model_or_modules.modules() if hasattr(model_or_modules, "modules") else model_or_modules
    results = [m._ress_status for m in mods if getattr(m, "_ress_status", None) is not None]
    per = [r._status_values() for r in results]
    vals = [v for vs in per for v in vs]
    if not vals:
        return
    got = torch.stack(vals).tolist()
    i = 0
    for r, vs in zip(results, per):
        r._raise_status(got[i:i + len(vs)])
        i += len(vs)


def _device_patch_order(module, order, grid, device):
    """The device table of a module's patch order, validated and copied once per (order,
    device) and kept on the module (no host-to-device copy per call)."""
    if order is None:
        return None
    cache = module.__dict__.setdefault("_ress_patch_order_tables", {})
    key = (id(order), str(device))
    hit = cache.get(key)
    if hit is None or hit[0] is not order:
        hit = (order, kernels.patch_order_table(order, grid, device))
        cache[key] = hit
    return hit[1]


def _in_block_order(patch, order, frames):
    """Patch tokens (..., frames*HW, C) in the order the blocks were formed in."""
    if order is None:
        return patch
    hw = order.numel()
    idx = (torch.arange(frames, device=patch.device)[:, None] * hw + order.long()[None]).reshape(-1)
    return patch.index_select(-2, idx)


# ---------------------------------------------------------------------------
# Reference-compatible standalone helpers (plain sequences, GPU kernels)
# ---------------------------------------------------------------------------

def _plain_pools(query, key):
    B, nh, Tq, C = query.shape
    Tk = key.shape[-2]
    if C != 64:
        raise ValueError("head_dim must be 64")
    dev = query.device
    q = query.to(torch.bfloat16)
    k = key.to(torch.bfloat16)
    nq, nk = -(-Tq // KS_Q), -(-Tk // KS_K)
    BH = B * nh
    q_i8 = torch.empty(BH, nq, KS_Q, 64, dtype=torch.int8, device=dev)
    q_scale = torch.empty(BH, nq, device=dev)
    k_i8 = torch.empty(BH, nk, KS_K, 64, dtype=torch.int8, device=dev)
    k_scale = torch.empty(BH, nk, device=dev)
    pooled_q = torch.empty(BH, nq, 64, device=dev)
    P = _lib.ptr
    _lib.call("ress_per_block_int8", P(q), P(k), None, B, nh, Tq, Tk, *q.stride()[:3], *k.stride()[:3], P(q_i8),
              P(q_scale), P(k_i8), P(k_scale), P(pooled_q), _lib.stream_handle(dev))
    ksum = torch.empty(BH, nk, 64, device=dev)
    km = torch.empty(BH, 64, device=dev)
    pooled_k = torch.empty(BH, nk, 64, device=dev)
    pooled_v = torch.empty(BH, nk, 64, device=dev)
    v_pack = torch.empty(BH, nk, 4096, dtype=torch.bfloat16, device=dev)
    _lib.call("ress_prep_kv_plain", P(k), P(k), B, nh, Tk, *k.stride()[:3], *k.stride()[:3], P(ksum), P(km),
              P(pooled_k), P(pooled_v), P(v_pack), _lib.stream_handle(dev))
    return pooled_q, pooled_k, (B, nh, nq, nk)


def predict_attention(query, key, ks_q=KS_Q, ks_k=KS_K, pool_mode="avg"):
    """Pooled block map softmax(pool(Q) pool(K)^T / sqrt(C)) (reference attention.py:82-100).
    query (B, nh, Tq, 64), key (B, nh, Tk, 64) -> (B, nh, ceil(Tq/128), ceil(Tk/64)) fp32."""
    if (ks_q, ks_k, pool_mode) != (KS_Q, KS_K, "avg"):
        raise NotImplementedError("the kernels pool with 128/64 averages")
    pooled_q, pooled_k, (B, nh, nq, nk) = _plain_pools(query, key)
    dev = query.device
    full = torch.empty(B, nh, nq, nk, device=dev)
    cond = torch.empty(B, nh, nq, nk, device=dev)
    _lib.call("ress_pooled_scores", _lib.ptr(pooled_q), _lib.ptr(pooled_k), B * nh, nq, nk, nk,
              1.0 / math.sqrt(64), _lib.ptr(full), _lib.ptr(cond), _lib.stream_handle(dev))
    return full


def block_mean_value(value, ks_k=KS_K):
    """Per-64-key-block mean of V (reference attention.py:103-109): (B, nh, Tk, 64) ->
    (B, nh, ceil(Tk/64), 64) fp32."""
    if ks_k != KS_K:
        raise NotImplementedError("block size is 64")
    B, nh, Tk, C = value.shape
    v = value.to(torch.bfloat16)
    dev = v.device
    nk = -(-Tk // KS_K)
    BH = B * nh
    ksum = torch.empty(BH, nk, 64, device=dev)
    km = torch.empty(BH, 64, device=dev)
    pk = torch.empty(BH, nk, 64, device=dev)
    pv = torch.empty(BH, nk, 64, device=dev)
    vp = torch.empty(BH, nk, 4096, dtype=torch.bfloat16, device=dev)
    _lib.call("ress_prep_kv_plain", _lib.ptr(v), _lib.ptr(v), B, nh, Tk, *v.stride()[:3], *v.stride()[:3],
              _lib.ptr(ksum), _lib.ptr(km), _lib.ptr(pk), _lib.ptr(pv), _lib.ptr(vp), _lib.stream_handle(dev))
    return pv.view(B, nh, nk, 64)


def build_block_mask(pooled_score, num_to_select, sink_blocks, rank_by=None):
    """Top num_to_select of each row by (rank_by or pooled_score), ties to the lowest
    index, plus `sink_blocks` trailing all-True columns (reference attention.py:147-174).
    Returns (B, nh, q_blk, k_blk + sink_blocks) bool."""
    key = pooled_score if rank_by is None else rank_by
    B, nh, q_blk, k_blk = key.shape
    grid_cols = k_blk + sink_blocks
    dev = key.device
    fmap = torch.empty(B, nh, q_blk, grid_cols, dtype=torch.uint8, device=dev)
    lut = torch.empty(B * nh, q_blk, grid_cols, dtype=torch.int32, device=dev)
    nvalid = torch.empty(B * nh, q_blk, dtype=torch.int32, device=dev)
    rk = key.float().contiguous()
    cn = num_to_select.to(torch.int32).contiguous()
    _lib.call("ress_select_blocks", _lib.ptr(rk), _lib.ptr(cn), B * nh, q_blk, q_blk, k_blk, grid_cols, 0, 0,
              _lib.ptr(fmap), _lib.ptr(lut), _lib.ptr(nvalid), _lib.stream_handle(dev))
    return fmap.bool()


def compute_baseline_num_to_select(pooled_score, sparse_ratio=None, cdf_threshold=None, eps=1e-5):
    from ress_amd.budget import compute_baseline_num_to_select as _c
    return _c(pooled_score, sparse_ratio, cdf_threshold, eps)


def run_block_sparse_kernel(query, key, value, final_map, dtype=torch.float16, out_dtype=torch.float32):
    """Reference attention.py:217-243 on the GPU kernels: LUT of final_map, key mean,
    per-block INT8 Q and K - km, block-sparse attention. query (B,nh,Tq,64), key/value
    (B,nh,Tk,64), final_map (B,nh,ceil(Tq/128),ceil(Tk/64)). Returns (o, sparsity).
    One stated deviation: the reference casts q and k to `dtype` (fp16 by default) and takes
    km and k - km in that dtype; here q and k are taken in bf16 and km, k - km in fp32 before
    the per-block quantiser, so the INT8 codes can differ in the last code step from the
    reference's on the same inputs. V and o follow `dtype` as in the reference."""
    from ress_amd import sparge
    B, nh, Tq, C = query.shape
    q = query.contiguous().to(torch.bfloat16)
    k = key.contiguous().to(torch.bfloat16)
    v = value.contiguous().to(dtype)
    lut, valid_block_num = sparge.block_map_lut_triton(final_map)
    km = sparge.key_mean(k)
    q_int8, q_scale, k_int8, k_scale = sparge.per_block_int8(q, k, km=km)
    # o in `dtype` then out_dtype, as the reference rounds it (empty_like(query), .to(out_dtype))
    o = torch.empty(B, nh, Tq, C, dtype=dtype if dtype in (torch.float16, torch.bfloat16) else out_dtype,
                    device=q.device)
    sparge.qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold(
        q_int8, k_int8, v, o, lut, valid_block_num, sparge.hyperparameter_check(1e10, nh, q.device), q_scale,
        k_scale, 1, 0, 1, 1.0 / math.sqrt(C), 0)
    # one synchronisation for the sparsity the reference returns and the mirror's input check
    mean, status = torch.stack([final_map.float().mean(), sparge.last_call_status()[0].float()]).tolist()
    sparge.raise_for_status(int(status))
    return o.to(out_dtype), 1 - mean
