"""ReSS's residual-drift score and the restore-swap block ranking
(reference src/ress/scoring/projected.py).

M_h = (W_O^h)^T W_O^h is baked once per model; the per-candidate score is
s_ij = P_ij * sqrt(d^T M_h d), d = v_bar_query_i - v_bar_j.
"""

import contextlib

import torch

from ress_amd import _lib
from ress_amd.wiring import global_blocks

KEPT_MASS_EPS = 1e-6


def bake_M(model):
    """(n_blocks, nh, hd, hd): M_h = W_O[:, h*hd:(h+1)*hd]^T W_O[:, h*hd:(h+1)*hd] per global
    block (reference projected.py:214-232)."""
    Ms = []
    with torch.no_grad():
        for block in global_blocks(model):
            W_O = block.attn.proj.weight
            nh = block.attn.num_heads
            hd = W_O.shape[1] // nh
            Ms.append(torch.stack([W_O[:, h * hd:(h + 1) * hd].T @ W_O[:, h * hd:(h + 1) * hd]
                                   for h in range(nh)], dim=0))
    return torch.stack(Ms, dim=0)


def bake_and_attach_M(model):
    """Attach each layer's (nh, hd, hd) M as `block.attn.M` (reference projected.py:235-244)."""
    M = bake_M(model)
    for i, block in enumerate(global_blocks(model)):
        block.attn.M = M[i].to(next(block.attn.parameters()).device)
    return M


def quadratic_deviation(v_bar_query, v_bar, M):
    """sqrt(e^T M e), e = v_bar_query_i - v_bar_j, by the expanded form
    (reference projected.py:259-288)."""
    Mvq = torch.einsum("hij,...hqj->...hqi", M, v_bar_query)
    Mvk = torch.einsum("hij,...hkj->...hki", M, v_bar)
    term_q = (Mvq * v_bar_query).sum(dim=-1)
    term_k = (Mvk * v_bar).sum(dim=-1)
    cross = torch.einsum("...hqi,...hki->...hqk", Mvq, v_bar)
    quad = (term_q.unsqueeze(-1) - 2.0 * cross + term_k.unsqueeze(-2)).clamp(min=0)
    return quad.sqrt()


def dense_reference(attn_pooled, v_bar, n_cand=None):
    """(P candidates, V candidates, v_bar_query over all blocks, total mass)
    (reference projected.py:313-356)."""
    if n_cand is None:
        n_cand = attn_pooled.shape[-1]
    return (attn_pooled[..., :n_cand], v_bar[..., :n_cand, :], attn_pooled @ v_bar, attn_pooled.sum(dim=-1))


def projected_score(attn_pooled, v_bar, M, n_cand=None, renormalize=True):
    """s_ij / (1 - p_ij) (reference projected.py:359-388)."""
    P, V, vq, _ = dense_reference(attn_pooled.float(), v_bar.float(), n_cand)
    score = P * quadratic_deviation(vq, V, M.float())
    if renormalize:
        score = score / (1.0 - P).clamp(min=1e-4)
    return score


# The list record_realized_drift has active, or None: the forward appends to it only while
# a recorder is open (reference projected.py:84-93).
_realized_records = None


@contextlib.contextmanager
def record_realized_drift():
    """While active, every block-sparse attention layer that has an M (bake_and_attach_M)
    appends one float to the yielded list, in forward order: the mean over its (batch,
    head, query-block) rows of J = ||g||^2_M / K^2 for the kept set the attention kernel
    was handed, sinks included (reference projected.py:95-109, attention.py:199-214, 620-623).
    Each recorded layer synchronises once; nothing changes while no recorder is open."""
    global _realized_records
    prev = _realized_records
    records = []
    _realized_records = records
    try:
        yield records
    finally:
        _realized_records = prev


def realized_objective(attn_pooled, v_bar, M, keep_mask, n_cand=None, dtype=torch.float32):
    """J = ||g||^2_M / K^2 per (..., nh, q_blk) for any kept set (reference
    projected.py:112-129): g = (sum of the dropped P) * v_bar_query - (dropped P) @ V over
    the candidates, K = total mass - dropped mass (floored at KEPT_MASS_EPS before squaring).
    attn_pooled / v_bar: the pooled map and block means over the whole pooled grid
    (candidates first); keep_mask (..., nh, q_blk, n_cand) bool over the candidates only.
    The same J the restore-swap kernel reports for its own set, here in torch fp32 for a
    set made by any criterion: a diagnostic, off the layer's hot path."""
    P, V, vq, total = dense_reference(attn_pooled.to(dtype), v_bar.to(dtype), n_cand)
    Pd = P * (~keep_mask.bool()).to(dtype)
    sum_pd = Pd.sum(dim=-1)
    g = sum_pd.unsqueeze(-1) * vq - torch.matmul(Pd, V)
    Mg = torch.matmul(g, M.to(dtype).transpose(-1, -2))
    obj = (g * Mg).sum(dim=-1)
    return obj / (total - sum_pd).clamp(min=KEPT_MASS_EPS).pow(2)


def record_layer_drift(M, attn_full, v_bar_full, final_map, n_cand):
    """Append the layer's mean realized J to the open recorder; a no-op when none is open
    or the layer has no M (reference attention.py:199-214)."""
    if _realized_records is None or M is None:
        return
    with torch.no_grad():
        J = realized_objective(attn_full, v_bar_full, M, final_map[..., :n_cand].bool(), n_cand=n_cand)
    _realized_records.append(J.float().mean().item())


def kept_mass_norm_quality(G, K, delta_G, u, eps=KEPT_MASS_EPS):
    """J - J_new = [G*u*(2K+u)/K^2 - delta_G] / (K+u)^2 (reference projected.py:191-211)."""
    K_ = K.unsqueeze(-1)
    K_new = (K_ + u).clamp(min=eps)
    return (G.unsqueeze(-1) * u * (2.0 * K_ + u) / K_.pow(2) - delta_G) / K_new.pow(2)


_RS_BF16, _RS_TRACK_BEST, _RS_MAXIMIZE, _RS_INVERT_CUT, _RS_NO_RENORM = 1, 2, 4, 8, 16


def _restore_swap(attn_pooled, v_bar, M, num_to_select, restore_frac, n_iters, track_best, big_dtype, decay,
                  renormalize, n_cand, maximize, invert_cut, want_s):
    """Run the restore-swap kernel (ress_swap.hip). Returns (keep_key, s) with keep_key
    (..., nh, q_blk, n_cand) fp32 = 1 kept / 0 dropped, and s the drift scores (or None)."""
    if big_dtype not in (None, torch.float32, torch.bfloat16):
        raise NotImplementedError(f"big_dtype {big_dtype} (fp32 and bf16 are implemented)")
    *lead, nh, q_blk, kb_p = attn_pooled.shape
    if v_bar.shape[-2:] != (kb_p, 64) or M.shape != (nh, 64, 64):
        raise ValueError("v_bar must be (..., nh, k_blk, 64) and M (nh, 64, 64)")
    if n_cand is None:
        n_cand = kb_p
    dev = attn_pooled.device
    A = attn_pooled.float().contiguous()
    V = v_bar.float().contiguous()
    Mf = M.float().contiguous()
    nts = num_to_select.to(torch.int32).expand(*lead, nh, q_blk).contiguous()
    BH = A.numel() // (q_blk * kb_p) if q_blk else nh
    keep = torch.empty(*lead, nh, q_blk, n_cand, dtype=torch.float32, device=dev)
    s = torch.empty_like(keep) if want_s else None
    flags = ((_RS_BF16 if big_dtype == torch.bfloat16 else 0) | (_RS_TRACK_BEST if track_best else 0)
             | (_RS_MAXIMIZE if maximize else 0) | (_RS_INVERT_CUT if invert_cut else 0)
             | (0 if (True if renormalize is None else renormalize) else _RS_NO_RENORM))
    ws_bytes = _lib.lib().ress_restore_swap_workspace_size(BH, q_blk, kb_p, n_cand)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    _lib.call("ress_restore_swap", _lib.ptr(A), _lib.ptr(V), _lib.ptr(Mf), _lib.ptr(nts), BH, nh, q_blk, kb_p, n_cand,
              int(n_iters), float(restore_frac), float(decay), flags, _lib.ptr(keep), None, _lib.ptr(s), _lib.ptr(ws),
              ws_bytes, _lib.stream_handle(dev))
    return keep, s


def restore_swap_keep(attn_pooled, v_bar, M, num_to_select, restore_frac=0.5, n_iters=1, track_best=False,
                      big_dtype=None, decay=0.5, renormalize=None, n_cand=None, maximize=False, invert_cut=False):
    """The restore-swap keep set as a rank key (1 = kept, 0 = dropped): the top
    num_to_select of it is exactly the set restore_swap_rank_by's rank_by selects."""
    keep, _ = _restore_swap(attn_pooled, v_bar, M, num_to_select, restore_frac, n_iters, track_best, big_dtype, decay,
                            renormalize, n_cand, maximize, invert_cut, want_s=False)
    return keep


def restore_swap_rank_by(attn_pooled, v_bar, M, num_to_select, restore_frac=0.5, n_iters=1, dtype=torch.float32,
                         track_best=False, big_dtype=None, decay=0.5, renormalize=None, n_cand=None,
                         maximize=False, invert_cut=False):
    """ReSS restore-swap ranking (reference projected.py:395-1058), on the GPU kernel.

    attn_pooled (..., nh, q_blk, k_blk) the pooled map over the kernel's patch key blocks,
    v_bar (..., nh, k_blk, 64), M (nh, 64, 64), num_to_select (..., nh, q_blk). Initial
    cut by s/(1-P) (s with renormalize=False), then n_iters restore/compensate rounds on
    J = ||g||^2_M / K^2 with the geometric schedule restore_frac * decay * (1-decay)^i,
    track_best keeping each row's best state. big_dtype=torch.bfloat16 rounds the
    k-wide tensors as the reference's _bf16 recipes do. Returns rank_by (..., nh, q_blk,
    n_cand) = where(drop, s, s + max|s| + 1), in big_dtype (fp32 if None)."""
    if dtype != torch.float32:
        raise NotImplementedError("the accumulation dtype is fp32")
    keep, s = _restore_swap(attn_pooled, v_bar, M, num_to_select, restore_frac, n_iters, track_best, big_dtype,
                            decay, renormalize, n_cand, maximize, invert_cut, want_s=True)
    s = s.to(big_dtype or torch.float32)
    offset = (s.abs().amax() + 1.0) if s.numel() else torch.ones((), dtype=s.dtype, device=s.device)
    return torch.where(keep > 0.5, s + offset, s)
