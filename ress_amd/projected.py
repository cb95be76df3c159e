"""ReSS's residual-drift score and the restore-swap block ranking
(reference src/ress/scoring/projected.py).

M_h = (W_O^h)^T W_O^h is baked once per model; the per-candidate score is
s_ij = P_ij * sqrt(d^T M_h d), d = v_bar_query_i - v_bar_j.
"""

import torch

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


def kept_mass_norm_quality(G, K, delta_G, u, eps=KEPT_MASS_EPS):
    """J - J_new = [G*u*(2K+u)/K^2 - delta_G] / (K+u)^2 (reference projected.py:191-211)."""
    K_ = K.unsqueeze(-1)
    K_new = (K_ + u).clamp(min=eps)
    return (G.unsqueeze(-1) * u * (2.0 * K_ + u) / K_.pow(2) - delta_G) / K_new.pow(2)


def restore_swap_rank_by(attn_pooled, v_bar, M, num_to_select, restore_frac=0.5, n_iters=1, dtype=torch.float32,
                         track_best=False, big_dtype=None, decay=0.5, renormalize=None, n_cand=None,
                         maximize=False, invert_cut=False):
    """ReSS restore-swap ranking (reference projected.py:395-1058)."""
    raise NotImplementedError("restore-swap ranking is not implemented yet")
