"""The whole ReSS-forward block-map pipeline on the CPU oracle (test helper)."""

import numpy as np

import oracle
from ress_amd.kernels import LayerGrid


def oracle_layer(q, k, v, frames, P, S, sparse_ratio=None, cdf_threshold=None, head_scores=None, B=1, H=16,
                 sink_lead=0, criterion="probability", M=None, rank_key=None, max_iters=1000, sink_mass=False):
    """Returns a dict with prep outputs, attn_full/attn_cond, baseline, counts, map, lut, nvalid.

    criterion: "probability" ranks by attn_cond; "ress" by the restore_swap_iter5_bf16_trackbest
    keep set (M: (H, 64, 64)); "key" by the given rank_key (B*H, q_blk_p, n_cand). sink_lead:
    leading key blocks forced on (the attention sink). sink_mass: the map pooled over every key."""
    g = LayerGrid(B, H, frames, P, S, sink_mass=sink_mass)
    o = oracle.prep_qkv(q, k, v, frames, P, S, pool_all=sink_mass)
    full, cond = oracle.pooled_scores(o["pooled_q"], o["pooled_k"], g.n_cand)
    base = oracle.baseline_budget(cond, sparse_ratio, cdf_threshold).reshape(B, H, g.q_blk_p)
    if head_scores is not None:
        counts, it = oracle.head_budget(base, oracle.scores_norm_seq(head_scores), 1.0, g.n_cand, max_iters=max_iters)
        assert it >= 0
    else:
        counts = base
    min_sel = min(2, g.n_cand)
    sel_counts = counts.reshape(B * H, g.q_blk_p)
    if criterion == "probability":
        rank = cond
    elif criterion == "ress":
        sel_counts = np.maximum(sel_counts, min_sel).astype(np.int32)
        keep, _ = oracle.restore_swap(full.reshape(B * H, g.q_blk_p, g.kb_p), o["pooled_v"].reshape(B * H, g.kb_p, 64),
                                      np.tile(np.asarray(M, np.float32), (B, 1, 1)), sel_counts, g.n_cand, n_iters=5,
                                      big_bf16=True, track_best=True)
        rank = keep.astype(np.float32)
    elif criterion == "key":
        sel_counts = np.maximum(sel_counts, min_sel).astype(np.int32)
        rank = np.asarray(rank_key, np.float32).reshape(B * H, g.q_blk_p, g.n_cand)
    else:
        raise ValueError(criterion)
    fmap, lut, nvalid = oracle.select_blocks(rank, sel_counts, g.q_blk_total, g.kb_tot, sink_lead=sink_lead,
                                             min_select=min_sel)
    o.update(attn_full=full, attn_cond=cond, baseline=base, counts=counts, map=fmap, lut=lut, nvalid=nvalid,
             grid=g)
    return o


def row_sample(nvalid, n, seed=0):
    """A few (bh, qb) rows: first, last, the dense rows, and random ones."""
    BH, qt = nvalid.shape
    n = min(n, BH * qt)
    rng = np.random.default_rng(seed)
    rows = {(0, 0), (BH - 1, qt - 1), (0, qt - 1)}
    while len(rows) < n:
        rows.add((int(rng.integers(BH)), int(rng.integers(qt))))
    return sorted(rows)
