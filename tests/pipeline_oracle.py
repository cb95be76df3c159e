"""The whole ReSS-forward block-map pipeline on the CPU oracle (test helper)."""

import numpy as np

import oracle
from ress_amd.kernels import LayerGrid


def oracle_layer(q, k, v, frames, P, S, sparse_ratio=None, cdf_threshold=None, head_scores=None, B=1, H=16):
    """Returns a dict with prep outputs, attn_full/attn_cond, baseline, counts, map, lut, nvalid."""
    g = LayerGrid(B, H, frames, P, S)
    o = oracle.prep_qkv(q, k, v, frames, P, S)
    full, cond = oracle.pooled_scores(o["pooled_q"], o["pooled_k"], g.n_cand)
    base = oracle.baseline_budget(cond, sparse_ratio, cdf_threshold).reshape(B, H, g.q_blk_p)
    if head_scores is not None:
        counts, it = oracle.head_budget(base, oracle.scores_norm_seq(head_scores), 1.0, g.n_cand)
        assert it >= 0
    else:
        counts = base
    fmap, lut, nvalid = oracle.select_blocks(cond, counts.reshape(B * H, g.q_blk_p), g.q_blk_total, g.kb_tot,
                                             min_select=min(2, g.n_cand))
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
