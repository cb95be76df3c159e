"""protect_own_frame (reference src/ress/models/attention.py:112-144, 583-618): the
own-frame block mask against its interval-overlap definition, and the budget-neutral
swap against a per-row brute-force restatement in numpy (stable orders: ties to the
lower block index). Pure torch, so it runs on the CPU here; the GPU test runs it inside
the layer."""

import numpy as np
import torch

from ress_amd.attention import protect_own_frame_swap, same_frame_block_mask
from ress_amd.kernels import LayerGrid


def test_same_frame_mask_definition():
    N, H, W = 5, 7, 9          # 63 patch tokens per frame: blocks straddle frame boundaries
    T = N * H * W
    m = same_frame_block_mask(-(-T // 128), -(-T // 64), N, H, W, "cpu").numpy()
    for qb in range(m.shape[0]):
        qf = {t // (H * W) for t in range(qb * 128, min(qb * 128 + 128, T))}
        for kb in range(m.shape[1]):
            kf = {t // (H * W) for t in range(kb * 64, min(kb * 64 + 64, T))}
            # interval overlap of the frame ranges == the ranges share a frame
            assert m[qb, kb] == bool(qf & kf)


def _swap_ref(kept, same, pooled):
    """One row: kept/same bool (n,), pooled (n,) -> new kept."""
    missing = np.flatnonzero(same & ~kept)
    swappable = np.flatnonzero(kept & ~same)
    n_swap = min(len(missing), len(swappable))
    out = sorted(swappable, key=lambda c: (pooled[c], c))[:n_swap]
    inn = sorted(missing, key=lambda c: (-pooled[c], c))[:n_swap]
    new = kept.copy()
    new[out] = False
    new[inn] = True
    return new


def test_swap_matches_bruteforce_and_is_budget_neutral():
    rng = np.random.default_rng(0)
    g = LayerGrid(B=1, H=3, frames=4, P=1374, S=5)   # 85 candidates, 86 blocks
    n = g.n_cand
    for trial in range(3):
        fmap = rng.random((1, 3, g.q_blk_p, g.kb_tot)) < (0.15, 0.5, 0.9)[trial]
        fmap[..., n:] = True                                 # sink columns
        pooled = rng.random((1, 3, g.q_blk_p, n)).astype(np.float32)
        pooled[..., ::7] = pooled[..., 3:4]                  # ties
        got = protect_own_frame_swap(torch.from_numpy(fmap), torch.from_numpy(pooled), g).numpy()
        same = same_frame_block_mask(g.q_blk_p, n, g.frames, g.P - g.S, 1, "cpu").numpy()
        for h in range(3):
            for r in range(g.q_blk_p):
                want = _swap_ref(fmap[0, h, r, :n], same[r], pooled[0, h, r])
                assert np.array_equal(got[0, h, r, :n], want), (trial, h, r)
                assert got[0, h, r, :n].sum() == fmap[0, h, r, :n].sum()
        assert got[..., n:].all()
