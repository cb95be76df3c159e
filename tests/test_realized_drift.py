"""realized_objective and the per-layer realized-J recorder (reference
src/ress/scoring/projected.py:95-129, src/ress/models/attention.py:199-214, 620-623).

realized_objective is checked against J written as the direct sum over the dropped set,
g = sum_{j in D} p_j (v_bar_query - V_j) (not the sum_pd * v_bar_query - Pd @ V form it
computes), in float64, against the C oracle's J for the restore-swap keep sets, and on the
special cases the definition fixes (nothing dropped gives 0; one dropped block gives
p^2 ||v_bar_query - V_j||^2_M / (total - p)^2)."""

import numpy as np
import torch

import oracle
from ress_amd import projected


def _problem(seed, H=2, q_blk=4, kb_p=30, n_cand=27):
    rng = np.random.default_rng(seed)
    logits = rng.normal(size=(H, q_blk, kb_p)) * 1.5
    A = np.exp(logits)
    A = (A / A.sum(-1, keepdims=True) * rng.uniform(0.6, 1.0, size=(H, q_blk, 1))).astype(np.float32)
    V = rng.normal(size=(H, kb_p, 64)).astype(np.float32)
    W = (rng.normal(size=(H, 64, 64)) / 8).astype(np.float32)
    M = np.einsum("hji,hjk->hik", W, W).astype(np.float32)
    keep = rng.random(size=(H, q_blk, n_cand)) < 0.4
    return A, V, M, keep, n_cand


def _direct(A, V, M, keep, n_cand):
    A, V, M = A.astype(np.float64), V.astype(np.float64), M.astype(np.float64)
    H, q_blk, _ = A.shape
    out = np.zeros((H, q_blk))
    for h in range(H):
        for q in range(q_blk):
            vq = A[h, q] @ V[h]
            g = np.zeros(64)
            dropped = 0.0
            for j in range(n_cand):
                if not keep[h, q, j]:
                    g += A[h, q, j] * (vq - V[h, j])
                    dropped += A[h, q, j]
            out[h, q] = g @ M[h] @ g / max(A[h, q].sum() - dropped, projected.KEPT_MASS_EPS) ** 2
    return out


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x))


def test_realized_objective_is_the_direct_sum():
    for seed in range(4):
        A, V, M, keep, n_cand = _problem(seed)
        got = projected.realized_objective(_t(A), _t(V), _t(M), _t(keep), n_cand=n_cand, dtype=torch.float64)
        np.testing.assert_allclose(got.numpy(), _direct(A, V, M, keep, n_cand), rtol=1e-11, atol=1e-15)


def test_realized_objective_special_cases():
    A, V, M, keep, n_cand = _problem(7)
    all_kept = np.ones_like(keep)
    z = projected.realized_objective(_t(A), _t(V), _t(M), _t(all_kept), n_cand=n_cand, dtype=torch.float64)
    assert torch.count_nonzero(z) == 0
    one = all_kept.copy()
    one[..., 5] = False
    got = projected.realized_objective(_t(A), _t(V), _t(M), _t(one), n_cand=n_cand, dtype=torch.float64).numpy()
    A64, V64, M64 = A.astype(np.float64), V.astype(np.float64), M.astype(np.float64)
    e = np.einsum("hqk,hkd->hqd", A64, V64) - V64[:, None, 5]
    p = A64[..., 5]
    want = p ** 2 * np.einsum("hqi,hij,hqj->hq", e, M64, e) / (A64.sum(-1) - p) ** 2
    np.testing.assert_allclose(got, want, rtol=1e-11)


def test_realized_objective_matches_oracle_restore_swap_J():
    """The oracle's J of its own fp32 restore-swap keep set (its arithmetic order) against
    realized_objective in fp32 on that set."""
    for seed in range(3):
        A, V, M, _, n_cand = _problem(20 + seed, kb_p=50, n_cand=48)
        nts = np.random.default_rng(seed).integers(2, n_cand, size=A.shape[:2]).astype(np.int32)
        keep, J = oracle.restore_swap(A, V, M, nts, n_cand, n_iters=5, big_bf16=False, track_best=True)
        got = projected.realized_objective(_t(A), _t(V), _t(M), _t(keep.astype(bool)), n_cand=n_cand)
        np.testing.assert_allclose(got.numpy(), J, rtol=2e-4, atol=1e-9)


def test_recorder_collects_per_layer_means_and_nests():
    A, V, M, keep, n_cand = _problem(3)
    fmap = _t(np.concatenate([keep, np.ones(keep.shape[:2] + (3,), bool)], -1))
    J = projected.realized_objective(_t(A), _t(V), _t(M), _t(keep), n_cand=n_cand)
    projected.record_layer_drift(_t(M), _t(A), _t(V), fmap, n_cand)  # no recorder: no-op
    with projected.record_realized_drift() as outer:
        projected.record_layer_drift(_t(M), _t(A), _t(V), fmap, n_cand)
        projected.record_layer_drift(None, _t(A), _t(V), fmap, n_cand)  # no M: not recorded
        with projected.record_realized_drift() as inner:
            projected.record_layer_drift(_t(M), _t(A), _t(V), fmap.to(torch.uint8), n_cand)
        projected.record_layer_drift(_t(M), _t(A), _t(V), fmap, n_cand)
    assert projected._realized_records is None
    assert len(outer) == 2 and len(inner) == 1
    assert outer[0] == outer[1] == inner[0] == J.mean().item()
