"""The C oracle's ReSS restore-swap (oracle_restore_swap) pinned without the reference:

* against an independent float64 torch restatement of the reference's eager algorithm
  (oracle/reference.py: restore_swap_torch) across every mode the criterion grammar
  reaches (n_iters, restore_frac, decay, track_best, _antiswap, _anti, renormalize);
* the bf16 rounding ladder against the same restatement run with the reference's bf16
  casts, on inputs whose dot products are exact in fp32 (so torch's summation order
  cannot matter and only the rounding points are compared);
* invariants: the kept count is min(nts, n_cand); track_best never returns a set with a
  larger J than the initial cut; the reported J is the float64 J of the returned set."""

import numpy as np
import pytest
import torch

import oracle
from oracle import reference as ref


def _problem(seed, H=2, q_blk=6, kb_p=None, nice=False):
    rng = np.random.default_rng(seed)
    kb_p = kb_p or int(rng.integers(20, 120))
    n_cand = kb_p - int(rng.integers(0, 2))
    if nice:
        A = (rng.integers(0, 16, size=(H, q_blk, kb_p)) / 256.0).astype(np.float32)
        V = (rng.integers(-8, 9, size=(H, kb_p, 64)) / 8.0).astype(np.float32)
        M = np.zeros((H, 64, 64), np.float32)
        for h in range(H):
            m = rng.integers(-2, 3, size=(64, 64)) / 4.0
            M[h] = (m + m.T) / 2 + np.eye(64) * 4
    else:
        A = np.exp(rng.normal(size=(H, q_blk, kb_p)) * rng.uniform(0.5, 3))
        A = (A / A.sum(-1, keepdims=True)).astype(np.float32)
        V = rng.normal(size=(H, kb_p, 64)).astype(np.float32)
        W = rng.normal(size=(H, 64, 64)).astype(np.float32) / 8
        M = np.einsum("hji,hjk->hik", W, W).astype(np.float32)
    nts = rng.integers(2, n_cand + 3, size=(H, q_blk)).astype(np.int32)
    return A, V, M, nts, n_cand


MODES = [
    dict(n_iters=5, restore_frac=0.5, decay=0.5, track_best=True),
    dict(n_iters=1, restore_frac=0.5, decay=0.5, track_best=False),
    dict(n_iters=6, restore_frac=0.3, decay=0.3, track_best=True),
    dict(n_iters=3, restore_frac=0.8, decay=0.5, track_best=False),
    dict(n_iters=5, restore_frac=0.5, decay=0.5, track_best=True, maximize=True),
    dict(n_iters=5, restore_frac=0.5, decay=0.5, track_best=True, maximize=True, invert_cut=True),
    dict(n_iters=2, restore_frac=0.5, decay=0.5, track_best=True, renormalize=False),
]


@pytest.mark.parametrize("mode", range(len(MODES)))
def test_matches_float64_restatement(mode):
    kw = MODES[mode]
    for seed in range(4):
        A, V, M, nts, n_cand = _problem(10 * mode + seed)
        keep, _ = oracle.restore_swap(A, V, M, nts, n_cand, big_bf16=False, **kw)
        tkw = {k: v for k, v in kw.items() if k != "renormalize"}
        want = ref.restore_swap_torch(A, V, M, nts, n_cand, renormalize=kw.get("renormalize", True), **tkw).numpy()
        assert np.array_equal(keep.astype(bool), want), (mode, seed)


def test_bf16_ladder_on_exact_sums():
    for seed in range(12):
        A, V, M, nts, n_cand = _problem(100 + seed, H=2, q_blk=4, kb_p=int(10 + 4 * seed), nice=True)
        keep, _ = oracle.restore_swap(A, V, M, nts, n_cand, big_bf16=True)
        want = ref.restore_swap_torch(A, V, M, nts, n_cand, dtype=torch.float32, big=torch.bfloat16).numpy()
        assert np.array_equal(keep.astype(bool), want), seed


def test_invariants_and_objective():
    for seed in range(6):
        A, V, M, nts, n_cand = _problem(300 + seed)
        for bf in (False, True):
            keep0, J0 = oracle.restore_swap(A, V, M, nts, n_cand, n_iters=0, big_bf16=bf)
            keep, J = oracle.restore_swap(A, V, M, nts, n_cand, n_iters=5, big_bf16=bf, track_best=True)
            assert np.array_equal(keep.sum(-1), np.minimum(nts, n_cand))
            assert np.array_equal(keep0.sum(-1), np.minimum(nts, n_cand))
            assert (J <= J0).all()
            J64 = ref.drift_objective64(A, V, M, keep, n_cand).numpy()
            if not bf:  # fp32 oracle arithmetic vs float64 on the same set
                np.testing.assert_allclose(J, J64, rtol=2e-4, atol=1e-9)
