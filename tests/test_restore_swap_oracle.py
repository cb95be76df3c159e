"""The C oracle's ReSS restore-swap (oracle_restore_swap) pinned without the reference:

* against an independent float64 torch restatement of the reference's eager algorithm
  (oracle/reference.py: restore_swap_torch) across every mode the criterion grammar
  reaches (n_iters, restore_frac, decay, track_best, _antiswap, _anti, renormalize);
* the bf16 rounding ladder against the same restatement run with the reference's bf16
  casts, on inputs whose dot products are exact in fp32 (so torch's summation order
  cannot matter and only the rounding points are compared);
* the bf16 ladder against its float64 definition on the same bf16 inputs: the scores, the
  cut key and J of the cut within per-term rounding bounds, and the cut's keep set equal to
  the float64 top-nts wherever the margin at the threshold exceeds the bounds;
* invariants: the kept count is min(nts, n_cand); track_best never returns a set with a
  larger J than the initial cut; the reported J is the float64 J of the returned set;
* the identities the reference states, each computed from its definition in float64
  through oracle_rs_probe (the helpers the rounds themselves rank with): the expanded
  quadratic form equals the direct one and s_k^2 = ||e_k||^2_M (projected.py:259-288,
  415-420); J({j}) = (s_j/(1-p_j))^2, the square of the cut key (:294-302); each round
  marginal equals the brute-force J(D) - J(D -/+ {k}) (:191-211); M = I gives the
  head-space damage p ||v_bar_query - V_k|| (attention.py:562-564). Planting a wrong sign,
  grouping, index or mass term in the C oracle's score, objective or marginals fails them."""

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


# ---- first-principles identities (float64), through oracle_rs_probe --------------------
# The probe runs the helpers oracle_restore_swap itself ranks with (rs_row_setup for s,
# rs_round_qualities for J and the round marginals), so these pin the rounds' arithmetic
# against the definitions in src/ress/scoring/projected.py, not against a second
# transcription of its expanded formulas.


def _softmax_problem(seed, H=2, q_blk=3, kb_p=40, sinks=2, identity_M=False, partial_mass=False):
    """Rows of A are full softmaxes over all kb_p blocks (total mass 1, the last `sinks`
    blocks never droppable), V random, M = W^T W (PSD) or the identity. partial_mass: each
    row scaled to a total mass in [0.5, 0.95], as when part of the mass lies outside the
    map, so K = total mass - dropped mass differs from 1 - dropped mass."""
    rng = np.random.default_rng(seed)
    logits = rng.normal(size=(H, q_blk, kb_p)) * rng.uniform(0.5, 2.5, size=(H, q_blk, 1))
    A = np.exp(logits - logits.max(-1, keepdims=True))
    A = A / A.sum(-1, keepdims=True)
    if partial_mass:
        A = A * rng.uniform(0.5, 0.95, size=(H, q_blk, 1))
    A = A.astype(np.float32)
    V = rng.normal(size=(H, kb_p, 64)).astype(np.float32)
    if identity_M:
        M = np.broadcast_to(np.eye(64, dtype=np.float32), (H, 64, 64)).copy()
    else:
        W = (rng.normal(size=(H, 64, 64)) / 8).astype(np.float32)
        M = np.einsum("hji,hjk->hik", W, W).astype(np.float32)
    return A, V, M, kb_p - sinks


def _J64(A, V, M, drop, n_cand):
    """J(D) = ||g||^2_M / K^2 by its definition (projected.py:290-302): g = sum_{j in D}
    p_j (v_bar_query - V_j) with v_bar_query = sum over all blocks of p V, K = total mass
    minus the dropped mass; float64, direct (no expansion). drop (..., n_cand) bool."""
    A64, V64, M64 = A.astype(np.float64), V.astype(np.float64), M.astype(np.float64)
    vq = np.einsum("hqk,hkd->hqd", A64, V64)
    Pd = A64[..., :n_cand] * drop
    g = Pd.sum(-1)[..., None] * vq - np.einsum("hqk,hkd->hqd", Pd, V64[:, :n_cand])
    G = np.einsum("hqi,hij,hqj->hq", g, M64, g)
    K = A64.sum(-1) - Pd.sum(-1)
    return G / K ** 2


def test_score_is_direct_quadratic_form():
    """s_k = p_k sqrt((v_bar_query - V_k)^T M (v_bar_query - V_k)): the oracle's expanded
    term_q - 2 cross + term_k (quadratic_deviation, projected.py:259-288) equals the direct
    form, and s_k^2 = ||e_k||^2_M for e_k = p_k (v_bar_query - V_k) (projected.py:415-420).
    Tolerance: fp32 cancellation of the expansion, eps32-scaled by its three terms."""
    for seed in range(6):
        A, V, M, n = _softmax_problem(seed)
        s, _, _, _, _ = oracle.rs_probe(A, V, M, np.zeros(A.shape[:2] + (n,), bool), n)
        A64, V64, M64 = A.astype(np.float64), V.astype(np.float64), M.astype(np.float64)
        vq = np.einsum("hqk,hkd->hqd", A64, V64)
        e = vq[:, :, None, :] - V64[:, None, :n, :]
        quad = np.einsum("hqki,hij,hqkj->hqk", e, M64, e)
        p = A64[..., :n]
        tq = np.einsum("hqi,hij,hqj->hq", vq, M64, vq)[..., None]
        tk = np.einsum("hki,hij,hkj->hk", V64[:, :n], M64, V64[:, :n])[:, None, :]
        cr = np.abs(np.einsum("hqi,hij,hkj->hqk", vq, M64, V64[:, :n]))
        tol = p ** 2 * 4e-6 * (tq + 2 * cr + tk) + 1e-30
        assert (np.abs(s.astype(np.float64) ** 2 - p ** 2 * quad) <= tol).all(), seed


def test_single_drop_objective_is_renormalized_score():
    """J({j}) = (s_j / (1 - p_j))^2 (projected.py:294-302): the objective of dropping one
    candidate alone, by definition and as the oracle's rs_objective computes it, equals the
    square of the renormalised cut key the initial cut ranks by. J is held to the float64
    definition at rtol 2e-5; against the closed forms built from the fp32 s, the tolerance
    adds the expanded quadratic form's cancellation bound on s^2
    (test_score_is_direct_quadratic_form), relative to s^2."""
    for seed in range(3):
        A, V, M, n = _softmax_problem(50 + seed, kb_p=24)
        H, Q = A.shape[:2]
        A64, V64, M64 = A.astype(np.float64), V.astype(np.float64), M.astype(np.float64)
        vq = np.einsum("hqk,hkd->hqd", A64, V64)
        tq = np.einsum("hqi,hij,hqj->hq", vq, M64, vq)
        for j in range(n):
            drop = np.zeros((H, Q, n), bool)
            drop[..., j] = True
            s, scut, J, _, _ = oracle.rs_probe(A, V, M, drop, n)
            p = A[..., j].astype(np.float64)
            sj = s[..., j].astype(np.float64)
            tk = np.einsum("hi,hij,hj->h", V64[:, j], M64, V64[:, j])[:, None]
            cr = np.abs(np.einsum("hqi,hij,hj->hq", vq, M64, V64[:, j]))
            rel = 2e-5 + p ** 2 * 4e-6 * (tq + 2 * cr + tk) / np.maximum(sj ** 2, 1e-300)
            closed = (sj / (1.0 - p)) ** 2
            assert (np.abs(J - closed) <= rel * closed + 1e-30).all(), (seed, j)
            sc2 = scut[..., j].astype(np.float64) ** 2
            assert (np.abs(J - sc2) <= (rel + 2e-5) * sc2 + 1e-30).all(), (seed, j)
            np.testing.assert_allclose(J, _J64(A, V, M, drop, n), rtol=2e-5, atol=1e-30)


def test_round_qualities_are_bruteforce_objective_differences():
    """kept_mass_norm_quality (projected.py:191-211) as the round uses it: restoring dropped
    k scores J(D) - J(D - {k}), dropping kept k scores J(D) - J(D + {k}), both by the
    float64 definition of J. Tolerance: the fp32 grouped form's rounding, relative to the
    row's largest marginal."""
    rng = np.random.default_rng(7)
    for seed in range(6):
        A, V, M, n = _softmax_problem(80 + seed, kb_p=36, partial_mass=seed % 2 == 1)
        H, Q = A.shape[:2]
        drop = rng.random((H, Q, n)) < rng.uniform(0.3, 0.8)
        _, _, J, rq, cq = oracle.rs_probe(A, V, M, drop, n)
        J0 = _J64(A, V, M, drop, n)
        np.testing.assert_allclose(J, J0, rtol=2e-5, atol=1e-30)
        want = np.zeros((H, Q, n))
        for k in range(n):
            d2 = drop.copy()
            d2[..., k] = ~drop[..., k]
            want[..., k] = J0 - _J64(A, V, M, d2, n)
        got = np.where(drop, rq, cq).astype(np.float64)
        scale = np.abs(want).max(-1, keepdims=True)
        assert (np.abs(got - want) <= 2e-4 * scale + 1e-6 * np.abs(J0)[..., None]).all(), seed
        # the marginal has the sign of the change of J, so a beneficial move is a positive one
        big = np.abs(want) > 1e-2 * scale
        assert (np.sign(got[big]) == np.sign(want[big])).all(), seed


def test_identity_metric_is_head_space_damage():
    """M = I reduces the score to the head-space damage p_k ||v_bar_query - V_k||_2
    (src/ress/models/attention.py:562-564, the _nowo recipes)."""
    for seed in range(4):
        A, V, M, n = _softmax_problem(120 + seed, identity_M=True)
        s, _, _, _, _ = oracle.rs_probe(A, V, M, np.zeros(A.shape[:2] + (n,), bool), n)
        A64, V64 = A.astype(np.float64), V.astype(np.float64)
        vq = np.einsum("hqk,hkd->hqd", A64, V64)
        dmg = A64[..., :n] * np.linalg.norm(vq[:, :, None, :] - V64[:, None, :n, :], axis=-1)
        np.testing.assert_allclose(s, dmg, rtol=5e-5, atol=1e-7)


# ---- the _bf16 ladder against its float64 definition -------------------------------------
# The production recipe (restore_swap_iter5_bf16_trackbest) rounds the k-wide tensors to
# bf16 at the reference's points (projected.py:763-783, 868-878). test_bf16_ladder_on_exact_sums
# pins where the roundings sit; these pin how far they may move the result: every quantity
# the cut and the objective rank by stays within a rounding bound of its float64 definition
# on the same bf16 inputs (P, V and M rounded to bf16, as the recipe casts them), and the cut
# keeps the float64 top-nts wherever the ranking margin at the threshold exceeds the bounds.
_U = 2.0 ** -8  # bf16 unit roundoff (8 significand bits, round to nearest)


def _bf(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).double().numpy()


def _ladder_bounds(A, V, M, n):
    """float64 s (and the cut key) on the bf16 inputs, and per-candidate bounds. With
    m = Mb vq, mk = Mb V_k and e = vq - V_k, the ladder's roundings move the expanded
    quadratic form term_q - 2 cross + term_k by at most u times: 2 sum|vq_i (Mb e)_i|
    (v_bar_query itself), 2 sum|m_i vq_i| + |term_q| (M vq, the products, their sum),
    2 (sum|m_i V_ki| + |cross|) (M vq, the cross sum), 2 sum|mk_i V_ki| + |term_k| (the key
    side), |term_q - 2 cross| + |quad| (the two additions); 1.25 of that covers the fp32 sums.
    |sqrt a - sqrt b| <= min(sqrt |a - b|, |a - b| / sqrt b) carries it through the root, and
    the last roundings (sqrt, P * sqrt, s / (1 - P)) add a few u relative."""
    Pb, Vb, Mb = _bf(A), _bf(V), _bf(M)
    vq = np.einsum("hqk,hkd->hqd", Pb, Vb)
    Vn = Vb[:, :n]
    m = np.einsum("hij,hqj->hqi", Mb, vq)
    mk = np.einsum("hij,hkj->hki", Mb, Vn)
    tq = np.einsum("hqi,hqi->hq", m, vq)[..., None]
    cr = np.einsum("hqi,hki->hqk", m, Vn)
    tk = np.einsum("hki,hki->hk", mk, Vn)[:, None, :]
    quad_raw = tq - 2 * cr + tk
    quad = np.maximum(quad_raw, 0.0)
    me = m[:, :, None, :] - mk[:, None, :, :]                      # Mb e_k
    d = (2 * np.einsum("hqi,hqki->hqk", np.abs(vq), np.abs(me))
         + 2 * np.einsum("hqi,hqi->hq", np.abs(m), np.abs(vq))[..., None] + np.abs(tq)
         + 2 * (np.einsum("hqi,hki->hqk", np.abs(m), np.abs(Vn)) + np.abs(cr))
         + 2 * np.einsum("hki,hki->hk", np.abs(mk), np.abs(Vn))[:, None, :] + np.abs(tk)
         + np.abs(tq - 2 * cr) + quad)
    dq = 1.25 * _U * d
    p = Pb[..., :n]
    s64 = p * np.sqrt(quad)
    tol_s = p * np.minimum(np.sqrt(dq), dq / np.maximum(np.sqrt(quad), 1e-300)) + 4 * _U * s64
    om = np.maximum(1.0 - p, 1e-4)
    return s64, tol_s, s64 / om, tol_s / om + 3 * _U * s64 / om


def _flat_problem(seed, H=2, q_blk=4, kb_p=48):
    """Softmax rows with logits of scale 0.3: v_bar_query is a broad average, well away from
    every V_k, so the expanded form's terms do not cancel and the bounds are informative."""
    rng = np.random.default_rng(seed)
    logits = rng.normal(size=(H, q_blk, kb_p)) * 0.3
    A = np.exp(logits)
    A = (A / A.sum(-1, keepdims=True)).astype(np.float32)
    V = rng.normal(size=(H, kb_p, 64)).astype(np.float32)
    W = (rng.normal(size=(H, 64, 64)) / 8).astype(np.float32)
    M = np.einsum("hji,hjk->hik", W, W).astype(np.float32)
    return A, V, M, kb_p - 2


def test_bf16_scores_within_rounding_bound_of_float64():
    for seed in range(6):
        for A, V, M, n in (_softmax_problem(700 + seed, H=2, q_blk=4, kb_p=48), _flat_problem(750 + seed)):
            s, scut, _, _, _ = oracle.rs_probe(A, V, M, np.zeros(A.shape[:2] + (n,), bool), n, big_bf16=True)
            s64, tol_s, c64, tol_c = _ladder_bounds(A, V, M, n)
            assert (np.abs(s.astype(np.float64) - s64) <= tol_s).all(), seed
            assert (np.abs(scut.astype(np.float64) - c64) <= tol_c).all(), seed
        # on the flat rows the bound is informative: a few percent of s
        assert np.median(tol_s / np.maximum(s64, 1e-30)) < 0.05


def test_bf16_cut_keeps_float64_top_where_margin_exceeds_bound():
    decided = 0
    for seed in range(8):
        A, V, M, n = _flat_problem(800 + seed, H=4, q_blk=8, kb_p=12)
        H, Q = A.shape[:2]
        rng = np.random.default_rng(seed)
        nts = rng.integers(2, n, size=(H, Q)).astype(np.int32)
        keep, _ = oracle.restore_swap(A, V, M, nts, n, n_iters=0, big_bf16=True, track_best=False)
        _, _, c64, tol_c = _ladder_bounds(A, V, M, n)
        for h in range(H):
            for q in range(Q):
                order = np.argsort(-c64[h, q], kind="stable")
                m = int(nts[h, q])
                lo, hi = order[m - 1], order[m]   # the last kept, the first dropped (float64)
                if c64[h, q, lo] - tol_c[h, q, lo] > c64[h, q, hi] + tol_c[h, q, hi]:
                    want = np.zeros(n, bool)
                    want[order[:m]] = True
                    assert np.array_equal(keep[h, q].astype(bool), want), (seed, h, q)
                    decided += 1
    assert decided >= 40  # most rows have a margin above the bound


def test_bf16_objective_within_rounding_bound_of_float64():
    """J = ||g||^2_M / K^2 of the cut's drop set, the _bf16 ladder (bf16 sum_Pd, Pd @ v_bar and
    v_bar_query; fp32 M) against the float64 J on the same bf16 P and V. g = sum_Pd vq - Pd @ V
    moves by |dg_i| <= u (2.5 sum_Pd |vq_i| + 1.25 |(Pd @ V)_i|) (the three roundings and the
    fp32 sums), so g^T M g moves by at most 2 |dg|^T |M g| + |dg|^T |M| |dg|."""
    for seed in range(6):
        A, V, M, n = _flat_problem(900 + seed)
        H, Q = A.shape[:2]
        nts = np.full((H, Q), n // 2, np.int32)
        keep, _ = oracle.restore_swap(A, V, M, nts, n, n_iters=0, big_bf16=True, track_best=False)
        drop = ~keep.astype(bool)
        _, _, J, _, _ = oracle.rs_probe(A, V, M, drop, n, big_bf16=True)
        Pb, Vb = _bf(A), _bf(V)
        M64 = M.astype(np.float64)
        vq = np.einsum("hqk,hkd->hqd", Pb, Vb)
        Pd = Pb[..., :n] * drop
        g = Pd.sum(-1)[..., None] * vq - np.einsum("hqk,hkd->hqd", Pd, Vb[:, :n])
        K = Pb.sum(-1) - Pd.sum(-1)
        J64 = np.einsum("hqi,hij,hqj->hq", g, M64, g) / K ** 2
        mv = np.einsum("hqk,hkd->hqd", Pd, Vb[:, :n])
        gabs = _U * (2.5 * Pd.sum(-1)[..., None] * np.abs(vq) + 1.25 * np.abs(mv))
        Mg = np.einsum("hij,hqj->hqi", M64, g)
        dG = 2 * np.einsum("hqi,hqi->hq", gabs, np.abs(Mg)) + np.einsum("hqi,hij,hqj->hq", gabs, np.abs(M64), gabs)
        tol = dG / K ** 2 + 4 * _U * J64 + 1e-30
        assert (np.abs(J.astype(np.float64) - J64) <= tol).all(), seed
        assert np.median(tol / np.maximum(J64, 1e-30)) < 0.2
