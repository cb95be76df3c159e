"""Pins the C oracle (oracle/ress_oracle.c) to the mathematics and to the reference's own
torch expressions. CPU only."""

import math

import numpy as np
import pytest
import torch

import oracle
from oracle import reference as ref
from ress_amd import synth
from ress_amd.kernels import LayerGrid


def _ulp_diff(a, b):
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


# ---------------------------------------------------------------- exp

def test_expf_within_one_ulp_of_libm():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-103.0, 88.5, 200_000), rng.uniform(-1, 1, 50_000),
                        np.linspace(-87.5, -86.5, 10_000)]).astype(np.float32)
    y = oracle.expf_array(x)
    exact = np.array([math.exp(float(v)) for v in x], dtype=np.float64)
    normal = exact >= 1.1754943508222875e-38
    d = _ulp_diff(y[normal], exact[normal].astype(np.float32))
    assert d.max() <= 1, d.max()
    # subnormal results: absolute error within one subnormal step
    assert np.all(np.abs(y[~normal].astype(np.float64) - exact[~normal]) <= 2 ** -149)


def test_expf_special_values():
    assert oracle.expf(0.0) == 1.0
    assert oracle.expf(-np.inf) == 0.0
    assert np.isinf(oracle.expf(np.inf)) and oracle.expf(np.inf) > 0
    assert np.isnan(oracle.expf(np.nan))
    assert oracle.expf(-104.0) == 0.0
    assert np.isinf(oracle.expf(89.0))


def test_round_bf16_matches_torch():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(100_000) * np.exp(rng.uniform(-20, 20, 100_000))).astype(np.float32)
    x[:4] = [0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8]  # ties to even
    y = oracle.round_bf16_array(x)
    t = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(y.view(np.uint32), t.view(np.uint32))


# ---------------------------------------------------------------- geometry

@pytest.mark.parametrize("F,q_blk,n_cand,kb_p,kb_tot,sink,topk,sr", [
    (4, 43, 85, 86, 86, 1, 42, 0.5),
    (16, 172, 342, 343, 344, 2, 102, 0.7),
    (32, 343, 684, 685, 687, 3, 136, 0.8),
    (200, 2140, 4278, 4279, 4294, 16, 427, 0.9),
])
def test_grid_matches_survey_table(F, q_blk, n_cand, kb_p, kb_tot, sink, topk, sr):
    g = LayerGrid(1, 16, F, 1374, 5)
    assert (g.q_blk_p, g.n_cand, g.kb_p, g.kb_tot, g.sink_blocks) == (q_blk, n_cand, kb_p, kb_tot, sink)
    assert int(g.n_cand * (1 - sr)) == topk  # Python double product, then truncation


def test_sink_protect_off_uses_ceil():
    g = LayerGrid(1, 16, 16, 1374, 5, sink_protect=False)
    assert g.n_cand == 343 and g.sink_blocks == 1
    g0 = LayerGrid(1, 16, 1, 1024, 0)
    assert g0.n_cand == 16 and g0.sink_blocks == 0


# ---------------------------------------------------------------- preparation

def _rand_bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


@pytest.fixture(scope="module")
def small_layer():
    frames, P, S = 3, 203, 5  # T_p = 594 (partial q and k blocks), T_s = 15
    B, H = 1, 2
    q = _rand_bf16((B, H, frames * P, 64), 1)
    k = _rand_bf16((B, H, frames * P, 64), 2)
    v = _rand_bf16((B, H, frames * P, 64), 3)
    return q, k, v, frames, P, S, oracle.prep_qkv(q, k, v, frames, P, S)


def test_pooling_matches_torch_avg_pool(small_layer):
    q, k, v, frames, P, S, o = small_layer
    qp, _ = ref.split_tokens(q.float(), frames, P, S)
    kp, _ = ref.split_tokens(k.float(), frames, P, S)
    vp, _ = ref.split_tokens(v.float(), frames, P, S)
    for x, pooled, ks in ((qp, o["pooled_q"], 128), (kp, o["pooled_k"], 64), (vp, o["pooled_v"], 64)):
        t = torch.nn.functional.avg_pool1d(x[0].transpose(-1, -2), ks, ceil_mode=True).transpose(-1, -2)
        np.testing.assert_allclose(pooled, t.numpy(), rtol=0, atol=2e-6)
        # partial last block divides by its valid count: fp64 check
        T = x.shape[2]
        last = x[0, :, (T - 1) // ks * ks:].double().mean(dim=1).numpy()
        np.testing.assert_allclose(pooled[:, -1], last, rtol=0, atol=2e-6)



def test_sink_mass_pooling_covers_every_key(small_layer):
    """pool_all (the sink-mass grid, reference attention.py:451-452, 481): K and V pooled
    over cat(patch, special) in kernel order, kb_tot blocks, the block straddling the patch
    tail and the first special keys mixing both; the other outputs do not change."""
    q, k, v, frames, P, S, o = small_layer
    om = oracle.prep_qkv(q, k, v, frames, P, S, pool_all=True)
    g = LayerGrid(1, 2, frames, P, S, sink_mass=True)
    assert om["pooled_k"].shape == (2, g.kb_tot, 64) and g.kb_p == g.kb_tot
    for x, pooled in ((k, om["pooled_k"]), (v, om["pooled_v"])):
        xp, xs = ref.split_tokens(x.float(), frames, P, S)
        key = torch.cat([xp, xs], dim=2)[0]
        t = torch.nn.functional.avg_pool1d(key.transpose(-1, -2), 64, ceil_mode=True).transpose(-1, -2)
        np.testing.assert_allclose(pooled, t.numpy(), rtol=0, atol=2e-6)
        T_p = xp.shape[2]
        b = T_p // 64  # the straddling block: patch tail and leading special keys together
        mixed = key[:, b * 64:b * 64 + 64].double().mean(dim=1).numpy()
        np.testing.assert_allclose(pooled[:, b], mixed, rtol=0, atol=2e-6)
    for name in ("q_i8", "q_scale", "pooled_q", "k_i8", "k_scale", "v_pack", "ksum", "km"):
        assert np.array_equal(om[name], o[name]), name
    # the patch-only grid is the leading kb_p blocks where no block straddles
    n_whole = (frames * (P - S)) // 64
    np.testing.assert_array_equal(om["pooled_k"][:, :n_whole], o["pooled_k"][:, :n_whole])

def _sage_quant(x, scale):
    """SageAttention per-block rule, vectorised numpy fp32."""
    x = x.astype(np.float32)
    if scale == 0:
        return np.zeros(x.shape, np.int8)
    y = (x / np.float32(scale)).astype(np.float32)
    y = (y + np.where(y >= 0, np.float32(0.5), np.float32(-0.5))).astype(np.float32)
    return np.trunc(y).astype(np.int8)


def test_quantisation_rule_and_roundtrip(small_layer):
    q, k, v, frames, P, S, o = small_layer
    qp, qs = ref.split_tokens(q.float(), frames, P, S)
    T_p, T_s = qp.shape[2], qs.shape[2]
    BH = 2
    qbp = -(-T_p // 128)
    for bh in range(BH):
        for qb in range(o["q_scale"].shape[1]):
            if qb < qbp:
                x = qp[0, bh, qb * 128:min(T_p, qb * 128 + 128)].numpy()
            else:
                r0 = (qb - qbp) * 128
                x = qs[0, bh, r0:min(T_s, r0 + 128)].numpy()
            scale = o["q_scale"][bh, qb]
            assert scale == np.float32(np.abs(x).max()) / np.float32(127)
            codes = o["q_i8"][bh, qb, :x.shape[0]]
            assert np.array_equal(codes, _sage_quant(x, scale))
            assert np.abs(codes).max() == 127
            assert np.all(np.abs(x - scale * codes.astype(np.float32)) <= scale * 0.5 * (1 + 1e-5))
            assert np.all(o["q_i8"][bh, qb, x.shape[0]:] == 0)
    # K: smoothed by the key mean over all keys (patch then special)
    kp, ks = ref.split_tokens(k.float(), frames, P, S)
    key = torch.cat([kp, ks], dim=-2)[0].numpy()
    km = key.astype(np.float64).mean(axis=1)
    np.testing.assert_allclose(o["km"], km, rtol=0, atol=1e-6)
    for bh in range(BH):
        for kb in range(o["k_scale"].shape[1]):
            x = key[bh, kb * 64:kb * 64 + 64] - o["km"][bh]
            scale = o["k_scale"][bh, kb]
            assert scale == np.float32(np.abs(x).max()) / np.float32(127)
            assert np.array_equal(o["k_i8"][bh, kb, :x.shape[0]], _sage_quant(x, scale))


def test_split_codes_bound_the_residual(small_layer):
    q, k, v, frames, P, S, o = small_layer
    for hi, lo, sc in ((o["q_i8"], o["q_lo"], o["q_scale"]), (o["k_i8"], o["k_lo"], o["k_scale"])):
        assert np.abs(lo.astype(np.int32)).max() <= 127
    qp, _ = ref.split_tokens(q.float(), frames, P, S)
    x = qp[0, 0, :128].numpy()
    s = o["q_scale"][0, 0]
    approx = s * o["q_i8"][0, 0].astype(np.float64) + (s / 254) * o["q_lo"][0, 0].astype(np.float64)
    err = np.abs(x - approx)
    assert err.max() <= s / 508 * 1.001 + 1e-12
    # the two-term code is ~254x finer than the single term
    assert err.max() < np.abs(x - s * o["q_i8"][0, 0]).max() / 100


def test_zero_block_quantises_to_zero():
    q = torch.zeros(1, 1, 256, 64, dtype=torch.bfloat16)
    k = _rand_bf16((1, 1, 256, 64), 5)
    o = oracle.prep_qkv(q, k, k, 1, 256, 0)
    assert np.all(o["q_scale"] == 0) and np.all(o["q_i8"] == 0)


def test_v_pack_permutation(small_layer):
    q, k, v, frames, P, S, o = small_layer
    vp_, vs_ = ref.split_tokens(v, frames, P, S)
    val = torch.cat([vp_, vs_], dim=-2)[0].contiguous().view(torch.int16).numpy().view(np.uint16)
    Tk = val.shape[1]
    for kb in (0, o["v_pack"].shape[1] - 1):
        blk = o["v_pack"][1, kb].reshape(64, 64)  # [dim][pos]
        for t in range(64):
            u = t % 16
            pos = (t // 16) * 16 + [0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15].index(u)
            want = val[1, kb * 64 + t] if kb * 64 + t < Tk else np.zeros(64, np.uint16)
            assert np.array_equal(blk[:, pos], want)


# ---------------------------------------------------------------- pooled map

def test_pooled_scores_match_reference_formula():
    q, k, v, meta = synth.make_layer_qkv(2, H=4)
    frames, P, S = meta["frames"], meta["P"], meta["S"]
    o = oracle.prep_qkv(q, k, v, frames, P, S)
    g = LayerGrid(1, 4, frames, P, S)
    full, cond = oracle.pooled_scores(o["pooled_q"], o["pooled_k"], g.n_cand)
    qp, _ = ref.split_tokens(q, frames, P, S)
    kp, _ = ref.split_tokens(k, frames, P, S)
    t = ref.predict_attention_torch(qp, kp)[0].numpy()
    np.testing.assert_allclose(full, t, rtol=2e-5, atol=1e-8)
    # fp64 restatement
    pq, pk = o["pooled_q"].astype(np.float64), o["pooled_k"].astype(np.float64)
    s = np.einsum("hqd,hkd->hqk", pq, pk) / 8.0
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(full, p, rtol=1e-5, atol=1e-9)
    c = p[..., :g.n_cand] / np.maximum(p[..., :g.n_cand].sum(-1, keepdims=True), 1e-6)
    np.testing.assert_allclose(cond, c, rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(cond.sum(-1), 1.0, atol=2e-6)


# ---------------------------------------------------------------- budgets

def test_baseline_budget_definition():
    rng = np.random.default_rng(3)
    a = rng.dirichlet(np.full(97, 0.3), size=(2, 5, 11)).astype(np.float32)
    a[0, 0, 0] = np.float32(1.0 / 97)  # uniform row: many ties
    for sr, cdf in ((0.5, 0.9), (None, 0.9), (0.7, None), (0.3, 0.5), (None, 0.999)):
        got = oracle.baseline_budget(a, sr, cdf)
        want = np.zeros(a.shape[:-1], np.int64)
        for idx in np.ndindex(a.shape[:-1]):
            n = -1
            if cdf is not None:
                c = np.cumsum(np.sort(a[idx])[::-1].astype(np.float32), dtype=np.float32)
                thr = np.float32(np.float32(cdf) + np.float32(1e-5))
                n = int(np.searchsorted(c, thr, side="right"))
            if sr is not None:
                n = max(n, int(97 * (1 - sr)))
            want[idx] = n
        assert np.array_equal(got, want), (sr, cdf)
        # vs the torch expression (which accumulates its CPU cumsum in double): counts
        # may only differ where a prefix sum lies within rounding of the threshold
        tt = ref.baseline_torch(torch.from_numpy(a), sr, cdf).numpy()
        for idx in zip(*np.nonzero(tt != got)):
            c64 = np.cumsum(np.sort(a[idx].astype(np.float64))[::-1])
            assert np.min(np.abs(c64 - (cdf + 1e-5))) < 1e-6


def test_head_budget_closed_form_without_caps():
    rng = np.random.default_rng(4)
    base = rng.integers(20, 40, size=(1, 16, 9)).astype(np.int32)
    scores = oracle.scores_norm_seq(rng.uniform(0.5, 1.5, 16).astype(np.float32))
    out, it = oracle.head_budget(base, scores, 1.0, 1000)
    total = base.sum(axis=1)[0].astype(np.float32)
    want = np.floor((scores[:, None] * total[None, :]).astype(np.float32)).astype(np.int32)
    assert it == 0 and np.array_equal(out[0], want)


def test_head_budget_matches_reference_expression_on_exact_sums():
    # dyadic scores and integer budgets keep every head sum exact, so the reference's
    # torch expression (any summation order) and the oracle agree bit for bit
    rng = np.random.default_rng(5)
    for trial in range(20):
        raw = rng.integers(1, 64, size=16).astype(np.float32)
        raw[rng.integers(0, 16)] = 600.0  # one dominant head -> caps and redistribution
        base = rng.integers(0, 60, size=(1, 16, 7)).astype(np.int32)
        max_val = int(rng.integers(40, 90))
        sn = oracle.scores_norm_seq(raw)
        got, it = oracle.head_budget(base, sn, 1.0, max_val)
        want = ref.adjust_attention_selection_torch(torch.from_numpy(base).long(), torch.from_numpy(raw), 1.0,
                                                    max_val).numpy()
        assert it >= 0
        assert np.array_equal(got, want), trial
        assert got.max() <= max_val
        assert np.all(got.sum(axis=1) <= base.sum(axis=1))


def test_head_budget_degenerate_scores_fall_back_to_uniform():
    base = np.full((1, 16, 3), 10, np.int32)
    sn = oracle.scores_norm_seq(np.zeros(16, np.float32))
    assert np.all(sn == np.float32(1.0 / 16))
    out, _ = oracle.head_budget(base, sn, 1.0, 100)
    assert np.all(out == 10)
    sn = oracle.scores_norm_seq(np.full(16, np.nan, np.float32))
    assert np.all(sn == np.float32(1.0 / 16))


def test_head_budget_reports_non_convergence():
    base = np.full((1, 4, 1), 50, np.int32)
    sn = oracle.scores_norm_seq(np.array([8, 1, 1, 1], np.float32))
    _, it = oracle.head_budget(base, sn, 1.0, 60, max_iters=1)
    assert it == -1
    _, it = oracle.head_budget(base, sn, 1.0, 60, max_iters=1000)
    assert it > 0


def test_head_budget_floor_and_beta():
    base = np.array([[[1], [0], [5], [2]]], np.int32)
    out, _ = oracle.head_budget(base, None, 1.0, 10, min_select=2)
    assert out[0, :, 0].tolist() == [2, 2, 5, 2]
    sn = oracle.scores_norm_seq(np.array([1, 1, 1, 1], np.float32))
    out, _ = oracle.head_budget(base, sn, 0.0, 10)  # beta 0: unchanged
    assert out[0, :, 0].tolist() == [1, 0, 5, 2]


# ---------------------------------------------------------------- selection

def test_select_matches_bruteforce_with_ties():
    rng = np.random.default_rng(6)
    BH, q, n_cand, kb_tot = 3, 9, 70, 73
    keys = rng.integers(0, 6, size=(BH, q, n_cand)).astype(np.float32)  # heavy ties
    keys[0, 0] = 0.0
    keys[1, 1, ::2] = -0.0  # -0 ties with +0
    counts = rng.integers(-3, n_cand + 5, size=(BH, q)).astype(np.int32)
    counts[0, :4] = [0, 1, n_cand, n_cand + 5]
    fmap, lut, nvalid = oracle.select_blocks(keys, counts, q + 1, kb_tot, min_select=2)
    want = ref.rank_select_numpy(keys, counts, kb_tot, min_select=2)
    assert np.array_equal(fmap, want)
    for b in range(BH):
        for r in range(q):
            kept = np.nonzero(want[b, r])[0]
            assert nvalid[b, r] == kept.size and np.array_equal(lut[b, r, :kept.size], kept)
        assert nvalid[b, q] == kb_tot and np.array_equal(lut[b, q], np.arange(kb_tot))  # dense row


def test_select_leading_sink():
    keys = np.linspace(0, 1, 40, dtype=np.float32)[None, None]  # ascending: top are the last
    fmap, lut, nv = oracle.select_blocks(keys, np.array([[3]], np.int32), 1, 40, sink_lead=5)
    assert np.nonzero(fmap[0, 0])[0].tolist() == [0, 1, 2, 3, 4, 37, 38, 39]


# ---------------------------------------------------------------- generator

def test_hilbert_order_is_a_bijection_with_unit_steps():
    for w, h in ((37, 37), (8, 8), (12, 5), (5, 12), (1, 7)):
        cells = synth.gilbert_order(w, h)
        assert len(cells) == w * h and len(set(cells)) == w * h
        steps = [abs(a[0] - b[0]) + abs(a[1] - b[1]) for a, b in zip(cells, cells[1:])]
        assert max(steps) <= 2 and sum(s > 1 for s in steps) <= 1
        if w % 2 == 0 and h % 2 == 0:
            assert max(steps) == 1
    assert synth.gilbert_order(37, 37)[0] == (0, 0)


def test_hilbert_order_matches_reference_vectors():
    """The curve equals the reference's own (src/ress/models/hilbert.py gilbert2d and
    make_hilbert_gather_idx), cell for cell, on the 37x37 patch grid and two odd rectangles:
    vectors written by tests/golden/make_hilbert_orders.py. The gather table the kernels read
    in place (patch_order: kernel patch j = storage patch perm[j]) is the reference's
    forward gather, and its inverse is the reference's inverse gather."""
    import json
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hilbert_orders.json")
    grids = json.load(open(path))["grids"]
    assert [(g["width"], g["height"]) for g in grids] == [(37, 37), (13, 11), (23, 7)]
    for g in grids:
        w, h = g["width"], g["height"]
        assert [list(c) for c in synth.gilbert_order(w, h)] == g["cells"]
        perm = synth.hilbert_permutation(w, h)
        assert perm.tolist() == g["gather"]
        inv = np.empty_like(perm)
        inv[perm] = np.arange(w * h)
        assert inv.tolist() == g["gather_inverse"]


def test_generator_is_deterministic_and_shaped():
    q1, k1, v1, m = synth.make_layer_qkv(2, H=2)
    q2, _, _, _ = synth.make_layer_qkv(2, H=2)
    assert q1.shape == (1, 2, 2 * 1374, 64) and q1.dtype == torch.bfloat16
    assert torch.equal(q1.view(torch.int16), q2.view(torch.int16))
    assert m == {"frames": 2, "P": 1374, "S": 5}
    cam, pc = synth.make_hess_tables()
    assert cam.shape == (3, 24, 16) and torch.all(cam > 0)


def test_reciprocal_quantiser_fast_path_is_exact():
    """The kernels quantise with x * (1/scale) and fall back to the division x / scale when
    |y| + 0.5 has a fraction within 2^-12 of an integer (common.h quant_i8_rcp, and the
    equivalent form of quant_i8x8_rcp). In float32 (numpy, round to nearest like the GPU),
    the fast path's code equals the division's on random blocks and on values placed at and
    around every half-integer boundary, and both forms trust the same elements."""
    rng = np.random.default_rng(3)
    f32 = np.float32

    def exact(x, s):
        y = (x / s).astype(f32)
        y = (y + np.where(y >= 0, f32(0.5), f32(-0.5))).astype(f32)
        return np.trunc(y).astype(np.int64)

    def fast(x, s):
        r = (f32(1.0) / s).astype(f32)
        y = (x * r).astype(f32)
        a = (np.abs(y) + f32(0.5)).astype(f32)
        f = (a - np.floor(a)).astype(f32)
        ok = (f > f32(2.0 ** -12)) & (f < f32(1.0) - f32(2.0 ** -12))
        m = np.trunc(a).astype(np.int64)
        return np.where(ok, np.where(y >= 0, m, -m), exact(x, s)), ok

    def fast8(x, s):
        """quant_i8x8_rcp's form: a = y + copysign(0.5, y) (sign(y) * (|y| + 0.5), the same
        rounding), the fraction of |a| tested as |f - 0.5| < 0.5 - 2^-12, the code trunc(a)."""
        r = (f32(1.0) / s).astype(f32)
        y = (x * r).astype(f32)
        a = (y + np.copysign(f32(0.5), y)).astype(f32)
        aa = np.abs(a)
        f = (aa - np.floor(aa)).astype(f32)
        ok = np.abs((f - f32(0.5)).astype(f32)) < f32(0.5) - f32(2.0 ** -12)
        return np.where(ok, np.trunc(a).astype(np.int64), exact(x, s)), ok

    for trial in range(200):
        x = (rng.standard_normal(4096) * 10.0 ** rng.uniform(-6, 4)).astype(f32)
        s = f32(np.abs(x).max() / f32(127.0))
        got, ok = fast(x, s)
        assert np.array_equal(got, exact(x, s))
        got8, ok8 = fast8(x, s)
        assert np.array_equal(got8, exact(x, s)) and np.array_equal(ok8, ok)
    # adversarial: x just around (k + 1/2) * s for every k, a few ulps either side
    for s in (f32(0.0137), f32(3.3e-5), f32(1.0), f32(7.77)):
        k = np.arange(-127, 128, dtype=f32)
        base = ((k + f32(0.5)) * s).astype(f32)
        xs = [base]
        for n in range(1, 6):
            xs.append(np.nextafter(base, np.inf, dtype=f32))
            xs.append(np.nextafter(base, -np.inf, dtype=f32))
            base = xs[-2]
        x = np.concatenate(xs)
        got, ok = fast(x, s)
        assert np.array_equal(got, exact(x, s))
        assert not ok.all()  # the boundary values do take the division
        got8, ok8 = fast8(x, s)
        assert np.array_equal(got8, exact(x, s)) and np.array_equal(ok8, ok)
