"""Host-side API, no GPU: the restore-swap criterion grammar, wiring and mode switching on a
fake model, the calibration tables and HeSS lambda mixing, the leading attention sink,
the deferred HeSS convergence check and the random criterion's generator.

References: src/ress/scoring/criterion.py:3-7,96-124 (grammar), src/ress/models/wiring.py
:49-109 and src/ress/runtime/static.py:20-77 (wiring, resets), src/ress/api.py:60-144 and
src/ress/budget/hess.py:46-100 (budgets, tables, lambda), external/patches/
spargeattn.patch:61-65 (sink), src/ress/budget/_proportional.py:112-113 (convergence),
src/ress/models/attention.py:177-196 (random criterion)."""

import itertools
import math
import os

import numpy as np
import pytest
import torch
import torch.nn as nn
from hypothesis import given, settings
from hypothesis import strategies as st

import ress_amd as ress
from ress_amd import attention, backbones, budget, criterion, static, wiring
from ress_amd.criterion import RestoreSwapSpec, is_restore_swap, parse_restore_swap
from ress_amd.kernels import LayerGrid

# ---- criterion grammar --------------------------------------------------------------------

KNOWN = {
    # the published recipe (api.py:44)
    "restore_swap_iter5_bf16_trackbest": dict(n_iters=5, big_dtype=torch.bfloat16, track_best=True),
    "restore_swap": dict(),
    "restore_swap_iter1": dict(n_iters=1),
    "restore_swap_iter12": dict(n_iters=12),
    "damage_restore_swap_iter3": dict(n_iters=3, use_wo=False),
    "restore_swap_iter5_nowo": dict(n_iters=5, use_wo=False),
    "damage_restore_swap_wo": dict(use_wo=True),
    "restore_swap_rf30_dc25": dict(restore_frac=0.30, decay=0.25),
    "restore_swap_iter5_bf16_trackbest_antiswap": dict(n_iters=5, big_dtype=torch.bfloat16, track_best=True,
                                                       maximize=True),
    "restore_swap_iter5_bf16_trackbest_anti": dict(n_iters=5, big_dtype=torch.bfloat16, track_best=True,
                                                   maximize=True, invert_cut=True),
    "restore_swap_trackbest_iter5": None,   # iter is part of the base, not a suffix
    "restore_swap_iter": None,
    "restore_swap_rf": None,
    "restore_swap_xyz": None,
    "damage_damage_restore_swap": None,
    "restore__swap": None,
    "restore_swap__bf16": None,
    "probability": None,
    "random": None,
    "projected": None,
    "": None,
}


@pytest.mark.parametrize("name", list(KNOWN))
def test_criterion_known_names(name):
    want = KNOWN[name]
    if want is None:
        assert not is_restore_swap(name)
        with pytest.raises(ValueError):
            parse_restore_swap(name)
        return
    assert is_restore_swap(name)
    got = parse_restore_swap(name)
    exp = RestoreSwapSpec(**want)
    assert got == exp, (got, exp)


def test_criterion_leftmost_suffix_wins():
    """Conflicting suffixes: the leftmost setter of a field decides (suffixes are read off the
    end of the name, each overriding the ones read before it)."""
    assert parse_restore_swap("restore_swap_nowo_wo").use_wo is False
    assert parse_restore_swap("restore_swap_wo_nowo").use_wo is True
    assert parse_restore_swap("damage_restore_swap_wo_nowo").use_wo is True
    assert parse_restore_swap("restore_swap_rf10_rf90").restore_frac == pytest.approx(0.10)
    assert parse_restore_swap("restore_swap_dc75_dc20").decay == pytest.approx(0.75)


_FLAGS = ["bf16", "trackbest", "antiswap", "rf40", "dc30"]


@settings(max_examples=200, deadline=None)
@given(st.lists(st.sampled_from(_FLAGS), unique=True), st.one_of(st.none(), st.integers(0, 99)),
       st.booleans(), st.randoms())
def test_criterion_suffix_order_is_irrelevant(suffixes, iters, damage, rnd):
    """Non-conflicting suffixes in any order name the same spec, and each sets exactly its
    field."""
    base = ("damage_" if damage else "") + "restore_swap" + ("" if iters is None else f"_iter{iters}")
    perm = list(suffixes)
    rnd.shuffle(perm)
    a = parse_restore_swap("_".join([base] + suffixes))
    b = parse_restore_swap("_".join([base] + perm))
    assert a == b
    assert a.n_iters == (1 if iters is None else iters)
    assert a.use_wo is (not damage)
    assert (a.big_dtype == torch.bfloat16) == ("bf16" in suffixes)
    assert a.track_best == ("trackbest" in suffixes)
    assert a.maximize == ("antiswap" in suffixes) and a.invert_cut is False
    assert a.restore_frac == (0.40 if "rf40" in suffixes else 0.5)
    assert a.decay == (0.30 if "dc30" in suffixes else 0.5)


@settings(max_examples=200, deadline=None)
@given(st.text(alphabet="abdegimnoprstuvwxy_0123456789", max_size=40))
def test_criterion_rejects_or_parses_consistently(name):
    """is_restore_swap and parse_restore_swap agree on every string."""
    if is_restore_swap(name):
        assert isinstance(parse_restore_swap(name), RestoreSwapSpec)
    else:
        with pytest.raises(ValueError):
            parse_restore_swap(name)


# ---- wiring and mode switching on a fake model -------------------------------------------

class _FakeAttn(nn.Module):
    def __init__(self, dim=128, heads=2):
        super().__init__()
        self.num_heads = heads
        self.proj = nn.Linear(dim, dim)

    def forward(self, x, pos=None):  # replaced by wiring
        raise AssertionError("not wired")


class _FakeBlock(nn.Module):
    def __init__(self):
        super().__init__()
        self.attn = _FakeAttn()


class _FakeModel(nn.Module):
    def __init__(self, n=3):
        super().__init__()
        self.blocks = nn.ModuleList(_FakeBlock() for _ in range(n))


def _wired(n=3):
    m = _FakeModel(n)
    wiring.wire_ress_attention(m, m.blocks)
    return m


def test_wiring_installs_forward_and_reads_config(monkeypatch):
    m = _wired()
    assert wiring.global_blocks(m) == list(m.blocks)
    assert wiring.global_attns(m) == [b.attn for b in m.blocks]
    calls = []

    def fake_forward(attn, x, pos, **kw):
        calls.append((attn, x, pos, kw))
        return x

    monkeypatch.setattr(wiring, "ress_attention_forward", fake_forward)
    a = m.blocks[1].attn
    a.block_criterion = "restore_swap_iter5"
    a.attention_sink = 1374
    x = torch.zeros(1, 4, 128)
    assert a(x, xpos="P") is x                     # Pi3 spelling of the positions
    attn, _, pos, kw = calls[-1]
    assert attn is a and pos == "P"
    assert kw["block_criterion"] == "restore_swap_iter5" and kw["attention_sink"] == 1374
    assert kw["num_heads"] == 2 and kw["num_special_tokens"] == 5 and kw["dense"] is False
    a(x, pos="Q", xpos="P")
    assert calls[-1][2] == "Q"                      # pos wins over xpos
    with pytest.raises(AssertionError):
        a(x, pos="Q", attn_mask=torch.ones(1))
    with pytest.raises(AssertionError):
        a(x, pos="Q", attn_bias=torch.ones(1))
    assert set(dict(wiring.CALL_ATTRIBUTES)) <= set(attention.ress_attention_forward.__code__.co_varnames)


def test_set_static_budget_resets_every_knob():
    """Every mode starts from the same knobs (reference static.py:49-66): a joint selector, a
    fixed count, dense or a sink left behind by an earlier mode never survives."""
    m = _wired()

    class Bud:
        def num_to_select(self, layer, attn_pooled, sr, cdf, beta):
            return (layer, sr, cdf, beta)

    for b in m.blocks:
        a = b.attn
        a.dense, a.num_to_select, a.joint_select_fn, a.perhead_budget_fn = True, 7, object(), object()
        a.retain_output_grad, a.attention_sink = True, 99
    static.set_static_budget(m, Bud(), 0.6, 0.9, beta=0.5, block_criterion="random")
    for i, b in enumerate(m.blocks):
        a = b.attn
        assert a.dense is False and a.num_to_select is None and a.joint_select_fn is None
        assert a.perhead_budget_fn is None and a.retain_output_grad is False and a.attention_sink == 0
        assert a.block_criterion == "random" and a.protect_own_frame is False and a.pooled_fallback is False
        assert a.budget_fn("P") == (i, 0.6, 0.9, 0.5)

    class VBud:
        needs_v_bar = True

        def num_to_select(self, layer, attn_pooled, sr, cdf, beta, v_bar=None):
            return (layer, v_bar)

    static.set_static_budget(m, VBud(), 0.6)
    assert m.blocks[2].attn.budget_fn is None
    assert m.blocks[2].attn.perhead_budget_fn("P", "V") == (2, "V")


# ---- calibration tables, HeSS lambda --------------------------------------------------------

def test_calibration_tables_load_weights_only():
    """The package's tables (the six the reference ships, src/ress/calibration/) are plain
    float32 (3, n_global_blocks, n_heads) tensors readable with weights_only=True."""
    for name, spec in backbones.BACKBONES.items():
        for path in spec.calibration_paths():
            assert os.path.exists(path), path
            t = torch.load(path, map_location="cpu", weights_only=True)
            assert t.dtype == torch.float32 and tuple(t.shape) == (3, spec.n_global_blocks, spec.n_heads)
            assert bool(torch.isfinite(t).all()) and bool((t > 0).all())


@pytest.mark.parametrize("name", ["vggt", "pi3", "da3"])
@pytest.mark.parametrize("lam", [0.0, 0.5, 1.0, 0.3])
def test_hess_lambda_mix_closed_form(name, lam):
    """HessBudget(cam, pc, lam).head_scores = sum_normalize(lam*cam + (1-lam)*pc) of the
    per-layer sum-normalised W_Q slices, float64 closed form; lam = 1 is the camera table
    alone and lam = 0 the point-cloud table alone (DA3 and Pi3's settings)."""
    pcd_path, cam_path = backbones.get_backbone(name).calibration_paths()
    hb = budget.HessBudget(cam_path, pcd_path, lam=lam)
    cam = torch.load(cam_path, weights_only=True)[0].double()
    pc = torch.load(pcd_path, weights_only=True)[0].double()
    cam, pc = cam / cam.sum(-1, keepdim=True), pc / pc.sum(-1, keepdim=True)
    mix = lam * cam + (1 - lam) * pc
    want = mix / mix.sum(-1, keepdim=True)
    np.testing.assert_allclose(hb.head_scores.double().numpy(), want.numpy(), rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(hb.head_scores.sum(-1).numpy(), 1.0, rtol=1e-5)
    if lam == 1.0:
        np.testing.assert_allclose(hb.head_scores.double().numpy(), cam.numpy(), rtol=1e-5, atol=1e-9)
    if lam == 0.0:
        np.testing.assert_allclose(hb.head_scores.double().numpy(), pc.numpy(), rtol=1e-5, atol=1e-9)


def test_hess_tables_from_tensors_equal_paths():
    pcd_path, cam_path = backbones.get_backbone("vggt").calibration_paths()
    a = budget.HessBudget(cam_path, pcd_path, lam=0.5)
    b = budget.HessBudget(torch.load(cam_path, weights_only=True), torch.load(pcd_path, weights_only=True), lam=0.5)
    assert torch.equal(a.head_scores, b.head_scores)


def test_apply_modes_pick_tables_and_cache_per_lambda():
    """apply_hess / apply_ress on a tagged model: the backbone's tuned lambda by default, one
    budget per lambda, tables in the reference's (cam, pc) argument order, M baked once."""
    m = _wired(2)
    m._ress_backbone = "pi3"   # 18 x 16 tables; the fake model has 2 global blocks
    ress.apply_hess(m, 0.5)
    st = m._ress_state
    assert list(st.hess) == [0.0]                           # Pi3's hess_lam
    pcd_path, cam_path = backbones.get_backbone("pi3").calibration_paths()
    pc = torch.load(pcd_path, weights_only=True)[0]
    np.testing.assert_allclose(st.hess[0.0].head_scores.numpy(), (pc / pc.sum(-1, keepdim=True)).numpy(), rtol=1e-6)
    M0 = m.blocks[0].attn.M
    assert M0.shape == (2, 64, 64)
    W = m.blocks[0].attn.proj.weight.detach()
    torch.testing.assert_close(M0[1], W[:, 64:].T @ W[:, 64:])
    ress.apply_ress(m, 0.5, n_iters=3, lam=1.0)
    assert sorted(st.hess) == [0.0, 1.0] and m.blocks[0].attn.M is M0
    assert m.blocks[1].attn.block_criterion == "restore_swap_iter3_bf16_trackbest"
    ress.apply_hess(m, 0.5)
    assert m._ress_state is st and len(st.hess) == 2
    ress.apply_sparse_vggt(m, 0.5, 0.9)
    assert m.blocks[0].attn.block_criterion == "probability" and st.uniform is not None
    with pytest.raises(ValueError):
        ress.apply_dense(_wired(1))                          # untagged model


def test_model_tables_override_backbone_files():
    m = _wired(2)
    m._ress_backbone = "vggt"
    cam = torch.rand(3, 24, 16) + 0.1
    pc = torch.rand(3, 24, 16) + 0.1
    m._ress_calibration_tables = (pc, cam)   # (point cloud, camera), like calibration_paths()
    ress.apply_hess(m, 0.5, lam=1.0)
    hb = m._ress_state.hess[1.0]
    torch.testing.assert_close(hb.head_scores, cam[0] / cam[0].sum(-1, keepdim=True))


# ---- attention sink, convergence, random criterion ---------------------------------------

def test_sink_lead_blocks():
    g = LayerGrid(1, 16, 4, 1374, 5)           # 4 frames: n_cand = 85
    assert attention.sink_lead_blocks(0, g) == 0
    assert attention.sink_lead_blocks(1374, g) == 22   # ceil(1374 / 64), the configs' sink
    assert attention.sink_lead_blocks(64, g) == 1 and attention.sink_lead_blocks(65, g) == 2
    assert attention.sink_lead_blocks(10 ** 6, g) == g.n_cand
    with pytest.raises(ValueError):
        attention.sink_lead_blocks(-1, g)


def test_layer_result_raises_on_unconverged_budget():
    fmap = torch.ones(1, 2, 3, 4, dtype=torch.uint8)
    ok = attention.LayerResult(out=None, final_map=fmap, unconverged=torch.tensor(0, dtype=torch.int32),
                               max_iters=1000)
    assert ok.sparsity() == 0.0
    ok.check()
    bad = attention.LayerResult(out=None, final_map=fmap, unconverged=torch.tensor(3, dtype=torch.int32),
                                max_iters=7)
    with pytest.raises(RuntimeError, match="did not converge in 7 iterations"):
        bad.sparsity()
    with pytest.raises(RuntimeError, match="did not converge"):
        bad.check()
    assert attention.LayerResult(out=None, final_map=fmap).sparsity() == 0.0


def test_layer_result_counts_unconverged_columns_at_the_sync():
    # HeSS budgets hand over per-column iteration counts (negative = not converged); the
    # layer counts them only when it synchronises
    fmap = torch.ones(1, 2, 3, 4, dtype=torch.uint8)
    ok = attention.LayerResult(out=None, final_map=fmap, budget_iters=torch.tensor([[4, 9, 1]], dtype=torch.int32),
                               max_iters=10)
    assert ok.sparsity() == 0.0
    bad = attention.LayerResult(out=None, final_map=fmap,
                                budget_iters=torch.tensor([[4, -10, -10]], dtype=torch.int32), max_iters=10)
    with pytest.raises(RuntimeError, match=r"did not converge in 10 iterations \(2 query-block columns\)"):
        bad.check()
    mod = torch.nn.Module()
    mod._ress_status = bad
    with pytest.raises(RuntimeError, match="did not converge"):
        attention.check_layers([mod])


def test_random_criterion_generator():
    """One generator per device, seeded 20260826 on first use and advanced by every draw: the
    same call order reproduces the same keys, consecutive layers get different keys
    (reference attention.py:177-196)."""
    cond = torch.rand(1, 2, 5, 40)
    g = LayerGrid(1, 2, 1, 400, 0)
    saved = dict(attention._random_gens)
    try:
        attention._random_gens.clear()
        a1 = attention._rank_key("random", cond, None, None, None, g, None, 64)
        a2 = attention._rank_key("random", cond, None, None, None, g, None, 64)
        attention._random_gens.clear()
        b1 = attention._rank_key("random", cond, None, None, None, g, None, 64)
        b2 = attention._rank_key("random", cond, None, None, None, g, None, 64)
        want = torch.rand(2 * cond.numel(), generator=torch.Generator().manual_seed(20260826))
    finally:
        attention._random_gens.clear()
        attention._random_gens.update(saved)
    assert torch.equal(a1, b1) and torch.equal(a2, b2) and not torch.equal(a1, a2)
    assert a1.shape == cond.shape and a1.dtype == torch.float32
    assert torch.equal(torch.cat([a1.flatten(), a2.flatten()]), want)


def test_mirror_status_word_names_every_problem():
    """The SpargeAttn mirror's device-side input check (status word bits 1, 2, 4: counts,
    LUT entries, PV threshold) is decoded into one ValueError naming each problem."""
    from ress_amd import sparge
    sparge.raise_for_status(0)  # a clean call
    with pytest.raises(ValueError, match="valid_block_num outside"):
        sparge.raise_for_status(1)
    with pytest.raises(ValueError, match="not strictly ascending"):
        sparge.raise_for_status(2)
    with pytest.raises(ValueError, match="pv_threshold below 1e9") as e:
        sparge.raise_for_status(7)
    assert "valid_block_num" in str(e.value) and "LUT entry" in str(e.value)


def test_patch_order_table_validates_the_permutation():
    """kernels.patch_order_table: a per-frame permutation of the P-S patch positions becomes
    the int32 table the kernels read; anything else is refused on the host."""
    from ress_amd import kernels, synth
    g = LayerGrid(B=1, H=2, frames=3, P=13 * 11 + 5, S=5)
    perm = synth.hilbert_permutation(13, 11)
    t = kernels.patch_order_table(perm, g, "cpu")
    assert t.dtype == torch.int32 and torch.equal(t.long(), torch.from_numpy(perm))
    assert kernels.patch_order_table(None, g, "cpu") is None
    bad = perm.copy()
    bad[3] = bad[4]
    with pytest.raises(ValueError, match="permutation"):
        kernels.patch_order_table(bad, g, "cpu")
    with pytest.raises(ValueError, match="permutation"):
        kernels.patch_order_table(perm[:-1], g, "cpu")
    assert ("patch_order", None) in wiring.CALL_ATTRIBUTES


def test_layer_result_reports_fp16_operand_range():
    """LayerResult decodes the 16-bit kernel's operand status (1 key, 2 query)."""
    attention.LayerResult._raise_range(0)
    with pytest.raises(ValueError, match="a key element"):
        attention.LayerResult._raise_range(1)
    with pytest.raises(ValueError, match="a query element"):
        attention.LayerResult._raise_range(2)
    with pytest.raises(ValueError, match="a key and query element"):
        attention.LayerResult._raise_range(3)


def test_check_layers_raises_what_the_forwards_left():
    """ress_amd.check_layers: one synchronisation over the status the last forward of each
    block-sparse attention module kept (HeSS convergence, 16-bit operand range)."""
    class Mod(nn.Module):
        pass

    ok, bad_range, bad_hess = Mod(), Mod(), Mod()
    ok._ress_status = attention.LayerResult(out=None, unconverged=torch.tensor(0, dtype=torch.int32),
                                            attn_status=torch.zeros(1, dtype=torch.int32))
    ress.check_layers([ok])
    bad_range._ress_status = attention.LayerResult(out=None, attn_status=torch.tensor([2], dtype=torch.int32))
    with pytest.raises(ValueError, match="a query element"):
        ress.check_layers([ok, bad_range])
    bad_hess._ress_status = attention.LayerResult(out=None, unconverged=torch.tensor(3, dtype=torch.int32),
                                                  max_iters=1000)
    with pytest.raises(RuntimeError, match="did not converge"):
        ress.check_layers(nn.ModuleList([ok, bad_hess]))


def test_declare_rope_marks_a_foreign_rotation():
    """A module that is not this package's RoPE2D is fused only once declared; the
    declaration names the layout and base the fused kernel implements and rejects others."""
    from ress_amd.aggregator import RoPE2D
    from ress_amd.qkv import ROPE_LAYOUT, rope_base

    class Foreign(nn.Module):
        def forward(self, t, pos):
            return t

    r = Foreign()
    assert rope_base(r) is None
    assert rope_base(RoPE2D(50.0)) == 50.0
    assert ress.declare_rope(r, base=100) is r and rope_base(r) == 100.0
    assert r.ress_rope == (ROPE_LAYOUT, 100.0)
    with pytest.raises(ValueError):
        ress.declare_rope(Foreign(), base=100.0, layout="interleaved_2d")
    with pytest.raises(ValueError):
        ress.declare_rope(Foreign(), base=1.0)


def test_sink_mass_and_protect_reach_the_forward_grid():
    """The module attributes sink_mass / sink_protect (the reference's RESS_SINK_MASS /
    RESS_SINK_PROTECT flags, attention.py:50-79) reach the layer grid: the pooled map's
    width and the candidate count."""
    assert [n for n, _ in wiring.CALL_ATTRIBUTES if n.startswith("sink")] == ["sink_mass", "sink_protect"]
    g = LayerGrid(1, 16, 4, 1374, 5)
    gm = LayerGrid(1, 16, 4, 1374, 5, sink_mass=True)
    gp = LayerGrid(1, 16, 4, 1374, 5, sink_protect=False)
    assert (g.kb_p, g.n_cand, g.kb_tot) == (86, 85, 86)
    assert (gm.kb_p, gm.n_cand, gm.sink_blocks) == (86, 85, 1)
    assert gp.n_cand == 86 and gp.sink_blocks == 0
    big = LayerGrid(1, 16, 12, 1374, 5)  # 60 special keys: one whole special block past the straddler
    bigm = LayerGrid(1, 16, 12, 1374, 5, sink_mass=True)
    assert (big.kb_p, bigm.kb_p, big.kb_tot, big.n_cand) == (257, 258, 258, 256)
