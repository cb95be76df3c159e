"""GPU parity: every HIP stage against the CPU oracle on the same inputs.

Block maps, budgets, LUTs, INT8 codes, scales and pooled values are compared bit for
bit; the attention output against the fp32 block-masked softmax reference with
max-abs <= 2e-2 and cosine >= 0.999."""

import numpy as np
import pytest
import torch

import oracle
from oracle import reference as ref
from pipeline_oracle import oracle_layer, row_sample
from ress_amd import _lib, budget, kernels, synth
from ress_amd.attention import sparse_global_attention
from ress_amd.kernels import LayerGrid

pytestmark = pytest.mark.gpu

ATOL = 2e-2
MIN_COS = 0.999


def _np(t):
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _bits_equal(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    if a.dtype == np.float32:
        return np.array_equal(a.view(np.uint32), b.astype(np.float32).view(np.uint32))
    return np.array_equal(a, b)


def _rand_layer(frames, P, S, H, seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda s: torch.randn(1, H, frames * P, 64, generator=g).mul(s).to(torch.bfloat16)  # noqa: E731
    return mk(1.0), mk(1.3), mk(0.7)


SHAPES = [
    ("vggt_f4", None),            # 4 frames of VGGT token geometry, synthetic field
    ("ragged", (3, 203, 5, 2)),   # partial q/k blocks, straddling special block
    ("plain", (1, 320, 0, 3)),    # no special tokens
    ("tiny", (2, 40, 5, 1)),      # fewer tokens than one q block
]


@pytest.fixture(scope="module", params=SHAPES, ids=[s[0] for s in SHAPES])
def layer(request, dev):
    name, spec = request.param
    if spec is None:
        q, k, v, meta = synth.make_layer_qkv(4)
        frames, P, S, H = meta["frames"], meta["P"], meta["S"], 16
    else:
        frames, P, S, H = spec
        q, k, v = _rand_layer(frames, P, S, H, seed=len(name))
    print(f"[layer {name}] frames={frames} P={P} S={S} H={H}", flush=True)
    return name, q, k, v, frames, P, S, H


def test_prep_bit_exact(layer, dev):
    name, q, k, v, frames, P, S, H = layer
    g = LayerGrid(1, H, frames, P, S)
    blocks = kernels.prepare_blocks(q.to(dev), k.to(dev), v.to(dev), g, mode="i8x2")
    torch.cuda.synchronize()
    o = oracle.prep_qkv(q, k, v, frames, P, S)
    for field in ("q_i8", "q_lo", "q_scale", "pooled_q", "k_i8", "k_lo", "k_scale", "pooled_k", "pooled_v", "ksum", "km"):
        assert _bits_equal(_np(getattr(blocks, field)), o[field]), field
    assert _bits_equal(_np(blocks.v_pack), o["v_pack"])


def test_prep_f16_operands(layer, dev):
    """16-bit mode: the pools and v_pack equal the INT8 modes' (oracle) bit for bit; k_pack
    is K in kernel key order cat(patch, special) rounded to fp16, zero-padded to whole
    blocks; k_scale holds each key block's largest key norm, bit-exact against the oracle
    and within one ulp of the float64 norm."""
    name, q, k, v, frames, P, S, H = layer
    g = LayerGrid(1, H, frames, P, S)
    blocks = kernels.prepare_blocks(q.to(dev), k.to(dev), v.to(dev), g, mode="f16")
    torch.cuda.synchronize()
    assert blocks.q_i8 is None and blocks.k_i8 is None
    o = oracle.prep_qkv(q, k, v, frames, P, S)
    for field in ("pooled_q", "pooled_k", "pooled_v", "v_pack"):
        assert _bits_equal(_np(getattr(blocks, field)), o[field]), field
    assert _bits_equal(_np(blocks.k_scale), o["k_norm"])
    kp, ks = ref.split_tokens(k, frames, P, S)
    keys = kp if ks is None else torch.cat([kp, ks], dim=-2)
    want = torch.zeros(H, g.kb_tot * 64, 64, dtype=torch.float16)
    want[:, :g.Tk] = keys[0].to(torch.float16)
    assert torch.equal(blocks.k_pack.cpu().reshape(H, -1, 64), want)
    norms = torch.zeros(H, g.kb_tot * 64, dtype=torch.float64)
    norms[:, :g.Tk] = keys[0].double().norm(dim=-1)
    np.testing.assert_allclose(o["k_norm"], norms.view(H, g.kb_tot, 64).amax(-1).numpy(), rtol=2e-7)


def test_pooled_scores_bit_exact(layer, dev):
    name, q, k, v, frames, P, S, H = layer
    g = LayerGrid(1, H, frames, P, S)
    blocks = kernels.prepare_blocks(q.to(dev), k.to(dev), v.to(dev), g)
    full, cond = kernels.pooled_scores(blocks)
    o = oracle.prep_qkv(q, k, v, frames, P, S)
    ofull, ocond = oracle.pooled_scores(o["pooled_q"], o["pooled_k"], g.n_cand)
    assert _bits_equal(_np(full).reshape(ofull.shape), ofull)
    assert _bits_equal(_np(cond).reshape(ocond.shape), ocond)


@pytest.mark.parametrize("q_blk,kb_p", [(5, 1), (7, 70), (3, 687), (9, 1024), (3, 1025), (2, 2048), (17, 4300)])
def test_pooled_scores_row_lengths(q_blk, kb_p, dev):
    """Rows of one tile, a ragged tile, a 32-frame row (687 blocks), the tiled kernel's limit (1024)
    and the row kernel beyond it; q_blk not a multiple of the rows per workgroup."""
    rng = np.random.default_rng(kb_p)
    pq = (rng.normal(size=(2, q_blk, 64)) * 2).astype(np.float32)
    pk = (rng.normal(size=(2, kb_p, 64)) * 2).astype(np.float32)
    n_cand = max(kb_p - 3, 0)
    full = torch.empty(2, q_blk, kb_p, device=dev)
    cond = torch.empty(2, q_blk, max(n_cand, 1), device=dev)
    tq, tk = torch.from_numpy(pq).to(dev), torch.from_numpy(pk).to(dev)
    _lib.call("ress_pooled_scores", _lib.ptr(tq), _lib.ptr(tk), 2, q_blk, kb_p, n_cand, 0.125, _lib.ptr(full),
              _lib.ptr(cond), _lib.stream_handle(dev))
    ofull, ocond = oracle.pooled_scores(pq, pk, n_cand)
    assert _bits_equal(_np(full), ofull)
    assert _bits_equal(_np(cond)[:, :, :n_cand], ocond)


def test_pooled_scores_two_rows_per_wave(dev):
    """Enough rows for the tiled kernel's two-rows-per-wave instance (>= 512 workgroups),
    q_blk not a multiple of its eight rows per workgroup."""
    BH, q_blk, kb_p = 16, 257, 333
    rng = np.random.default_rng(7)
    pq = (rng.normal(size=(BH, q_blk, 64)) * 2).astype(np.float32)
    pk = (rng.normal(size=(BH, kb_p, 64)) * 2).astype(np.float32)
    n_cand = kb_p - 1
    full = torch.empty(BH, q_blk, kb_p, device=dev)
    cond = torch.empty(BH, q_blk, n_cand, device=dev)
    tq, tk = torch.from_numpy(pq).to(dev), torch.from_numpy(pk).to(dev)
    _lib.call("ress_pooled_scores", _lib.ptr(tq), _lib.ptr(tk), BH, q_blk, kb_p, n_cand, 0.125, _lib.ptr(full),
              _lib.ptr(cond), _lib.stream_handle(dev))
    ofull, ocond = oracle.pooled_scores(pq, pk, n_cand)
    assert _bits_equal(_np(full), ofull)
    assert _bits_equal(_np(cond), ocond)


@pytest.mark.parametrize("sr,cdf", [(0.5, 0.9), (None, 0.9), (0.7, None), (0.2, 0.5)])
def test_baseline_budget_bit_exact(sr, cdf, dev):
    rng = np.random.default_rng(7)
    a = rng.dirichlet(np.full(342, 0.2), size=(1, 16, 40)).astype(np.float32)
    a[0, 0, 0] = np.float32(1 / 342)
    got = budget.compute_baseline_num_to_select(torch.from_numpy(a).to(dev), sr, cdf)
    want = oracle.baseline_budget(a, sr, cdf)
    assert np.array_equal(_np(got), want)


def test_head_budget_bit_exact(dev):
    rng = np.random.default_rng(8)
    cam, pc = synth.make_hess_tables()
    hb = budget.HessBudget(cam, pc, lam=0.5)
    for layer_idx in (0, 5, 23):
        base = rng.integers(0, 342, size=(1, 16, 50)).astype(np.int32)
        base[0, 3] = 340  # force caps
        got = kernels.head_budget(torch.from_numpy(base).to(dev), hb._scores_norm(layer_idx, dev), 1.0, 342)
        want, it = oracle.head_budget(base, oracle.scores_norm_seq(hb.head_scores[layer_idx].numpy()), 1.0, 342)
        assert it >= 0
        assert np.array_equal(_np(got), want)
    # host-side normalisation equals the oracle's
    assert np.array_equal(budget.scores_norm(hb.head_scores[3]), oracle.scores_norm_seq(hb.head_scores[3].numpy()))


def test_head_budget_non_convergence_is_reported(dev):
    base = torch.full((1, 4, 1), 50, dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="did not converge"):
        budget.adjust_attention_selection(base, torch.tensor([8.0, 1.0, 1.0, 1.0]), 1.0, 60, max_iters=1, check=True)
    out = budget.adjust_attention_selection(base, torch.tensor([8.0, 1.0, 1.0, 1.0]), 1.0, 60, check=True)
    want, _ = oracle.head_budget(np.full((1, 4, 1), 50, np.int32), oracle.scores_norm_seq(np.array([8, 1, 1, 1.0])),
                                 1.0, 60)
    assert np.array_equal(_np(out), want)


# rows below 1024 candidates run on one wave, longer rows on four (a cross-wave tie order)
@pytest.mark.parametrize("n_cand,kb_tot,sink_lead", [(342, 344, 0), (85, 86, 0), (64, 64, 5), (1, 3, 0), (700, 710, 22),
                                                     (1500, 1503, 3), (4293, 4294, 22)])
def test_select_bit_exact_with_ties(n_cand, kb_tot, sink_lead, dev):
    rng = np.random.default_rng(n_cand)
    BH, q_sel, q_tot = 4, 11, 12
    keys = rng.integers(0, 7, size=(BH, q_sel, n_cand)).astype(np.float32) * np.float32(0.125)
    keys[0, 1] = rng.random(n_cand).astype(np.float32)
    counts = rng.integers(-2, n_cand + 3, size=(BH, q_sel)).astype(np.int32)
    counts[0, :3] = [0, 1, n_cand]
    g = LayerGrid(1, BH, 1, 64, 0)  # only BH / shapes are used below
    dev_keys = torch.from_numpy(keys).to(dev)
    fmap = torch.empty(BH, q_sel, kb_tot, dtype=torch.uint8, device=dev)
    lut = torch.empty(BH, q_tot, kb_tot, dtype=torch.int32, device=dev)
    nv = torch.empty(BH, q_tot, dtype=torch.int32, device=dev)
    from ress_amd import _lib
    _lib.call("ress_select_blocks", _lib.ptr(dev_keys), _lib.ptr(torch.from_numpy(counts).to(dev)), BH, q_sel, q_tot,
              n_cand, kb_tot, sink_lead, 2, _lib.ptr(fmap), _lib.ptr(lut), _lib.ptr(nv), _lib.stream_handle(dev))
    omap, olut, onv = oracle.select_blocks(keys, counts, q_tot, kb_tot, sink_lead=sink_lead, min_select=2)
    assert np.array_equal(_np(fmap), omap)
    assert np.array_equal(_np(nv), onv)
    l = _np(lut)
    for b in range(BH):
        for r in range(q_tot):
            assert np.array_equal(l[b, r, :onv[b, r]], olut[b, r, :onv[b, r]])
    del g


def _check_attention(out, q, k, v, frames, P, S, lut, nvalid, rows):
    o = out.float().cpu()
    refs = ref.masked_attention_rows(q, k, v, frames, P, S, lut, nvalid, rows)
    worst, cos_min = 0.0, 1.0
    for (bh, qb), (tok, r) in refs.items():
        got = o.reshape(-1, o.shape[2], 64)[bh, torch.from_numpy(tok)]
        err = (got - r).abs().max().item()
        cos = torch.nn.functional.cosine_similarity(got.flatten(), r.flatten(), dim=0).item()
        worst, cos_min = max(worst, err), min(cos_min, cos)
    assert worst <= ATOL, worst
    assert cos_min >= MIN_COS, cos_min
    return worst, cos_min


@pytest.mark.parametrize("mode", ["f16", "i8x2"])
def test_attention_matches_fp32_masked_softmax(layer, mode, dev):
    name, q, k, v, frames, P, S, H = layer
    g = LayerGrid(1, H, frames, P, S)
    o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=0.5, cdf_threshold=0.9, H=H)
    blocks = kernels.prepare_blocks(q.to(dev), k.to(dev), v.to(dev), g, mode=mode)
    lut = torch.from_numpy(o["lut"].reshape(g.BH, g.q_blk_total, g.kb_tot)).to(dev)
    nv = torch.from_numpy(o["nvalid"]).to(dev)
    out = kernels.sparse_attention(blocks, lut, nv)
    torch.cuda.synchronize()
    rows = row_sample(o["nvalid"], 12 if name == "vggt_f4" else 30)
    w, c = _check_attention(out, q, k, v, frames, P, S, o["lut"], o["nvalid"], rows)
    print(f"[{name} {mode}] attention max-abs {w:.3e} min-cos {c:.6f}")


@pytest.mark.parametrize("mode", ["f16", "i8x2"])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_attention_low_precision_outputs(out_dtype, mode, dev):
    frames, P, S, H = 2, 200, 4, 2
    q, k, v = _rand_layer(frames, P, S, H, seed=11)
    g = LayerGrid(1, H, frames, P, S)
    o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=0.5, H=H)
    blocks = kernels.prepare_blocks(q.to(dev), k.to(dev), v.to(dev), g, mode=mode)
    lut = torch.from_numpy(o["lut"]).to(dev)
    nv = torch.from_numpy(o["nvalid"]).to(dev)
    out32 = kernels.sparse_attention(blocks, lut, nv)
    out = kernels.sparse_attention(blocks, lut, nv, out_dtype=out_dtype)
    assert out.dtype == out_dtype
    if out_dtype == torch.bfloat16:
        assert torch.equal(out, out32.to(out_dtype))
    else:
        # fp16: the epilogue rounds o*inv to half once (v_fma_mixlo_f16); rounding the
        # fp32 output to half rounds twice, so the two may differ by one half ulp
        assert torch.allclose(out.float(), out32, rtol=2.0 ** -10, atol=2.0 ** -24)


@pytest.mark.parametrize("cfg,mode", [("sparse_vggt_f4", "f16"), ("hess_f16", "f16"), ("hess_f16", "i8x2")])
def test_layer_pipeline_matches_oracle(cfg, mode, dev):
    if cfg == "sparse_vggt_f4":
        frames, sr, cdf, hess = 4, 0.5, 0.9, False
    else:
        frames, sr, cdf, hess = 16, 0.7, None, True
    q, k, v, meta = synth.make_layer_qkv(frames)
    P, S = meta["P"], meta["S"]
    g = LayerGrid(1, 16, frames, P, S)
    if hess:
        cam, pc = synth.make_hess_tables()
        bud = budget.HessBudget(cam, pc, lam=0.5)
        head_scores = bud.head_scores[0].numpy()
    else:
        bud = budget.UniformBudget()
        head_scores = None
    res = sparse_global_attention(q.to(dev), k.to(dev), v.to(dev), g,
                                  budget_fn=lambda a: bud.num_to_select(0, a, sr, cdf, 1.0), keep_intermediates=True,
                                  qk_mode=mode)
    torch.cuda.synchronize()
    o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=sr, cdf_threshold=cdf, head_scores=head_scores)
    assert np.array_equal(_np(res.counts).reshape(o["counts"].shape), o["counts"])
    assert np.array_equal(_np(res.final_map).reshape(o["map"].shape), o["map"])
    assert np.array_equal(_np(res.nvalid), o["nvalid"])
    sparsity = res.sparsity()
    print(f"[{cfg}] realized sparsity {sparsity:.4f}")
    rows = row_sample(o["nvalid"], 10)
    w, c = _check_attention(res.out, q, k, v, frames, P, S, o["lut"], o["nvalid"], rows)
    print(f"[{cfg} {mode}] attention max-abs {w:.3e} min-cos {c:.6f}")


@pytest.mark.parametrize("criterion", ["probability", "ress"])
def test_sink_mass_layer_matches_oracle(criterion, dev):
    """sink_mass (the reference's RESS_SINK_MASS, attention.py:451-452, 481): the pools,
    the map over every key block and the restore-swap keep sets bit-exact against the
    oracle pipeline on the same grid; the budget reads the renormalised candidate map."""
    frames, sr = 4, 0.7
    q, k, v, meta = synth.make_layer_qkv(frames)
    P, S = meta["P"], meta["S"]
    g = LayerGrid(1, 16, frames, P, S, sink_mass=True)
    assert g.kb_p == g.kb_tot > g.n_cand
    W_O = synth.make_w_o()
    M = torch.stack([W_O[:, h * 64:(h + 1) * 64].T @ W_O[:, h * 64:(h + 1) * 64] for h in range(16)])
    bud = budget.UniformBudget()
    crit = "restore_swap_iter5_bf16_trackbest" if criterion == "ress" else "probability"
    print(f"[sink_mass {criterion}] frames={frames} kb_p={g.kb_p} n_cand={g.n_cand}", flush=True)
    res = sparse_global_attention(q.to(dev), k.to(dev), v.to(dev), g,
                                  budget_fn=lambda a: bud.num_to_select(0, a, sr, None, 1.0), block_criterion=crit,
                                  M=M.to(dev), keep_intermediates=True)
    torch.cuda.synchronize()
    o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=sr, criterion=criterion, M=M.numpy(), sink_mass=True)
    assert _bits_equal(_np(res.blocks.pooled_k), o["pooled_k"])
    assert _bits_equal(_np(res.blocks.pooled_v), o["pooled_v"])
    assert _bits_equal(_np(res.attn_full).reshape(o["attn_full"].shape), o["attn_full"])
    assert np.array_equal(_np(res.final_map).reshape(o["map"].shape), o["map"])
    assert np.array_equal(_np(res.nvalid), o["nvalid"])
    rows = row_sample(o["nvalid"], 8)
    w, c = _check_attention(res.out, q, k, v, frames, P, S, o["lut"], o["nvalid"], rows)
    print(f"[sink_mass {criterion}] sparsity {res.sparsity():.4f} max-abs {w:.3e} min-cos {c:.6f}")


def test_realized_drift_is_recorded_for_the_kernels_keep_set(dev):
    """record_realized_drift around one layer (fp32 restore-swap, track_best): one value, the
    mean J of the keep set the attention kernel ran with, equal within fp32 reassociation to
    the oracle's J of the oracle's keep set on the same pooled map (the two keep sets are
    bit-exact; reference attention.py:199-214, projected.py:112-129)."""
    from ress_amd import projected
    frames, sr = 4, 0.6
    q, k, v, meta = synth.make_layer_qkv(frames)
    P, S = meta["P"], meta["S"]
    g = LayerGrid(1, 16, frames, P, S)
    W_O = synth.make_w_o()
    M = torch.stack([W_O[:, h * 64:(h + 1) * 64].T @ W_O[:, h * 64:(h + 1) * 64] for h in range(16)])
    bud = budget.UniformBudget()
    print(f"[realized drift] frames={frames} n_cand={g.n_cand}", flush=True)
    with projected.record_realized_drift() as rec:
        res = sparse_global_attention(q.to(dev), k.to(dev), v.to(dev), g,
                                      budget_fn=lambda a: bud.num_to_select(0, a, sr, None, 1.0),
                                      block_criterion="restore_swap_iter5_trackbest", M=M.to(dev),
                                      keep_intermediates=True)
    torch.cuda.synchronize()
    assert len(rec) == 1
    o = oracle.prep_qkv(q, k, v, frames, P, S)
    full, _ = oracle.pooled_scores(o["pooled_q"], o["pooled_k"], g.n_cand)
    counts = np.maximum(_np(res.counts).reshape(16, g.q_blk_p), min(2, g.n_cand)).astype(np.int32)
    keep, J = oracle.restore_swap(full.reshape(16, g.q_blk_p, g.kb_p), o["pooled_v"].reshape(16, g.kb_p, 64),
                                  M.numpy(), counts, g.n_cand, n_iters=5, big_bf16=False, track_best=True)
    assert np.array_equal(_np(res.final_map).reshape(16, g.q_blk_p, g.kb_tot)[..., :g.n_cand], keep)
    np.testing.assert_allclose(rec[0], float(J.astype(np.float64).mean()), rtol=2e-4)
    print(f"[realized drift] recorded {rec[0]:.6e} oracle {J.mean():.6e}")


def test_layer_protect_own_frame(dev):
    """protect_own_frame inside the layer: the swapped map is the oracle map after the
    budget-neutral own-frame swap, the LUT is rebuilt from it, per-row kept counts are
    unchanged, and the attention follows the new LUT."""
    from ress_amd.attention import protect_own_frame_swap
    frames, sr = 4, 0.8
    q, k, v, meta = synth.make_layer_qkv(frames)
    P, S = meta["P"], meta["S"]
    g = LayerGrid(1, 16, frames, P, S)
    bud = budget.UniformBudget()
    res = sparse_global_attention(q.to(dev), k.to(dev), v.to(dev), g,
                                  budget_fn=lambda a: bud.num_to_select(0, a, sr, None, 1.0), keep_intermediates=True,
                                  protect_own_frame=True)
    torch.cuda.synchronize()
    o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=sr, cdf_threshold=None)
    want = protect_own_frame_swap(torch.from_numpy(o["map"]).reshape(1, 16, g.q_blk_p, g.kb_tot),
                                  torch.from_numpy(o["attn_full"]).reshape(1, 16, g.q_blk_p, -1)[..., :g.n_cand], g)
    got = _np(res.final_map).astype(bool)
    assert np.array_equal(got, want.numpy())
    assert np.array_equal(got.sum(-1).reshape(-1), o["map"].reshape(-1, g.kb_tot).sum(-1))
    lut, nv = _np(res.lut), _np(res.nvalid)
    gm = got.reshape(16, g.q_blk_p, g.kb_tot)
    for bh in range(16):
        for r in range(g.q_blk_p):
            cols = np.flatnonzero(gm[bh, r])
            assert nv[bh, r] == cols.size and np.array_equal(lut[bh, r, :cols.size], cols)
    rows = row_sample(nv, 8)
    _check_attention(res.out, q, k, v, frames, P, S, lut, nv, rows)


@pytest.mark.parametrize("mode", ["f16", "i8x2"])
@pytest.mark.parametrize("B,H,frames", [(2, 16, 3), (1, 5, 2), (1, 1, 1)])
def test_attention_writes_every_row(B, H, frames, mode, dev):
    """The persistent row schedule covers every (batch, head, q-block) exactly once:
    a NaN-filled output has no NaN left, and rows match the per-row fp32 reference."""
    P, S = 203, 5
    g = torch.Generator().manual_seed(B * 100 + H)
    mk = lambda: torch.randn(B, H, frames * P, 64, generator=g).to(torch.bfloat16)  # noqa: E731
    q, k, v = mk(), mk(), mk()
    grid = LayerGrid(B, H, frames, P, S)
    blocks = kernels.prepare_blocks(q.to(dev), k.to(dev), v.to(dev), grid, mode=mode)
    rng = np.random.default_rng(1)
    keys = torch.from_numpy(rng.random((B, H, grid.q_blk_p, grid.n_cand)).astype(np.float32)).to(dev)
    counts = torch.from_numpy(rng.integers(0, grid.n_cand + 1, (B, H, grid.q_blk_p)).astype(np.int32)).to(dev)
    _, lut, nv = kernels.select_blocks(keys, counts, grid, 2)
    out = torch.full((B, H, grid.Tk, 64), float("nan"), device=dev)
    kernels.sparse_attention(blocks, lut, nv, out=out)
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    rows = row_sample(nv.cpu().numpy(), 12)
    _check_attention(out, q, k, v, frames, P, S, lut.cpu().numpy(), nv.cpu().numpy(), rows)


def test_random_criterion_layer(dev):
    """block_criterion="random" (reference attention.py:177-196, 576-578): the rank key is the
    per-device generator's next draw (seed 20260826 on first use); the map is the oracle's
    selection of that key, every row keeps exactly max(counts, 2) candidates plus the sinks."""
    from ress_amd import attention as attn_mod
    frames, sr = 4, 0.6
    q, k, v, meta = synth.make_layer_qkv(frames)
    P, S = meta["P"], meta["S"]
    g = LayerGrid(1, 16, frames, P, S)
    bud = budget.UniformBudget()
    saved = dict(attn_mod._random_gens)
    try:
        attn_mod._random_gens.clear()
        res = sparse_global_attention(q.to(dev), k.to(dev), v.to(dev), g,
                                      budget_fn=lambda a: bud.num_to_select(0, a, sr, None, 1.0),
                                      block_criterion="random", keep_intermediates=True)
        torch.cuda.synchronize()
        gen = torch.Generator(device=dev).manual_seed(20260826)
        key = torch.rand((1, 16, g.q_blk_p, g.n_cand), device=dev, dtype=torch.float32, generator=gen)
        assert torch.equal(attn_mod._random_gens[dev].get_state(), gen.get_state())
    finally:
        attn_mod._random_gens.clear()
        attn_mod._random_gens.update(saved)
    o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=sr, criterion="key", rank_key=key.cpu().numpy())
    fmap = _np(res.final_map).reshape(o["map"].shape)
    assert np.array_equal(fmap, o["map"])
    want = np.maximum(o["counts"].reshape(-1, g.q_blk_p), 2) + g.sink_blocks
    assert np.array_equal(fmap.sum(-1), want)


def test_hess_non_convergence_raises_at_layer_sync(dev):
    """A HeSS budget that cannot converge within its iteration cap makes the layer's deferred
    check raise RuntimeError (reference _proportional.py:112-113). The cap is forced to 1
    from the host: two heads' ideal budgets exceed the candidate count, so every column needs
    one redistribution step and the loop ends before the pass that finds no excess left. The
    default cap converges on the same input."""
    frames, sr = 4, 0.2
    q, k, v, meta = synth.make_layer_qkv(frames)
    P, S = meta["P"], meta["S"]
    g = LayerGrid(1, 16, frames, P, S)
    scores = torch.full((3, 1, 16), 1.0)
    scores[0, 0, :2] = 50.0   # two heads want far more than max_val -> repeated caps
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    for cap, ok in ((1, False), (1000, True)):
        hb = budget.HessBudget(scores, scores, lam=0.5, max_iters=cap)
        res = sparse_global_attention(qd, kd, vd, g, budget_fn=lambda a: hb.num_to_select(0, a, sr, None, 1.0))
        if ok:
            res.check()
            assert 0.0 < res.sparsity() < 1.0
        else:
            with pytest.raises(RuntimeError, match="did not converge in 1 iterations"):
                res.sparsity()
            with pytest.raises(RuntimeError, match="did not converge"):
                res.check()


@pytest.mark.parametrize("name", ["vggt", "pi3", "da3"])
def test_head_budget_on_shipped_tables(name, dev):
    """k_head_budget with every layer's head scores from the shipped calibration tables, at
    the backbone's tuned lambda, against the oracle, with budgets that force caps."""
    from ress_amd import backbones
    spec = backbones.get_backbone(name)
    pcd, cam = spec.calibration_paths()
    hb = budget.HessBudget(cam, pcd, lam=spec.hess_lam)
    rng = np.random.default_rng(len(name))
    H, n_cand = spec.n_heads, 342
    for layer in range(spec.n_global_blocks):
        base = rng.integers(0, n_cand, size=(1, H, 40)).astype(np.int32)
        got = kernels.head_budget(torch.from_numpy(base).to(dev), hb._scores_norm(layer, dev), 1.0, n_cand)
        want, it = oracle.head_budget(base, oracle.scores_norm_seq(hb.head_scores[layer].numpy()), 1.0, n_cand)
        assert it >= 0
        assert np.array_equal(_np(got), want), (name, layer)


@pytest.mark.parametrize("q_mul", [1.0, 8.0, 0.0], ids=["mixed", "running_max", "zero_q"])
def test_f16_bounded_and_running_max_rows(q_mul, dev):
    """16-bit mode rows run bounded (pre-scaled fp16 queries, P = exp2(logit) with no offset
    and no running max) when |q'| * max key norm is at most 64 for every query of the row, or
    otherwise with exact fp16 queries and the running max. Queries scaled by 8 push every row past the bound (running max everywhere);
    zero queries give uniform attention on bounded rows; unscaled data mixes both. Every row
    against the fp32 masked softmax."""
    from device_reference import row_errors
    frames, P, S, H = 4, 1374, 5, 4
    q, k, v, meta = synth.make_layer_qkv(frames, H=H, seed=3)
    q = (q.float() * q_mul).to(torch.bfloat16)
    g = LayerGrid(1, H, frames, P, S)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    blocks = kernels.prepare_blocks(qd, kd, vd, g, mode="f16")
    rng = np.random.default_rng(5)
    keys = torch.from_numpy(rng.random((1, H, g.q_blk_p, g.n_cand)).astype(np.float32)).to(dev)
    counts = torch.from_numpy(rng.integers(2, g.n_cand + 1, (1, H, g.q_blk_p)).astype(np.int32)).to(dev)
    _, lut, nv = kernels.select_blocks(keys, counts, g, 2)
    out = kernels.sparse_attention(blocks, lut, nv)
    torch.cuda.synchronize()
    # which rows ran bounded: every query's |q * c|_fp16 * max kept key norm <= 64
    c = 0.125 * 1.4426950408889634
    qc = (q.float() * c).to(torch.float16).float()[0]
    kn = blocks.k_scale.view(H, g.kb_tot).cpu()
    lutc, nvc = lut.cpu(), nv.cpu()
    order = torch.cat([torch.arange(f * P + S, (f + 1) * P) for f in range(frames)] +
                      [torch.arange(f * P, f * P + S) for f in range(frames)])
    qn = qc[:, order].norm(dim=-1)
    bounded = np.zeros((H, g.q_blk_total), bool)
    for h in range(H):
        for r in range(g.q_blk_total):
            kmax = kn[h, lutc[h, r, :nvc[h, r]].long()].max() if nvc[h, r] else torch.tensor(0.0)
            r0 = r * 128 if r < g.q_blk_p else g.T_p + (r - g.q_blk_p) * 128
            bounded[h, r] = bool((qn[h, r0:r0 + 128] * kmax <= 64).all())
    err, cos = row_errors(out, qd, kd, vd, g, lut, nv)
    print(f"[f16 q*{q_mul}] bounded rows {bounded.sum()}/{bounded.size}: max-abs {np.nanmax(err):.3e} "
          f"min-cos {np.nanmin(cos):.6f}")
    if q_mul == 8.0:
        assert not bounded.any()
    if q_mul == 0.0:
        assert bounded.all()
    assert np.nanmax(err) <= ATOL and np.nanmin(cos) >= MIN_COS


def test_f16_outlier_query_off_the_vote_lane_takes_running_max(dev):
    """The bounded/running-max vote covers all 128 queries of a row, not only the first query
    of each 32-query group. Every patch row gets one outlier query at index 77 (lane 13 of its
    query group) aligned with a kept key, so that its logits reach ~200 in log2 units while the
    rest of the row stays far inside the bound. A row that ran bounded would give exp2 overflow
    (inf/NaN) for that query; the running-max path gives the fp32 masked softmax."""
    from device_reference import kernel_order, row_errors
    frames, P, S, H = 4, 1374, 5, 2
    q, k, v, meta = synth.make_layer_qkv(frames, H=H, seed=4)
    q = (q.float() * 0.25).to(torch.bfloat16)
    g = LayerGrid(1, H, frames, P, S)
    rng = np.random.default_rng(6)
    keys = torch.from_numpy(rng.random((1, H, g.q_blk_p, g.n_cand)).astype(np.float32)).to(dev)
    counts = torch.from_numpy(rng.integers(2, g.n_cand + 1, (1, H, g.q_blk_p)).astype(np.int32)).to(dev)
    _, lut, nv = kernels.select_blocks(keys, counts, g, 2)
    lutc, nvc = lut.cpu(), nv.cpu()
    order = kernel_order(frames, P, S, "cpu")
    c = 0.125 * 1.4426950408889634
    qf, kf = q.float(), k.float()
    worst_logit = np.inf
    for h in range(H):
        for r in range(g.q_blk_p):
            kb = int(lutc[h, r, 0])                    # a kept key block of the row
            kk = kf[0, h, order[kb * 64]]              # its first key (kernel order)
            scale = 200.0 / (c * float(kk.dot(kk)))
            q[0, h, order[r * 128 + 77]] = (kk * scale).to(torch.bfloat16)
            qo = q[0, h, order[r * 128 + 77]].float()
            kept = torch.cat([torch.arange(int(b) * 64, min(int(b) * 64 + 64, g.Tk)) for b in lutc[h, r, :nvc[h, r]]])
            worst_logit = min(worst_logit, float((kf[0, h, order[kept]] @ qo).max()) * c)
    assert worst_logit > 128.0, worst_logit   # exp2 of the outlier's logits overflows fp32
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    blocks = kernels.prepare_blocks(qd, kd, vd, g, mode="f16")
    out = kernels.sparse_attention(blocks, lut, nv)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    err, cos = row_errors(out, qd, kd, vd, g, lut, nv)
    print(f"[f16 outlier q77] min outlier logit {worst_logit:.1f} log2 units: max-abs {np.nanmax(err):.3e} "
          f"min-cos {np.nanmin(cos):.6f}")
    assert np.nanmax(err) <= ATOL and np.nanmin(cos) >= MIN_COS


@pytest.mark.parametrize("mode", ["f16", "i8x2"])
def test_patch_order_read_in_place_matches_permuted_copy(mode, dev):
    """The Hilbert order read in place (patch_order) gives exactly what the reference's
    hilbert_permute copy gives (src/ress/models/hilbert.py:128-162): the layer on raster-order
    Q/K/V with the curve's gather table equals the layer on the permuted tensors with the
    output permuted back, bit for bit (maps, LUTs, pools, attention)."""
    from ress_amd.synth import hilbert_permutation
    gw, gh, S, frames, H = 13, 11, 5, 3, 4
    HW = gw * gh
    P = HW + S
    perm = torch.from_numpy(hilbert_permutation(gw, gh))
    gen = torch.Generator().manual_seed(11)
    q, k, v = (torch.randn(1, H, frames * P, 64, generator=gen).to(torch.bfloat16) for _ in range(3))
    print(f"[patch_order {mode}] frames={frames} P={P} S={S} H={H}", flush=True)
    # the reference's copy: per frame, the special tokens, then the patch tokens gathered
    idx = torch.cat([torch.cat([f * P + torch.arange(S), f * P + S + perm]) for f in range(frames)])
    g = LayerGrid(1, H, frames, P, S)
    counts = torch.full((1, H, g.q_blk_p), max(2, g.n_cand // 3), dtype=torch.int32, device=dev)
    a = sparse_global_attention(q.to(dev), k.to(dev), v.to(dev), g, num_to_select=counts, qk_mode=mode,
                                keep_intermediates=True, patch_order=perm)
    b = sparse_global_attention(q[:, :, idx].contiguous().to(dev), k[:, :, idx].contiguous().to(dev),
                                v[:, :, idx].contiguous().to(dev), g, num_to_select=counts, qk_mode=mode,
                                keep_intermediates=True)
    torch.cuda.synchronize()
    assert torch.equal(a.blocks.pooled_q, b.blocks.pooled_q) and torch.equal(a.blocks.pooled_k, b.blocks.pooled_k)
    assert torch.equal(a.attn_full, b.attn_full)
    assert torch.equal(a.final_map, b.final_map) and torch.equal(a.nvalid, b.nvalid)
    listed = torch.arange(g.kb_tot, device=dev) < a.nvalid[..., None]  # entries past nvalid are unused
    assert torch.equal(torch.where(listed, a.lut, -1), torch.where(listed, b.lut, -1))
    back = torch.empty_like(b.out)
    back[:, :, idx] = b.out
    assert torch.equal(a.out, back)


def test_layer_step_replays_from_a_hip_graph(dev):
    """The layer step (prep, pooled map, HeSS budget, selection, attention) captured once in
    a HIP graph: every replay, with eager work and synchronisations between replays, equals
    the eager step bit for bit (no memset nodes or host reads inside the step)."""
    frames = 4
    q, k, v, meta = synth.make_layer_qkv(frames)
    g = LayerGrid(1, 16, frames, meta["P"], meta["S"])
    cam, pc = synth.make_hess_tables()
    bud = budget.HessBudget(cam, pc, lam=0.5)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out = torch.empty(1, 16, g.Tk, 64, dtype=torch.float32, device=dev)

    def step():
        return sparse_global_attention(qd, kd, vd, g, budget_fn=lambda a: bud.num_to_select(0, a, 0.7, None, 1.0),
                                       out=out, attention_sink=64)

    step()
    torch.cuda.synchronize()
    want = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for rep in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep} differs from the eager step"
        step()  # eager work between the replays
        torch.cuda.synchronize()
        assert torch.equal(out, want)


@pytest.mark.parametrize("which", ["key", "query"])
def test_f16_operand_outside_fp16_range_is_reported(which, dev):
    """A key or query element fp16 cannot hold (|x| >= 65520; bf16 can) makes the 16-bit
    layer raise at its next synchronisation instead of returning inf/NaN rows silently;
    the same layer without it reports nothing."""
    frames, H = 2, 4
    q, k, v, meta = synth.make_layer_qkv(frames, H=H)
    g = LayerGrid(1, H, frames, meta["P"], meta["S"])
    counts = torch.full((1, H, g.q_blk_p), max(2, g.n_cand // 2), dtype=torch.int32, device=dev)
    clean = sparse_global_attention(q.to(dev), k.to(dev), v.to(dev), g, num_to_select=counts)
    clean.check()
    q2, k2 = q.clone(), k.clone()
    (k2 if which == "key" else q2)[0, 1, 7, 3] = 70000.0
    print(f"[f16 range] {which} element 70000", flush=True)
    res = sparse_global_attention(q2.to(dev), k2.to(dev), v.to(dev), g, num_to_select=counts)
    with pytest.raises(ValueError, match=f"a {which} element lies outside the fp16 range"):
        res.check()
    with pytest.raises(ValueError, match="outside the fp16 range"):
        res.sparsity()
