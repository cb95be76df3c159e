"""The BASELINE workloads on the GPU, at their real shapes, against the CPU oracle.

* configs[0] (4 frames, SparseVGGT uniform budget, sr 0.5, cdf 0.9, attention_sink 1374):
  block map bit-exact including the 22 forced leading blocks; every attention row within
  max-abs 2e-2 / cosine 0.999 of the fp32 masked softmax, in the bf16 and two-term INT8 modes.
* configs[1] (16 frames, HeSS, sr 0.7): map bit-exact; every row checked in the bf16 and
  two-term INT8 modes; the reference's single-term INT8 arithmetic is measured against the
  same bar (it is known to miss it: xfail with the measured error).
* configs[2] (32 frames, ReSS restore_swap_iter5_bf16_trackbest, sr 0.8): map bit-exact
  against the oracle's restore-swap pipeline; every row checked.
* configs[4] (200 frames, N = 274,800, SparseVGGT sr 0.9, attention_sink 1374): map
  bit-exact with the leading blocks; a stratified sample of rows checked (every dense row,
  every split row, every 16th patch row) in the 16-bit and two-term INT8 modes, and the
  reference's single-term INT8 arithmetic measured on the same rows.
* configs[3] (the VGGT-1B-style aggregator, 24 global layers, dim 1024, 64 frames of
  518x518, ReSS at sr 0.8): finite output, per-layer realised sparsity near 0.8, close to the
  dense model; global layer 0's captured Q/K/V rerun through the oracle bit-exactly.

Every check of the rows the attention launch splits into parts (device_reference.split_rows)
is reported separately. References: src/ress/models/attention.py:217-243,446-659;
external/patches/spargeattn.patch:61-65."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from device_reference import row_errors, split_rows
from pipeline_oracle import oracle_layer
from ress_amd import budget, kernels, synth
from ress_amd.attention import sink_lead_blocks, sparse_global_attention
from ress_amd.kernels import LayerGrid

pytestmark = pytest.mark.gpu

ATOL, MIN_COS = 2e-2, 0.999
SINK = 1374   # the configs' attention_sink: the first frame's tokens


def _np(t):
    return t.detach().cpu().numpy()


def _say(msg):
    print(msg, flush=True)


def _check_rows(name, res, q, k, v, grid, rows=None):
    err, cos = row_errors(res.out, q, k, v, grid, res.lut, res.nvalid, rows=rows)
    checked = ~np.isnan(err)
    split = split_rows(_np(res.nvalid), grid.q_blk_p)
    assert split.any()
    assert checked[split].all(), "every split (merged) row must be among the checked rows"
    worst, cmin = np.nanmax(err), np.nanmin(cos)
    _say(f"[{name}] {int(checked.sum())} rows checked: max-abs {worst:.3e} min-cos {cmin:.6f}; "
         f"{int(split.sum())} split rows: max-abs {err[split].max():.3e} min-cos {cos[split].min():.6f}")
    return worst, cmin


def _layer(frames, corr="shared"):
    q, k, v, meta = synth.make_layer_qkv(frames, corr=corr)
    return q, k, v, meta["P"], meta["S"]


@pytest.fixture(scope="module")
def config1(dev):
    _say("[configs[1]] generating 16 frames")
    q, k, v, P, S = _layer(16)
    cam, pc = synth.make_hess_tables()
    bud = budget.HessBudget(cam, pc, lam=0.5)
    o = oracle_layer(q, k, v, 16, P, S, sparse_ratio=0.7, head_scores=bud.head_scores[0].numpy())
    return q, k, v, P, S, bud, o


@pytest.mark.parametrize("mode", ["f16", "i8x2"])
def test_config0_uniform_with_sink(mode, dev):
    frames, sr, cdf = 4, 0.5, 0.9
    _say(f"[configs[0] {mode}] frames={frames} sr={sr} cdf={cdf} attention_sink={SINK}")
    q, k, v, P, S = _layer(frames)
    g = LayerGrid(1, 16, frames, P, S)
    lead = sink_lead_blocks(SINK, g)
    assert lead == 22
    bud = budget.UniformBudget()
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    res = sparse_global_attention(qd, kd, vd, g, budget_fn=lambda a: bud.num_to_select(0, a, sr, cdf, 1.0),
                                  keep_intermediates=True, qk_mode=mode, attention_sink=SINK)
    torch.cuda.synchronize()
    o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=sr, cdf_threshold=cdf, sink_lead=lead)
    fmap = _np(res.final_map).reshape(o["map"].shape)
    assert np.array_equal(fmap, o["map"])
    assert np.array_equal(_np(res.nvalid), o["nvalid"])
    assert fmap[..., :lead].all() and fmap[..., g.n_cand:].all()
    worst, cmin = _check_rows(f"configs[0] {mode}", res, qd, kd, vd, g)
    assert worst <= ATOL and cmin >= MIN_COS


@pytest.mark.parametrize("mode", ["f16", "i8x2", "i8"])
def test_config1_hess_every_row(config1, mode, dev):
    q, k, v, P, S, bud, o = config1
    _say(f"[configs[1] {mode}] 16 frames HeSS sr=0.7")
    g = LayerGrid(1, 16, 16, P, S)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    res = sparse_global_attention(qd, kd, vd, g, budget_fn=lambda a: bud.num_to_select(0, a, 0.7, None, 1.0),
                                  keep_intermediates=True, qk_mode=mode)
    torch.cuda.synchronize()
    assert np.array_equal(_np(res.counts).reshape(o["counts"].shape), o["counts"])
    assert np.array_equal(_np(res.final_map).reshape(o["map"].shape), o["map"])
    res.check()
    worst, cmin = _check_rows(f"configs[1] {mode}", res, qd, kd, vd, g)
    if mode == "i8" and (worst > ATOL or cmin < MIN_COS):
        pytest.xfail(f"single-term per-block INT8 QK^T (the reference's SpargeAttn quantiser) misses the "
                     f"tolerance: max-abs {worst:.3e}, min-cos {cmin:.6f}")
    assert worst <= ATOL and cmin >= MIN_COS


def test_config2_ress_layer(dev):
    frames, sr = 32, 0.8
    _say(f"[configs[2]] frames={frames} ReSS restore_swap_iter5_bf16_trackbest sr={sr}")
    q, k, v, P, S = _layer(frames)
    g = LayerGrid(1, 16, frames, P, S)
    cam, pc = synth.make_hess_tables()
    bud = budget.HessBudget(cam, pc, lam=0.5)
    W_O = synth.make_w_o()
    M = torch.stack([W_O[:, h * 64:(h + 1) * 64].T @ W_O[:, h * 64:(h + 1) * 64] for h in range(16)])
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    res = sparse_global_attention(qd, kd, vd, g, budget_fn=lambda a: bud.num_to_select(0, a, sr, None, 1.0),
                                  block_criterion="restore_swap_iter5_bf16_trackbest", M=M.to(dev),
                                  keep_intermediates=True)
    torch.cuda.synchronize()
    _say("[configs[2]] GPU layer done; oracle pipeline")
    o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=sr, head_scores=bud.head_scores[0].numpy(),
                     criterion="ress", M=M.numpy())
    assert np.array_equal(_np(res.final_map).reshape(o["map"].shape), o["map"])
    assert np.array_equal(_np(res.nvalid), o["nvalid"])
    _say(f"[configs[2]] map bit-exact, realised sparsity {res.sparsity():.4f}")
    worst, cmin = _check_rows("configs[2] f16", res, qd, kd, vd, g)
    assert worst <= ATOL and cmin >= MIN_COS


def test_config4_long_sequence(dev):
    frames, sr = 200, 0.9
    _say(f"[configs[4]] generating {frames} frames (AR(1) correlation 0.98)")
    q, k, v, P, S = _layer(frames, corr="ar1")
    g = LayerGrid(1, 16, frames, P, S)
    lead = sink_lead_blocks(SINK, g)
    bud = budget.UniformBudget()
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    _say(f"[configs[4]] GPU layer N={g.Tk} q_blk={g.q_blk_p} n_cand={g.n_cand} sink_lead={lead}")
    res = sparse_global_attention(qd, kd, vd, g, budget_fn=lambda a: bud.num_to_select(0, a, sr, None, 1.0),
                                  keep_intermediates=True, attention_sink=SINK)
    torch.cuda.synchronize()
    _say("[configs[4]] GPU layer done; oracle pipeline")
    o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=sr, sink_lead=lead)
    fmap = _np(res.final_map).reshape(o["map"].shape)
    assert np.array_equal(fmap, o["map"])
    assert np.array_equal(_np(res.nvalid), o["nvalid"])
    assert fmap[..., :lead].all()
    _say(f"[configs[4]] map bit-exact, realised sparsity {res.sparsity():.4f}")
    nv = _np(res.nvalid)
    rows = split_rows(nv, g.q_blk_p)
    rows[:, g.q_blk_p:] = True
    rows[:, :g.q_blk_p:16] = True
    worst, cmin = _check_rows("configs[4] f16", res, qd, kd, vd, g, rows=rows)
    assert worst <= ATOL and cmin >= MIN_COS
    # the INT8 QK^T the config names, on the same map and rows: two-term codes within the bar;
    # the reference's single-term codes measured and reported (they miss the 2e-2 bar by
    # construction; the emulation of every single-term granularity in tests/int8_variant_study.py)
    for mode in ("i8x2", "i8"):
        blocks = kernels.prepare_blocks(qd, kd, vd, g, mode=mode)
        out = kernels.sparse_attention(blocks, res.lut, res.nvalid)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        worst, cmin = _check_rows(f"configs[4] {mode}", SimpleNamespace(out=out, lut=res.lut, nvalid=res.nvalid),
                                  qd, kd, vd, g, rows=rows)
        if mode == "i8x2":
            assert worst <= ATOL and cmin >= MIN_COS
        del blocks, out


def test_config3_aggregator(dev):
    """The full-size aggregator under ReSS on every global layer."""
    import ress_amd as ress
    import ress_amd.attention as attn_mod
    import ress_amd.wiring as wiring
    from ress_amd.aggregator import build_vggt_aggregator, synthetic_frames
    S_frames, depth, sr = 64, 24, 0.8
    _say(f"[configs[3]] building the aggregator: depth {depth}, dim 1024, {S_frames} frames of 518x518")
    cam, pc = synth.make_hess_tables()
    model = build_vggt_aggregator(depth, 1024, 16, device=dev, tables=(pc, cam))
    images = synthetic_frames(S_frames, size=518, device=dev)
    ress.apply_ress(model, sr, n_iters=5)
    seen, captured = [], {}
    orig_fwd, orig_layer = wiring.ress_attention_forward, attn_mod.sparse_global_attention

    def spy_forward(*a, **kw):
        store = {}
        kw["aux_store"], kw["aux_full"] = store, False
        out = orig_fwd(*a, **kw)
        seen.append(store["value"].sparsity)
        return out

    def spy_layer(q, k, v, grid, **kw):
        if captured:
            return orig_layer(q, k, v, grid, **kw)
        kw["keep_intermediates"] = True
        res = orig_layer(q, k, v, grid, **kw)
        captured.update(q=q.cpu(), k=k.cpu(), v=v.cpu(), grid=grid, res=res, M=kw["M"].float().cpu())
        return res

    wiring.ress_attention_forward, attn_mod.sparse_global_attention = spy_forward, spy_layer
    try:
        with torch.no_grad():
            got = model(images)
    finally:
        wiring.ress_attention_forward, attn_mod.sparse_global_attention = orig_fwd, orig_layer
    torch.cuda.synchronize()
    assert len(seen) == depth and torch.isfinite(got).all()
    _say(f"[configs[3]] realised sparsity per layer: min {min(seen):.4f} max {max(seen):.4f}")
    for s in seen:
        assert abs(s - sr) <= 0.05, seen
    del model
    torch.cuda.empty_cache()
    plain = build_vggt_aggregator(depth, 1024, 16, device=dev, wire=False)
    with torch.no_grad():
        want = plain(images)
    torch.cuda.synchronize()
    cosine = torch.nn.functional.cosine_similarity(got.float().flatten(), want.float().flatten(), dim=0).item()
    _say(f"[configs[3]] cosine to the dense-attention model {cosine:.6f}")
    assert cosine >= 0.95
    del plain, want, got
    torch.cuda.empty_cache()
    # layer 0 through the oracle: the same Q/K/V, HeSS budget and M give the same map
    g, res = captured["grid"], captured["res"]
    _say(f"[configs[3]] oracle pipeline on global layer 0 (N={g.Tk}, q_blk={g.q_blk_p}, n_cand={g.n_cand})")
    hb = budget.HessBudget(cam, pc, lam=0.5)
    o = oracle_layer(captured["q"], captured["k"], captured["v"], g.frames, g.P, g.S, sparse_ratio=sr,
                     head_scores=hb.head_scores[0].numpy(), criterion="ress", M=captured["M"].numpy())
    assert np.array_equal(_np(res.final_map).reshape(o["map"].shape), o["map"])
    assert np.array_equal(_np(res.nvalid), o["nvalid"])
