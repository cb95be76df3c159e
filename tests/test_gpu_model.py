"""The public API on a whole model (reference src/ress/api.py:95-144 through the patched
global-attention forward, wiring.py:76-106): a small VGGT-style aggregator with random
weights, its global blocks wired to the block-sparse forward.

* apply_dense and apply_sparse_vggt at sparse_ratio 0 (every block kept, so the HIP
  sparse kernels compute full attention) reproduce the unwired model's plain-SDPA
  forward within bf16 tolerance;
* apply_sparse_vggt / apply_hess / apply_ress at a real sparse ratio run on every
  global layer, keep about the requested fraction of blocks, and stay close to dense;
* switching modes back to dense restores the dense output exactly (modes do not leak)."""

import numpy as np
import pytest
import torch

import ress_amd as ress
import ress_amd.wiring as wiring
from ress_amd import budget, synth
from ress_amd.aggregator import build_vggt_aggregator, synthetic_frames

pytestmark = pytest.mark.gpu

DEPTH, DIM, HEADS, FRAMES, SIZE = 2, 256, 4, 8, 196   # 8 frames x (14*14 + 5) = 1608 tokens


def _cos(a, b):
    return torch.nn.functional.cosine_similarity(a.float().flatten(), b.float().flatten(), dim=0).item()


@pytest.fixture(scope="module")
def models(dev):
    tables = synth.make_hess_tables(n_layers=DEPTH, n_heads=HEADS)
    wired = build_vggt_aggregator(DEPTH, DIM, HEADS, device=dev, tables=(tables[1], tables[0]))
    plain = build_vggt_aggregator(DEPTH, DIM, HEADS, device=dev, wire=False)
    images = synthetic_frames(FRAMES, size=SIZE, device=dev)
    with torch.no_grad():
        want = plain(images)
    torch.cuda.synchronize()
    return wired, images, want


def test_dense_and_all_blocks_match_plain_sdpa(models):
    model, images, want = models
    with torch.no_grad():
        ress.apply_dense(model)
        got_dense = model(images)
        ress.apply_sparse_vggt(model, 0.0)
        got_sparse = model(images)
    torch.cuda.synchronize()
    for got in (got_dense, got_sparse):
        assert torch.isfinite(got).all()
        assert _cos(got, want) >= 0.999
        assert (got.float() - want.float()).abs().max().item() <= 5e-2 * want.float().abs().max().item()


@pytest.mark.parametrize("mode", ["sparse_vggt", "hess", "ress"])
def test_sparse_modes_run_every_layer(models, mode):
    model, images, want = models
    sr = 0.5
    seen = []  # each global layer's realised sparsity, through the forward's aux store
    with torch.no_grad():
        if mode == "sparse_vggt":
            ress.apply_sparse_vggt(model, sr)
        elif mode == "hess":
            ress.apply_hess(model, sr)
        else:
            ress.apply_ress(model, sr, n_iters=5)
        orig = wiring.ress_attention_forward

        def spy(*a, **kw):
            store = {}
            kw["aux_store"] = store
            kw["aux_full"] = False
            out = orig(*a, **kw)
            seen.append(store["value"].sparsity)
            return out

        wiring.ress_attention_forward = spy
        try:
            got = model(images)
        finally:
            wiring.ress_attention_forward = orig
    torch.cuda.synchronize()
    assert len(seen) == DEPTH
    assert torch.isfinite(got).all()
    # about half of the candidate blocks dropped (sinks and dense special rows keep some)
    for s in seen:
        assert 0.2 <= s <= 0.6, seen
    assert _cos(got, want) >= 0.95


def test_realized_drift_recorded_per_layer(models):
    """record_realized_drift over a ReSS forward: one finite J >= 0 per global layer, in
    forward order; nothing is recorded once the recorder is closed."""
    from ress_amd import projected
    model, images, _ = models
    with torch.no_grad():
        ress.apply_ress(model, 0.5, n_iters=5)
        with projected.record_realized_drift() as rec:
            model(images)
        model(images)
    torch.cuda.synchronize()
    assert len(rec) == DEPTH, rec
    assert all(np.isfinite(j) and j >= 0.0 for j in rec), rec


@pytest.mark.parametrize("max_pos", [38, 5000], ids=["grid", "large_positions"])
def test_fused_qk_norm_rope_matches_modules(max_pos, dev):
    """The fused q/k LayerNorm + 2D RoPE kernel against the torch modules it replaces:
    v is copied exactly; q and k agree to bf16 rounding (the kernel's hardware cos/sin for
    patch-grid positions, the library functions beyond 256, and its LayerNorm reduction
    order are its own)."""
    from ress_amd.aggregator import Attention, RoPE2D
    from ress_amd.qkv import fused_qk_norm_rope
    torch.manual_seed(3)
    attn = Attention(256, 4, RoPE2D()).to(dev, torch.bfloat16)
    with torch.no_grad():
        for n in (attn.q_norm, attn.k_norm):
            n.weight.uniform_(0.5, 1.5)
            n.bias.uniform_(-0.2, 0.2)
    B, T = 2, 300
    x = torch.randn(B, T, 256, device=dev).to(torch.bfloat16)
    pos = torch.randint(0, max_pos, (B, T, 2), device=dev)
    with torch.no_grad():
        qkv = attn.qkv(x)
        q, k, v = fused_qk_norm_rope(attn, qkv, pos, 4)
        rq, rk, rv = qkv.reshape(B, T, 3, 4, 64).permute(2, 0, 3, 1, 4).unbind(0)
        rq, rk = attn.rope(attn.q_norm(rq), pos), attn.rope(attn.k_norm(rk), pos)
    torch.cuda.synchronize()
    assert torch.equal(v, rv.contiguous())
    for got, want in ((q, rq), (k, rk)):
        err = (got.float() - want.float()).abs()
        assert err.max().item() <= 2 ** -6 * want.float().abs().max().item()
        assert (err > 0).float().mean().item() < 0.02  # nearly all bit-identical


class _RowColRotary(torch.nn.Module):
    """A backbone-style 2D rotary module written apart from this package's RoPE2D: angle
    tables per position built once per call, the halves taken with chunk, positions read
    as (row, column). round_tables rounds cos/sin to the token dtype before use, as some
    backbones cache them."""

    def __init__(self, frequency=100.0, round_tables=False):
        super().__init__()
        self.frequency = frequency
        self.round_tables = round_tables

    def _one(self, x, p):
        d = x.shape[-1]
        inv = self.frequency ** (-torch.arange(0, d, 2, device=x.device, dtype=torch.float32) / d)
        ang = torch.einsum("bt,f->btf", p.to(torch.float32), inv)
        ang = torch.cat((ang, ang), dim=-1)[:, None]
        cos, sin = ang.cos(), ang.sin()
        if self.round_tables:
            cos, sin = cos.to(x.dtype).float(), sin.to(x.dtype).float()
        a, b = x.float().chunk(2, dim=-1)
        return x.float() * cos + torch.cat((-b, a), dim=-1) * sin

    def forward(self, tokens, positions):
        rows, cols = tokens.chunk(2, dim=-1)
        return torch.cat((self._one(rows, positions[..., 0]), self._one(cols, positions[..., 1])),
                         dim=-1).to(tokens.dtype)


@pytest.mark.parametrize("round_tables", [False, True], ids=["fp32_tables", "bf16_tables"])
def test_fused_path_takes_a_declared_foreign_rope(round_tables, dev):
    """A RoPE module that is not this package's, declared with declare_rope, takes the fused
    kernel; its q and k against the module's own torch norms and rotation: with fp32
    angle tables nearly all bit-identical, with tables rounded to bf16 within the bf16
    rounding of cos/sin. An undeclared module keeps the torch path."""
    from ress_amd.aggregator import Attention
    from ress_amd.qkv import _fusable, declare_rope, fused_qk_norm_rope
    torch.manual_seed(5)
    rope = _RowColRotary(100.0, round_tables)
    attn = Attention(256, 4, rope).to(dev, torch.bfloat16)
    with torch.no_grad():
        for n in (attn.q_norm, attn.k_norm):
            n.weight.uniform_(0.5, 1.5)
            n.bias.uniform_(-0.2, 0.2)
    B, T = 2, 300
    x = torch.randn(B, T, 256, device=dev).to(torch.bfloat16)
    pos = torch.randint(0, 38, (B, T, 2), device=dev)
    assert not _fusable(attn, x, 64)
    declare_rope(rope, base=rope.frequency)
    assert _fusable(attn, x, 64)
    with torch.no_grad():
        qkv = attn.qkv(x)
        q, k, v = fused_qk_norm_rope(attn, qkv, pos, 4)
        rq, rk, rv = qkv.reshape(B, T, 3, 4, 64).permute(2, 0, 3, 1, 4).unbind(0)
        rq, rk = rope(attn.q_norm(rq), pos), rope(attn.k_norm(rk), pos)
    torch.cuda.synchronize()
    assert torch.equal(v, rv.contiguous())
    for got, want in ((q, rq), (k, rk)):
        err = (got.float() - want.float()).abs()
        scale = want.float().abs().max().item()
        print(f"[declared rope {round_tables}] max-abs {err.max().item():.3e} of {scale:.3e}")
        assert err.max().item() <= (2 ** -5 if round_tables else 2 ** -6) * scale
        if not round_tables:
            assert (err > 0).float().mean().item() < 0.02  # nearly all bit-identical


def test_modes_do_not_leak(models):
    model, images, _ = models
    with torch.no_grad():
        ress.apply_dense(model)
        a = model(images)
        ress.apply_ress(model, 0.7)
        model(images)
        ress.apply_dense(model)
        b = model(images)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_eager_check_raises_in_the_forward_and_dense_clears_status(models):
    """A HeSS budget that cannot converge (iteration cap 1, one head wanting far more than
    the candidate count) is reported by check_layers after the forward by default, and by the
    forward itself with the module attribute eager_check (the reference raises at once,
    _proportional.py:112-113). A later dense forward leaves nothing to report."""
    model, images, _ = models
    scores = torch.full((3, DEPTH, HEADS), 1.0)
    scores[0, :, 0] = 50.0
    hb = budget.HessBudget(scores, scores, lam=0.5, max_iters=1)
    attns = wiring.global_attns(model)
    try:
        with torch.no_grad():
            ress.apply_hess(model, 0.2)
            for a in attns:
                a.budget_fn = lambda ap: hb.num_to_select(0, ap, 0.2, None, 1.0)
            model(images)
            with pytest.raises(RuntimeError, match="did not converge"):
                ress.check_layers(model)
            for a in attns:
                a.eager_check = True
            with pytest.raises(RuntimeError, match="did not converge"):
                model(images)
            for a in attns:
                a.eager_check = False
            ress.apply_dense(model)
            model(images)
        ress.check_layers(model)
    finally:
        for a in attns:
            a.eager_check = False
        ress.apply_dense(model)
