"""GPU parity of the ReSS restore-swap kernel (ress_swap.hip) against the C oracle.

Keep sets, the drift scores s and the objective J of the returned set are compared bit
for bit, across row counts and lengths that exercise every tiling edge of the kernels and
the modes the criterion grammar reaches; then the whole ReSS layer (HeSS budget +
restore_swap_iter5_bf16_trackbest + selection + attention) against the oracle pipeline."""

import numpy as np
import pytest
import torch

import oracle
from oracle import reference as ref
from pipeline_oracle import oracle_layer, row_sample
from ress_amd import _lib, budget, synth
from ress_amd.attention import sparse_global_attention
from ress_amd.kernels import LayerGrid

pytestmark = pytest.mark.gpu

ATOL, MIN_COS = 2e-2, 0.999


def _problem(seed, H, q_blk, kb_p, n_cand):
    rng = np.random.default_rng(seed)
    A = np.exp(rng.normal(size=(H, q_blk, kb_p)) * 2.0)
    A = (A / A.sum(-1, keepdims=True)).astype(np.float32)
    V = rng.normal(size=(H, kb_p, 64)).astype(np.float32)
    W = rng.normal(size=(H, 64, 64)).astype(np.float32) / 8
    M = np.einsum("hji,hjk->hik", W, W).astype(np.float32)
    nts = rng.integers(2, n_cand + 2, size=(H, q_blk)).astype(np.int32)
    return A, V, M, nts


def _gpu_restore_swap(A, V, M, nts, n_cand, n_iters, restore_frac, decay, flags, dev):
    H, q_blk, kb_p = A.shape
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    key = torch.empty(H, q_blk, n_cand, device=dev)
    s = torch.empty(H, q_blk, n_cand, device=dev)
    obj = torch.empty(H, q_blk, device=dev)
    ws_bytes = _lib.lib().ress_restore_swap_workspace_size(H, q_blk, kb_p, n_cand)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    Ad, Vd, Md, nd = t(A), t(V), t(M), t(nts)
    _lib.call("ress_restore_swap", _lib.ptr(Ad), _lib.ptr(Vd), _lib.ptr(Md), _lib.ptr(nd), H, H, q_blk, kb_p,
              n_cand, n_iters, restore_frac, decay, flags, _lib.ptr(key), _lib.ptr(obj), _lib.ptr(s), _lib.ptr(ws),
              ws_bytes, _lib.stream_handle(dev))
    torch.cuda.synchronize()
    return key.cpu().numpy(), s.cpu().numpy(), obj.cpu().numpy()


# (heads, rows, key blocks, candidates): row lengths across every selection width (candidate
# slots per lane 4..32), key-block chunks of the P @ v_bar sums (partial last chunk),
# candidate tiles of the product GEMM (partial last tile), row groups of the sums (16 rows,
# ragged last group) and row tiles of the GEMM (128 rows, ragged last tile)
SHAPES = [(2, 7, 40, 39), (3, 9, 130, 129), (2, 37, 300, 299), (2, 5, 685, 684), (1, 3, 900, 899),
          (1, 150, 700, 700), (1, 3, 1100, 1100), (1, 2, 1369, 1368), (1, 2, 1800, 1799)]
MODES = {
    "ress_recipe": (5, 0.5, 0.5, 1 | 2),
    "fp32": (5, 0.5, 0.5, 2),
    "single_round": (1, 0.5, 0.5, 1),
    "flat_schedule": (6, 0.3, 0.3, 1 | 2),
    "antiswap": (5, 0.5, 0.5, 1 | 2 | 4),
    "anti": (5, 0.5, 0.5, 1 | 2 | 4 | 8),
    "no_renorm": (3, 0.5, 0.5, 1 | 2 | 16),
    "cut_only": (0, 0.5, 0.5, 1 | 2),
}


@pytest.mark.parametrize("shape", SHAPES, ids=[f"k{s[2]}" for s in SHAPES])
@pytest.mark.parametrize("mode", list(MODES))
def test_kernel_matches_oracle(shape, mode, dev):
    H, q_blk, kb_p, n_cand = shape
    n_iters, rf, dc, flags = MODES[mode]
    print(f"[restore-swap {mode}] H={H} q_blk={q_blk} kb_p={kb_p} n_cand={n_cand}", flush=True)
    A, V, M, nts = _problem(kb_p + flags, H, q_blk, kb_p, n_cand)
    key, s, obj = _gpu_restore_swap(A, V, M, nts, n_cand, n_iters, rf, dc, flags, dev)
    keep, J, s_o = oracle.restore_swap(A, V, M, nts, n_cand, n_iters=n_iters, restore_frac=rf, decay=dc,
                                       big_bf16=bool(flags & 1), track_best=bool(flags & 2),
                                       maximize=bool(flags & 4), invert_cut=bool(flags & 8),
                                       renormalize=not (flags & 16), want_s=True)
    assert np.array_equal(s.view(np.uint32), s_o.view(np.uint32))
    assert np.array_equal(key > 0.5, keep.astype(bool))
    assert np.array_equal(obj.view(np.uint32), J.view(np.uint32))


def test_rank_by_api_reproduces_reference_form(dev):
    """restore_swap_rank_by returns where(drop, s, s + max|s| + 1) in big_dtype, whose
    top-nts is the keep set."""
    from ress_amd.projected import restore_swap_rank_by
    H, q_blk, kb_p, n_cand = 2, 6, 70, 69
    A, V, M, nts = _problem(5, H, q_blk, kb_p, n_cand)
    t = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
    rb = restore_swap_rank_by(t(A), t(V), t(M), t(nts), n_iters=5, track_best=True, big_dtype=torch.bfloat16,
                              n_cand=n_cand)
    keep, _, s_o = oracle.restore_swap(A, V, M, nts, n_cand, want_s=True)
    assert rb.dtype == torch.bfloat16 and rb.shape == (H, q_blk, n_cand)
    s_b = torch.from_numpy(s_o).to(torch.bfloat16)
    want = torch.where(torch.from_numpy(keep.astype(bool)), s_b + (s_b.abs().amax() + 1.0), s_b)
    assert torch.equal(rb.cpu(), want)


def test_ress_layer_pipeline(dev):
    """ReSS on one layer: HeSS budget, restore_swap_iter5_bf16_trackbest on the pooled map,
    selection, attention -- final map bit-exact against the oracle pipeline, output within
    the attention tolerance."""
    frames, H, sr = 8, 4, 0.8
    q, k, v, meta = synth.make_layer_qkv(frames, H=H)
    P, S = meta["P"], meta["S"]
    g = LayerGrid(1, H, frames, P, S)
    W_O = synth.make_w_o(dim=H * 64)
    M = torch.stack([W_O[:, h * 64:(h + 1) * 64].T @ W_O[:, h * 64:(h + 1) * 64] for h in range(H)])
    cam, pc = synth.make_hess_tables(n_heads=H)
    bud = budget.HessBudget(cam, pc, lam=0.5)
    res = sparse_global_attention(q.to(dev), k.to(dev), v.to(dev), g,
                                  budget_fn=lambda a: bud.num_to_select(0, a, sr, None, 1.0),
                                  block_criterion="restore_swap_iter5_bf16_trackbest", M=M.to(dev),
                                  keep_intermediates=True)
    torch.cuda.synchronize()
    o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=sr, head_scores=bud.head_scores[0].numpy(), H=H)
    counts = np.maximum(o["counts"].reshape(H, g.q_blk_p), min(2, g.n_cand)).astype(np.int32)
    keep, _ = oracle.restore_swap(o["attn_full"].reshape(H, g.q_blk_p, g.kb_p), o["pooled_v"].reshape(H, g.kb_p, 64),
                                  M.numpy(), counts, g.n_cand, n_iters=5, big_bf16=True, track_best=True)
    fmap, lut, nvalid = oracle.select_blocks(keep.astype(np.float32), counts, g.q_blk_total, g.kb_tot,
                                             min_select=min(2, g.n_cand))
    assert np.array_equal(res.final_map.cpu().numpy().reshape(fmap.shape), fmap)
    assert np.array_equal(res.nvalid.cpu().numpy(), nvalid)
    print(f"[ress f{frames} H{H}] realized sparsity {res.sparsity():.4f}")
    rows = row_sample(nvalid, 10)
    refs = ref.masked_attention_rows(q, k, v, frames, P, S, lut, nvalid, rows)
    out = res.out.float().cpu().reshape(-1, g.Tk, 64)
    for (bh, qb), (tok, r) in refs.items():
        got = out[bh, torch.from_numpy(tok)]
        assert (got - r).abs().max().item() <= ATOL
        assert torch.nn.functional.cosine_similarity(got.flatten(), r.flatten(), dim=0).item() >= MIN_COS
