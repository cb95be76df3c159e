"""GPU parity of the SpargeAttn-convention meansim block map (meansim.hip,
ress_amd.sparge.get_block_map_meansim_fuse_quant) against the C oracle.

Everything the entry point returns is compared bit for bit: the map, the INT8 codes and
scales of Q and K - km, the pooled block means and the similarity flags. Cases cover
ragged sequence ends, zero tokens and an all-zero block, duplicated key blocks (tied
probabilities, broken by block index), per-head thresholds, rows where every key block
is non-similar, attention sinks that are and are not multiples of 64, strided (NHD)
inputs, and the full-sequence grid of the north-star shape (16 frames, 172 x 344)."""

import numpy as np
import pytest
import torch

import oracle
from ress_amd import sparge, synth

pytestmark = pytest.mark.gpu


def _qk(seed, B, H, Tq, Tk, dup=False, zeros=False):
    """bf16 q, k whose blocks mix near-parallel tokens (similar) and isotropic ones."""
    rng = np.random.default_rng(seed)

    def seq(T, bs):
        nb = -(-T // bs)
        strength = rng.choice([0.0, 0.3, 1.0, 3.0], size=(B, H, nb, 1))
        base = rng.normal(size=(B, H, nb, 64)) * strength
        x = np.repeat(base, bs, axis=2)[:, :, :T] + rng.normal(size=(B, H, T, 64))
        return x

    q, k = seq(Tq, 128), seq(Tk, 64)
    if dup and Tk >= 192:
        k[:, :, 128:192] = k[:, :, 0:64]          # key block 2 duplicates block 0
    if zeros:
        q[:, :, 5] = 0.0
        k[:, :, 7] = 0.0
        if Tk >= 128:
            k[:, :, 64:128] = 0.0                 # an all-zero key block (scale 0, norm 0)
    to = lambda a: torch.from_numpy(a.astype(np.float32)).to(torch.bfloat16)  # noqa: E731
    return to(q), to(k)


def _check(q, k, km, simth, cdfth, sink, dev, qdev=None, kdev=None):
    B, H, Tq, _ = q.shape
    Tk = k.shape[2]
    qd = q.to(dev) if qdev is None else qdev
    kd = k.to(dev) if kdev is None else kdev
    kmd = None if km is None else km.to(dev)
    fm, qi8, qs, ki8, ks = sparge.get_block_map_meansim_fuse_quant(
        qd, kd, km=kmd, simthreshd1=simth, cdfthreshd=cdfth, attention_sink=sink)
    torch.cuda.synchronize()
    want = oracle.meansim_map(q.reshape(B * H, Tq, 64), k.reshape(B * H, Tk, 64),
                              None if km is None else km.reshape(B * H, 64).numpy(),
                              simthreshd1=simth, cdfthreshd=cdfth, attention_sink=sink, H=H)
    nq, nk = want["map"].shape[1:]
    got_map = fm.cpu().numpy().reshape(B * H, nq, nk).astype(np.uint8)
    assert np.array_equal(got_map, want["map"]), np.argwhere(got_map != want["map"])[:5]
    assert np.array_equal(qi8.cpu().numpy().reshape(B * H, Tq, 64), want["q_i8"][:, :Tq])
    assert np.array_equal(ki8.cpu().numpy().reshape(B * H, Tk, 64), want["k_i8"][:, :Tk])
    # the padded rows behind the views are zero codes, as the attention kernel reads them
    assert np.array_equal(qi8.as_strided((B, H, nq * 128, 64), qi8.stride()).cpu().numpy().reshape(B * H, -1, 64),
                          want["q_i8"])
    assert np.array_equal(qs.cpu().numpy().reshape(B * H, nq).view(np.uint32), want["q_scale"].view(np.uint32))
    assert np.array_equal(ks.cpu().numpy().reshape(B * H, nk).view(np.uint32), want["k_scale"].view(np.uint32))
    return fm, want


# key-block counts 4, 3, 24 (one column per lane), 65, 188, 625 (2, 4, 16 per lane) and
# 1026 (the workgroup-per-row kernel beyond 1024)
@pytest.mark.parametrize("B,H,Tq,Tk,sink", [(1, 2, 300, 250, 0), (2, 3, 128, 130, 1), (1, 4, 1000, 1500, 150),
                                            (1, 2, 513, 4097, 128), (1, 2, 700, 12000, 64), (1, 1, 1030, 40000, 0),
                                            (1, 1, 300, 65636, 0)])
def test_meansim_bit_exact(dev, B, H, Tq, Tk, sink):
    q, k = _qk(B * 1000 + Tq + Tk, B, H, Tq, Tk, dup=True, zeros=True)
    km = k.float().mean(2, keepdim=True)
    simth = [0.3, 0.05, 0.4, 0.1][:H]
    cdfth = [0.9, 0.5, 0.98, 0.7][:H]
    fm, want = _check(q, k, km, simth, cdfth, sink, dev)
    # the cases reach both similarity outcomes, CDF-selected and forced blocks
    assert 0 < want["sim_k"].mean() < 1 and 0 < want["sim_q"].mean() <= 1
    assert 0 < fm.float().mean().item() < 1


# Tied probabilities across most of a row and thresholds at the edges of the cut's
# definition: negative (nothing cut in), 0, inside a tie group, exactly 1, above 1 and above
# the 8192 clamp. Both map kernels: 63 key blocks (one wave per row) and 1094 (a workgroup).
@pytest.mark.parametrize("Tk", [4000, 70000])
def test_meansim_cut_with_ties_and_edge_thresholds(dev, Tk):
    H, Tq = 6, 500
    rng = np.random.default_rng(Tk)
    q = rng.normal(size=(1, H, Tq, 64))
    blk = rng.normal(size=(1, H, 64, 64)) + 2.0 * rng.normal(size=(1, H, 1, 64))
    nk = -(-Tk // 64)
    k = np.tile(blk, (1, 1, nk, 1))[:, :, :Tk]             # every key block the same ...
    for j in (3, 17, nk - 2):                              # ... but three
        k[:, :, 64 * j:64 * j + 64] += 1.5 * rng.normal(size=(1, H, 1, 64))
    to = lambda a: torch.from_numpy(a.astype(np.float32)).to(torch.bfloat16)  # noqa: E731
    q, k = to(q), to(k)
    cdfth = [-0.5, 0.0, 0.37, 1.0, 5.0, 1.0e5]
    fm, want = _check(q, k, None, [0.0] * H, cdfth, 0, dev)
    kept = want["map"].reshape(H, -1, nk).sum(-1)
    assert (kept[0] == 0).all()                           # tau < 0: nothing is cut in, nothing forced
    assert (kept[5] == nk).all() and (kept[4] == nk).all()  # tau >= 1 keeps every block


def test_meansim_longest_rows(dev):
    """4100 key blocks (the workgroup kernel: radix CDF descent over the row in LDS, ties
    ranked by a workgroup scan)."""
    q, k = _qk(12, 1, 1, 1030, 4100 * 64, dup=True, zeros=True)
    _check(q, k, k.float().mean(2, keepdim=True), 0.2, 0.95, 1374, dev)


@pytest.mark.parametrize("with_workspace", [True, False], ids=["gemm_scores", "row_scores"])
def test_meansim_long_rows_both_score_paths(dev, with_workspace, monkeypatch):
    """Rows past 1024 key blocks, with the workspace (the scores of every row by one
    matrix-core GEMM, DOT64 exactly) and without it (each row's workgroup scores its own
    columns): the same map and codes as the oracle either way; ragged row and column tiles
    (q blocks not a multiple of 128, key blocks not a multiple of 128)."""
    if not with_workspace:
        monkeypatch.setattr(sparge, "_meansim_workspace", lambda *a: (None, 0))
    q, k = _qk(21, 1, 2, 300 * 128 - 77, 1100 * 64 + 13, dup=True, zeros=True)
    print(f"[meansim long rows workspace={with_workspace}] nq=300 nk=1101", flush=True)
    _check(q, k, k.float().mean(2, keepdim=True), [0.1, 0.3], [0.9, 0.5], 200, dev)


def test_meansim_no_km_scalar_thresholds(dev):
    q, k = _qk(7, 1, 3, 700, 900)
    _check(q, k, None, 0.1, 0.9, 0, dev)


def test_meansim_all_nonsimilar_rows(dev):
    """A head whose threshold no block reaches: every K block is forced on, every row full."""
    q, k = _qk(8, 1, 2, 400, 640)
    fm, want = _check(q, k, None, [2.0, 0.1], [0.9, 0.9], 0, dev)
    assert fm[0, 0].all()
    assert not fm[0, 1].all()


def test_meansim_strided_inputs(dev):
    """NHD storage viewed as HND: non-contiguous head and token strides."""
    q, k = _qk(9, 2, 4, 384, 576)
    qn = q.transpose(1, 2).contiguous().to(dev).transpose(1, 2)
    kn = k.transpose(1, 2).contiguous().to(dev).transpose(1, 2)
    km = k.float().mean(2, keepdim=True)
    _check(q, k, km, 0.15, 0.8, 70, dev, qdev=qn, kdev=kn)


def test_meansim_return_lut(dev):
    q, k = _qk(10, 1, 2, 600, 800)
    qd, kd = q.to(dev), k.to(dev)
    fm, *_ = sparge.get_block_map_meansim_fuse_quant(qd, kd, simthreshd1=0.1, cdfthreshd=0.9, attention_sink=64)
    lut, nv, *_ = sparge.get_block_map_meansim_fuse_quant(qd, kd, simthreshd1=0.1, cdfthreshd=0.9, attention_sink=64,
                                                          return_lut=True)
    m = fm.cpu().numpy()
    lut, nv = lut.cpu().numpy(), nv.cpu().numpy()
    for b in range(m.shape[0]):
        for h in range(m.shape[1]):
            for r in range(m.shape[2]):
                cols = np.flatnonzero(m[b, h, r])
                assert nv[b, h, r] == cols.size and np.array_equal(lut[b, h, r, :cols.size], cols)
                assert m[b, h, r, 0]  # the sink block


def test_meansim_codes_match_per_block_int8(dev):
    """The fused pass quantises exactly as the standalone per_block_int8 entry point."""
    q, k = _qk(11, 1, 2, 700, 900, zeros=True)
    qd, kd = q.to(dev), k.to(dev)
    km = kd.float().mean(2).reshape(2, 64).contiguous()
    _, qi8, qs, ki8, ks = sparge.get_block_map_meansim_fuse_quant(qd, kd, km=km)
    qi8b, qsb, ki8b, ksb = sparge.per_block_int8(qd, kd, km=km)
    for a, b in ((qi8, qi8b), (ki8, ki8b)):
        assert torch.equal(a, b)
    for a, b in ((qs, qsb), (ks, ksb)):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_meansim_full_sequence(dev):
    """The north-star shape: 16 frames of 1374 tokens, H=16, full 172 x 344 grid, K smoothed
    by its mean, the leading 1374 tokens (22 blocks) as sinks."""
    q, k, _, _ = synth.make_layer_qkv(16)
    km = k.float().mean(2, keepdim=True)
    print("meansim full sequence: q", tuple(q.shape), flush=True)
    fm, want = _check(q, k, km, 0.1, 0.9, 1374, dev)
    assert fm.shape == (1, 16, 172, 344)
    assert fm[..., :22].all()
