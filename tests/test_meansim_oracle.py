"""The oracle's SpargeAttn-convention meansim block map (oracle_meansim_map) against its
definition, computed independently in float64 numpy: block means, the mean pairwise
cosine similarity (brute force over all token pairs), the masked pooled softmax, the
CDF count and the forced blocks (non-similar K blocks and Q rows, leading sinks).
SpargeAttn itself is not in the reference, so these pin the restatement, not upstream
(parity unpinned against SpargeAttn)."""

import numpy as np
import torch

import oracle


def _seq(seed, BH, T, corr):
    """bf16 tokens with block-correlated directions: a shared per-64-token direction plus noise."""
    rng = np.random.default_rng(seed)
    base = np.repeat(rng.normal(size=(BH, -(-T // 64), 64)), 64, axis=1)[:, :T]
    x = corr * base + rng.normal(size=(BH, T, 64))
    return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)


def _f64(x):
    return x.float().numpy().astype(np.float64)


def _block_stats64(x, BS, km=None):
    BH, T, _ = x.shape
    nb = -(-T // BS)
    pooled = np.zeros((BH, nb, 64))
    sim = np.zeros((BH, nb))
    for b in range(BH):
        for j in range(nb):
            xs = x[b, j * BS:(j + 1) * BS]
            if km is not None:
                xs = xs - km[b]
            pooled[b, j] = xs.mean(0)
            nrm = np.linalg.norm(xs, axis=1, keepdims=True)
            xh = np.where(nrm > 0, xs / np.where(nrm > 0, nrm, 1), 0)
            sim[b, j] = (xh @ xh.T).mean()  # mean pairwise cosine similarity, self pairs included
    return pooled, sim


def test_block_means_and_similarity():
    q, k = _seq(1, 3, 300, 1.5), _seq(2, 3, 200, 0.7)
    km = np.random.default_rng(3).normal(size=(3, 64)).astype(np.float32)
    pq, sq = _block_stats64(_f64(q), 128)
    pk, sk = _block_stats64(_f64(k), 64, km.astype(np.float64))
    for margin, want in ((-1e-3, 1), (1e-3, 0)):
        # per-block thresholds just below / above the float64 similarity -> flag 1 / 0
        for b in range(sq.shape[1]):
            o = oracle.meansim_map(q, k, km, simthreshd1=[sq[h, b] + margin for h in range(3)], H=3)
            assert (o["sim_q"][:, b] == want).all()
        for b in range(sk.shape[1]):
            o = oracle.meansim_map(q, k, km, simthreshd1=[sk[h, b] + margin for h in range(3)], H=3)
            assert (o["sim_k"][:, b] == want).all()
    o = oracle.meansim_map(q, k, km, H=3)
    np.testing.assert_allclose(o["pooled_q"], pq, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(o["pooled_k"], pk, rtol=1e-5, atol=1e-6)


def test_map_matches_definition():
    BH, Tq, Tk = 4, 700, 900
    q, k = _seq(5, BH, Tq, 0.6), _seq(6, BH, Tk, 0.9)
    km = _f64(k).mean(1).astype(np.float32)
    th, cd, sink = [0.02, 0.05, 0.3, 0.9], [0.9, 0.5, 0.95, 0.8], 150
    o = oracle.meansim_map(q, k, km, simthreshd1=th, cdfthreshd=cd, attention_sink=sink, H=BH)
    pq, sq = _block_stats64(_f64(q), 128)
    pk, sk = _block_stats64(_f64(k), 64, km.astype(np.float64))
    nq, nk = sq.shape[1], sk.shape[1]
    assert (o["sim_q"] == (sq > np.array(th)[:, None])).all() and (o["sim_k"] == (sk > np.array(th)[:, None])).all()
    for b in range(BH):
        for r in range(nq):
            s = pq[b, r] @ pk[b].T / 8.0
            simk = o["sim_k"][b].astype(bool)
            want = np.zeros(nk, bool)
            if simk.any():
                e = np.where(simk, np.exp(s - s[simk].max()), 0.0)
                p = e / e.sum()
                order = np.lexsort((np.arange(nk), -p))
                n = int((np.cumsum(p[order]) <= cd[b]).sum())
                want[order[:n]] = True
            want |= ~simk
            if not o["sim_q"][b, r]:
                want[:] = True
            want[:-(-sink // 64)] = True
            assert np.array_equal(o["map"][b, r].astype(bool), want), (b, r)


def test_codes_follow_the_block_quantiser():
    q, k = _seq(7, 2, 260, 0.5), _seq(8, 2, 130, 0.5)
    km = np.random.default_rng(9).normal(size=(2, 64)).astype(np.float32)
    o = oracle.meansim_map(q, k, km, H=2)
    ks = k.float().numpy() - km[:, None, :]
    for b in range(2):
        for j in range(3):
            blk = ks[b, 64 * j:64 * (j + 1)]
            scale = np.float32(np.abs(blk).max()) / np.float32(127)
            assert o["k_scale"][b, j] == scale
            y = blk / scale
            codes = np.trunc(y + np.where(y >= 0, 0.5, -0.5)).astype(np.int8)
            assert np.array_equal(o["k_i8"][b, 64 * j:64 * j + blk.shape[0]], codes)
