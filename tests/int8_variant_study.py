"""Study (not a pytest module): single-term INT8 QK^T variants against the unquantised softmax on
BASELINE rows -- TEST INFRASTRUCTURE, CPU only.

    python tests/int8_variant_study.py CONFIG [ROWS]     # CONFIG 0, 1 or 4

For a seeded sample of (head, q-block) rows of the BASELINE layer (its block map from the C oracle's
pipeline, every head's dense special row included), each variant quantises Q and K - km with amax/127
scales (round half away from zero: SpargeAttn's per_block_int8 rule, external/patches/spargeattn.patch:38-41)
at the granularity it names, forms the logits exactly in float64 from the codes, and the script prints the
worst max-abs, the median max-abs and the worst cosine of the rows' outputs against the float64 softmax of
the unquantised logits:

  ref_blockQ_blockK   one scale per 128-query block and per 64-key block (the reference's arithmetic)
  rowQ_blockK         one scale per query, per 64-key block
  rowQ_keyK           one scale per query and per key (a multiply per score)
  rowQ_blockK2        per query; K two-term (hi + lo/254) per block
  rowQ2_blockK        Q two-term per query; K single-term per block
  rowQ_blockK_smooth  per query, per block, after a per-dim rescale sqrt(amax_k / amax_q) moved from K to Q

The attention tolerance is 2e-2 max-abs and cosine 0.999.
"""

import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

from oracle import reference as ref  # noqa: E402
from pipeline_oracle import oracle_layer  # noqa: E402
from ress_amd import budget, synth  # noqa: E402

VARIANTS = ("ref_blockQ_blockK", "rowQ_blockK", "rowQ_keyK", "rowQ_blockK2", "rowQ2_blockK", "rowQ_blockK_smooth")


def quant(x, axes):
    """Symmetric INT8 of float64 `x` with one scale amax/127 per group, the groups being the
    slices over `axes`; returns the dequantised values."""
    amax = np.abs(x).max(axis=axes, keepdims=True)
    s = np.where(amax > 0, amax / 127.0, 1.0)
    y = x / s
    return np.trunc(y + 0.5 * np.sign(y)) * s


def quant2(x, axes):
    """Two-term INT8: hi at scale s, the residual at s/254 (clamped to +-127)."""
    amax = np.abs(x).max(axis=axes, keepdims=True)
    s = np.where(amax > 0, amax / 127.0, 1.0)
    y = x / s
    hi = np.trunc(y + 0.5 * np.sign(y))
    r = x - hi * s
    lo = np.clip(np.trunc(r / (s / 254.0) + 0.5 * np.sign(r)), -127, 127)
    return hi * s + lo * (s / 254.0)


def softmax_out(logits, val):
    p = np.exp(logits - logits.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return p @ val


class HeadKeys:
    """The smoothed keys of one head and their per-block / per-key quantisations."""

    def __init__(self, key, val):
        self.K, self.V = key, val
        self.nk = key.shape[0]
        nkb = -(-self.nk // 64)
        self.Ks = key - key.mean(0, keepdims=True)
        self.Kpad = np.zeros((nkb * 64, 64))
        self.Kpad[:self.nk] = self.Ks
        blocks = self.Kpad.reshape(nkb, 64, 64)
        self.K_block = quant(blocks, (1, 2)).reshape(-1, 64)[:self.nk]
        self.K_key = quant(self.Kpad, (1,))[:self.nk]
        self.K_block2 = quant2(blocks, (1, 2)).reshape(-1, 64)[:self.nk]


def row_logits(qq, hk, idx):
    """Every variant's logits of the queries qq (n, 64) against the kept keys idx."""
    q_row = quant(qq, (1,))
    out = {
        "ref_blockQ_blockK": quant(qq, (0, 1)) @ hk.K_block[idx].T,
        "rowQ_blockK": q_row @ hk.K_block[idx].T,
        "rowQ_keyK": q_row @ hk.K_key[idx].T,
        "rowQ_blockK2": q_row @ hk.K_block2[idx].T,
        "rowQ2_blockK": quant2(qq, (1,)) @ hk.K_block[idx].T,
    }
    a = np.sqrt((np.abs(hk.Ks[idx]).max(0) + 1e-12) / (np.abs(qq).max(0) + 1e-12))
    nkb = hk.Kpad.shape[0] // 64
    k_smooth = quant((hk.Kpad / a).reshape(nkb, 64, 64), (1, 2)).reshape(-1, 64)[:hk.nk]
    out["rowQ_blockK_smooth"] = quant(qq * a, (1,)) @ k_smooth[idx].T
    return {n: v * 0.125 for n, v in out.items()}


def evaluate(q, k, v, frames, P, S, o, rows):
    qp, qs = ref.split_tokens(q.double(), frames, P, S)
    kp, ks = ref.split_tokens(k.double(), frames, P, S)
    vp, vs = ref.split_tokens(v.double(), frames, P, S)
    key = kp if ks is None else torch.cat([kp, ks], -2)
    val = vp if vs is None else torch.cat([vp, vs], -2)
    T_p, T_s, Tk = frames * (P - S), frames * S, frames * P
    qbp = -(-T_p // 128)
    H = q.shape[1]
    err = {n: [] for n in VARIANTS}
    cos = {n: [] for n in VARIANTS}
    head = None
    for bh, qb in rows:  # sorted by head: each head's keys are quantised once
        b, h = divmod(bh, H)
        if head is None or head[0] != (b, h):
            head = ((b, h), HeadKeys(key[b, h].numpy(), val[b, h].numpy()))
        hk = head[1]
        if qb < qbp:
            qq = qp[b, h, qb * 128:min(qb * 128 + 128, T_p)].numpy()
        else:
            r0 = (qb - qbp) * 128
            qq = qs[b, h, r0:min(r0 + 128, T_s)].numpy()
        blocks = np.asarray(o["lut"][bh, qb, :o["nvalid"][bh, qb]])
        idx = np.concatenate([np.arange(c * 64, min(c * 64 + 64, Tk)) for c in blocks])
        want = softmax_out(qq @ hk.K[idx].T * 0.125, hk.V[idx])
        for n, logits in row_logits(qq, hk, idx).items():
            got = softmax_out(logits, hk.V[idx])
            err[n].append(np.abs(got - want).max())
            cos[n].append((got * want).sum() / np.sqrt((got * got).sum() * (want * want).sum()))
    return {n: (max(err[n]), float(np.median(err[n])), min(cos[n])) for n in VARIANTS}


def layer(cfg):
    """The BASELINE layer's inputs and the oracle's block map (configs[0], [1] or [4])."""
    frames = {0: 4, 1: 16, 4: 200}[cfg]
    q, k, v, meta = synth.make_layer_qkv(frames)
    P, S = meta["P"], meta["S"]
    if cfg == 1:
        cam, pc = synth.make_hess_tables()
        bud = budget.HessBudget(cam, pc, lam=0.5)
        o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=0.7, head_scores=bud.head_scores[0].numpy())
    elif cfg == 0:
        o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=0.5, cdf_threshold=0.9, sink_lead=22)
    else:
        o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=0.9, sink_lead=22)
    return q, k, v, frames, P, S, o


def main(cfg, n_rows=200):
    t0 = time.time()
    q, k, v, frames, P, S, o = layer(cfg)
    BH, qt = o["nvalid"].shape
    rng = np.random.default_rng(1)
    rows = sorted({(int(rng.integers(BH)), int(rng.integers(qt))) for _ in range(n_rows)}
                  | {(bh, qt - 1) for bh in range(BH)})
    print(f"configs[{cfg}]: layer ready in {time.time() - t0:.0f} s; {len(rows)} rows", flush=True)
    for n, (worst, med, cmin) in evaluate(q, k, v, frames, P, S, o, rows).items():
        print(f"  {n:22s} max-abs {worst:.4f}  median {med:.4f}  min-cos {cmin:.6f}", flush=True)


if __name__ == "__main__":
    main(int(sys.argv[1]), int(sys.argv[2]) if len(sys.argv) > 2 else 200)
