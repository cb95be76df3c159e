"""Study (not a pytest module): single-term INT8 QK^T variants against the fp64 masked softmax on
BASELINE rows -- TEST INFRASTRUCTURE, CPU only.

    python tests/int8_variant_study.py CONFIG [ROWS]     # CONFIG 0, 1 or 4

For a seeded sample of (head, q-block) rows of the BASELINE layer (its block map from the C oracle's
pipeline), every variant quantises Q and K - km with amax/127 scales (round half away from zero,
SpargeAttn's per_block_int8 rule, external/patches/spargeattn.patch:38-41) at the granularity it names,
forms the logits exactly in float64 from the codes, and prints the worst max-abs / median max-abs / worst
cosine of the output against the unquantised softmax:
  ref_blockQ_blockK   one scale per 128-query block and per 64-key block (the reference's arithmetic)
  rowQ_blockK         one scale per query, per 64-key block
  rowQ_keyK           one scale per query and per key (a multiply per score)
  rowQ_blockK2        per query; K two-term (hi + lo/254) per block
  rowQ2_blockK        Q two-term per query; K single-term per block
  rowQ_blockK_smooth  per query, per block, after a per-dim rescale sqrt(amax_k/amax_q) moved from K to Q
The output tolerance is 2e-2 max-abs and cosine 0.999."""
import sys, time, math
import numpy as np, torch
ROOT = __import__('os').path.dirname(__import__('os').path.dirname(__import__('os').path.abspath(__file__)))
sys.path.insert(0, ROOT); sys.path.insert(0, ROOT + '/tests')
from ress_amd import synth, budget
from oracle import reference as ref
from pipeline_oracle import oracle_layer

def quant(x, axis_keep):
    """per-group symmetric int8: scale = amax/127, round half away from zero. x float64 (..,64);
    groups = all axes not in axis_keep are reduced for amax."""
    amax = np.abs(x).max(axis=axis_keep, keepdims=True)
    s = np.where(amax > 0, amax / 127.0, 1.0)
    y = x / s
    qv = np.trunc(y + 0.5 * np.sign(y))
    return qv, s

def quant2(x, axis_keep):
    hi, s = quant(x, axis_keep)
    r = x - hi * s
    s2 = s / 254.0
    lo = np.clip(np.trunc(r / s2 + 0.5 * np.sign(r)), -127, 127)
    return hi * s + lo * s2

def rows_eval(q, k, v, frames, P, S, o, rows):
    qp, qs = ref.split_tokens(q.double(), frames, P, S)
    kp, ks = ref.split_tokens(k.double(), frames, P, S)
    vp, vs = ref.split_tokens(v.double(), frames, P, S)
    key = kp if ks is None else torch.cat([kp, ks], -2)
    val = vp if vs is None else torch.cat([vp, vs], -2)
    T_p, T_s, Tk = frames * (P - S), frames * S, frames * P
    qbp = -(-T_p // 128)
    H = q.shape[1]
    names = ['ref_blockQ_blockK', 'rowQ_blockK', 'rowQ_keyK', 'rowQ_blockK2', 'rowQ2_blockK', 'rowQ_blockK_smooth']
    err = {n: [] for n in names}
    cosm = {n: [] for n in names}
    cache = {}
    for bh, qb in rows:
        b, h = divmod(bh, H)
        blocks = np.asarray(o['lut'][bh, qb, :o['nvalid'][bh, qb]])
        if qb < qbp:
            qq = qp[b, h, qb*128:min(qb*128+128, T_p)].numpy()
        else:
            r0 = (qb - qbp)*128; qq = qs[b, h, r0:min(r0+128, T_s)].numpy()
        if cache.get('bh') != (b, h):
            K = key[b, h].numpy(); V = val[b, h].numpy()
            km = K.mean(0, keepdims=True)
            Ks = K - km
            nk = Ks.shape[0]; nkb = -(-nk // 64)
            Kpad = np.zeros((nkb*64, 64)); Kpad[:nk] = Ks
            Kb = Kpad.reshape(nkb, 64, 64)
            kh, ksc = quant(Kb, (1, 2)); Kr = (kh * ksc).reshape(-1, 64)[:nk]
            kh2, ksc2 = quant(Kpad, (1,)); Kk = (kh2 * ksc2)[:nk]
            K2 = quant2(Kb, (1, 2)).reshape(-1, 64)[:nk]
            cache.update(bh=(b, h), K=K, V=V, Ks=Ks, nk=nk, nkb=nkb, Kpad=Kpad, Kr=Kr, Kk=Kk, K2=K2)
        K, V, Ks, nk, nkb, Kpad = (cache[x] for x in ('K', 'V', 'Ks', 'nk', 'nkb', 'Kpad'))
        Kr, Kk, K2 = cache['Kr'], cache['Kk'], cache['K2']
        idx = np.concatenate([np.arange(c*64, min(c*64+64, Tk)) for c in blocks])
        exact = qq @ K[idx].T * 0.125
        def out_of(sc):
            p = np.exp(sc - sc.max(-1, keepdims=True)); p /= p.sum(-1, keepdims=True)
            return p @ V[idx]
        o_ref = out_of(exact)
        # reference: per-block Q (the 128-query block), per-block K
        qh, qsc = quant(qq, (0, 1)); Qr = qh * qsc
        variants = {}
        variants['ref_blockQ_blockK'] = Qr @ Kr[idx].T * 0.125
        qh, qsc = quant(qq, (1,)); Qq = qh * qsc
        variants['rowQ_blockK'] = Qq @ Kr[idx].T * 0.125
        variants['rowQ_keyK'] = Qq @ Kk[idx].T * 0.125
        variants['rowQ_blockK2'] = Qq @ K2[idx].T * 0.125
        Q2 = quant2(qq, (1,))
        variants['rowQ2_blockK'] = Q2 @ Kr[idx].T * 0.125
        # per-dim smoothing (SmoothQuant-style): q_d * a_d, k_d / a_d, a_d = sqrt(amax_k_d / amax_q_d)
        aq = np.abs(qq).max(0) + 1e-12; ak = np.abs(Ks[idx]).max(0) + 1e-12
        a = np.sqrt(ak / aq)
        qh, qsc = quant(qq * a, (1,)); Qs = qh * qsc
        Kbs = (Kpad / a).reshape(nkb, 64, 64)
        kh, ksc = quant(Kbs, (1, 2)); Ksm = (kh * ksc).reshape(-1, 64)[:nk]
        variants['rowQ_blockK_smooth'] = Qs @ Ksm[idx].T * 0.125
        for n, sc in variants.items():
            od = out_of(sc)
            err[n].append(np.abs(od - o_ref).max())
            c = (od * o_ref).sum() / np.sqrt((od*od).sum() * (o_ref*o_ref).sum())
            cosm[n].append(c)
    return {n: (max(err[n]), min(cosm[n]), float(np.median(err[n]))) for n in names}

def main(cfg):
    t0 = time.time()
    if cfg == 1:
        frames = 16
        q, k, v, meta = synth.make_layer_qkv(frames)
        P, S = meta['P'], meta['S']
        cam, pc = synth.make_hess_tables()
        bud = budget.HessBudget(cam, pc, lam=0.5)
        o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=0.7, head_scores=bud.head_scores[0].numpy())
    elif cfg == 0:
        frames = 4
        q, k, v, meta = synth.make_layer_qkv(frames)
        P, S = meta['P'], meta['S']
        o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=0.5, cdf_threshold=0.9, sink_lead=22)
    else:
        frames = 200
        q, k, v, meta = synth.make_layer_qkv(frames)
        P, S = meta['P'], meta['S']
        o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=0.9, sink_lead=22)
    BH, qt = o['nvalid'].shape
    rng = np.random.default_rng(1)
    nrows = int(sys.argv[2]) if len(sys.argv) > 2 else 200
    rows = sorted({(int(rng.integers(BH)), int(rng.integers(qt))) for _ in range(nrows)} | {(bh, qt-1) for bh in range(BH)})
    print(f'cfg {cfg}: layer ready in {time.time()-t0:.0f}s; {len(rows)} rows', flush=True)
    r = rows_eval(q, k, v, frames, P, S, o, rows)
    for n, (e, c, med) in r.items():
        print(f'  {n:22s} max-abs {e:.4f}  median {med:.4f}  min-cos {c:.6f}', flush=True)

if __name__ == '__main__':
    main(int(sys.argv[1]))
