"""CPU oracle for the block-sparse global-attention path -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg import this
package, and only as the checker; the product (ress_amd) never does.

* ress_oracle.c -- the reference algorithm restated in C under the GPU library's
  numerics contract, so block maps, budgets and INT8 codes compare bit-exactly.
  Each function cites the reference lines it follows.
* reference.py -- float32/float64 restatements in numpy/torch-CPU used to pin the C
  oracle (closed forms, brute force) and the fp32 masked-softmax attention reference.
* cpu_baseline.py -- the PyTorch-CPU block-masked SDPA baseline bench.py reports.
"""

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            from oracle.build import build_oracle
            build_oracle()
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_expf.restype = ctypes.c_float
        L.oracle_expf.argtypes = [ctypes.c_float]
        L.oracle_round_bf16.restype = ctypes.c_float
        L.oracle_round_bf16.argtypes = [ctypes.c_float]
        L.oracle_head_budget.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _u16(a):
    """bf16 data (torch tensor or uint16 ndarray) -> contiguous uint16 ndarray."""
    try:
        import torch
        if isinstance(a, torch.Tensor):
            a = a.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    except ImportError:
        pass
    return np.ascontiguousarray(a, dtype=np.uint16)


def expf(x):
    return np.float32(lib().oracle_expf(ctypes.c_float(float(x))))


def prep_qkv(q, k, v, frames, P, S, pool_all=False):
    """q,k,v: bf16 (B,H,frames*P,64) (torch tensors or uint16 arrays). Returns a dict of
    the ress_prep_qkv outputs, shapes as in include/ress_hip.h (pool_all: pooled K/V over
    every key block, the sink-mass grid)."""
    qu, ku, vu = _u16(q), _u16(k), _u16(v)
    B, H, N, D = qu.shape
    assert D == 64 and N == frames * P
    BH = B * H
    T_p, T_s = frames * (P - S), frames * S
    qbp, qbs = -(-T_p // 128), -(-T_s // 128)
    kbt, kbp = -(-N // 64), -(-(N if pool_all else T_p) // 64)
    out = dict(
        q_i8=np.zeros((BH, qbp + qbs, 128, 64), np.int8),
        q_lo=np.zeros((BH, qbp + qbs, 128, 64), np.int8),
        q_scale=np.zeros((BH, qbp + qbs), np.float32),
        pooled_q=np.zeros((BH, qbp, 64), np.float32),
        k_i8=np.zeros((BH, kbt, 64, 64), np.int8),
        k_lo=np.zeros((BH, kbt, 64, 64), np.int8),
        k_scale=np.zeros((BH, kbt), np.float32),
        pooled_k=np.zeros((BH, kbp, 64), np.float32),
        pooled_v=np.zeros((BH, kbp, 64), np.float32),
        v_pack=np.zeros((BH, kbt, 4096), np.uint16),
        ksum=np.zeros((BH, kbt, 64), np.float32),
        km=np.zeros((BH, 64), np.float32),
        k_norm=np.zeros((BH, kbt), np.float32),
    )
    lib().oracle_prep_qkv(_p(qu), _p(ku), _p(vu), BH, frames, P, S, *[_p(out[n]) for n in (
        "q_i8", "q_lo", "q_scale", "pooled_q", "k_i8", "k_lo", "k_scale", "pooled_k", "pooled_v", "v_pack", "ksum",
        "km", "k_norm")], 1 if pool_all else 0)
    return out


def pooled_scores(pooled_q, pooled_k, n_cand, scale=0.125):
    pq = np.ascontiguousarray(pooled_q, np.float32)
    pk = np.ascontiguousarray(pooled_k, np.float32)
    BH, q_blk, _ = pq.shape
    kb_p = pk.shape[1]
    full = np.zeros((BH, q_blk, kb_p), np.float32)
    cond = np.zeros((BH, q_blk, n_cand), np.float32)
    lib().oracle_pooled_scores(_p(pq), _p(pk), BH, q_blk, kb_p, n_cand, ctypes.c_float(scale), _p(full), _p(cond))
    return full, cond


def baseline_budget(attn_cond, sparse_ratio=None, cdf_threshold=None):
    a = np.ascontiguousarray(attn_cond, np.float32)
    n = a.shape[-1]
    rows = a.size // n
    topk = int(n * (1 - sparse_ratio)) if sparse_ratio is not None else -1
    cdf = float(cdf_threshold) if cdf_threshold is not None else -1.0
    out = np.zeros(a.shape[:-1], np.int32)
    lib().oracle_baseline_budget(_p(a), ctypes.c_longlong(rows), n, ctypes.c_float(cdf), topk, _p(out))
    return out


def head_budget(baseline, scores_norm, beta, max_val, max_iters=1000, min_select=0):
    """Returns (counts, worst_iterations) -- worst_iterations is -1 on non-convergence."""
    b = np.ascontiguousarray(baseline, np.int32)
    B, H, q_blk = b.shape
    s = None if scores_norm is None else np.ascontiguousarray(scores_norm, np.float32)
    out = np.zeros_like(b)
    it = lib().oracle_head_budget(_p(b), B, H, q_blk, _p(s), ctypes.c_double(beta), max_val, max_iters, min_select,
                                  _p(out))
    return out, it


def select_blocks(rank_key, counts, q_blk_total, kb_tot, sink_lead=0, min_select=0):
    """rank_key (BH, q_blk_sel, n_cand), counts (BH, q_blk_sel). Returns (map, lut, nvalid)."""
    rk = np.ascontiguousarray(rank_key, np.float32)
    cn = np.ascontiguousarray(counts, np.int32)
    BH, q_sel, n_cand = rk.shape
    fmap = np.zeros((BH, q_sel, kb_tot), np.uint8)
    lut = np.full((BH, q_blk_total, kb_tot), -1, np.int32)
    nvalid = np.zeros((BH, q_blk_total), np.int32)
    lib().oracle_select_blocks(_p(rk), _p(cn), BH, q_sel, q_blk_total, n_cand, kb_tot, sink_lead, min_select, _p(fmap),
                               _p(lut), _p(nvalid))
    return fmap, lut, nvalid


def scores_norm_seq(head_scores):
    """adjust_attention_selection's score normalisation (src/ress/budget/_proportional.py:84-88)
    with a sequential fp32 sum: uniform 1/H when the sum is non-finite or <= 0."""
    hs = np.asarray(head_scores, np.float32)
    s = np.float32(0.0)
    for x in hs:
        s = np.float32(s + x)
    if not np.isfinite(s) or s <= 0:
        return np.full(hs.shape, np.float32(1.0 / hs.size), np.float32)
    return (hs / s).astype(np.float32)


def expf_array(x):
    a = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(a)
    lib().oracle_expf_array(_p(a), _p(y), ctypes.c_longlong(a.size))
    return y


def round_bf16_array(x):
    a = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(a)
    lib().oracle_round_bf16_array(_p(a), _p(y), ctypes.c_longlong(a.size))
    return y


RS_BF16, RS_TRACK_BEST, RS_MAXIMIZE, RS_INVERT_CUT, RS_NO_RENORM = 1, 2, 4, 8, 16


def restore_swap(A, V, M, nts, n_cand, n_iters=5, restore_frac=0.5, decay=0.5, big_bf16=True, track_best=True,
                 maximize=False, invert_cut=False, renormalize=True, want_s=False):
    """ReSS restore-swap keep sets. A (H,q_blk,kb_p) f32, V (H,kb_p,64) f32, M (H,64,64) f32,
    nts (H,q_blk) int. Returns (keep (H,q_blk,n_cand) uint8, J (H,q_blk) f32[, s])."""
    A = np.ascontiguousarray(A, np.float32)
    V = np.ascontiguousarray(V, np.float32)
    M = np.ascontiguousarray(M, np.float32)
    nts = np.ascontiguousarray(nts, np.int32)
    H, q_blk, kb_p = A.shape
    keep = np.zeros((H, q_blk, n_cand), np.uint8)
    obj = np.zeros((H, q_blk), np.float32)
    s = np.zeros((H, q_blk, n_cand), np.float32) if want_s else None
    flags = ((RS_BF16 if big_bf16 else 0) | (RS_TRACK_BEST if track_best else 0) | (RS_MAXIMIZE if maximize else 0)
             | (RS_INVERT_CUT if invert_cut else 0) | (0 if renormalize else RS_NO_RENORM))
    lib().oracle_restore_swap(_p(A), _p(V), _p(M), _p(nts), H, q_blk, kb_p, n_cand, n_iters,
                              ctypes.c_double(restore_frac), ctypes.c_double(decay), flags, _p(keep), _p(obj), _p(s))
    return (keep, obj, s) if want_s else (keep, obj)


def rs_probe(A, V, M, drop, n_cand, big_bf16=False, renormalize=True):
    """What oracle_restore_swap ranks by, for a given drop set (oracle_rs_probe): returns
    (s, scut (H,q_blk,n_cand), J (H,q_blk), rq, cq (H,q_blk,n_cand)): the drift scores, the
    initial cut's key, the objective ||g||^2_M / K^2 of the drop set, and the round's
    restore / drop marginals of every candidate (minimisation sign, unmasked).
    drop (H,q_blk,n_cand) bool, True = dropped."""
    A = np.ascontiguousarray(A, np.float32)
    V = np.ascontiguousarray(V, np.float32)
    M = np.ascontiguousarray(M, np.float32)
    d = np.ascontiguousarray(drop, np.uint8)
    H, q_blk, kb_p = A.shape
    s = np.zeros((H, q_blk, n_cand), np.float32)
    scut = np.zeros((H, q_blk, n_cand), np.float32)
    J = np.zeros((H, q_blk), np.float32)
    rq = np.zeros((H, q_blk, n_cand), np.float32)
    cq = np.zeros((H, q_blk, n_cand), np.float32)
    flags = (RS_BF16 if big_bf16 else 0) | (0 if renormalize else RS_NO_RENORM)
    lib().oracle_rs_probe(_p(A), _p(V), _p(M), _p(d), H, q_blk, kb_p, n_cand, flags, _p(s), _p(scut), _p(J), _p(rq),
                          _p(cq))
    return s, scut, J, rq, cq


def meansim_map(q, k, km=None, simthreshd1=0.1, cdfthreshd=0.9, attention_sink=0, H=None):
    """SpargeAttn-convention meansim block map (oracle_meansim_map). q (BH,Tq,64), k (BH,Tk,64)
    bf16 (torch or uint16); km (BH,64) f32 or None; thresholds scalar or per head.
    Returns a dict of map, q_i8, q_scale, k_i8, k_scale, pooled_q, pooled_k, sim_q, sim_k."""
    qa, ka = _u16(q), _u16(k)
    BH, Tq, _ = qa.shape
    Tk = ka.shape[1]
    H = H or BH
    nq, nk = -(-Tq // 128), -(-Tk // 64)
    th = np.ascontiguousarray(np.broadcast_to(np.asarray(simthreshd1, np.float32), (H,)))
    cd = np.ascontiguousarray(np.broadcast_to(np.asarray(cdfthreshd, np.float32), (H,)))
    kmv = None if km is None else np.ascontiguousarray(km, np.float32).reshape(BH, 64)
    o = dict(map=np.zeros((BH, nq, nk), np.uint8), q_i8=np.zeros((BH, nq * 128, 64), np.int8),
             q_scale=np.zeros((BH, nq), np.float32), k_i8=np.zeros((BH, nk * 64, 64), np.int8),
             k_scale=np.zeros((BH, nk), np.float32), pooled_q=np.zeros((BH, nq, 64), np.float32),
             pooled_k=np.zeros((BH, nk, 64), np.float32), sim_q=np.zeros((BH, nq), np.uint8),
             sim_k=np.zeros((BH, nk), np.uint8))
    lib().oracle_meansim_map(_p(qa), _p(ka), _p(kmv), BH, H, Tq, Tk, _p(th), _p(cd), int(attention_sink),
                             *(_p(o[n]) for n in ("map", "q_i8", "q_scale", "k_i8", "k_scale", "pooled_q", "pooled_k",
                                                  "sim_q", "sim_k")))
    return o
