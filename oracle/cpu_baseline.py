"""CPU baseline for bench.py: the layer's block-sparse attention as PyTorch-CPU
block-masked SDPA -- TEST / MEASUREMENT INFRASTRUCTURE.

For each (head, 128-query block) row the kept 64-key blocks (the LUT, sinks included)
are gathered and F.scaled_dot_product_attention runs in fp32: exactly block-masked
softmax without an N x N mask. The reference has no CPU sparse path (its sparse kernel
is CUDA-only), so this is a port of its semantics, timed on a bounded sample of rows
and extrapolated linearly to the whole layer.
"""

import os
import time

import numpy as np
import torch
import torch.nn.functional as F

from oracle.reference import split_tokens


def time_block_masked_sdpa(q, k, v, frames, P, S, lut, nvalid, budget_s=15.0, max_rows=None, seed=0):
    """Times fp32 block-masked SDPA over a random sample of kernel rows until about
    `budget_s` seconds of CPU work, then extrapolates to all rows.

    lut/nvalid: numpy [BH][q_blk_total][kb_tot] / [BH][q_blk_total]. Returns a dict with
    the extrapolated ms per layer, the sample size and the threads used."""
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    B, H = q.shape[:2]
    qp, qs = split_tokens(q.float().cpu(), frames, P, S)
    kp, ks = split_tokens(k.float().cpu(), frames, P, S)
    vp, vs = split_tokens(v.float().cpu(), frames, P, S)
    key = kp if ks is None else torch.cat([kp, ks], dim=-2)
    val = vp if vs is None else torch.cat([vp, vs], dim=-2)
    T_p, T_s, Tk = frames * (P - S), frames * S, frames * P
    q_blk_p = -(-T_p // 128)
    BH, q_blk_total = nvalid.shape
    all_rows = [(bh, qb) for bh in range(BH) for qb in range(q_blk_total)]
    rng = np.random.default_rng(seed)
    order = rng.permutation(len(all_rows))

    def run(bh, qb):
        b, h = divmod(bh, H)
        blocks = lut[bh, qb, :nvalid[bh, qb]]
        idx = torch.from_numpy(np.concatenate([np.arange(c * 64, min(c * 64 + 64, Tk)) for c in blocks]))
        if qb < q_blk_p:
            qq = qp[b, h, qb * 128:min(qb * 128 + 128, T_p)]
        else:
            r0 = (qb - q_blk_p) * 128
            qq = qs[b, h, r0:min(r0 + 128, T_s)]
        return F.scaled_dot_product_attention(qq[None], key[b, h, idx][None], val[b, h, idx][None])

    run(*all_rows[order[0]])  # warm-up
    done, work_done = 0, 0
    total_work = float(nvalid.sum())
    t0 = time.perf_counter()
    for i in order:
        bh, qb = all_rows[i]
        run(bh, qb)
        done += 1
        work_done += float(nvalid[bh, qb])
        if time.perf_counter() - t0 > budget_s or (max_rows and done >= max_rows):
            break
    elapsed = time.perf_counter() - t0
    # extrapolate by kept-block work (rows differ in length)
    ms_layer = elapsed * 1e3 * total_work / work_done
    return {"ms_per_layer": ms_layer, "rows_timed": done, "rows_total": len(all_rows), "threads": threads,
            "elapsed_s": elapsed}
