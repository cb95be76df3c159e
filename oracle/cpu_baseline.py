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
    """Times fp32 block-masked SDPA over a fixed random sample of kernel rows (about a
    quarter of `budget_s` per pass: one warm-up pass that picks the sample, then three
    timed passes, median taken), then extrapolates to all rows.

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

    # warm-up pass, which also fixes the sample: rows in a seeded random order until
    # about a quarter of the budget is spent; the sample is then timed three more times
    t0 = time.perf_counter()
    sample = []
    for i in order:
        run(*all_rows[i])
        sample.append(all_rows[i])
        if time.perf_counter() - t0 > budget_s / 4 or (max_rows and len(sample) >= max_rows):
            break
    runs = []
    for _ in range(3):
        t1 = time.perf_counter()
        for bh, qb in sample:
            run(bh, qb)
        runs.append(time.perf_counter() - t1)
    elapsed = time.perf_counter() - t0
    work_done = float(sum(nvalid[bh, qb] for bh, qb in sample))
    total_work = float(nvalid.sum())
    # extrapolate by kept-block work (rows differ in length)
    ms_layer = sorted(runs)[1] * 1e3 * total_work / work_done
    return {"ms_per_layer": ms_layer, "rows_timed": len(sample), "rows_total": len(all_rows), "threads": threads,
            "elapsed_s": elapsed, "runs": len(runs), "cpu_model": _cpu_model()}


def _cpu_model():
    """The host CPU's model name (/proc/cpuinfo), for the report."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"
