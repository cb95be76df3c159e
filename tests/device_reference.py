"""fp32 block-masked softmax attention on the device, checking every row (test helper).

For each (batch*head, query block) row of a layer, the reference is
softmax(Q K^T / 8 masked to the row's kept key blocks) V in float32, computed by torch on
the GPU over the kernel's token order (queries: patch tokens then special tokens; keys:
cat(patch, special), reference src/ress/models/attention.py:405-406), in chunks of query
rows so that one chunk's score matrix stays under `max_elems` elements. The kernel's
output (storage order) is compared row block by row block.

`split_rows` restates the attention launch's work split (the row schedule's 8 equal-work
ranges and the last rows of each, which run as parts merged afterwards), so a test can
name the rows that went through the merge.
"""

import numpy as np
import torch

SPLIT_ROWS = 32      # rows split at the end of each XCD range (attn.hip RESS_SPLIT_ROWS)
ROW_COST = 2         # per-row cost in the equal-work split (attn.hip RESS_ROW_COST)


def kernel_order(frames, P, S, device):
    """Storage indices of the kernel's rows: every frame's patch tokens, then every frame's
    special tokens."""
    HW = P - S
    f = torch.arange(frames, device=device)[:, None] * P
    patch = (f + S + torch.arange(HW, device=device)[None]).reshape(-1)
    special = (f + torch.arange(S, device=device)[None]).reshape(-1)
    return torch.cat([patch, special])


def block_mask(lut, nvalid, kb_tot):
    """[BH][q_blk_total][kb_tot] bool: the blocks each LUT row lists."""
    BH, QT, _ = lut.shape
    pos = torch.arange(kb_tot, device=lut.device)
    idx = torch.where(pos[None, None] < nvalid[..., None].long(), lut.long(), kb_tot)
    m = torch.zeros(BH, QT, kb_tot + 1, dtype=torch.bool, device=lut.device)
    m.scatter_(2, idx, True)
    return m[..., :kb_tot]


def row_errors(out, q, k, v, grid, lut, nvalid, rows=None, max_elems=1 << 27):
    """Per (bh, q-block) row: max-abs error and cosine of `out` against the fp32 masked
    softmax. out, q, k, v: (B, H, frames*P, 64) device tensors in storage order; lut / nvalid:
    the kernel's [BH][q_blk_total][kb_tot] / [BH][q_blk_total] (device). rows: None for every
    row, or a bool array [BH][q_blk_total]. Returns numpy (err, cos), NaN where unchecked."""
    dev = out.device
    B, H = grid.B, grid.H
    T_p, Tk = grid.T_p, grid.Tk
    order = kernel_order(grid.frames, grid.P, grid.S, dev)
    r = torch.arange(Tk, device=dev)
    rowblk = torch.where(r < T_p, r // 128, grid.q_blk_p + (r - T_p) // 128)
    keyblk = r // 64
    bm = block_mask(lut.to(dev), nvalid.to(dev), grid.kb_tot)
    QT = grid.q_blk_total
    err = np.full((grid.BH, QT), np.nan)
    cos = np.full((grid.BH, QT), np.nan)
    chunk = max(128, (max_elems // Tk) // 128 * 128)
    want_rows = None if rows is None else torch.from_numpy(np.asarray(rows, bool)).to(dev)
    for bh in range(grid.BH):
        b, h = divmod(bh, H)
        if want_rows is not None and not bool(want_rows[bh].any()):
            continue
        qo = q[b, h, order].float()
        ko = k[b, h, order].float()
        vo = v[b, h, order].float()
        kT = ko.t().contiguous()
        got_all = out[b, h, order].float()
        sel = torch.arange(Tk, device=dev) if want_rows is None else torch.nonzero(want_rows[bh][rowblk])[:, 0]
        e_blk = torch.zeros(QT, device=dev)
        dot = torch.zeros(QT, device=dev, dtype=torch.float64)
        n1 = torch.zeros_like(dot)
        n2 = torch.zeros_like(dot)
        for c0 in range(0, sel.numel(), chunk):
            idx = sel[c0:c0 + chunk]
            s = (qo[idx] @ kT) * 0.125
            mask = bm[bh][rowblk[idx]][:, keyblk]
            s.masked_fill_(~mask, float("-inf"))
            ref = torch.softmax(s, dim=-1) @ vo
            del s, mask
            got = got_all[idx]
            blk = rowblk[idx]
            e_blk.scatter_reduce_(0, blk, (got - ref).abs().amax(-1), reduce="amax")
            dot.index_add_(0, blk, (got.double() * ref.double()).sum(-1))
            n1.index_add_(0, blk, (got.double() ** 2).sum(-1))
            n2.index_add_(0, blk, (ref.double() ** 2).sum(-1))
        done = torch.zeros(QT, dtype=torch.bool, device=dev)
        done[rowblk[sel]] = True
        e = e_blk.cpu().numpy()
        c = (dot / (n1.sqrt() * n2.sqrt()).clamp(min=1e-300)).cpu().numpy()
        d = done.cpu().numpy()
        err[bh, d] = e[d]
        cos[bh, d] = c[d]
    return err, cos


def split_rows(nvalid, q_blk_p):
    """The (bh, q-block) rows the attention launch splits into parts: the row schedule lists
    every head's dense special rows, then the patch rows head-major; it cuts the list into 8
    ranges of equal work (kept blocks + ROW_COST per row), and the last min(SPLIT_ROWS,
    range length) rows of each range are split. nvalid: numpy [BH][q_blk_total]."""
    BH, QT = nvalid.shape
    items = [(bh, q_blk_p + j) for bh in range(BH) for j in range(QT - q_blk_p)]
    items += [(bh, qb) for bh in range(BH) for qb in range(q_blk_p)]
    n = len(items)
    work = np.array([nvalid[bh, qb] + ROW_COST for bh, qb in items], np.int64)
    W = int(work.sum())
    excl = np.concatenate([[0], np.cumsum(work)[:-1]])
    bounds = [0] + [n] * 8
    for j in range(1, 8):
        hit = np.nonzero((excl * 8 >= j * W) & (np.concatenate([[-1], excl[:-1]]) * 8 < j * W))[0]
        if hit.size:
            bounds[j] = int(hit[0])
    L = min(n, SPLIT_ROWS)
    out = np.zeros((BH, QT), bool)
    for x in range(8):
        lx = min(L, bounds[x + 1] - bounds[x])
        for i in range(bounds[x + 1] - lx, bounds[x + 1]):
            out[items[i]] = True
    return out
