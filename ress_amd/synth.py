"""Seeded synthetic inputs for one VGGT-style global-attention layer.

Generator (everything in float64 numpy with a PCG64 stream, so this container and the
GPU host build identical tensors; bf16 only at the end):

* per frame a latent field z_f on the 37x37 patch grid with `rank` (16) channels:
    "shared": z_f = rho * z_shared + sqrt(1 - rho^2) * eps_f        (rho = 0.6)
    "ar1":    z_0 = eps_0,  z_f = a * z_{f-1} + sqrt(1 - a^2) * eps_f   (a = 0.98,
              i.e. correlation a^|df| between frames)
* an 8x8 box blur over the grid ("same" size: the window covers offsets -4..+3 on each
  axis and divides by its in-bounds cell count), then each channel rescaled to unit
  standard deviation over the whole field
* per head, Q/K/V = z @ W + noise * N(0,1), W (rank x 64) ~ N(0, 1/rank), with
  W_K = W_Q + 0.5 * N(0, 1/rank) so nearby tokens attend to each other; noise = 0.1.
  Each (batch, head) draws from its own stream, SeedSequence([seed, 1, b*H + h]), so the
  heads are generated in parallel and head h is the same tensor whatever H is.
* 5 special tokens per frame (1 camera + 4 register) projected from N(0,1) latents
* patch tokens of every frame in generalized-Hilbert order; storage per frame is
  [5 special, 1369 patch] -> tensors (B, H, frames*1374, 64) bf16.

The Hilbert order is the generalized Hilbert ("gilbert") curve for arbitrary rectangles
(J. Cerveny's published construction), computed here with an explicit work stack.
"""

import concurrent.futures
import math
import os

import numpy as np
import torch

GRID = 37
N_SPECIAL = 5
TOKENS_PER_FRAME = GRID * GRID + N_SPECIAL  # 1374


def _sgn(v):
    return (v > 0) - (v < 0)


def gilbert_order(width, height):
    """Cells (x, y) of a width x height grid along the generalized Hilbert curve: a
    bijection onto the grid in which consecutive cells are 4-neighbours whenever the
    construction allows (always for even sides)."""
    out = []
    if width >= height:
        stack = [(0, 0, width, 0, 0, height)]
    else:
        stack = [(0, 0, 0, height, width, 0)]
    while stack:
        x, y, ax, ay, bx, by = stack.pop()
        w, h = abs(ax + ay), abs(bx + by)
        dax, day = _sgn(ax), _sgn(ay)
        dbx, dby = _sgn(bx), _sgn(by)
        if h == 1:
            out.extend((x + i * dax, y + i * day) for i in range(w))
            continue
        if w == 1:
            out.extend((x + i * dbx, y + i * dby) for i in range(h))
            continue
        ax2, ay2 = ax // 2, ay // 2
        bx2, by2 = bx // 2, by // 2
        w2, h2 = abs(ax2 + ay2), abs(bx2 + by2)
        if 2 * w > 3 * h:
            if (w2 % 2) and w > 2:
                ax2, ay2 = ax2 + dax, ay2 + day
            parts = [(x, y, ax2, ay2, bx, by),
                     (x + ax2, y + ay2, ax - ax2, ay - ay2, bx, by)]
        else:
            if (h2 % 2) and h > 2:
                bx2, by2 = bx2 + dbx, by2 + dby
            parts = [(x, y, bx2, by2, ax2, ay2),
                     (x + bx2, y + by2, ax, ay, bx - bx2, by - by2),
                     (x + (ax - dax) + (bx2 - dbx), y + (ay - day) + (by2 - dby),
                      -bx2, -by2, -(ax - ax2), -(ay - ay2))]
        stack.extend(reversed(parts))  # first part is processed first
    return out


def hilbert_permutation(width, height):
    """perm[i] = raster index (y*width + x) of the i-th cell along the curve."""
    return np.array([y * width + x for x, y in gilbert_order(width, height)], dtype=np.int64)


def _box_blur(z, k=8):
    """'same'-size box blur over axes 0,1 of (G, G, C): window offsets -k/2..k/2-1,
    divided by the in-bounds count."""
    G = z.shape[0]
    lo, hi = -(k // 2), k - k // 2 - 1
    c = np.zeros((G + 1, G + 1, z.shape[2]))
    c[1:, 1:] = z.cumsum(0).cumsum(1)
    out = np.empty_like(z)
    for i in range(G):
        i0, i1 = max(0, i + lo), min(G - 1, i + hi)
        for j in range(G):
            j0, j1 = max(0, j + lo), min(G - 1, j + hi)
            s = c[i1 + 1, j1 + 1] - c[i0, j1 + 1] - c[i1 + 1, j0] + c[i0, j0]
            out[i, j] = s / ((i1 - i0 + 1) * (j1 - j0 + 1))
    return out


def _project(z, W, chunk=512):
    """z (..., rank) @ W (rank, D) as an explicit sum over rank (deterministic order:
    ((z_0 W_0 + z_1 W_1) + z_2 W_2) + ..., each product rounded before its add), in
    place over cache-sized row chunks."""
    zf = z.reshape(-1, z.shape[-1])
    out = np.empty((zf.shape[0], W.shape[1]))
    tmp = np.empty((min(chunk, zf.shape[0]), W.shape[1]))
    for i in range(0, zf.shape[0], chunk):
        o = out[i:i + chunk]
        t = tmp[:o.shape[0]]
        zc = zf[i:i + chunk]
        np.multiply(zc[:, 0:1], W[0], out=o)
        for r in range(1, W.shape[0]):
            np.multiply(zc[:, r:r + 1], W[r], out=t)
            np.add(o, t, out=o)
    return out.reshape(z.shape[:-1] + (W.shape[1],))


def make_layer_qkv(frames, H=16, D=64, B=1, rank=16, seed=0, corr="shared", rho=0.6, ar=0.98, noise=0.1,
                   blur=8, hilbert=True, device="cpu", progress=None):
    """(q, k, v): bf16 (B, H, frames*1374, D) in VGGT storage order, plus the meta dict
    {frames, P, S}. `progress`, if given, is called with a short string per head."""
    rng = np.random.default_rng(seed)
    G, S = GRID, N_SPECIAL
    fields = np.empty((frames, G, G, rank))
    if corr == "shared":
        shared = rng.standard_normal((G, G, rank))
        for f in range(frames):
            fields[f] = rho * shared + math.sqrt(1 - rho * rho) * rng.standard_normal((G, G, rank))
    elif corr == "ar1":
        fields[0] = rng.standard_normal((G, G, rank))
        for f in range(1, frames):
            fields[f] = ar * fields[f - 1] + math.sqrt(1 - ar * ar) * rng.standard_normal((G, G, rank))
    else:
        raise ValueError(corr)
    for f in range(frames):
        fields[f] = _box_blur(fields[f], blur)
    fields /= fields.reshape(-1, rank).std(axis=0)
    patch = fields.reshape(frames, G * G, rank)
    if hilbert:
        patch = patch[:, hilbert_permutation(G, G)]
    special = rng.standard_normal((frames, S, rank))
    lat = np.concatenate([special, patch], axis=1)  # (frames, P, rank)
    P = G * G + S
    out = [torch.empty((B, H, frames * P, D), dtype=torch.bfloat16) for _ in range(3)]

    def one_head(bh):
        b, h = divmod(bh, H)
        hrng = np.random.default_rng(np.random.SeedSequence([seed, 1, bh]))
        Wq = hrng.standard_normal((rank, D)) / math.sqrt(rank)
        Wk = Wq + 0.5 * hrng.standard_normal((rank, D)) / math.sqrt(rank)
        Wv = hrng.standard_normal((rank, D)) / math.sqrt(rank)
        for t, W in enumerate((Wq, Wk, Wv)):
            x = _project(lat, W)
            x += noise * hrng.standard_normal((frames, P, D))
            out[t][b, h] = torch.from_numpy(x.reshape(frames * P, D).astype(np.float32))
        return bh

    workers = max(1, min(B * H, os.cpu_count() or 1, 16))
    with concurrent.futures.ThreadPoolExecutor(workers) as ex:
        for i, _ in enumerate(ex.map(one_head, range(B * H))):
            if progress:
                progress(f"head {i + 1}/{B * H}")
    q, k, v = (a.to(device) for a in out)
    return q, k, v, {"frames": frames, "P": P, "S": S}


def make_hess_tables(n_layers=24, n_heads=16, seed=1, sigma=0.5):
    """Two synthetic (3, n_layers, n_heads) log-normal(0, sigma) Fisher tables
    (camera, point cloud), fp32 -- the calibration-table format HessBudget reads."""
    rng = np.random.default_rng(seed)
    cam = np.exp(sigma * rng.standard_normal((3, n_layers, n_heads))).astype(np.float32)
    pc = np.exp(sigma * rng.standard_normal((3, n_layers, n_heads))).astype(np.float32)
    return torch.from_numpy(cam), torch.from_numpy(pc)


def make_w_o(dim=1024, seed=2):
    """A seeded N(0, 1/dim) output projection W_O (dim x dim), fp32."""
    rng = np.random.default_rng(seed)
    return torch.from_numpy((rng.standard_normal((dim, dim)) / math.sqrt(dim)).astype(np.float32))


# BASELINE.json configurations (frames, sparse_ratio, cdf_threshold, budget mode, frame
# correlation, attention_sink = leading tokens whose key blocks every row keeps)
CONFIGS = {
    0: dict(frames=4, sparse_ratio=0.5, cdf_threshold=0.9, mode="sparse_vggt", corr="shared", attention_sink=1374),
    1: dict(frames=16, sparse_ratio=0.7, cdf_threshold=None, mode="hess", corr="shared"),
    2: dict(frames=32, sparse_ratio=0.8, cdf_threshold=None, mode="ress", corr="shared", n_iters=5),
    4: dict(frames=200, sparse_ratio=0.9, cdf_threshold=None, mode="sparse_vggt", corr="ar1", attention_sink=1374),
}
