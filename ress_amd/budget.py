"""Per-head block budgets: the `.num_to_select(layer_idx, attn_pooled, sparse_ratio,
cdf_threshold, beta)` plug-in protocol of the reference (src/ress/runtime/static.py:7-9,
src/ress/budget/uniform.py, src/ress/budget/hess.py), computed by the GPU kernels.

Counts come back as int32 device tensors shaped attn_pooled.shape[:-1] (the reference
returns int64; every consumer here takes either). The MIN_NUM_TO_SELECT floor is not
applied here -- the forward applies it, as the reference does (attention.py:525).
"""

import numpy as np
import torch

from ress_amd import kernels


def compute_baseline_num_to_select(pooled_score, sparse_ratio=None, cdf_threshold=None, eps=1e-5):
    """Baseline per-(head, query-block) budget (reference src/ress/models/attention.py:268-293):
    the CDF count (sort descending, cumulative sum, searchsorted(fp32(tau) + 1e-5, right))
    and/or topk = int(k_blk * (1 - sparse_ratio)); with both, the larger count."""
    if eps != 1e-5:
        raise ValueError("the CDF epsilon is fixed at 1e-5 (the reference default)")
    return kernels.baseline_budget(pooled_score, sparse_ratio, cdf_threshold)


def sum_normalize(scores):
    """Per-layer sum=1 normalisation (reference src/ress/budget/hess.py:46-48)."""
    return scores / scores.sum(dim=-1, keepdim=True)


def combine_lambda(score_cam, score_pc, lam):
    """HeSS Eq. (9), continuous lambda, renormalised (reference hess.py:51-56)."""
    return sum_normalize(lam * score_cam + (1 - lam) * score_pc)


def scores_norm(head_scores):
    """adjust_attention_selection's score normalisation (reference
    src/ress/budget/_proportional.py:84-88), as an fp32 vector: head_scores / sum, the
    sum taken sequentially in fp32; uniform 1/H when the sum is non-finite or <= 0."""
    hs = np.asarray(torch.as_tensor(head_scores, dtype=torch.float32).cpu().numpy(), np.float32)
    s = np.float32(0.0)
    for x in hs:
        s = np.float32(s + x)
    if not np.isfinite(s) or s <= 0:
        return np.full(hs.shape, np.float32(1.0 / hs.size), np.float32)
    return (hs / s).astype(np.float32)


def adjust_attention_selection(num_to_select, head_scores, beta, max_val, max_iters=1000, floor_frac=None,
                               check=False):
    """HeSS cap-and-redistribute (reference src/ress/budget/_proportional.py:49-115) on the
    GPU. num_to_select (B, nh, q_blk) int; head_scores (nh,). `check=True` synchronises
    and raises RuntimeError if some column did not converge within max_iters (the
    reference's behaviour, which it pays for with a host sync per iteration)."""
    if floor_frac is not None:
        raise NotImplementedError("floor_frac is not on the HeSS path (HessBudget passes None)")
    nts = num_to_select if num_to_select.dim() == 3 else num_to_select.unsqueeze(0)
    sn = torch.from_numpy(scores_norm(head_scores)).to(nts.device)
    iters = torch.empty(nts.shape[0], nts.shape[2], dtype=torch.int32, device=nts.device) if check else None
    out = kernels.head_budget(nts, sn, beta, max_val, max_iters=max_iters, iters_out=iters)
    if check and bool((iters < 0).any()):
        raise RuntimeError(f"adjust_attention_selection did not converge in {max_iters} iterations")
    return out if num_to_select.dim() == 3 else out.squeeze(0)


class UniformBudget:
    """One budget for every head (reference src/ress/budget/uniform.py:23-37)."""

    def __init__(self, n_blocks=24, n_heads=16):
        self.head_scores = torch.ones(n_blocks, n_heads)

    @property
    def needs_v_bar(self):
        return False

    def num_to_select(self, layer_idx, attn_pooled, sparse_ratio=None, cdf_threshold=None, beta=1.0):
        return compute_baseline_num_to_select(attn_pooled, sparse_ratio, cdf_threshold)


def _load_table(src, qkv_idx):
    if isinstance(src, torch.Tensor):
        t = src
    else:
        # calibration tables are plain tensors; never unpickle arbitrary objects
        t = torch.load(src, map_location="cpu", weights_only=True)
    return t[qkv_idx].to(torch.float32)


class HessBudget:
    """HeSS: the baseline budget of this input, reallocated across heads in proportion
    to calibrated head importance (reference src/ress/budget/hess.py:59-100).

    score_cam / score_pc: (3, n_layers, n_heads) tables, as tensors or `.pt` paths (read
    with torch.load(weights_only=True)); index `qkv_idx` (0 = W_Q) is used."""

    def __init__(self, score_cam, score_pc, lam=0.5, qkv_idx=0, floor_frac=None, layer_slice=None, max_iters=1000):
        raw_cam = _load_table(score_cam, qkv_idx)
        raw_pc = _load_table(score_pc, qkv_idx)
        if layer_slice is not None:
            raw_cam, raw_pc = raw_cam[layer_slice], raw_pc[layer_slice]
        self.score_cam = sum_normalize(raw_cam)
        self.score_pc = sum_normalize(raw_pc)
        self.lam = lam
        self.head_scores = combine_lambda(self.score_cam, self.score_pc, self.lam)
        if floor_frac is not None:
            raise NotImplementedError("floor_frac is not on the HeSS path")
        self.floor_frac = None
        self.max_iters = max_iters
        self._norm_cache = {}
        self._uniform_baseline = {}

    @property
    def needs_v_bar(self):
        return False

    def _scores_norm(self, layer_idx, device):
        key = (layer_idx, str(device))
        t = self._norm_cache.get(key)
        if t is None:
            t = torch.from_numpy(scores_norm(self.head_scores[layer_idx])).to(device)
            self._norm_cache[key] = t
        return t

    def num_to_select(self, layer_idx, attn_pooled, sparse_ratio=None, cdf_threshold=None, beta=1.0):
        """Counts (B, nh, q_blk) int32 on the device, without a host sync. The reference
        raises RuntimeError when the redistribution does not converge within max_iters
        (_proportional.py:112-113), which costs it a sync per iteration. Here the kernel
        reports each column's iteration count on the device (negative where it did not
        converge) and the returned tensor carries those counts as `ress_iters` ((B, q_blk)
        int32); the layer counts them and raises at its next host sync (LayerResult.check /
        .sparsity), so the budget launches only its own kernels: the head budget, and the
        baseline count when a CDF threshold makes it depend on the scores."""
        if cdf_threshold is None and sparse_ratio is not None:
            # a sparse-ratio baseline does not depend on the scores: every row gets
            # int(k_blk * (1 - sparse_ratio)). It is made once per shape and device and
            # only read afterwards, so the step launches no fill for it.
            # Under HIP graph capture the fill kernel would only be recorded, not run, and
            # the tensor would belong to the graph's pool: such a baseline is made for the
            # graph alone and not kept.
            key = (tuple(attn_pooled.shape), float(sparse_ratio), str(attn_pooled.device))
            baseline = self._uniform_baseline.get(key)
            if baseline is None:
                baseline = compute_baseline_num_to_select(attn_pooled, sparse_ratio, None)
                if not (attn_pooled.is_cuda and torch.cuda.is_current_stream_capturing()):
                    self._uniform_baseline[key] = baseline
        else:
            baseline = compute_baseline_num_to_select(attn_pooled, sparse_ratio, cdf_threshold)
        max_val = attn_pooled.shape[-1]
        nts = baseline if baseline.dim() == 3 else baseline.unsqueeze(0)
        iters = torch.empty(nts.shape[0], nts.shape[2], dtype=torch.int32, device=nts.device)
        out = kernels.head_budget(nts, self._scores_norm(layer_idx, attn_pooled.device), beta, max_val,
                                  max_iters=self.max_iters, iters_out=iters)
        out = out if baseline.dim() == 3 else out.squeeze(0)
        out.ress_iters = iters
        out.ress_max_iters = self.max_iters
        return out
