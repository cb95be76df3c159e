"""The SpargeAttn entry points the reference binds (src/ress/models/attention.py:28-32),
implemented on libress_hip:

    per_block_int8(q, k)                      spas_sage_attn.quant_per_block.per_block_int8
    block_map_lut_triton(map)                 spas_sage_attn.utils.block_map_lut_triton
    fill_block_map_triton(map, n, idx)        spas_sage_attn.utils.fill_block_map_triton
    hyperparameter_check(x, H, device)        spas_sage_attn.utils.hyperparameter_check
    get_block_map_meansim_fuse_quant(q, k)    spas_sage_attn.utils.get_block_map_meansim_fuse_quant
                                              (as patched, external/patches/spargeattn.patch:50-67)
    qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold(...)
                                              spas_sage_attn._qattn (the CUDA kernel)

Same argument meaning and return values as the reference's call sites use them. Two
layout facts differ and are stated where they matter: the INT8 tensors returned by
per_block_int8 are views of buffers padded to whole blocks (128 query / 64 key rows),
which the attention kernel reads; and the LUT holds absolute kept block indices.
"""

import math

import torch

from ress_amd import _lib

BLKQ, BLKK = 128, 64


def _cdiv(a, b):
    return -(-a // b)


def hyperparameter_check(hyper, H, device):
    """Broadcast a scalar (or per-head tensor) hyperparameter to a (H,) fp32 tensor."""
    if isinstance(hyper, (int, float)):
        return torch.full((H,), float(hyper), device=device)
    t = torch.as_tensor(hyper, device=device, dtype=torch.float32)
    if t.numel() != H:
        raise ValueError(f"hyperparameter has {t.numel()} values for {H} heads")
    return t.reshape(H)


def key_mean(k):
    """Mean over the sequence of a (B, H, Tk, 64) key tensor, fp32 (B*H, 64), with the
    block-sum order of the fused path (reference attention.py:231)."""
    B, H, Tk, C = k.shape
    kb = k.to(torch.bfloat16)
    nk = _cdiv(Tk, BLKK)
    dev = k.device
    ksum = torch.empty(B * H, nk, 64, device=dev)
    km = torch.empty(B * H, 64, device=dev)
    pk = torch.empty(B * H, nk, 64, device=dev)
    pv = torch.empty(B * H, nk, 64, device=dev)
    vp = torch.empty(B * H, nk, 4096, dtype=torch.bfloat16, device=dev)
    _lib.call("ress_prep_kv_plain", _lib.ptr(kb), _lib.ptr(kb), B, H, Tk, *kb.stride()[:3], *kb.stride()[:3],
              _lib.ptr(ksum), _lib.ptr(km), _lib.ptr(pk), _lib.ptr(pv), _lib.ptr(vp), _lib.stream_handle(dev))
    return km


def per_block_int8(q, k, km=None, BLKQ=BLKQ, BLKK=BLKK, sm_scale=None, tensor_layout="HND"):
    """Per-block symmetric INT8 of Q (128-token blocks) and K (64-token blocks):
    scale = amax/127, codes rounded half away from zero. Q is NOT pre-scaled by
    sm_scale*log2(e) (external/patches/spargeattn.patch:38-41); the attention kernel
    applies sm_scale itself. `km` (B*H, 64), if given, is subtracted from K first (the
    reference subtracts it in torch before the call, attention.py:232).
    Returns (q_int8, q_scale, k_int8, k_scale): (B,H,Tq,64) int8, (B,H,nq) fp32,
    (B,H,Tk,64) int8, (B,H,nk) fp32."""
    if (BLKQ, BLKK) != (128, 64) or tensor_layout != "HND":
        raise NotImplementedError("blocks are 128/64, layout HND")
    if sm_scale not in (None, 1.0):
        raise NotImplementedError("Q is quantised with sm_scale = 1 (the patched SpargeAttn convention)")
    B, H, Tq, C = q.shape
    Tk = k.shape[-2]
    if C != 64:
        raise ValueError("head_dim must be 64")
    qb = q.to(torch.bfloat16)
    kb = k.to(torch.bfloat16)
    dev = q.device
    nq, nk = _cdiv(Tq, 128), _cdiv(Tk, 64)
    q_buf = torch.empty(B, H, nq * 128, 64, dtype=torch.int8, device=dev)
    k_buf = torch.empty(B, H, nk * 64, 64, dtype=torch.int8, device=dev)
    q_scale = torch.empty(B, H, nq, device=dev)
    k_scale = torch.empty(B, H, nk, device=dev)
    pooled_q = torch.empty(B * H, nq, 64, device=dev)
    _lib.call("ress_per_block_int8", _lib.ptr(qb), _lib.ptr(kb), _lib.ptr(km), B, H, Tq, Tk, *qb.stride()[:3],
              *kb.stride()[:3], _lib.ptr(q_buf), _lib.ptr(q_scale), _lib.ptr(k_buf), _lib.ptr(k_scale),
              _lib.ptr(pooled_q), _lib.stream_handle(dev))
    return q_buf[:, :, :Tq], q_scale, k_buf[:, :, :Tk], k_scale


def block_map_lut_triton(block_map):
    """(B,H,q,k) bool -> (lut (B,H,q,k) int32 ascending kept block indices,
    valid_block_num (B,H,q) int32)."""
    B, H, nq, nk = block_map.shape
    m = block_map.to(torch.uint8).contiguous()
    lut = torch.empty(B, H, nq, nk, dtype=torch.int32, device=m.device)
    nv = torch.empty(B, H, nq, dtype=torch.int32, device=m.device)
    _lib.call("ress_block_map_lut", _lib.ptr(m), B * H * nq, nk, _lib.ptr(lut), _lib.ptr(nv),
              _lib.stream_handle(m.device))
    return lut, nv


def fill_block_map_triton(final_map, num_to_select, sorted_idx):
    """final_map[..., sorted_idx[..., :n]] = True per row; returns the map (bool)."""
    shp = final_map.shape
    k = shp[-1]
    m = final_map.to(torch.uint8).contiguous()
    n = num_to_select.to(torch.int64).contiguous()
    idx = sorted_idx.to(torch.int64).contiguous()
    _lib.call("ress_fill_block_map", _lib.ptr(m), _lib.ptr(n), _lib.ptr(idx), m.numel() // k, k,
              _lib.stream_handle(m.device))
    return m.bool().view(shp)


def _padded(t, rows_needed):
    """t (B,H,T,64) int8; returns a tensor whose storage holds rows_needed rows per (b,h)
    with t's values in the first T (copying into a padded buffer when t's own storage
    cannot be read that far)."""
    B, H, T, C = t.shape
    blocked = t.stride() == (H * rows_needed * C, rows_needed * C, C, 1)
    if blocked and t.untyped_storage().nbytes() >= t.storage_offset() + B * H * rows_needed * C:
        return t
    buf = torch.zeros(B, H, rows_needed, C, dtype=t.dtype, device=t.device)
    buf[:, :, :T] = t
    return buf


def qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold(
        q_int8, k_int8, v, o, lut, valid_block_num, pv_threshold, q_scale, k_scale, tensor_layout, is_causal,
        qk_quant_gran, sm_scale, return_pv_count):
    """Block-sparse attention writing `o` in place (reference call attention.py:238-241).
    q_int8 (B,H,Tq,64), k_int8 (B,H,Tk,64), v (B,H,Tk,64) fp16/bf16, o (B,H,Tq,64)
    fp32/bf16/fp16, lut/valid_block_num from block_map_lut_triton, pv_threshold (H,)
    (must be the disabled value, >= 1e9), q_scale (B,H,nq), k_scale (B,H,nk)."""
    B, H, Tq, C = q_int8.shape
    Tk = k_int8.shape[-2]
    dev = q_int8.device
    nq, nk = _cdiv(Tq, 128), _cdiv(Tk, 64)
    q8 = _padded(q_int8, nq * 128)
    k8 = _padded(k_int8, nk * 64)
    if v.dtype not in (torch.float16, torch.bfloat16):
        v = v.to(torch.float16)
    if lut.shape[-2:] != (nq, nk):
        raise ValueError(f"lut must be (B,H,{nq},{nk})")
    # the thresholds stay on the device (no host copy, no synchronisation): the kernel's
    # check records a non-disabled value in the status word
    pv_dev = torch.as_tensor(pv_threshold, dtype=torch.float32, device=dev).reshape(-1).contiguous()
    if pv_dev.numel() != H:
        raise ValueError("pv_threshold must have one value per head")
    ws_bytes = _lib.lib().ress_qattn_workspace_size(B, H, Tq, Tk)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    code = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[o.dtype]
    lut_c = lut.to(torch.int32).contiguous()
    nv_c = valid_block_num.to(torch.int32).contiguous()
    qs = q_scale.float().contiguous()
    ks = k_scale.float().contiguous()
    _lib.call("ress_qattn_block_sparse_fwd", _lib.ptr(q8), _lib.ptr(k8), _lib.ptr(v), int(v.dtype == torch.float16),
              _lib.ptr(o), code, _lib.ptr(lut_c), _lib.ptr(nv_c), _lib.ptr(pv_dev), _lib.ptr(qs), _lib.ptr(ks),
              B, H, Tq, Tk, *v.stride()[:3], *o.stride()[:3], int(tensor_layout), int(is_causal), int(qk_quant_gran),
              float(sm_scale), int(return_pv_count), _lib.ptr(ws), ws_bytes, _lib.stream_handle(dev))
    global _last_status
    _last_status = ws[:4].view(torch.int32).clone()  # kept past the workspace; read at the next sync
    return None


# Status word of the last mirror call (device int32), and what its bits mean.
_last_status = None
_STATUS_BITS = (
    (1, "valid_block_num outside [0, ceil(Tk/64)]"),
    (2, "a LUT entry outside [0, ceil(Tk/64)) or not strictly ascending within valid_block_num"),
    (4, "pv_threshold below 1e9: PV-threshold skipping is not implemented (the reference passes 1e10)"),
)


def raise_for_status(status):
    """Raise ValueError naming every problem the status word `status` (an int) records."""
    status = int(status)
    if status:
        msgs = [m for bit, m in _STATUS_BITS if status & bit]
        raise ValueError("qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold: " + "; ".join(msgs))


def last_call_status():
    """The status word of the last mirror call as a device tensor (0 = the LUT, counts and
    thresholds were valid); None before the first call."""
    return _last_status


def check_last_call():
    """Synchronise on the last mirror call's status word and raise if its inputs were invalid
    (the call itself never synchronises; it ran on a copy of the LUT clamped into range)."""
    if _last_status is not None:
        raise_for_status(_last_status.item())


def _meansim_workspace(B, H, Tq, Tk, dev):
    """(buffer or None, bytes): the scores workspace ress_meansim_block_map uses for long
    rows (ress_meansim_workspace_size), allocated per call."""
    n = _lib.lib().ress_meansim_workspace_size(B, H, Tq, Tk)
    return (torch.empty(n, dtype=torch.uint8, device=dev) if n else None), n


def get_block_map_meansim_fuse_quant(q, k, km=None, is_causal=False, BLKQ=BLKQ, BLKK=BLKK, simthreshd1=0.1,
                                     cdfthreshd=0.9, is_sparse=True, return_lut=False, attention_sink=0):
    """SpargeAttn's fused block map, as the reference patches it (spargeattn.patch:50-67):
    per-block mean pooling, mean intra-block cosine similarity and INT8 quantisation of
    Q (128-token blocks) and K - km (64-token blocks), then per (head, q-block) row the
    softmax of the pooled scores over the similar K blocks, the longest prefix of the
    sorted probabilities whose cumulative sum stays <= cdfthreshd (the sums taken exactly,
    at 2^-50 resolution, so the cut depends on the values alone), and the forced
    blocks: non-similar K blocks, every block of a non-similar Q row, and the
    ceil(attention_sink/64) leading blocks (attention_sink counts tokens, :63-65).

    q (B,H,Tq,64), k (B,H,Tk,64) (computed in bf16), km (B,H,1,64) / (B*H,64) or None,
    simthreshd1 / cdfthreshd scalars or per-head. Returns (final_map bool (B,H,nq,nk),
    q_int8, q_scale, k_int8, k_scale), or with return_lut (lut, valid_block_num, q_int8,
    q_scale, k_int8, k_scale); the INT8 tensors are views of block-padded buffers, the
    layout per_block_int8 returns. Only the non-causal sparse form is provided
    (is_causal=True / is_sparse=False raise): the reference calls neither, and
    SpargeAttn's causal block mask is not in the reference to be matched."""
    if (BLKQ, BLKK) != (128, 64):
        raise NotImplementedError("blocks are 128/64")
    if is_causal or not is_sparse:
        raise NotImplementedError("only the non-causal sparse block map is provided")
    attention_sink = int(attention_sink)
    if attention_sink < 0:
        raise ValueError("attention_sink counts leading tokens (>= 0)")
    B, H, Tq, C = q.shape
    Tk = k.shape[-2]
    if C != 64 or k.shape[:2] != (B, H) or k.shape[-1] != 64:
        raise ValueError("q, k must be (B,H,T,64) with matching B, H")
    dev = q.device
    qb, kb = q.to(torch.bfloat16), k.to(torch.bfloat16)
    if qb.stride(-1) != 1 or any(s % 8 for s in qb.stride()[:3]) or qb.data_ptr() % 16:
        qb = qb.contiguous()
    if kb.stride(-1) != 1 or any(s % 8 for s in kb.stride()[:3]) or kb.data_ptr() % 16:
        kb = kb.contiguous()
    kmf = None
    if km is not None:
        kmf = km.to(device=dev, dtype=torch.float32).reshape(B * H, 64).contiguous()
    simth = hyperparameter_check(simthreshd1, H, dev).float().contiguous()
    cdfth = hyperparameter_check(cdfthreshd, H, dev).float().contiguous()
    nq, nk = _cdiv(Tq, 128), _cdiv(Tk, 64)
    final_map = torch.empty(B, H, nq, nk, dtype=torch.uint8, device=dev)
    q_buf = torch.empty(B, H, nq * 128, 64, dtype=torch.int8, device=dev)
    k_buf = torch.empty(B, H, nk * 64, 64, dtype=torch.int8, device=dev)
    q_scale = torch.empty(B, H, nq, device=dev)
    k_scale = torch.empty(B, H, nk, device=dev)
    pooled_q = torch.empty(B * H, nq, 64, device=dev)
    pooled_k = torch.empty(B * H, nk, 64, device=dev)
    sim_q = torch.empty(B * H, nq, dtype=torch.uint8, device=dev)
    sim_k = torch.empty(B * H, nk, dtype=torch.uint8, device=dev)
    ws, ws_bytes = _meansim_workspace(B, H, Tq, Tk, dev)
    _lib.call("ress_meansim_block_map", _lib.ptr(qb), _lib.ptr(kb), _lib.ptr(kmf), B, H, Tq, Tk, *qb.stride()[:3],
              *kb.stride()[:3], _lib.ptr(simth), _lib.ptr(cdfth), attention_sink, _lib.ptr(final_map),
              _lib.ptr(q_buf), _lib.ptr(q_scale), _lib.ptr(k_buf), _lib.ptr(k_scale), _lib.ptr(pooled_q),
              _lib.ptr(pooled_k), _lib.ptr(sim_q), _lib.ptr(sim_k), _lib.ptr(ws), ws_bytes, _lib.stream_handle(dev))
    q_int8, k_int8 = q_buf[:, :, :Tq], k_buf[:, :, :Tk]
    if not return_lut:
        return final_map.bool(), q_int8, q_scale, k_int8, k_scale
    lut, valid_block_num = block_map_lut_triton(final_map)
    return lut, valid_block_num, q_int8, q_scale, k_int8, k_scale


def sm_scale_default(head_dim=64):
    return 1.0 / math.sqrt(head_dim)
