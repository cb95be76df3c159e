"""The single-term INT8 attention (the reference's SpargeAttn semantics) and the
SpargeAttn-API mirror (ress_amd.sparge) on the GPU."""

import numpy as np
import pytest
import torch

import oracle
from oracle import reference as ref
from pipeline_oracle import oracle_layer, row_sample
from ress_amd import kernels, sparge, synth
from ress_amd.kernels import LayerGrid

pytestmark = pytest.mark.gpu


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).mul(scale).to(torch.bfloat16)


def _emulation_gap(out, prep, q, v, frames, P, S, lut, nvalid, rows, split):
    emu = ref.int8_attention_rows(prep, v, frames, P, S, lut, nvalid, rows, split=split)
    o = out.float().cpu().reshape(-1, out.shape[2], 64)
    worst = 0.0
    T_p = frames * (P - S)
    q_blk_p = -(-T_p // 128)
    HW = P - S
    for (bh, qb), e in emu.items():
        if qb < q_blk_p:
            tok = [(p // HW) * P + S + p % HW for p in range(qb * 128, qb * 128 + e.shape[0])]
        else:
            r0 = (qb - q_blk_p) * 128
            tok = [(s // S) * P + s % S for s in range(r0, r0 + e.shape[0])]
        worst = max(worst, (o[bh, torch.tensor(tok)] - e).abs().max().item())
    return worst


@pytest.mark.parametrize("split", [False, True])
def test_kernel_matches_exact_dequantised_softmax(split, dev):
    """Given the INT8 codes, the kernel's only approximations are exp2, bf16 P and the
    accumulation order: it must agree with the exact-arithmetic emulation closely."""
    q, k, v, meta = synth.make_layer_qkv(4)
    frames, P, S = meta["frames"], meta["P"], meta["S"]
    g = LayerGrid(1, 16, frames, P, S)
    o = oracle_layer(q, k, v, frames, P, S, sparse_ratio=0.5, cdf_threshold=0.9)
    blocks = kernels.prepare_blocks(q.to(dev), k.to(dev), v.to(dev), g, split=split)
    out = kernels.sparse_attention(blocks, torch.from_numpy(o["lut"]).to(dev), torch.from_numpy(o["nvalid"]).to(dev))
    torch.cuda.synchronize()
    rows = row_sample(o["nvalid"], 16)
    gap = _emulation_gap(out, o, q, v, frames, P, S, o["lut"], o["nvalid"], rows, split)
    print(f"[split={split}] kernel vs exact-dequantised emulation max-abs {gap:.3e}")
    assert gap <= 1.2e-2
    # single-term INT8 (the reference's numerics) is within cosine 0.999 of fp32
    refs = ref.masked_attention_rows(q, k, v, frames, P, S, o["lut"], o["nvalid"], rows)
    oo = out.float().cpu().reshape(16, -1, 64)
    for (bh, qb), (tok, r) in refs.items():
        got = oo[bh, torch.from_numpy(tok)]
        assert torch.nn.functional.cosine_similarity(got.flatten(), r.flatten(), dim=0).item() >= 0.999


def test_per_block_int8_matches_oracle_codes(dev):
    B, H, Tq, Tk = 1, 3, 300, 200
    q = _rand((B, H, Tq, 64), 1)
    k = _rand((B, H, Tk, 64), 2, 1.5)
    km = sparge.key_mean(k.to(dev))
    q8, qs, k8, ks = sparge.per_block_int8(q.to(dev), k.to(dev), km=km)
    assert q8.shape == (B, H, Tq, 64) and k8.shape == (B, H, Tk, 64)
    assert qs.shape == (B, H, 3) and ks.shape == (B, H, 4)
    # the oracle's plain-sequence preparation (S = 0) gives the same codes and scales
    oq = oracle.prep_qkv(q, q, q, 1, Tq, 0)
    ok = oracle.prep_qkv(k, k, k, 1, Tk, 0)
    assert np.array_equal(q8.cpu().numpy().reshape(H, -1), oq["q_i8"].reshape(H, -1)[:, :Tq * 64])
    assert np.array_equal(qs.cpu().numpy().reshape(H, -1).view(np.uint32), oq["q_scale"].view(np.uint32))
    assert np.array_equal(km.cpu().numpy().view(np.uint32), ok["km"].view(np.uint32))
    assert np.array_equal(k8.cpu().numpy().reshape(H, -1), ok["k_i8"].reshape(H, -1)[:, :Tk * 64])
    assert np.array_equal(ks.cpu().numpy().reshape(H, -1).view(np.uint32), ok["k_scale"].view(np.uint32))


def test_block_map_lut_and_fill(dev):
    rng = np.random.default_rng(3)
    m = torch.from_numpy(rng.random((2, 3, 5, 70)) < 0.3).to(dev)
    lut, nv = sparge.block_map_lut_triton(m)
    mm = m.cpu().numpy()
    for idx in np.ndindex(mm.shape[:-1]):
        kept = np.nonzero(mm[idx])[0]
        assert nv[idx].item() == kept.size
        assert np.array_equal(lut[idx][:kept.size].cpu().numpy(), kept)
    scores = torch.from_numpy(rng.random((2, 3, 5, 70)).astype(np.float32)).to(dev)
    srt = torch.sort(scores, dim=-1, descending=True)
    n = torch.from_numpy(rng.integers(0, 71, size=(2, 3, 5))).to(dev)
    filled = sparge.fill_block_map_triton(torch.zeros_like(m), n, srt.indices)
    want = torch.zeros_like(m)
    for idx in np.ndindex(mm.shape[:-1]):
        want[idx][srt.indices[idx][:n[idx]]] = True
    assert torch.equal(filled, want)
    assert torch.equal(sparge.hyperparameter_check(0.5, 3, dev), torch.full((3,), 0.5, device=dev))


@pytest.mark.parametrize("v_dtype,o_dtype", [(torch.float16, torch.float16), (torch.bfloat16, torch.float32)])
def test_qattn_mirror_matches_emulation(v_dtype, o_dtype, dev):
    """run_block_sparse_kernel's call sequence on plain sequences (reference
    attention.py:217-243): per_block_int8(q, k - km), LUT, the kernel writing o."""
    B, H, Tq, Tk = 1, 2, 260, 330
    q = _rand((B, H, Tq, 64), 4)
    k = _rand((B, H, Tk, 64), 5)
    v = _rand((B, H, Tk, 64), 6)
    rng = np.random.default_rng(9)
    fmap = torch.from_numpy(rng.random((B, H, 3, 6)) < 0.5)
    fmap[..., 0] = True
    km = sparge.key_mean(k.to(dev))
    q8, qs, k8, ks = sparge.per_block_int8(q.to(dev), k.to(dev), km=km)
    lut, nv = sparge.block_map_lut_triton(fmap.to(dev))
    o = torch.empty(B, H, Tq, 64, dtype=o_dtype, device=dev)
    sparge.qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold(
        q8, k8, v.to(dev).to(v_dtype), o, lut, nv, sparge.hyperparameter_check(1e10, H, dev), qs, ks, 1, 0, 1,
        0.125, 0)
    torch.cuda.synchronize()
    # emulate from the oracle's codes of the same plain sequences
    oq = oracle.prep_qkv(q, q, q, 1, Tq, 0)
    ok = oracle.prep_qkv(k, k, k, 1, Tk, 0)
    prep = {"q_i8": oq["q_i8"], "q_scale": oq["q_scale"], "k_i8": ok["k_i8"], "k_scale": ok["k_scale"]}
    lut_np, nv_np = lut.cpu().numpy().reshape(H, 3, 6), nv.cpu().numpy().reshape(H, 3)
    emu = ref.int8_attention_rows(prep, v.to(v_dtype).float(), 1, Tk, 0, lut_np, nv_np,
                                  [(h, r) for h in range(H) for r in range(3)], Tq=Tq)
    for (h, r), e in emu.items():
        got = o[0, h, r * 128:r * 128 + e.shape[0]].float().cpu()
        assert (got - e).abs().max().item() <= 1.5e-2
    sparge.check_last_call()  # a valid call records no problem
    # invalid inputs are found on the device without a synchronisation; the attention runs on
    # a copy clamped into range, and the problem is raised at the caller's next check
    sparge.qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold(
        q8, k8, v.to(dev), o, lut, nv, sparge.hyperparameter_check(50.0, H, dev), qs, ks, 1, 0, 1, 0.125, 0)
    with pytest.raises(ValueError, match="pv_threshold below 1e9"):
        sparge.check_last_call()
    bad_nv = nv.clone()
    bad_nv[0, 1, 2] = 7  # more than the 6 key blocks
    sparge.qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold(
        q8, k8, v.to(dev), o, lut, bad_nv, sparge.hyperparameter_check(1e10, H, dev), qs, ks, 1, 0, 1, 0.125, 0)
    with pytest.raises(ValueError, match="valid_block_num outside"):
        sparge.check_last_call()
    bad_lut = lut.clone()
    bad_lut[0, 0, 0, 0] = 6  # a block past the last one
    sparge.qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold(
        q8, k8, v.to(dev), o, bad_lut, nv, sparge.hyperparameter_check(1e10, H, dev), qs, ks, 1, 0, 1, 0.125, 0)
    with pytest.raises(ValueError, match="LUT entry"):
        sparge.check_last_call()
    unsorted = lut.clone()
    row = int(torch.nonzero(nv[0, 0] >= 2)[0, 0])
    unsorted[0, 0, row, :2] = unsorted[0, 0, row, :2].flip(0)  # two listed blocks swapped
    sparge.qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold(
        q8, k8, v.to(dev), o, unsorted, nv, sparge.hyperparameter_check(1e10, H, dev), qs, ks, 1, 0, 1, 0.125, 0)
    with pytest.raises(ValueError, match="not strictly ascending"):
        sparge.check_last_call()
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="is_causal"):
        sparge.qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold(
            q8, k8, v.to(dev), o, lut, nv, sparge.hyperparameter_check(1e10, H, dev), qs, ks, 1, 1, 1, 0.125, 0)
