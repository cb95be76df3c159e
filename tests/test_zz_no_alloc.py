"""The allocation-free attention entry point (ress_sparse_attn_fwd_f16_noalloc) against
the workspace entry point it shares its kernels with (ress_sparse_attn_fwd_f16), through
the C ABI: bit-identical outputs on two calls in a row, the second on a smaller layer, so
the shared static scratch is reused with different shapes."""

import numpy as np
import pytest
import torch

from ress_amd import _lib, kernels, synth
from ress_amd.kernels import LayerGrid

pytestmark = pytest.mark.gpu


def _layer(frames, H, dev, seed):
    q, k, v, meta = synth.make_layer_qkv(frames, H=H, seed=seed)
    g = LayerGrid(1, H, frames, meta["P"], meta["S"])
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    blocks = kernels.prepare_blocks(q, k, v, g, mode="f16")
    rng = np.random.default_rng(seed)
    keys = torch.from_numpy(rng.random((1, H, g.q_blk_p, g.n_cand)).astype(np.float32)).to(dev)
    counts = torch.from_numpy(rng.integers(0, g.n_cand + 1, (1, H, g.q_blk_p)).astype(np.int32)).to(dev)
    _, lut, nvalid = kernels.select_blocks(keys, counts, g, 2, sink_lead=3)
    return g, blocks, lut, nvalid


def _run(entry, g, blocks, lut, nvalid, dev):
    out = torch.full((g.B, g.H, g.Tk, 64), float("nan"), device=dev)
    P = _lib.ptr
    args = [P(blocks.q), *blocks.q.stride()[:3], P(blocks.k_pack), P(blocks.k_scale), P(blocks.v_pack), P(lut),
            P(nvalid), g.B, g.H, g.frames, g.P, g.S, None, 0.125, P(out), 0, *out.stride()[:3]]
    if entry == "ress_sparse_attn_fwd_f16":
        sched = torch.empty(_lib.lib().ress_attn_sched_bytes(g.B, g.H, g.Tk), dtype=torch.uint8, device=dev)
        args.append(P(sched))
    _lib.call(entry, *args, _lib.stream_handle(dev))
    torch.cuda.synchronize()
    return out


def test_noalloc_matches_workspace_entry_point(dev):
    assert _lib.lib().ress_noalloc_scratch_bytes() >= _lib.lib().ress_attn_sched_bytes(8, 64, 1 << 22)
    for frames, H, seed in ((16, 16, 0), (3, 4, 1)):   # the second call is smaller
        print(f"[noalloc] frames={frames} H={H}", flush=True)
        g, blocks, lut, nvalid = _layer(frames, H, dev, seed)
        want = _run("ress_sparse_attn_fwd_f16", g, blocks, lut, nvalid, dev)
        got = _run("ress_sparse_attn_fwd_f16_noalloc", g, blocks, lut, nvalid, dev)
        assert not torch.isnan(got).any()
        assert torch.equal(got, want)


def _read_status_word():
    """The noalloc call's operand-status word, read from its device address with a 4-byte
    hipMemcpy (device to host)."""
    import ctypes
    addr = ctypes.c_void_p()
    _lib.call("ress_noalloc_status_address", ctypes.byref(addr))
    hip = ctypes.CDLL("libamdhip64.so")
    word = ctypes.c_int(-1)
    assert hip.hipMemcpy(ctypes.byref(word), addr, ctypes.c_size_t(4), 2) == 0   # hipMemcpyDeviceToHost
    return word.value


def test_noalloc_reports_fp16_range_through_its_status_word(dev):
    """A key element fp16 cannot hold (70000; bf16 can) is reported in the noalloc call's
    status word, as ress_sparse_attn_fwd_f16 reports it in its workspace; the next call on
    clean data clears the word."""
    frames, H, seed = 2, 4, 2
    q, k, v, meta = synth.make_layer_qkv(frames, H=H, seed=seed)
    g = LayerGrid(1, H, frames, meta["P"], meta["S"])
    k_bad = k.clone()
    k_bad[0, 1, 7, 3] = 70000.0
    counts = torch.full((1, H, g.q_blk_p), max(2, g.n_cand // 2), dtype=torch.int32, device=dev)
    keys = torch.ones(1, H, g.q_blk_p, g.n_cand, device=dev)
    _, lut, nvalid = kernels.select_blocks(keys, counts, g, 2)
    for kk, want in ((k_bad, 1), (k, 0)):
        print(f"[noalloc status] key element {float(kk[0, 1, 7, 3]):.0f}", flush=True)
        blocks = kernels.prepare_blocks(q.to(dev), kk.to(dev), v.to(dev), g, mode="f16")
        _run("ress_sparse_attn_fwd_f16_noalloc", g, blocks, lut, nvalid, dev)
        assert _read_status_word() == want
