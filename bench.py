"""Benchmark: one VGGT global-attention layer through the block-sparse path on one MI355X.

Workload (the metric's configuration): N = 16 frames x 1374
tokens = 21,984, H = 16, D = 64, bf16 Q/K/V already resident in HBM, HeSS per-head
budgets from synthetic (3,24,16) log-normal tables (lambda 0.5, layer 0), sparse_ratio
0.7. A step is one full layer forward of the hot path: preparation (pools, packed
K/V or INT8 codes), pooled map, budgets, selection + LUT, sparse attention with the
special-query rows dense, output in storage order.

    python bench.py [--steps K] [--warmup W] [--config 1] [--no-cpu-baseline]

Prints one JSON line. value = effective TFLOP/s = 4 N^2 H D / t (dense-equivalent);
ms_per_step = ms per layer (ms_per_step_median: the median of the per-step HIP-event
times), kernels launched eagerly; with --graph, ms_per_step_graph times the same step
captured once in a HIP graph and replayed (its output checked bit for bit against an
eager step first). roofline = the attention kernel's retained-block FLOPs over
its own HIP-event-timed duration against the dense MFMA peak of its arithmetic (QK^T
half at the bf16 or INT8 rate, PV half at the bf16 rate); frac_of_int8_peak prices the
same FLOPs against the INT8 peak, frac_of_measured_peak against the rates measured on
this GPU (measured_peaks: MFMA microbenchmark, 1 GiB copy). traffic (HBM bytes per
launch) and mfma_busy_pct_pmc (matrix-core busy cycles over active SIMD cycles) are read
from the committed rocprofv3 PMC summaries in profiles/ (the default 16-frame layer only).
"""

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_INT8_TOPS = 5000.0   # MI355X dense INT8 MFMA, TOPS
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, TFLOP/s
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E, GB/s


def mfma_peak(qk_mode):
    """Dense MFMA peak for the retained FLOPs, half of which are QK^T and half PV (bf16):
    QK^T at the bf16 or INT8 rate, harmonic combination of the two halves."""
    qk = PEAK_BF16_TFLOPS if qk_mode == "f16" else PEAK_INT8_TOPS
    return 1.0 / (0.5 / qk + 0.5 / PEAK_BF16_TFLOPS)


def measured_peaks(dev):
    """This GPU's measured dense MFMA rates (bf16, int8) from the libress_peak.so
    microbenchmark (four independent accumulator chains per wave, two workgroups of four
    waves per CU) and its HBM copy bandwidth (1 GiB device-to-device copy, read + write)."""
    import ctypes

    import torch

    from ress_amd.build import PEAK_LIB
    L = ctypes.CDLL(PEAK_LIB)
    L.ress_peak_mfma.restype = ctypes.c_int
    L.ress_peak_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    wgs = 2 * cus
    out = torch.empty(wgs * 256, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    res = {"cus": cus}
    for kind, name, per_mfma in ((0, "bf16_tflops", 32768), (1, "int8_tops", 65536)):
        iters = 20000
        if L.ress_peak_mfma(kind, 64, wgs, out.data_ptr(), stream) != 0:
            raise RuntimeError("ress_peak_mfma failed")
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        L.ress_peak_mfma(kind, iters, wgs, out.data_ptr(), stream)
        e.record()
        torch.cuda.synchronize()
        res[name] = round(wgs * 4 * iters * 4 * per_mfma / (s.elapsed_time(e) * 1e-3) / 1e12, 1)
    src = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    dst.copy_(src)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(5):
        dst.copy_(src)
    e.record()
    torch.cuda.synchronize()
    res["hbm_copy_GBs"] = round(5 * 2 * src.numel() * 4 / (s.elapsed_time(e) * 1e-3) / 1e9, 1)
    del src, dst
    return res


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget-s", type=float, default=15.0)
    ap.add_argument("--no-dense", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="also capture the step once in a HIP graph and time its replays (reported as "
                         "ms_per_step_graph; on this ROCm stack the replay measured slower than eager launches)")
    ap.add_argument("--qk-mode", default="f16", choices=["f16", "i8x2", "i8"],
                    help="QK^T operands of the attention kernel (16-bit: fp16 K blocks and per-row fp16 queries; "
                         "two-term or single-term INT8)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="run one plain device copy of this many MiB first (PMC traffic calibration)")
    return ap.parse_args()


def _profile_value(name, key):
    """The number on the `key:` line of profiles/<name>, or None."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return float(line.split(":", 1)[1])
    except OSError:
        return None
    return None


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel`, from the committed PMC summary (profiles/), or None.

    The summary holds FETCH_SIZE and WRITE_SIZE per dispatch, each divided by what the
    same counter read for a plain copy of known size; its 'traffic_bytes_per_launch'
    line is the sum."""
    return _profile_value(f"{kernel}_config1_pmc_traffic.txt", "traffic_bytes_per_launch")


def measured_mfma_busy(kernel):
    """Percent of SIMD cycles the matrix cores were busy during `kernel` (rocprofv3's
    MfmaUtil: SQ_VALU_MFMA_BUSY_CYCLES over the active cycles of every SIMD), from the
    committed PMC summary, or None."""
    return _profile_value(f"{kernel}_config1_pmc_mfma.txt", "mfma_busy_pct_per_launch")


def retained_flops(nvalid, lut, grid):
    """Sum over kept (row, key block) of 4*D*rows*cols with true partial sizes."""
    import numpy as np
    rows_p = [min(128, grid.T_p - 128 * i) for i in range(grid.q_blk_p)]
    rows_s = [min(128, grid.T_s - 128 * i) for i in range(grid.q_blk_s)]
    rows = np.array(rows_p + rows_s, dtype=np.float64)
    cols = np.array([min(64, grid.Tk - 64 * c) for c in range(grid.kb_tot)], dtype=np.float64)
    total = 0.0
    for bh in range(nvalid.shape[0]):
        for r in range(nvalid.shape[1]):
            total += rows[r] * cols[lut[bh, r, :nvalid[bh, r]]].sum()
    return 4.0 * 64 * total


def time_meansim(q, k, reps):
    """The fused meansim scoring pass (ress_meansim_block_map) over the layer's full sequence,
    buffers allocated once outside the timed region. Algorithmic bytes: read Q and K bf16,
    write their INT8 codes, the pooled means, scales, similarity flags and the map."""
    import torch

    from ress_amd import _lib
    B, H, T, _ = q.shape
    dev = q.device
    nq, nk = -(-T // 128), -(-T // 64)
    km = k.float().mean(2).reshape(B * H, 64).contiguous()
    th = torch.full((H,), 0.1, device=dev)
    cd = torch.full((H,), 0.9, device=dev)
    bufs = [torch.empty(B * H, nq, nk, dtype=torch.uint8, device=dev),
            torch.empty(B * H, nq * 128, 64, dtype=torch.int8, device=dev), torch.empty(B * H, nq, device=dev),
            torch.empty(B * H, nk * 64, 64, dtype=torch.int8, device=dev), torch.empty(B * H, nk, device=dev),
            torch.empty(B * H, nq, 64, device=dev), torch.empty(B * H, nk, 64, device=dev),
            torch.empty(B * H, nq, dtype=torch.uint8, device=dev), torch.empty(B * H, nk, dtype=torch.uint8, device=dev)]
    ws_bytes = _lib.lib().ress_meansim_workspace_size(B, H, T, T)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None

    def run():
        _lib.call("ress_meansim_block_map", _lib.ptr(q), _lib.ptr(k), _lib.ptr(km), B, H, T, T, *q.stride()[:3],
                  *k.stride()[:3], _lib.ptr(th), _lib.ptr(cd), 1374, *(_lib.ptr(b) for b in bufs), _lib.ptr(ws),
                  ws_bytes, _lib.stream_handle(dev))

    run()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        run()
    e.record()
    torch.cuda.synchronize()
    elems = B * H * T * 64
    nbytes = (elems * 2 * 2 + B * H * (nq * 128 + nk * 64) * 64 + B * H * (nq + nk) * (64 * 4 + 4 + 1)
              + B * H * nq * nk)
    return s.elapsed_time(e) / reps, nbytes


def run_aggregator(args):
    """a VGGT-1B-style aggregator (random init; 24 frame/global ViT-L
    block pairs, dim 1024, 16 heads) on 64 synthetic 518x518 frames (N = 87,936 tokens),
    ReSS (restore_swap_iter5_bf16_trackbest, HeSS budgets from synthetic per-layer tables)
    on all 24 global layers at sparse_ratio 0.8. A step is one forward; the global-attention
    share is the HIP-event time inside the 24 patched global-attention forwards (QKV
    projection to W_O included) over the step. The dense comparison is the same model
    (same seed) with plain SDPA global attention."""
    import torch

    import ress_amd as ress
    from ress_amd import synth
    from ress_amd.aggregator import build_vggt_aggregator, synthetic_frames
    from ress_amd.wiring import global_blocks

    dev = torch.device("cuda:0")
    S, depth = 64, 24
    cam, pc = synth.make_hess_tables()
    model = build_vggt_aggregator(depth, 1024, 16, device=dev, tables=(pc, cam))
    images = synthetic_frames(S, size=518, device=dev)
    ress.apply_ress(model, 0.8, n_iters=5)
    spans = []
    for block in global_blocks(model):
        fwd = block.attn.forward

        def timed(*a, _fwd=fwd, **kw):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            out = _fwd(*a, **kw)
            e.record()
            spans.append((s, e))
            return out

        block.attn.forward = timed
    with torch.no_grad():
        for _ in range(args.warmup):
            model(images)
        torch.cuda.synchronize()
        spans.clear()
        marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
        marks[0].record()
        for i in range(args.steps):
            model(images)
            marks[i + 1].record()
        torch.cuda.synchronize()
    ms = marks[0].elapsed_time(marks[-1]) / args.steps
    step_ms = sorted(marks[i].elapsed_time(marks[i + 1]) for i in range(args.steps))
    glob_ms = sum(s.elapsed_time(e) for s, e in spans) / args.steps
    result = {
        "metric": "ms per end-to-end aggregator forward (24 global layers under ReSS) + global-attention share",
        "value": round(ms, 2), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 2), "ms_per_step_median": round(step_ms[len(step_ms) // 2], 2),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 model; global attention fp16 QK (bf16 inputs) / bf16 PV / fp32 softmax",
        "data": "synthetic (64 frames 518x518: uniform [0,1] pixels + a shared low-frequency pattern); random weights",
        "config": {"workload": "BASELINE configs[3]: VGGT-1B-style aggregator, ReSS on all 24 global layers",
                   "frames": S, "tokens": S * 1374, "layers": depth, "dim": 1024, "heads": 16, "sparse_ratio": 0.8,
                   "criterion": "restore_swap_iter5_bf16_trackbest"},
        "global_attention_ms": round(glob_ms, 2), "global_attention_share": round(glob_ms / ms, 4),
    }
    if not args.no_dense:
        del model
        torch.cuda.empty_cache()
        plain = build_vggt_aggregator(depth, 1024, 16, device=dev, wire=False)
        with torch.no_grad():
            plain(images)
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            plain(images)
            e.record()
            torch.cuda.synchronize()
        result["dense_sdpa_forward_ms"] = round(s.elapsed_time(e), 2)
        result["speedup_vs_dense"] = round(s.elapsed_time(e) / ms, 3)
    print(json.dumps(result))


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU sharding (by heads, one "
                                   "all-gather of the HeSS counts) is not built", "n_gpus": args.gpus}))
        sys.exit(2)
    if args.config == 3:
        run_aggregator(args)
        return
    import numpy as np
    import torch
    import torch.nn.functional as F

    from ress_amd import budget, kernels, synth
    from ress_amd.attention import sparse_global_attention
    from ress_amd.kernels import LayerGrid

    cfg = synth.CONFIGS[args.config]
    dev = torch.device("cuda:0")
    t0 = time.time()
    q, k, v, meta = synth.make_layer_qkv(
        cfg["frames"], corr=cfg["corr"],
        progress=(lambda m: print(f"[bench] generating inputs: {m}", file=sys.stderr, flush=True))
        if cfg["frames"] > 32 else None)
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    if args.calib_copy_mib:
        src = torch.empty(args.calib_copy_mib << 18, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    print(f"[bench] inputs {tuple(q.shape)} generated in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    frames, P, S = meta["frames"], meta["P"], meta["S"]
    grid = LayerGrid(1, 16, frames, P, S)
    sr, cdf = cfg["sparse_ratio"], cfg["cdf_threshold"]
    if cfg["mode"] in ("hess", "ress"):
        cam, pc = synth.make_hess_tables()
        bud = budget.HessBudget(cam, pc, lam=0.5)
    else:
        bud = budget.UniformBudget()
    budget_fn = lambda a: bud.num_to_select(0, a, sr, cdf, 1.0)  # noqa: E731
    out = torch.empty(1, 16, grid.Tk, 64, dtype=torch.float32, device=dev)
    criterion, M = "probability", None
    if cfg["mode"] == "ress":  # restore-swap ranking with M_h from a seeded W_O
        criterion = f"restore_swap_iter{cfg['n_iters']}_bf16_trackbest"
        W_O = synth.make_w_o().to(dev)
        M = torch.stack([W_O[:, h * 64:(h + 1) * 64].T @ W_O[:, h * 64:(h + 1) * 64] for h in range(16)])

    # attention-kernel events: recorded on the stream the kernel is launched on
    ev = []
    orig_attn = kernels.sparse_attention

    def timed_attention(*a, **kw):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        r = orig_attn(*a, **kw)
        e.record()
        ev.append((s, e))
        return r

    import ress_amd.attention as attn_mod
    from ress_amd import projected
    attn_mod.kernels.sparse_attention = timed_attention
    rs_ev = []
    orig_rs = projected.restore_swap_keep

    def timed_restore_swap(*a, **kw):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        r = orig_rs(*a, **kw)
        e.record()
        rs_ev.append((s, e))
        return r

    projected.restore_swap_keep = timed_restore_swap

    sink = cfg.get("attention_sink", 0)

    def step():
        return sparse_global_attention(q, k, v, grid, budget_fn=budget_fn, out=out, qk_mode=args.qk_mode,
                                       block_criterion=criterion, M=M, attention_sink=sink)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev.clear()
    rs_ev.clear()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    marks[0].record()
    for i in range(args.steps):
        res = step()
        marks[i + 1].record()
    torch.cuda.synchronize()
    ms = marks[0].elapsed_time(marks[-1]) / args.steps
    step_ms = sorted(marks[i].elapsed_time(marks[i + 1]) for i in range(args.steps))
    ms_median = step_ms[len(step_ms) // 2]
    attn_ms = sum(s.elapsed_time(e) for s, e in ev) / len(ev)
    rs_ms = sum(s.elapsed_time(e) for s, e in rs_ev) / len(rs_ev) if rs_ev else None
    attn_mod.kernels.sparse_attention = orig_attn
    projected.restore_swap_keep = orig_rs
    # --graph: the same step captured once in a HIP graph and replayed (every kernel and
    # buffer of the eager step); the replay's output is checked against an eager step bit
    # for bit before it is timed. The eager step stays the headline figure.
    ms_graph = ms_graph_median = None
    if args.graph:
        step()
        torch.cuda.synchronize()
        want = out.clone()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        graph_checked = bool(torch.equal(out, want))
        if not graph_checked:
            raise RuntimeError("graph replay differs from the eager step")
        gm = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
        gm[0].record()
        for i in range(args.steps):
            g.replay()
            gm[i + 1].record()
        torch.cuda.synchronize()
        ms_graph = gm[0].elapsed_time(gm[-1]) / args.steps
        g_ms = sorted(gm[i].elapsed_time(gm[i + 1]) for i in range(args.steps))
        ms_graph_median = g_ms[len(g_ms) // 2]
        del g

    # work actually done (same map every step)
    res = sparse_global_attention(q, k, v, grid, budget_fn=budget_fn, out=out, keep_intermediates=True,
                                  qk_mode=args.qk_mode, block_criterion=criterion, M=M, attention_sink=sink)
    torch.cuda.synchronize()
    lut, nvalid = res.lut.cpu().numpy(), res.nvalid.cpu().numpy()
    flops_kept = retained_flops(nvalid, lut, grid)
    N = grid.Tk
    flops_dense = 4.0 * N * N * 16 * 64
    sparsity = res.sparsity()
    achieved = flops_kept / (attn_ms * 1e-3) / 1e12

    # preparation pass (HBM-bound). Algorithmic bytes, in units of one (N,H,64) tensor's
    # element count: bf16 reads Q,K,V (6) and writes packed K,V (4); the INT8 modes read
    # Q,K,V and K again (8) and write the codes (2 per term) and packed V (2).
    pe_s, pe_e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 20
    pe_s.record()
    for _ in range(reps):
        kernels.prepare_blocks(q, k, v, grid, mode=args.qk_mode)
    pe_e.record()
    torch.cuda.synchronize()
    prep_ms = pe_s.elapsed_time(pe_e) / reps
    elems = N * 16 * 64
    prep_bytes = elems * {"f16": 10, "i8x2": 14, "i8": 12}[args.qk_mode]
    peak = mfma_peak(args.qk_mode)
    ms_meansim, ms_bytes = time_meansim(q, k, 100)
    peaks = measured_peaks(dev)
    qk_meas = peaks["bf16_tflops"] if args.qk_mode == "f16" else peaks["int8_tops"]
    peak_meas = 1.0 / (0.5 / qk_meas + 0.5 / peaks["bf16_tflops"])

    result = {
        "metric": "ms/global-attn layer + effective TFLOPS, N=21984 H16 D64 @70% sparse, 1 GPU",
        "value": round(flops_dense / (ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s (effective, dense-equivalent 4*N^2*H*D per layer)",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "ms_per_step_median": round(ms_median, 4),
        "ms_per_step_graph": None if ms_graph is None else round(ms_graph, 4),
        "ms_per_step_graph_median": None if ms_graph is None else round(ms_graph_median, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"f16": "fp16 QK (bf16 inputs)", "i8x2": "two-term int8 QK", "i8": "int8 QK"}[args.qk_mode]
                 + " / bf16 PV / fp32 softmax",
        "data": "synthetic (seeded smoothed-field Q/K/V, Hilbert order; synthetic HeSS tables)",
        "config": {"workload": f"BASELINE configs[{args.config}]: one global-attention layer, {cfg['mode']} budget",
                   "frames": frames, "tokens": N, "heads": 16, "head_dim": 64, "sparse_ratio": sr,
                   "cdf_threshold": cdf, "attention_sink": sink, "realized_sparsity": round(sparsity, 4),
                   "qk_mode": args.qk_mode},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": round(peak, 1), "unit": "TFLOP/s",
                     "frac": round(achieved / peak, 4),
                     "traffic": measured_traffic(f"k_sparse_attn_{args.qk_mode}") if args.config == 1 else None,
                     "mfma_busy_pct_pmc": measured_mfma_busy(f"k_sparse_attn_{args.qk_mode}") if args.config == 1 else None,
                     "frac_of_int8_peak": round(achieved / PEAK_INT8_TOPS, 4),
                     "measured_peak": round(peak_meas, 1), "frac_of_measured_peak": round(achieved / peak_meas, 4),
                     "kernel": "k_sparse_attn_f16" if args.qk_mode == "f16" else "k_sparse_attn",
                     "kernel_ms": round(attn_ms, 4),
                     "retained_flop_per_launch": flops_kept},
        "restore_swap_ms": None if rs_ms is None else round(rs_ms, 4),
        "measured_peaks": peaks,
        "prep": {"ms": round(prep_ms, 4), "algorithmic_bytes": prep_bytes,
                 "achieved_GBs": round(prep_bytes / (prep_ms * 1e-3) / 1e9, 1), "peak_GBs": PEAK_HBM_GBS},
        "meansim_scoring": {"ms": round(ms_meansim, 4), "algorithmic_bytes": ms_bytes,
                            "achieved_GBs": round(ms_bytes / (ms_meansim * 1e-3) / 1e9, 1),
                            "peak_GBs": PEAK_HBM_GBS, "measured_copy_GBs": peaks["hbm_copy_GBs"],
                            "what": "SpargeAttn get_block_map_meansim_fuse_quant over the full sequence "
                                    "(K smoothed by its mean, sinks = first frame)"},
    }

    if not args.no_dense:
        qd = q.contiguous()
        for _ in range(3):
            F.scaled_dot_product_attention(qd, k, v)
        torch.cuda.synchronize()
        ds, de = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ds.record()
        for _ in range(10):
            F.scaled_dot_product_attention(qd, k, v)
        de.record()
        torch.cuda.synchronize()
        dense_ms = ds.elapsed_time(de) / 10
        result["dense_bf16_sdpa_ms"] = round(dense_ms, 4)
        result["speedup_vs_dense"] = round(dense_ms / ms, 3)

    if not args.no_cpu_baseline:
        from oracle.cpu_baseline import time_block_masked_sdpa
        cb = time_block_masked_sdpa(q.cpu(), k.cpu(), v.cpu(), frames, P, S, lut, nvalid, budget_s=args.cpu_budget_s)
        result["cpu_baseline"] = {
            "value": round(cb["ms_per_layer"], 1), "unit": "ms/layer", "cores": cb["threads"], "kind": "port",
            "cpu": cb["cpu_model"],
            "sample": f"fp32 block-masked SDPA (PyTorch CPU) on a fixed sample of {cb['rows_timed']} of "
                      f"{cb['rows_total']} (head, q-block) rows: median of {cb['runs']} timed runs after a "
                      f"warm-up ({cb['elapsed_s']:.1f}s in all), extrapolated by kept-block count"}
    print(json.dumps(result))


if __name__ == "__main__":
    main()
