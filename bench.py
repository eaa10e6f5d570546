"""Benchmark of the MI355X K-quant dequant-matvec + MoE hot path.

Headline (BASELINE.json metric "Q4_K matvec HBM GB/s (% peak); MoE layer
us/token at batch 1 and 512"): the Q4_K 4096x4096 decode matvec of
configs[0], fp32 x and y, measured cold from HBM.  One step = one matvec over
each of NCOPY distinct copies of the weight matrix (>= 2x the 256 MB
Infinity Cache), so no launch finds its weights in the MALL.  `value` is
algorithmic bytes (packed weights + x + y per matvec) / wall time of the
timed steps.  The same line carries the mixed-format sweep, the
MoE layer at batch 1 and 16 and 512 tokens, the
roofline fraction of the dominant kernel, and the reference CPU path timed
on this host.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"fp16": 2500.0, "int8": 5000.0}   # MI355X dense, per GPU
PMC_COPY_BYTES = 256 << 20
PROFILES = ("q4k", "q4k_graph", "q4k_big", "sweep", "seg", "moe_b1", "moe_b16", "moe_prefill", "moe_prefill_i8")
PMC_SUMMARY = os.path.join(ROOT, "profiles", "q4k_matvec_4096x4096_pmc.txt")


def pmc_traffic():
    """HBM bytes per launch of the headline kernel, from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, copy-calibrated), or
    None when that summary is absent."""
    try:
        with open(PMC_SUMMARY) as f:
            for ln in f:
                if ln.startswith("traffic_bytes_per_launch:"):
                    return int(float(ln.split(":", 1)[1]))
    except OSError:
        pass
    return None


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--quick", action="store_true", help="skip the sweep/MoE/CPU legs")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--moe-only", action="store_true", help="only the MoE leg (profiling)")
    p.add_argument("--dense-only", action="store_true", help="only the dense decode leg (profiling)")
    p.add_argument("--no-dense", action="store_true", help="skip the dense decode leg")
    p.add_argument("--pmc-calib", action="store_true", help="same as --profile q4k")
    p.add_argument("--profile", choices=sorted(PROFILES),
                   help="counter-collection run for rocprofv3: one workload as direct launches (no graph), "
                        "then a plain copy of PMC_COPY_BYTES (the HBM-byte calibration of FETCH_SIZE / "
                        "WRITE_SIZE); prints nothing on stdout")
    a = p.parse_args()
    if a.pmc_calib:
        a.profile = "q4k"
    return a


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def time_region(fn, steps, warmup, stream, graph=True):
    """Time exactly `steps` executions of fn() with HIP events recorded on the
    stream the kernels run on; returns seconds.  With graph=True, fn's launches
    are captured once into a HIP graph and the graph is replayed, so host-side
    launch cost (Python + ctypes) is not in the measurement."""
    import torch
    for _ in range(max(1, warmup)):
        fn()
    torch.cuda.synchronize()
    run = fn
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        run = g.replay
        for _ in range(warmup):
            run()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3


def matvec_bytes(qt, M, K):
    from trailblaze_amd import formats as fm
    return fm.weight_bytes(qt, M, K) + 4 * K + 4 * M


def gpu_leg(args):
    import torch

    import trailblaze_amd as tb
    from trailblaze_amd import formats as fm
    from trailblaze_amd import synth

    dev_name = tb.init()
    log("device", dev_name)
    stream = torch.cuda.current_stream()
    res = {"device": dev_name}
    if args.profile:
        profile_leg(args.profile, tb, fm, synth, torch)
        return res

    # ---- headline: Q4_K 4096x4096, cold HBM via rotated copies ----------
    qt, M, K = fm.Q4_K, 4096, 4096
    rng = np.random.default_rng(0)
    W0 = synth.kquant_matrix(qt, M, K, rng)
    x = torch.from_numpy(synth.activations(K, rng)).cuda()
    wbytes = fm.weight_bytes(qt, M, K)
    ncopy = max(2, int(np.ceil(2 * 256e6 / wbytes)) + 1)
    Wd = torch.from_numpy(W0).cuda()
    copies = [Wd] + [Wd.clone() for _ in range(ncopy - 1)]
    ys = torch.empty((ncopy, M), dtype=torch.float32, device="cuda")

    def step():
        for i in range(ncopy):
            tb.matvec(copies[i], qt, M, K, x, ys[i])

    # the kernel's own average duration over the timed region, from HIP
    # events on the stream it runs on (graph replay, one event pair)
    secs = time_region(step, args.steps, args.warmup, stream)
    per_launch = secs / (args.steps * ncopy)
    bpl = matvec_bytes(qt, M, K)
    gbs = bpl / per_launch / 1e9
    res["headline"] = dict(qt="Q4_K", M=M, K=K, ncopy=ncopy, ms_per_step=secs / args.steps * 1e3,
                           us_per_launch=per_launch * 1e6, bytes_per_launch=bpl, gbs=gbs)
    log(f"Q4_K 4096x4096 cold: {per_launch * 1e6:.2f} us/launch  {gbs:.0f} GB/s  ({gbs / HBM_PEAK_GBS:.1%} of 8 TB/s)")

    # warm (MALL-resident) number, same matrix every launch
    def warm():
        for _ in range(ncopy):
            tb.matvec(Wd, qt, M, K, x, ys[0])
    ws = time_region(warm, args.steps, args.warmup, stream)
    res["headline"]["warm_us_per_launch"] = ws / (args.steps * ncopy) * 1e6
    res["headline"]["warm_gbs"] = bpl / (ws / (args.steps * ncopy)) / 1e9
    del copies
    torch.cuda.empty_cache()

    if args.quick:
        return res

    # the reference ABI (host x in, host y out, synchronous): PCIe-inclusive
    # per-call time, never the headline value
    xh = np.ascontiguousarray(synth.activations(K, rng))
    yh = np.empty(M, np.float32)
    fn = tb.lib().tb_cuda_matvec_device
    for _ in range(20):
        fn(Wd.data_ptr(), qt, M, K, xh.ctypes.data, yh.ctypes.data)
    n_abi = 300
    t0 = time.perf_counter()
    for _ in range(n_abi):
        fn(Wd.data_ptr(), qt, M, K, xh.ctypes.data, yh.ctypes.data)
    res["abi_matvec_us"] = (time.perf_counter() - t0) / n_abi * 1e6
    log(f"tb_cuda_matvec_device (host x/y, synchronous): {res['abi_matvec_us']:.1f} us/call")

    if args.dense_only:
        res["dense"] = dense_leg(torch, stream)
        return res
    if args.moe_only:
        res["moe"] = moe_leg(tb, fm, synth, torch, rng, stream)
        return res
    # ---- HBM ceiling on this box: torch's read reduction and copy over
    # buffers larger than the MALL (a reference point for the fractions) --
    res["hbm_ceiling"] = hbm_ceiling(torch, stream)
    # ---- steady-state Q4_K stream: a matrix larger than the MALL --------
    res["q4k_steady"] = sweep_leg(tb, fm, synth, torch, rng, stream, [(fm.Q4_K, 151936, 4096),
                                                                      (fm.Q4_K, 65536, 4096)])
    # ---- configs[1] sweep ------------------------------------------------
    res["sweep"] = sweep_leg(tb, fm, synth, torch, rng, stream, SWEEP_SHAPES)
    # the same formats in ggml's on-disk layouts (TBQ_GGML ids)
    G = fm.GGML
    res["ggml_sweep"] = sweep_leg(tb, fm, synth, torch, rng, stream, [
        (G | fm.Q4_K, 4096, 4096), (G | fm.Q4_K, 12288, 4096), (G | fm.Q4_K, 4096, 12288),
        (G | fm.Q6_K, 12288, 4096), (G | fm.Q6_K, 4096, 12288), (G | fm.Q5_K, 12288, 4096),
        (G | fm.Q3_K, 12288, 4096), (G | fm.Q2_K, 12288, 4096), (G | fm.Q8_0, 12288, 4096)])

    res["moe"] = moe_leg(tb, fm, synth, torch, rng, stream)
    if not args.no_dense and not args.quick:
        res["dense"] = dense_leg(torch, stream)
    return res


def _sweep_shapes():
    from trailblaze_amd import formats as fm
    return [(fm.Q2_K, 12288, 4096), (fm.Q2_K, 4096, 12288), (fm.Q3_K, 12288, 4096), (fm.Q3_K, 4096, 12288),
            (fm.Q5_K, 12288, 4096), (fm.Q5_K, 4096, 12288), (fm.Q8_0, 12288, 4096), (fm.Q8_0, 4096, 12288),
            (fm.Q6_K, 151936, 4096)]


SWEEP_SHAPES = None   # filled in main() (formats import)


def hbm_ceiling(torch, stream):
    """Read and copy bandwidth of torch's own kernels on 512 MiB buffers
    (two alternating, so neither fits the 256 MB MALL)."""
    n = 512 << 20
    bufs = [torch.ones(n // 4, dtype=torch.float32, device="cuda") for _ in range(2)]
    dst = torch.empty(n // 4, dtype=torch.float32, device="cuda")
    acc = torch.zeros((), dtype=torch.float32, device="cuda")

    def rd():
        for b in bufs:
            torch.sum(b, dim=0, out=acc)

    def cp():
        for b in bufs:
            dst.copy_(b)
    r = time_region(rd, 10, 2, stream, graph=False) / 20
    c = time_region(cp, 10, 2, stream, graph=False) / 20
    out = dict(read_gbs=round(n / r / 1e9, 1), copy_gbs=round(2 * n / c / 1e9, 1), bytes=n,
               kernels="torch.sum (read), Tensor.copy_ (read + write)")
    log(f"HBM ceiling: torch.sum read {out['read_gbs']:.0f} GB/s, copy_ {out['copy_gbs']:.0f} GB/s (read+write)")
    del bufs, dst
    torch.cuda.empty_cache()
    return out


def hbm_roofline(nbytes, secs):
    gbs = nbytes / secs / 1e9
    return dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                frac=round(gbs / HBM_PEAK_GBS, 4))


def profile_leg(name, tb, fm, synth, torch):
    """One workload as direct launches for rocprofv3 (kernel trace or
    counters per dispatch), then the copy that calibrates FETCH_SIZE and
    WRITE_SIZE.  Weights are rotated over copies larger than the MALL where
    one matrix is smaller, as in the timed legs."""
    rng = np.random.default_rng(0)
    reps = 3
    if name == "q4k_graph":
        # the headline leg as timed: the 56-launch step in a HIP graph, replayed
        # (kernel trace: every dispatch of the timed region is a cold launch)
        qt, M, K = fm.Q4_K, 4096, 4096
        W = torch.from_numpy(synth.kquant_matrix(qt, M, K, rng)).cuda()
        nc = max(2, int(np.ceil(2 * 256e6 / fm.weight_bytes(qt, M, K))) + 1)
        cps = [W] + [W.clone() for _ in range(nc - 1)]
        x = torch.from_numpy(synth.activations(K, rng)).cuda()
        ys = torch.empty((nc, M), dtype=torch.float32, device="cuda")

        def step():
            for i in range(nc):
                tb.matvec(cps[i], qt, M, K, x, ys[i])
        steps = 20
        secs = time_region(step, steps, 3, torch.cuda.current_stream())
        log(f"profile {name}: Q4_K {M}x{K}, graph of {nc} launches replayed {steps} times after 3 warm-up "
            f"replays: event-timed {secs / (steps * nc) * 1e6:.3f} us/launch")
        del cps, W
    elif name in ("q4k", "q4k_big", "sweep", "seg"):
        # seg: rows the segmented mapping serves (K = 2560, Qwen3-4B's hidden)
        shapes = {"q4k": [(fm.Q4_K, 4096, 4096)], "q4k_big": [(fm.Q4_K, 151936, 4096)],
                  "sweep": _sweep_shapes(),
                  "seg": [(fm.Q4_K, 151936, 2560), (fm.Q5_K, 19456, 2560), (fm.Q3_K, 6144, 2560),
                          (fm.Q6_K, 151936, 2560)]}[name]
        for qt, M, K in shapes:
            W = torch.from_numpy(synth.kquant_matrix(qt, M, K, rng)).cuda()
            nc = max(1, int(np.ceil(2 * 256e6 / fm.weight_bytes(qt, M, K))) + (1 if M * K < 2 ** 26 else 0))
            cps = [W] + [W.clone() for _ in range(nc - 1)]
            x = torch.from_numpy(synth.activations(K, rng)).cuda()
            y = torch.empty(M, dtype=torch.float32, device="cuda")
            for _ in range(reps):
                for c in cps:
                    tb.matvec(c, qt, M, K, x, y)
            torch.cuda.synchronize()
            log(f"profile {name}: {fm.NAMES[qt]} {M}x{K}, {reps} x {nc} launches")
            del cps, W
            torch.cuda.empty_cache()
    else:
        H, F, E, k = 2048, 768, 128, 8
        prefill = name.startswith("moe_prefill")
        layers, keep = moe_layers(tb, fm, synth, torch, H, F, E, k, 1 if prefill else 3)
        T = 512 if prefill else {"moe_b1": 1, "moe_b16": 16}[name]
        mode = {"moe_prefill": tb.TBQ_MOE_BF16, "moe_prefill_i8": tb.TBQ_MOE_I8}.get(name, tb.TBQ_MOE_FP32)
        L = layers[0]
        if prefill:
            bias = torch.from_numpy(synth.zipf_router_bias(E, 1.1, 1.0, rng)).cuda()
            L = tb.moe_layer(H, F, E, k, fm.Q4_K, *L._keep[:4], bias=bias)
            layers = [L]
        n = 8 if prefill else 24
        xs = torch.from_numpy(synth.activations((n, T, H), rng)).cuda()
        out = torch.empty((T, H), dtype=torch.float32, device="cuda")
        ws = torch.zeros(tb.moe_workspace_size(L, T, mode), dtype=torch.uint8, device="cuda")
        for i in range(n):
            tb.moe_forward(layers[i % len(layers)], T, xs[i], xs[(i + 1) % n], out, workspace=ws, mode=mode)
        torch.cuda.synchronize()
        log(f"profile {name}: {n} MoE layer calls at T={T} over {len(layers)} layer copies")
        del keep
    torch.cuda.empty_cache()
    src = torch.empty(PMC_COPY_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"profile {name}: calibration copies 5 x {PMC_COPY_BYTES} B")


def sweep_leg(tb, fm, synth, torch, rng, stream, shapes):
    """Per-launch time of tbq_matvec at each (qtype, M, K), cold: enough
    rotated weight copies that every launch reads HBM."""
    out = []
    for qt2, M2, K2 in shapes:
        Wm = torch.from_numpy(synth.kquant_matrix(qt2, M2, K2, rng)).cuda()
        wb = fm.weight_bytes(qt2, M2, K2)
        nc = max(1, int(np.ceil(2 * 256e6 / wb)))
        cps = [Wm] + [Wm.clone() for _ in range(nc - 1)]
        xv = torch.from_numpy(synth.activations(K2, rng)).cuda()
        yv = torch.empty(M2, dtype=torch.float32, device="cuda")

        def st():
            for c in cps:
                tb.matvec(c, qt2, M2, K2, xv, yv)
        reps = max(3, int(2000 // max(1, nc)))
        s = time_region(st, reps, 2, stream)
        pl = s / (reps * nc)
        b = matvec_bytes(qt2, M2, K2)
        out.append(dict(qt=fm.NAMES[qt2], M=M2, K=K2, us=pl * 1e6, gbs=b / pl / 1e9,
                        frac=round(b / pl / 1e9 / HBM_PEAK_GBS, 4), copies=nc))
        log(f"{fm.NAMES[qt2]} {M2}x{K2}: {pl * 1e6:.2f} us  {b / pl / 1e9:.0f} GB/s "
            f"({b / pl / 1e9 / HBM_PEAK_GBS:.1%})")
        del cps, Wm
        torch.cuda.empty_cache()
    return out


def dense_leg(torch, stream):
    """Dense Qwen3-4B-shaped decode: one token at KV context 4096
    (the cache filled N(0,1), decoding position 4095), random-init Q4_K
    layers and Q6_K tied embedding/lm_head; one step = one token through 36
    layers and the lm_head, replayed from a HIP graph.  The matvecs alone
    (same shapes and weights, one graph) are timed beside it."""
    from trailblaze_amd import formats as fm
    from trailblaze_amd.dense import QWEN3_4B, SyntheticDense
    c = QWEN3_4B
    m = SyntheticDense(c, seed=4)
    m.k_cache.normal_()
    m.v_cache.normal_()
    logits = torch.empty(c.vocab, dtype=torch.float32, device="cuda")
    pos = c.max_ctx - 1
    reps = 20
    s = time_region(lambda: m.decode(1234, pos, logits), reps, 3, stream)
    us = s / reps * 1e6
    shapes = m.matvec_shapes()
    xs = torch.randn(max(K for _, _, K, _ in shapes), device="cuda")
    ys = torch.empty(max(M for _, M, _, _ in shapes), device="cuda")

    def mvs():
        for qt, M, K, W in shapes:
            tb_matvec(W, qt, M, K, xs, ys)
    smv = time_region(mvs, reps, 3, stream)
    mv_us = smv / reps * 1e6
    wbytes = sum(fm.weight_bytes(qt, M, K) for qt, M, K, _ in shapes)
    kv_bytes = 2 * c.n_layers * c.n_kv_heads * c.max_ctx * c.head_dim * 4
    bound_us = (wbytes + kv_bytes) / (HBM_PEAK_GBS * 1e3)
    log(f"dense Qwen3-4B decode @ctx {c.max_ctx}: {us:.0f} us/token = {1e6 / us:.0f} tok/s; "
        f"matvecs {mv_us:.0f} us ({wbytes / mv_us / 1e3:.0f} GB/s); HBM bound {bound_us:.0f} us")
    # batched prefill of a 512-token prompt from position 0 (the host token
    # copy keeps it out of a graph: timed as direct launches)
    T = 512
    toks = np.random.default_rng(5).integers(0, c.vocab, T)
    sp = time_region(lambda: m.prefill(toks, 0, logits), 5, 2, stream, graph=False)
    pf_ms = sp / 5 * 1e3
    layer_params = (c.hidden * (c.n_heads + 2 * c.n_kv_heads) * c.head_dim + c.n_heads * c.head_dim * c.hidden
                    + 3 * c.ffn * c.hidden)
    gemm_tflops = 2.0 * layer_params * c.n_layers * T / (pf_ms * 1e-3) / 1e12
    log(f"dense Qwen3-4B prefill T={T}: {pf_ms:.2f} ms = {T / pf_ms * 1e3:.0f} tok/s "
        f"(layer GEMMs {gemm_tflops:.0f} TFLOP/s over the whole step; token by token it would be "
        f"{T * us / 1e3:.0f} ms)")
    del m
    torch.cuda.empty_cache()
    # the same model in ggml's layouts (Q4_K layers, Q6_K embedding), as a
    # llama.cpp file holds it
    from dataclasses import replace
    mg = SyntheticDense(replace(c, qtype_layers=fm.GGML | fm.Q4_K, qtype_embd=fm.GGML | fm.Q6_K), seed=4)
    mg.k_cache.normal_()
    mg.v_cache.normal_()
    sg = time_region(lambda: mg.decode(1234, pos, logits), reps, 3, stream)
    ggml_us = sg / reps * 1e6
    log(f"dense Qwen3-4B decode, ggml layouts: {ggml_us:.0f} us/token = {1e6 / ggml_us:.0f} tok/s")
    del mg
    torch.cuda.empty_cache()
    return dict(us_per_token=us, tokens_per_s=1e6 / us, ggml_us_per_token=ggml_us,
                matvec_us=mv_us, matvec_gbs=wbytes / mv_us / 1e3,
                other_us=us - mv_us, weight_bytes=wbytes, kv_bytes=kv_bytes, hbm_bound_us=bound_us,
                frac_of_bound=bound_us / us,
                prefill_512=dict(ms=pf_ms, tokens_per_s=T / pf_ms * 1e3, layer_gemm_tflops=gemm_tflops))


def tb_matvec(W, qt, M, K, x, y):
    import trailblaze_amd as tb
    tb.matvec(W, qt, M, K, x, y)


def moe_layers(tb, fm, synth, torch, H, F, E, k, n):
    """n distinct copies of one random-init MoE layer on the device (the
    first from the seeded recipe, the others device clones): rotating over
    them keeps every call's experts out of the 256 MB MALL."""
    router, gate, up, down = synth.moe_layer(H, F, E, fm.Q4_K, seed=3)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    base = [d(router), d(gate), d(up), d(down)]
    keep, layers = [base], [tb.moe_layer(H, F, E, k, fm.Q4_K, *base)]
    for _ in range(n - 1):
        c = [t.clone() for t in base]
        keep.append(c)
        layers.append(tb.moe_layer(H, F, E, k, fm.Q4_K, *c))
    return layers, keep


EXPERT_BYTES = 3 * 768 * 2048 // 256 * 144   # one Q4_K expert at the Qwen3-30B-A3B shape: 2,654,208 B


def moe_leg(tb, fm, synth, torch, rng, stream):
    """MoE layer (configs[3] decode at batch 1 and 16, configs[4] prefill).
    Decode is timed cold: consecutive calls go to different copies of the
    layer (3 copies, 1 GB), so an expert's weights come from HBM, not from
    the MALL; the warm number repeats one layer.  Algorithmic bytes per call
    = router + U distinct experts x 2,654,208 B + xn, resid, out."""
    H, F, E, k = 2048, 768, 128, 8
    NL = 3
    layers, keep = moe_layers(tb, fm, synth, torch, H, F, E, k, NL)
    router_bytes = E * H * 4
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    moe = {}

    def distinct_experts(Lx, xs, T):
        idx = torch.empty(T * 8, dtype=torch.int32, device="cuda")
        w = torch.empty(T * 8, dtype=torch.float32, device="cuda")
        us = []
        for i in range(xs.shape[0]):
            tb.route(xs[i], Lx._keep[0], Lx._keep[4], T, H, E, k, idx, w)
            us.append(len(np.unique(idx.cpu().numpy().reshape(T, 8)[:, :k])))
        return float(np.mean(us))

    def decode(lx, T, name, expert_bytes=EXPERT_BYTES):
        # 64 different token batches per step
        ntok = 64
        xs = d(synth.activations((ntok, T, H), rng))
        rs = d(synth.activations((ntok, T, H), rng))
        out = torch.empty((T, H), dtype=torch.float32, device="cuda")
        ws_t = torch.zeros(tb.moe_workspace_size(lx[0], T), dtype=torch.uint8, device="cuda")
        U = distinct_experts(lx[0], xs, T)
        nbytes = router_bytes + U * expert_bytes + 3 * T * H * 4
        r = {}
        for temp, ls in (("cold", lx), ("warm", lx[:1])):
            def mstep():
                for i in range(ntok):
                    tb.moe_forward(ls[i % len(ls)], T, xs[i], rs[i], out, workspace=ws_t)
            reps = 20
            sec = time_region(mstep, reps, 2, stream) / (reps * ntok)
            r[temp] = dict(us_per_layer=round(sec * 1e6, 2), us_per_token=round(sec * 1e6 / T, 3),
                           roofline=hbm_roofline(nbytes, sec))
        moe[name] = dict(us_per_layer=r["cold"]["us_per_layer"], us_per_token=r["cold"]["us_per_token"],
                         distinct_experts=U, algorithmic_bytes=int(nbytes), layer_copies=len(lx), **r)
        log(f"MoE {name}: cold {r['cold']['us_per_layer']:.1f} us/layer ({r['cold']['roofline']['frac']:.1%} of "
            f"HBM, U={U:.1f}), warm {r['warm']['us_per_layer']:.1f} us/layer")
    for T in (1, 16):
        decode(layers, T, f"decode_b{T}")
    # the same expert bytes read in ggml's Q4_K layout
    lg = [tb.moe_layer(H, F, E, k, fm.GGML | fm.Q4_K, *c) for c in keep]
    decode(lg, 1, "decode_b1_ggml_q4k")
    del lg
    # a K-quant mix as llama.cpp writes it: Q4_K gate/up, Q6_K down (each
    # expert tensor in its own qtype)
    _, _, _, down6 = synth.moe_layer(H, F, E, fm.Q4_K, seed=3, qt_down=fm.Q6_K)
    d6 = d(down6)
    lm = [tb.moe_layer(H, F, E, k, fm.Q4_K, c[0], c[1], c[2], d6 if i == 0 else d6.clone(), qt_down=fm.Q6_K)
          for i, c in enumerate(keep)]
    mixed_bytes = 2 * fm.weight_bytes(fm.Q4_K, F, H) + fm.weight_bytes(fm.Q6_K, H, F)
    for T in (1, 16):
        decode(lm, T, f"decode_b{T}_q4k_q6k_down", mixed_bytes)
    del lm, d6
    # prefill, Zipf-skewed routing, grouped MFMA experts
    T = 512
    bias = d(synth.zipf_router_bias(E, 1.1, 1.0, rng))
    Lb = tb.moe_layer(H, F, E, k, fm.Q4_K, *keep[0], bias=bias)
    xs = d(synth.activations((T, H), rng))
    rs = d(synth.activations((T, H), rng))
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    U = distinct_experts(Lb, xs[None], T)
    nbytes = router_bytes + U * EXPERT_BYTES + 3 * T * H * 4
    flops = 2.0 * T * k * 3 * H * F + 2.0 * T * E * H
    # the same expert bytes read in ggml's Q4_K layout (fp16 MFMA only)
    Lg = tb.moe_layer(H, F, E, k, fm.GGML | fm.Q4_K, *keep[0], bias=bias)
    for name, mode, peak, Lx in (("prefill_512_fp16_mfma", tb.TBQ_MOE_BF16, MFMA_PEAK_TFLOPS["fp16"], Lb),
                                 ("prefill_512_int8_mfma", tb.TBQ_MOE_I8, MFMA_PEAK_TFLOPS["int8"], Lb),
                                 ("prefill_512_fp16_mfma_ggml_q4k", tb.TBQ_MOE_BF16, MFMA_PEAK_TFLOPS["fp16"], Lg)):
        ws_t = torch.zeros(tb.moe_workspace_size(Lx, T, mode), dtype=torch.uint8, device="cuda")
        sec = time_region(lambda: tb.moe_forward(Lx, T, xs, rs, out, workspace=ws_t, mode=mode), 20, 3,
                          stream) / 20
        tf = flops / sec / 1e12
        moe[name] = dict(us_per_layer=round(sec * 1e6, 2), us_per_token=round(sec * 1e6 / T, 4),
                         distinct_experts=U, algorithmic_bytes=int(nbytes), flops=flops,
                         roofline_hbm=hbm_roofline(nbytes, sec),
                         roofline_mfma=dict(bound="mfma", achieved=round(tf, 1), peak=peak, unit="TFLOP/s",
                                            frac=round(tf / peak, 4)),
                         bound_us=round(max(nbytes / HBM_PEAK_GBS / 1e3, flops / peak / 1e6), 2))
        log(f"MoE {name} T=512: {sec * 1e6:.1f} us/layer; HBM {moe[name]['roofline_hbm']['frac']:.1%}, "
            f"MFMA {tf:.0f} TFLOP/s ({tf / peak:.1%}); bound {moe[name]['bound_us']:.1f} us")
    del keep, layers
    torch.cuda.empty_cache()
    return moe


def _time_cpu(fn, budget_s):
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    return (time.perf_counter() - t0) / n, n


def cpu_leg(budget_s=10.0, row_budget_s=0.8):
    """The reference CPU path on this host, one pinned core: (i) the headline
    workload (whole Q4_K 4096x4096 matvecs) through tb_dispatch_matvec's
    AVX-512 kernels and the scalar tb_gguf_dequant_matvec, on a bounded
    sample; (ii) one row per configs[1] shape through the scalar matvec
    (tb_dispatch_matvec zero-fills Q2_K/Q5_K/Q6_K), plus the AVX dispatch
    for Q3_K and Q8_0; (iii) the MoE block at batch 1 (the reference's MoE
    branch composed of its own functions)."""
    from oracle.pyoracle import Oracle, Reference, host_has_avx512
    from trailblaze_amd import formats as fm
    from trailblaze_amd import synth

    try:
        os.sched_setaffinity(0, {sorted(os.sched_getaffinity(0))[0]})
    except (AttributeError, OSError):
        pass
    rng = np.random.default_rng(0)
    M, K = 4096, 4096
    W = synth.kquant_matrix(fm.Q4_K, M, K, rng)
    x = synth.activations(K, rng)
    b = matvec_bytes(fm.Q4_K, M, K)
    use_ref = Reference.available() and host_has_avx512()
    if use_ref:
        ref = Reference()
        kind = "reference"
        mv, avx = ref.matvec, ref.dispatch_matvec_avx512
        moe_fn = lambda *a, **kw: ref.moe_block(*a, **kw)
        fns = {"tb_dispatch_matvec (AVX-512 class)": lambda: avx(W, fm.Q4_K, M, K, x),
               "tb_gguf_dequant_matvec (scalar)": lambda: mv(W, fm.Q4_K, M, K, x)}
    else:
        orc = Oracle()
        kind = "port"
        mv = orc.matvec
        avx = None
        moe_fn = lambda *a, **kw: orc.moe(*a, **kw)[0]
        fns = {"AVX-512-structured restatement": lambda: orc.matvec_q4k_avx512s(W, M, K, x),
               "scalar restatement": lambda: orc.matvec(W, fm.Q4_K, M, K, x)}
    out = {}
    for name, fn in fns.items():
        dt, n = _time_cpu(fn, budget_s / len(fns))
        out[name] = dict(ms_per_matvec=dt * 1e3, gbs=b / dt / 1e9, reps=n)
        log(f"CPU {name}: {dt * 1e3:.1f} ms/matvec {b / dt / 1e9:.2f} GB/s")
    rows = []
    for qt, M2, K2 in _sweep_shapes():
        W2 = synth.kquant_matrix(qt, M2, K2, rng)
        x2 = synth.activations(K2, rng)
        b2 = matvec_bytes(qt, M2, K2)
        paths = [("scalar", lambda: mv(W2, qt, M2, K2, x2))]
        if avx is not None and qt in (fm.Q3_K, fm.Q8_0):
            paths.append(("avx", lambda: avx(W2, qt, M2, K2, x2)))
        for pname, fn in paths:
            dt, n = _time_cpu(fn, row_budget_s)
            rows.append(dict(qt=fm.NAMES[qt], M=M2, K=K2, path=pname, ms=round(dt * 1e3, 3),
                             gbs=round(b2 / dt / 1e9, 3), reps=n))
            log(f"CPU {fm.NAMES[qt]} {M2}x{K2} {pname}: {dt * 1e3:.1f} ms {b2 / dt / 1e9:.2f} GB/s")
        del W2
    H, F, E, k = 2048, 768, 128, 8
    router, gate, up, down = synth.moe_layer(H, F, E, fm.Q4_K, seed=3)
    xn = synth.activations((1, H), rng)
    rs = synth.activations((1, H), rng)
    dt, n = _time_cpu(lambda: moe_fn(xn, rs, router, gate, up, down, F=F, top_k=k, qtype=fm.Q4_K), 2 * row_budget_s)
    moe = dict(us_per_layer=round(dt * 1e6, 1), reps=n)
    log(f"CPU MoE block b=1: {dt * 1e3:.2f} ms/layer")
    # batches: the reference's MoE branch runs token by token
    # (layer4/tb_infer.c:1068-1075), so b=16 is timed whole and the 512-token
    # prefill on a 32-token sample of the same Zipf-routed batch, scaled
    x16 = synth.activations((16, H), rng)
    r16 = synth.activations((16, H), rng)
    dt16, n16 = _time_cpu(lambda: moe_fn(x16, r16, router, gate, up, down, F=F, top_k=k, qtype=fm.Q4_K),
                          2 * row_budget_s)
    moe_b16 = dict(us_per_layer=round(dt16 * 1e6, 1), us_per_token=round(dt16 * 1e6 / 16, 1), reps=n16)
    log(f"CPU MoE block b=16: {dt16 * 1e3:.2f} ms/layer")
    x32 = synth.activations((32, H), rng)
    r32 = synth.activations((32, H), rng)
    dt32, n32 = _time_cpu(lambda: moe_fn(x32, r32, router, gate, up, down, F=F, top_k=k, qtype=fm.Q4_K),
                          2 * row_budget_s)
    moe_t512 = dict(us_per_layer=round(dt32 * 1e6 * 512 / 32, 1), us_per_token=round(dt32 * 1e6 / 32, 1),
                    reps=n32, sample="32 of the 512 tokens (token by token, as the reference), scaled x16")
    log(f"CPU MoE block T=512 (32-token sample): {dt32 * 512 / 32 * 1e3:.1f} ms/layer")
    del router, gate, up, down
    # dense Qwen3-4B decode step, the reference's CPU matvecs
    # (tb_gguf_tensor_matvec -> tb_dispatch_matvec, layer4/tb_gguf.c:453-461):
    # one layer's Q4_K matrices timed, x 36 layers, plus the Q6_K lm_head
    # through the scalar matvec (the dispatch zero-fills Q6_K)
    from trailblaze_amd.dense import QWEN3_4B as c
    QR = (c.n_heads + 2 * c.n_kv_heads) * c.head_dim
    lay = [(QR, c.hidden), (c.hidden, c.n_heads * c.head_dim), (2 * c.ffn, c.hidden), (c.hidden, c.ffn)]
    mats = [(synth.kquant_matrix(fm.Q4_K, M3, K3, rng), M3, K3, synth.activations(K3, rng)) for M3, K3 in lay]
    layer_mv = avx if avx is not None else (lambda W3, q3, M3, K3, x3: mv(W3, q3, M3, K3, x3))
    dtl, nl = _time_cpu(lambda: [layer_mv(W3, fm.Q4_K, M3, K3, x3) for W3, M3, K3, x3 in mats], 2 * row_budget_s)
    del mats
    lm = synth.kquant_matrix(fm.Q6_K, c.vocab, c.hidden, rng)
    xl = synth.activations(c.hidden, rng)
    t0 = time.perf_counter()
    mv(lm, fm.Q6_K, c.vocab, c.hidden, xl)
    dt_lm = time.perf_counter() - t0
    del lm
    dense = dict(us_per_token=round((dtl * c.n_layers + dt_lm) * 1e6, 0), layer_ms=round(dtl * 1e3, 2),
                 lm_head_ms=round(dt_lm * 1e3, 1), reps=nl,
                 sample="one layer's Q4_K matvecs (qkv, o, gate|up, down) x 36 + the Q6_K lm_head, matvecs only")
    log(f"CPU dense Qwen3-4B step (matvecs): {dense['us_per_token'] / 1e3:.0f} ms/token")
    best = max(out, key=lambda k: out[k]["gbs"])
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return dict(value=out[best]["gbs"], unit="GB/s", cores=1, kind=kind,
                sample=f"{out[best]['reps']} whole Q4_K 4096x4096 matvecs via {best}, 1 pinned thread "
                       f"({cpu_model}, nproc={os.cpu_count()})",
                detail=out, rows=rows, moe_b1=moe, moe_b16=moe_b16, moe_t512=moe_t512, dense=dense)


def _proc_children(pid):
    """Descendants of pid from /proc (pid, command line), for hosts without
    psutil."""
    kids, parent = [], {}
    for d in os.listdir("/proc"):
        if not d.isdigit():
            continue
        try:
            with open(f"/proc/{d}/stat") as f:
                st = f.read()
            parent[int(d)] = int(st[st.rindex(")") + 2:].split()[1])
        except (OSError, ValueError, IndexError):
            pass
    todo = [pid]
    while todo:
        p = todo.pop()
        for c, pp in parent.items():
            if pp == p:
                try:
                    with open(f"/proc/{c}/cmdline", "rb") as f:
                        cmd = f.read().replace(b"\0", b" ").decode(errors="replace")[:120]
                except OSError:
                    cmd = "?"
                kids.append((c, cmd))
                todo.append(c)
    return kids


def _reap_children():
    """Wait for any child process of this one (the bench starts none itself;
    a library may) and name it on stderr, so the run ends with nothing left."""
    try:
        import psutil
    except ImportError:
        import signal
        kids = _proc_children(os.getpid())
        for pid, cmd in kids:
            log(f"child process left at exit: pid {pid} {cmd}")
            try:
                os.kill(pid, signal.SIGTERM)
            except OSError:
                pass
        log(f"child processes at exit: {len(kids)}")
        return
    kids = psutil.Process().children(recursive=True)
    for c in kids:
        try:
            log(f"child process left at exit: pid {c.pid} {c.name()} {' '.join(c.cmdline()[:4])}")
            c.terminate()
        except psutil.Error:
            pass
    psutil.wait_procs(kids, timeout=5)
    log(f"child processes at exit: {len(kids)}")


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU only (single-GPU hot path); --gpus must be 1",
              file=sys.stderr)
        sys.exit(2)
    global SWEEP_SHAPES
    SWEEP_SHAPES = _sweep_shapes()
    res = gpu_leg(args)
    if args.profile:
        _reap_children()
        return
    h = res["headline"]
    cpu = None
    if not args.no_cpu and not args.quick:
        cpu = cpu_leg()
    line = {
        "metric": "Q4_K matvec HBM GB/s",
        "value": round(h["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights, fp32 activations and accumulate",
        "data": "synthetic (seeded: fp16 scales U(1e-3,1e-2), uniform bytes, x ~ N(0,1))",
        "config": {"workload": f"Q4_K matvec 4096x4096 (BASELINE configs[0]) over {h['ncopy']} distinct "
                               f"weight copies per step (cold HBM)", "M": 4096, "K": 4096,
                   "copies_per_step": h["ncopy"]},
        "roofline": {"bound": "hbm", "achieved": round(h["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(h["gbs"] / HBM_PEAK_GBS, 4), "traffic": pmc_traffic(),
                     "traffic_source": "read from profiles/q4k_matvec_4096x4096_pmc.txt (rocprofv3 --pmc "
                                       "FETCH_SIZE + WRITE_SIZE per dispatch, copy-calibrated), not measured in "
                                       "this run",
                     "kernel": "k_mv_q4k_xr (Q4_K int-dot)", "us_per_launch": round(h["us_per_launch"], 3),
                     "bytes_per_launch": h["bytes_per_launch"]},
        "cpu_baseline": None if cpu is None else {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample")},
        "extra": {"device": res["device"], "warm_mall_gbs": round(h["warm_gbs"], 1),
                  "warm_us_per_launch": round(h["warm_us_per_launch"], 3),
                  "abi_matvec_us": None if res.get("abi_matvec_us") is None else round(res["abi_matvec_us"], 2),
                  "hbm_ceiling": res.get("hbm_ceiling"), "q4k_steady": res.get("q4k_steady"),
                  "sweep": res.get("sweep"), "ggml_sweep": res.get("ggml_sweep"), "moe": res.get("moe"),
                  "dense": res.get("dense"),
                  "cpu_detail": None if cpu is None else cpu["detail"],
                  "cpu_rows": None if cpu is None else cpu_rows_vs_gpu(cpu, res)},
    }
    print(json.dumps(line), flush=True)
    _reap_children()


def cpu_rows_vs_gpu(cpu, res):
    """The CPU rows with the GPU time of the same workload beside them."""
    gpu = {(r["qt"], r["M"], r["K"]): r["us"] for r in (res.get("sweep") or [])}
    rows = []
    for r in cpu["rows"]:
        g = gpu.get((r["qt"], r["M"], r["K"]))
        rows.append(dict(r, gpu_us=None if g is None else round(g, 2),
                         gpu_speedup=None if g is None else round(r["ms"] * 1e3 / g, 1)))
    def beside(row, gpu_us):
        r = dict(row, gpu_us=None if gpu_us is None else round(gpu_us, 2))
        if gpu_us:
            r["gpu_speedup"] = round(row["us_per_layer" if "us_per_layer" in row else "us_per_token"] / gpu_us, 1)
        return r
    moe_res = res.get("moe") or {}
    g = lambda name: (moe_res.get(name) or {}).get("us_per_layer")
    dense_gpu = (res.get("dense") or {}).get("us_per_token")
    return dict(matvec=rows, moe_b1=beside(cpu["moe_b1"], g("decode_b1")),
                moe_b16=beside(cpu["moe_b16"], g("decode_b16")),
                moe_t512=beside(cpu["moe_t512"], g("prefill_512_fp16_mfma")),
                dense_step=beside(cpu["dense"], dense_gpu), cores=1, kind=cpu["kind"])


if __name__ == "__main__":
    main()
