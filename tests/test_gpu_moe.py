"""GPU parity for the MoE block through the C-ABI: router indices and slot
order bit-exact against tb_route_experts semantics, MoE outputs within
rel-L2 1e-5 of the oracle on the output and on the MoE delta (out - resid),
at the reference's golden layer, at the Qwen3-30B-A3B shapes of
BASELINE.json (batch 1 and 16), with a Zipf-skewed router bias, on tied, nearly tied and
underflowing logits, and through the C11 host block."""
import ctypes as C

import numpy as np
import pytest

import trailblaze_amd as tb
from conftest import bits_equal, load_golden, rel_l2
from gpu_util import dev, empty, host
from trailblaze_amd import formats as fm
from trailblaze_amd import synth

pytestmark = pytest.mark.gpu
TOL = 1e-5
COUNTER_BYTES = 256 * 1024   # counter area at the start of the MoE workspace


@pytest.fixture(scope="module", autouse=True)
def _init():
    print("device:", tb.init(), flush=True)


def gpu_route(xn, router, bias, k):
    import torch
    T, H = xn.shape
    E = router.shape[0]
    idx = empty(T * 8, torch.int32)
    w = empty(T * 8, torch.float32)
    tb.route(dev(xn), dev(router), None if bias is None else dev(bias), T, H, E, k, idx, w)
    return host(idx).reshape(T, 8), host(w).reshape(T, 8)


def gpu_moe(xn, resid, router, gate, up, down, F, k, qt, bias=None, mode=tb.TBQ_MOE_FP32):
    import torch
    T, H = xn.shape
    E = router.shape[0]
    L = tb.moe_layer(H, F, E, k, qt, dev(router), dev(gate), dev(up), dev(down),
                     None if bias is None else dev(bias))
    out = empty(T * H, torch.float32)
    idx = empty(T * 8, torch.int32)
    w = empty(T * 8, torch.float32)
    ws = torch.zeros(tb.moe_workspace_size(L, T, mode), dtype=torch.uint8, device="cuda")
    tb.moe_forward(L, T, dev(xn), dev(resid), out, idx, w, workspace=ws, mode=mode)
    assert_counters_zero(ws)
    return host(out).reshape(T, H), host(idx).reshape(T, 8), host(w).reshape(T, 8)


def assert_counters_zero(ws):
    """The workspace's counter words (the router's per-token arrival
    counters) are zero after every call."""
    c = host(ws[:COUNTER_BYTES])
    assert not c.any(), np.flatnonzero(c.view(np.uint32))[:8]


def test_route_golden_logit_vectors(oracle):
    # identity router: logits = xn exactly, so the reference's own routing
    # vectors (route.npz) drive the device softmax/top-k directly
    g = load_golden("route.npz")
    off_l = off_s = 0
    for E, k in zip(g["E"], g["k"]):
        lg = g["logits"][off_l:off_l + E]
        Hp = ((E + 7) // 8) * 8
        xn = np.zeros((1, Hp), np.float32)
        xn[0, :E] = lg
        router = np.zeros((E, Hp), np.float32)
        router[np.arange(E), np.arange(E)] = 1.0
        kk = min(int(k), 8)
        idx, w = gpu_route(xn, router, None, int(k))
        ref_i, ref_w = g["idx"][off_s:off_s + kk], g["w"][off_s:off_s + kk]
        assert np.array_equal(idx[0, :kk], ref_i), (E, k, lg)
        assert bits_equal(w[0, :kk], ref_w)
        off_l += E
        off_s += kk


def tie_case_logits(case):
    """64 logits that exercise the slot scan's tie rule (first slot holding
    the minimum; strictly larger enters) or underflowing probabilities."""
    rng = np.random.default_rng(7)
    E = 64
    lg = rng.standard_normal(E).astype(np.float32)
    if case == "tie4":
        lg[:8] = 1.0          # the fill leaves equal minima; the next entry picks among them
        lg[20] = 3.0
    elif case == "tie_boundary":
        lg[:] = np.float32(-2.0)
        lg[::5] = np.float32(1.5)  # 13 equal leaders for 8 slots
    elif case == "near_tie":
        top = np.argsort(-lg)
        lg[top[8]] = np.nextafter(lg[top[7]], np.float32(-np.inf))   # 8th and 9th one ulp apart
    else:
        lg[:] = np.float32(-200.0)  # probabilities of the tail underflow to zero
        lg[3] = 0.0
        lg[40] = np.float32(-199.0)
    return lg


@pytest.mark.parametrize("case", ["tie4", "tie_boundary", "near_tie", "underflow"])
def test_route_ties_and_underflow(oracle, case):
    """The slot scan's tie rule and probabilities that underflow to zero."""
    lg = tie_case_logits(case)
    E, k = lg.size, 8
    H = 512
    xn = np.zeros((1, H), np.float32)
    xn[0, :E] = lg
    router = np.zeros((E, H), np.float32)
    router[np.arange(E), np.arange(E)] = 1.0
    idx, w = gpu_route(xn, router, None, k)
    ri, rw = oracle.route(lg, k)
    assert np.array_equal(idx[0], ri)
    assert bits_equal(w[0], rw)


@pytest.mark.parametrize("T", [1, 16, 512])
def test_route_config_bit_exact(oracle, T):
    rng = np.random.default_rng(T)
    H, E, k = 2048, 128, 8
    router = synth.router_weights(E, H, rng)
    xn = synth.activations((T, H), rng)
    bias = synth.zipf_router_bias(E, 1.1, 1.0, rng) if T == 512 else None
    idx, w = gpu_route(xn, router, bias, k)
    lg = oracle.router_logits(xn, router, bias)
    for t in range(T):
        ri, rw = oracle.route(lg[t], k)
        assert np.array_equal(idx[t], ri), t
        assert bits_equal(w[t], rw), t


def test_moe_golden_layer():
    g = load_golden("moe.npz")
    out, idx, w = gpu_moe(g["xn"], g["resid"], g["router"], g["gate"], g["up"], g["down"], int(g["F"]),
                          int(g["k"]), int(g["qtype"]), bias=g["bias"])
    k = int(g["k"])
    assert np.array_equal(idx[:, :k], g["idx"][:, :k])
    assert bits_equal(w[:, :k], g["w"][:, :k])
    assert rel_l2(out, g["out"]) <= TOL
    assert rel_l2(out - g["resid"], g["out"] - g["resid"]) <= TOL


@pytest.fixture(scope="module")
def qwen_layer():
    H, F, E = 2048, 768, 128
    router, gate, up, down = synth.moe_layer(H, F, E, fm.Q4_K, seed=30)
    return H, F, E, router, gate, up, down


@pytest.mark.parametrize("T", [1, 16])
def test_moe_decode_config(oracle, qwen_layer, T):
    H, F, E, router, gate, up, down = qwen_layer
    rng = np.random.default_rng(100 + T)
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    print("moe decode T=", T, flush=True)
    out, idx, w = gpu_moe(xn, resid, router, gate, up, down, F, 8, fm.Q4_K)
    ref, ridx, rw = oracle.moe(xn, resid, router, gate, up, down, F=F, top_k=8, qtype=fm.Q4_K)
    assert np.array_equal(idx, ridx)
    assert bits_equal(w, rw)
    assert rel_l2(out, ref) <= TOL
    assert rel_l2(out - resid, ref - resid) <= TOL


@pytest.mark.parametrize("T,H,F,E,k,qt,skew", [
    (8, 2048, 768, 128, 8, fm.Q4_K, False),
    (24, 1024, 512, 64, 6, fm.Q4_K, True),
    (32, 2048, 768, 128, 8, fm.Q4_K, True),
    (12, 4096, 1536, 256, 8, fm.Q4_K, False),
    (16, 2048, 768, 128, 8, fm.GGML | fm.Q4_K, True),
])
def test_moe_decode_expert_order(oracle, T, H, F, E, k, qt, skew):
    """Decode batches of 8..32 tokens run their expert kernels in expert
    order (a sorted pair list, down per pair, slot-ordered combine).  With a
    skewed router bias many tokens share an expert; every index and weight
    equals the reference's and the output is within tolerance."""
    router, gate, up, down = synth.moe_layer(H, F, E, qt, seed=T + E)
    rng = np.random.default_rng(T * 7 + k)
    bias = synth.zipf_router_bias(E, 1.1, 2.0, rng) if skew else None
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    print("moe expert order T=", T, "H=", H, "E=", E, "k=", k, "qt=", qt, flush=True)
    out, idx, w = gpu_moe(xn, resid, router, gate, up, down, F, k, qt, bias=bias)
    ref, ridx, rw = oracle.moe(xn, resid, router, gate, up, down, F=F, top_k=k, qtype=qt, bias=bias)
    assert np.array_equal(idx, ridx)
    assert bits_equal(w, rw)
    if skew:   # the bias concentrates the selections: some expert has several tokens
        assert np.bincount(idx[:, :k].ravel(), minlength=E).max() >= 3
    assert rel_l2(out - resid, ref - resid) <= TOL


def test_moe_decode_router_many_tokens(oracle):
    """Routing inside tbq_moe_forward over 512 decode tokens (32 batches of
    16): every index, slot and weight equal to the reference's."""
    H, F, E, k = 2048, 256, 128, 8
    router, gate, up, down = synth.moe_layer(H, F, E, fm.Q4_K, seed=41)
    import torch
    L = tb.moe_layer(H, F, E, k, fm.Q4_K, dev(router), dev(gate), dev(up), dev(down))
    rng = np.random.default_rng(41)
    T = 16
    ws = torch.zeros(tb.moe_workspace_size(L, T), dtype=torch.uint8, device="cuda")
    out = empty(T * H, torch.float32)
    for b in range(32):
        xn = synth.activations((T, H), rng)
        resid = np.zeros((T, H), np.float32)
        idx = empty(T * 8, torch.int32)
        w = empty(T * 8, torch.float32)
        tb.moe_forward(L, T, dev(xn), dev(resid), out, idx, w, workspace=ws)
        idx, w = host(idx).reshape(T, 8), host(w).reshape(T, 8)
        lg = oracle.router_logits(xn, router, None)
        for t in range(T):
            ri, rw = oracle.route(lg[t], k)
            assert np.array_equal(idx[t], ri), (b, t)
            assert bits_equal(w[t], rw), (b, t)


def test_moe_decode_repeated_calls(oracle):
    """One workspace across calls of different batch sizes (1, 16, 3, 1):
    outputs in tolerance every time and the counter words back at zero
    after each call."""
    import torch
    H, F, E, k = 2048, 256, 128, 8
    router, gate, up, down = synth.moe_layer(H, F, E, fm.Q4_K, seed=52)
    L = tb.moe_layer(H, F, E, k, fm.Q4_K, dev(router), dev(gate), dev(up), dev(down))
    ws = torch.zeros(tb.moe_workspace_size(L, 16), dtype=torch.uint8, device="cuda")
    rng = np.random.default_rng(52)
    for T in (1, 16, 3, 1):
        print("moe repeated call T=", T, flush=True)
        xn = synth.activations((T, H), rng)
        resid = synth.activations((T, H), rng)
        out = empty(T * H, torch.float32)
        idx = empty(T * 8, torch.int32)
        w = empty(T * 8, torch.float32)
        tb.moe_forward(L, T, dev(xn), dev(resid), out, idx, w, workspace=ws)
        ref, ridx, _ = oracle.moe(xn, resid, router, gate, up, down, F=F, top_k=k, qtype=fm.Q4_K)
        assert np.array_equal(host(idx).reshape(T, 8), ridx), T
        assert rel_l2(host(out).reshape(T, H) - resid, ref - resid) <= TOL, T
        assert_counters_zero(ws)


@pytest.mark.parametrize("case", ["tie4", "tie_boundary", "near_tie", "underflow"])
def test_moe_decode_router_ties(oracle, case):
    """Tied, nearly tied and underflowing logits through tbq_moe_forward:
    the reference's indices, slot order and weights bit for bit."""
    lg = tie_case_logits(case)
    E, k, H, F = lg.size, 8, 512, 256
    router = np.zeros((E, H), np.float32)
    router[np.arange(E), np.arange(E)] = 1.0
    _, gate, up, down = synth.moe_layer(H, F, E, fm.Q4_K, seed=13)
    xn = np.zeros((1, H), np.float32)
    xn[0, :E] = lg
    resid = synth.activations((1, H), np.random.default_rng(13))
    out, idx, w = gpu_moe(xn, resid, router, gate, up, down, F, k, fm.Q4_K)
    ref, ridx, rw = oracle.moe(xn, resid, router, gate, up, down, F=F, top_k=k, qtype=fm.Q4_K)
    assert np.array_equal(idx, ridx)
    assert bits_equal(w, rw)
    assert rel_l2(out - resid, ref - resid) <= TOL


@pytest.mark.parametrize("qt", [fm.Q2_K, fm.Q3_K, fm.Q5_K, fm.Q6_K, fm.Q8_0])
def test_moe_other_formats(oracle, qt):
    H, F, E, k, T = 512, 256, 16, 4, 3
    router, gate, up, down = synth.moe_layer(H, F, E, qt, seed=qt)
    rng = np.random.default_rng(qt)
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    out, idx, w = gpu_moe(xn, resid, router, gate, up, down, F, k, qt)
    ref, ridx, rw = oracle.moe(xn, resid, router, gate, up, down, F=F, top_k=k, qtype=qt)
    assert np.array_equal(idx, ridx)
    assert rel_l2(out - resid, ref - resid) <= TOL


def test_moe_host_block(oracle):
    """The C11 host substitution for tb_layer_forward's MoE branch."""
    g = load_golden("moe.npz")
    H, F, E, k = int(g["H"]), int(g["F"]), int(g["E"]), int(g["k"])
    T = g["xn"].shape[0]
    tensors = [dev(g[n]) for n in ("router", "gate", "up", "down", "bias")]
    L = tb.moe_layer(H, F, E, k, int(g["qtype"]), *tensors[:4], bias=tensors[4])
    import torch
    torch.cuda.synchronize()
    out = np.zeros((T, H), np.float32)
    idx = np.zeros((T, 8), np.int32)
    w = np.zeros((T, 8), np.float32)
    ok = tb.lib().tbq_moe_block_host(C.byref(L), T, g["xn"].ctypes.data, g["resid"].ctypes.data,
                                     out.ctypes.data, idx.ctypes.data, w.ctypes.data, tb.TBQ_MOE_FP32)
    assert ok == 1, tb.lib().tbq_last_error()
    assert np.array_equal(idx[:, :k], g["idx"][:, :k])
    assert rel_l2(out, g["out"]) <= TOL


@pytest.mark.parametrize("H", [512, 2048])
def test_moe_host_block_varying_batches(oracle, H):
    """tbq_moe_block_host over a sequence of calls whose T and mode change,
    so its cached buffer is reused at a smaller T and regrown at a larger
    one: every call routes exactly and stays within tolerance.  H = 512 and
    2048 take the router whose per-token arrival counters live in the
    workspace (T < 32), the path a misplaced or unzeroed counter area
    breaks."""
    F, E, k = 256, 16, 4
    router, gate, up, down = synth.moe_layer(H, F, E, fm.Q4_K, seed=H + 7)
    L = tb.moe_layer(H, F, E, k, fm.Q4_K, dev(router), dev(gate), dev(up), dev(down))
    import torch
    torch.cuda.synchronize()
    for i, (T, mode) in enumerate([(5, tb.TBQ_MOE_FP32), (1, tb.TBQ_MOE_FP32), (16, tb.TBQ_MOE_FP32),
                                   (1, tb.TBQ_MOE_FP32), (40, tb.TBQ_MOE_BF16), (1, tb.TBQ_MOE_FP32),
                                   (3, tb.TBQ_MOE_BF16), (2, tb.TBQ_MOE_FP32), (24, tb.TBQ_MOE_I8),
                                   (1, tb.TBQ_MOE_FP32)]):
        print(f"host block H={H} call {i}: T={T} mode={mode}", flush=True)
        rng = np.random.default_rng(1000 * H + i)
        xn = synth.activations((T, H), rng)
        resid = synth.activations((T, H), rng)
        out = np.zeros((T, H), np.float32)
        idx = np.full((T, 8), 77, np.int32)
        w = np.zeros((T, 8), np.float32)
        ok = tb.lib().tbq_moe_block_host(C.byref(L), T, xn.ctypes.data, resid.ctypes.data, out.ctypes.data,
                                         idx.ctypes.data, w.ctypes.data, mode)
        assert ok == 1, tb.lib().tbq_last_error()
        ref, ridx, rw = oracle.moe(xn, resid, router, gate, up, down, F=F, top_k=k, qtype=fm.Q4_K)
        assert np.array_equal(idx, ridx), (T, mode)
        assert bits_equal(w, rw), (T, mode)
        tol = TOL if mode == tb.TBQ_MOE_FP32 else 1e-2
        assert rel_l2(out - resid, ref - resid) <= tol, (T, mode)


# ---------------------------------------------------------------------------
# Prefill: grouped fp16 MFMA experts (tolerance 1e-2 rel-L2, routing exact)
# ---------------------------------------------------------------------------
PREFILL_TOL = 1e-2


def test_moe_prefill_mfma_golden_layer():
    g = load_golden("moe.npz")
    out, idx, w = gpu_moe(g["xn"], g["resid"], g["router"], g["gate"], g["up"], g["down"], int(g["F"]),
                          int(g["k"]), int(g["qtype"]), bias=g["bias"], mode=tb.TBQ_MOE_BF16)
    k = int(g["k"])
    assert np.array_equal(idx[:, :k], g["idx"][:, :k])
    assert rel_l2(out - g["resid"], g["out"] - g["resid"]) <= PREFILL_TOL


def test_moe_prefill_mfma_config(oracle, qwen_layer):
    """512 tokens, Zipf(1.1)-skewed router bias."""
    H, F, E, router, gate, up, down = qwen_layer
    T = 512
    rng = np.random.default_rng(512)
    bias = synth.zipf_router_bias(E, 1.1, 1.0, rng)
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    out, idx, w = gpu_moe(xn, resid, router, gate, up, down, F, 8, fm.Q4_K, bias=bias, mode=tb.TBQ_MOE_BF16)
    # routing: every token bit-exact
    lg = oracle.router_logits(xn, router, bias)
    for t in range(T):
        ri, rw = oracle.route(lg[t], 8)
        assert np.array_equal(idx[t], ri), t
        assert bits_equal(w[t], rw), t
    counts = np.bincount(idx.reshape(-1), minlength=E)
    assert counts.max() > 4 * counts.mean()      # the bias really skews the load
    # outputs: tokens are independent, so a sample checks the whole layer
    sample = np.sort(rng.choice(T, 32, replace=False))
    ref, _, _ = oracle.moe(xn[sample], resid[sample], router, gate, up, down, F=F, top_k=8, qtype=fm.Q4_K, bias=bias)
    assert rel_l2(out[sample] - resid[sample], ref - resid[sample]) <= PREFILL_TOL
    assert rel_l2(out[sample], ref) <= PREFILL_TOL


def test_moe_prefill_mfma_small_batches(oracle):
    """Tiles with 1..64 pairs, experts with zero tokens, several tiles per expert."""
    H, F, E, k = 512, 256, 8, 4
    router, gate, up, down = synth.moe_layer(H, F, E, fm.Q4_K, seed=91)
    for T in (1, 3, 17, 70):
        rng = np.random.default_rng(T)
        xn = synth.activations((T, H), rng)
        resid = synth.activations((T, H), rng)
        out, idx, w = gpu_moe(xn, resid, router, gate, up, down, F, k, fm.Q4_K, mode=tb.TBQ_MOE_BF16)
        ref, ridx, rw = oracle.moe(xn, resid, router, gate, up, down, F=F, top_k=k, qtype=fm.Q4_K)
        assert np.array_equal(idx, ridx)
        assert rel_l2(out - resid, ref - resid) <= PREFILL_TOL


@pytest.mark.parametrize("mode", ["BF16", "I8"])
def test_moe_prefill_many_pairs(oracle, mode):
    """More (token, slot) pairs than the dispatch keeps in LDS (8400 > 8192):
    the permutation goes through global memory.  Routing exact for every
    token; outputs checked on a sample (tokens are independent)."""
    H, F, E, k, T = 512, 256, 8, 4, 2100
    router, gate, up, down = synth.moe_layer(H, F, E, fm.Q4_K, seed=93)
    rng = np.random.default_rng(94)
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    out, idx, w = gpu_moe(xn, resid, router, gate, up, down, F, k, fm.Q4_K, mode=getattr(tb, "TBQ_MOE_" + mode))
    sample = np.sort(rng.choice(T, 48, replace=False))
    ref, ridx, rw = oracle.moe(xn[sample], resid[sample], router, gate, up, down, F=F, top_k=k, qtype=fm.Q4_K)
    assert np.array_equal(idx[sample], ridx)
    assert rel_l2(out[sample] - resid[sample], ref - resid[sample]) <= PREFILL_TOL


# ---------------------------------------------------------------------------
# Prefill on int8 MFMA with Q8_K activations (TBQ_MOE_I8): routing exact,
# outputs within 1e-2 rel-L2 (8-bit activations)
# ---------------------------------------------------------------------------
def test_quantize_q8k_device_matches_oracle(oracle):
    """tbq_quantize_q8k writes the Q8_K blocks the pinned oracle quantiser
    writes (d, every int8 quant, every 16-element sum), byte for byte, on
    N(0,1) blocks, tiny and huge scales, 1000x outliers, an all-zero block,
    a constant block and exact rounding ties."""
    import torch
    rng = np.random.default_rng(81)
    parts = [rng.standard_normal(4096).astype(np.float32),
             (rng.standard_normal(512) * 1e-30).astype(np.float32),
             (rng.standard_normal(512) * 1e30).astype(np.float32),
             np.zeros(256, np.float32), np.full(256, -3.25, np.float32)]
    o = rng.standard_normal(1024).astype(np.float32)
    o[rng.choice(1024, 9, replace=False)] *= 1000.0
    ties = np.zeros(256, np.float32)
    ties[0], ties[1], ties[2] = 127.0, 2.5, -3.5
    x = np.concatenate(parts + [o, ties])
    blocks = empty(x.size // 256 * 292, torch.uint8)
    assert tb.lib().tbq_quantize_q8k(dev(x).data_ptr(), x.size, blocks.data_ptr(), None) == 1
    got = host(blocks)
    want = oracle.quantize_q8k(x)
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:10]


def test_moe_prefill_i8_config(oracle, qwen_layer):
    """BASELINE configs[4] on the int8 path: 512 tokens, Zipf(1.1)-skewed
    router bias."""
    H, F, E, router, gate, up, down = qwen_layer
    T = 512
    rng = np.random.default_rng(512)
    bias = synth.zipf_router_bias(E, 1.1, 1.0, rng)
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    out, idx, w = gpu_moe(xn, resid, router, gate, up, down, F, 8, fm.Q4_K, bias=bias, mode=tb.TBQ_MOE_I8)
    lg = oracle.router_logits(xn, router, bias)
    for t in range(T):
        ri, rw = oracle.route(lg[t], 8)
        assert np.array_equal(idx[t], ri), t
        assert bits_equal(w[t], rw), t
    sample = np.sort(rng.choice(T, 32, replace=False))
    ref, _, _ = oracle.moe(xn[sample], resid[sample], router, gate, up, down, F=F, top_k=8, qtype=fm.Q4_K, bias=bias)
    e = rel_l2(out[sample] - resid[sample], ref - resid[sample])
    print("int8 prefill delta rel-L2", e, flush=True)
    assert e <= PREFILL_TOL
    assert rel_l2(out[sample], ref) <= PREFILL_TOL


@pytest.mark.parametrize("H,F,E,k", [(512, 256, 8, 4), (2048, 768, 16, 8), (1024, 512, 6, 2)])
def test_moe_prefill_i8_small_batches(oracle, H, F, E, k):
    """Tiles of 1..70 pairs (one and two 64-pair halves), experts with no
    tokens, several tiles per expert, K of 2..16 chunks."""
    router, gate, up, down = synth.moe_layer(H, F, E, fm.Q4_K, seed=H + E)
    for T in (1, 3, 17, 70):
        print(f"int8 prefill H={H} F={F} E={E} k={k} T={T}", flush=True)
        rng = np.random.default_rng(T + H)
        xn = synth.activations((T, H), rng)
        resid = synth.activations((T, H), rng)
        out, idx, w = gpu_moe(xn, resid, router, gate, up, down, F, k, fm.Q4_K, mode=tb.TBQ_MOE_I8)
        ref, ridx, rw = oracle.moe(xn, resid, router, gate, up, down, F=F, top_k=k, qtype=fm.Q4_K)
        assert np.array_equal(idx, ridx)
        assert rel_l2(out - resid, ref - resid) <= PREFILL_TOL
