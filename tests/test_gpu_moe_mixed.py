"""GPU parity for MoE layers whose expert tensors differ in qtype, as
llama.cpp's K-quant mixes write them (e.g. Q4_K gate/up with a Q6_K down)
and as the reference's MoE branch reads them: each tensor in its own qtype
and row stride (layer4/tb_infer.c:807-816).  Routing is bit-exact and the
outputs are within rel-L2 1e-5 of the oracle (tbo_moe_forward with one
qtype per tensor, pinned against the compiled reference in
tests/test_oracle.py), at the Qwen3-30B-A3B shape at batch 1 and 16, for a
down tensor with smaller and with larger blocks than gate's, for gate and up
in different qtypes, in ggml's layouts, and through the C11 host block,
whose prefill modes fall back to the fp32 kernels for such layers."""
import ctypes as C

import numpy as np
import pytest

import trailblaze_amd as tb
from conftest import bits_equal, rel_l2
from gpu_util import dev, empty, host
from trailblaze_amd import formats as fm
from trailblaze_amd import synth

pytestmark = pytest.mark.gpu
TOL = 1e-5
COUNTER_BYTES = 256 * 1024


@pytest.fixture(scope="module", autouse=True)
def _init():
    print("device:", tb.init(), flush=True)


def gpu_moe(xn, resid, layer, F, k, qts, bias=None, mode=tb.TBQ_MOE_FP32):
    import torch
    router, gate, up, down = layer
    T, H = xn.shape
    E = router.shape[0]
    qg, qu, qd = qts
    L = tb.moe_layer(H, F, E, k, qg, dev(router), dev(gate), dev(up), dev(down),
                     None if bias is None else dev(bias), qt_gate=qg, qt_up=qu, qt_down=qd)
    out = empty(T * H, torch.float32)
    idx = empty(T * 8, torch.int32)
    w = empty(T * 8, torch.float32)
    ws = torch.zeros(tb.moe_workspace_size(L, T, mode), dtype=torch.uint8, device="cuda")
    tb.moe_forward(L, T, dev(xn), dev(resid), out, idx, w, workspace=ws, mode=mode)
    assert not host(ws[:COUNTER_BYTES]).any()
    return host(out).reshape(T, H), host(idx).reshape(T, 8), host(w).reshape(T, 8)


def check(oracle, xn, resid, layer, F, k, qts, bias=None):
    qg, qu, qd = qts
    out, idx, w = gpu_moe(xn, resid, layer, F, k, qts, bias=bias)
    ref, ridx, rw = oracle.moe(xn, resid, *layer, F=F, top_k=k, qtype=qg, qt_up=qu, qt_down=qd, bias=bias)
    assert np.array_equal(idx, ridx)
    assert bits_equal(w, rw)
    assert rel_l2(out, ref) <= TOL
    assert rel_l2(out - resid, ref - resid) <= TOL
    return out, ref


@pytest.fixture(scope="module")
def qwen_q4_q6():
    """Qwen3-30B-A3B MoE shape, Q4_K gate/up and Q6_K down."""
    H, F, E = 2048, 768, 128
    return H, F, E, synth.moe_layer(H, F, E, fm.Q4_K, seed=606, qt_down=fm.Q6_K)


@pytest.mark.parametrize("T", [1, 16])
def test_moe_mixed_qwen_q4k_q6k_down(oracle, qwen_q4_q6, T):
    H, F, E, layer = qwen_q4_q6
    rng = np.random.default_rng(600 + T)
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    print("moe mixed Q4_K/Q4_K/Q6_K T=", T, flush=True)
    check(oracle, xn, resid, layer, F, 8, (fm.Q4_K, fm.Q4_K, fm.Q6_K))


@pytest.mark.parametrize("T", [1, 16])
@pytest.mark.parametrize("qts", [(fm.Q3_K, fm.Q3_K, fm.Q4_K), (fm.Q6_K, fm.Q6_K, fm.Q4_K),
                                 (fm.Q4_K, fm.Q5_K, fm.Q6_K), (fm.Q5_K, fm.Q4_K, fm.Q8_0),
                                 (fm.Q2_K, fm.Q3_K, fm.Q2_K)])
def test_moe_mixed_formats(oracle, qts, T):
    """down with smaller (Q3_K gate, Q4_K down) and larger (Q6_K gate, Q4_K
    down) blocks than gate's; gate and up in different qtypes (run one at a
    time, then SwiGLU); with a skewed router so the batch shares experts."""
    H, F, E, k = 2048, 768, 64, 8
    layer = synth.moe_layer(H, F, E, qts[0], seed=sum(qts) + T, qt_up=qts[1], qt_down=qts[2])
    rng = np.random.default_rng(sum(qts) * 3 + T)
    bias = synth.zipf_router_bias(E, 1.1, 2.0, rng)
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    print("moe mixed", qts, "T=", T, flush=True)
    check(oracle, xn, resid, layer, F, k, qts, bias=bias)


@pytest.mark.parametrize("F", [2048, 4096])
@pytest.mark.parametrize("qts", [(fm.Q4_K, fm.Q4_K, fm.Q6_K), (fm.Q5_K, fm.Q5_K, fm.Q3_K)])
def test_moe_mixed_wide_expert_rows(oracle, qts, F):
    """Down rows of 32 and 64 units (F = 2048, 4096) in a batch in expert
    order: the per-pair down kernel holds two or four units per lane and
    streams its passes' weights in batches (one or two passes at a time)."""
    H, E, k, T = 256, 16, 4, 16
    layer = synth.moe_layer(H, F, E, qts[0], seed=F + sum(qts), qt_up=qts[1], qt_down=qts[2])
    rng = np.random.default_rng(F + 7 * sum(qts))
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    print("moe wide rows", qts, "F=", F, flush=True)
    check(oracle, xn, resid, layer, F, k, qts)


@pytest.mark.parametrize("T", [1, 16])
def test_moe_mixed_ggml(oracle, T):
    """ggml's layouts: Q4_K gate/up with a Q6_K down, as llama.cpp writes."""
    H, F, E, k = 2048, 768, 64, 8
    qts = (fm.GGML | fm.Q4_K, fm.GGML | fm.Q4_K, fm.GGML | fm.Q6_K)
    layer = synth.moe_layer(H, F, E, qts[0], seed=31 + T, qt_down=qts[2])
    rng = np.random.default_rng(32 + T)
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    print("moe mixed ggml T=", T, flush=True)
    check(oracle, xn, resid, layer, F, k, qts)


def test_moe_mixed_refused_by_prefill_modes(qwen_q4_q6):
    """The MFMA prefill modes decode Q4_K for all three tensors: they refuse a
    mixed layer with a message instead of misreading it."""
    H, F, E, (router, gate, up, down) = qwen_q4_q6
    L = tb.moe_layer(H, F, E, 8, fm.Q4_K, dev(router), dev(gate), dev(up), dev(down), qt_down=fm.Q6_K)
    assert tb.moe_mode_supported(L, tb.TBQ_MOE_FP32)
    for mode in (tb.TBQ_MOE_BF16, tb.TBQ_MOE_I8):
        assert not tb.moe_mode_supported(L, mode)
        import torch
        T = 4
        x = torch.zeros(T * H, dtype=torch.float32, device="cuda")
        out = torch.empty_like(x)
        with pytest.raises(tb.TbqError, match="Q4_K"):
            tb.moe_forward(L, T, x, x, out, mode=mode)
    L2 = tb.moe_layer(H, F, E, 8, fm.Q4_K, dev(router), dev(gate), dev(up), dev(gate))
    assert tb.moe_mode_supported(L2, tb.TBQ_MOE_BF16)
    L3 = tb.moe_layer(H, F, E, 8, fm.Q4_K, dev(router), dev(gate), dev(up), dev(down), qt_down=fm.Q4_0)
    assert not tb.moe_mode_supported(L3, tb.TBQ_MOE_FP32)


@pytest.mark.parametrize("mode", [tb.TBQ_MOE_FP32, tb.TBQ_MOE_BF16])
def test_moe_mixed_host_block(oracle, qwen_q4_q6, mode):
    """tbq_moe_block_host (the substitution for the reference's MoE branch)
    on a Q4_K/Q6_K layer: a prefill mode runs the layer on the fp32 kernels,
    so the result is the decode path's, within 1e-5 of the oracle."""
    H, F, E, layer = qwen_q4_q6
    router, gate, up, down = layer
    T = 5
    rng = np.random.default_rng(77 + mode)
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    L = tb.moe_layer(H, F, E, 8, fm.Q4_K, dev(router), dev(gate), dev(up), dev(down), qt_down=fm.Q6_K)
    out = np.zeros((T, H), np.float32)
    idx = np.zeros((T, 8), np.int32)
    w = np.zeros((T, 8), np.float32)
    print("moe mixed host block mode", mode, flush=True)
    assert tb.lib().tbq_moe_block_host(C.byref(L), T, xn.ctypes.data, resid.ctypes.data, out.ctypes.data,
                                       idx.ctypes.data, w.ctypes.data, mode) == 1, tb.lib().tbq_last_error()
    ref, ridx, rw = oracle.moe(xn, resid, router, gate, up, down, F=F, top_k=8, qtype=fm.Q4_K, qt_down=fm.Q6_K)
    assert np.array_equal(idx, ridx)
    assert bits_equal(w, rw)
    assert rel_l2(out - resid, ref - resid) <= TOL


@pytest.mark.parametrize("mode,T,chunk", [(tb.TBQ_MOE_FP32, 40, 16), (tb.TBQ_MOE_BF16, 512, 200),
                                          (tb.TBQ_MOE_I8, 300, 128)])
def test_moe_token_chunks(oracle, monkeypatch, mode, T, chunk):
    """A batch run as consecutive token chunks (the path batches take whose
    activation rows exceed the prefill kernels' 2 GiB buffer range, or whose
    pair count exceeds a grid column; forced small here) routes exactly and
    stays within the mode's tolerance of the oracle."""
    import torch
    H, F, E, k = 2048, 768, 128, 8
    router, gate, up, down = synth.moe_layer(H, F, E, fm.Q4_K, seed=900 + T)
    rng = np.random.default_rng(901 + T)
    bias = synth.zipf_router_bias(E, 1.1, 2.0, rng)
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    L = tb.moe_layer(H, F, E, k, fm.Q4_K, dev(router), dev(gate), dev(up), dev(down), dev(bias))
    ws = torch.zeros(tb.moe_workspace_size(L, T, mode), dtype=torch.uint8, device="cuda")
    outs = []
    for c in (None, chunk):
        if c is not None:
            monkeypatch.setenv("TBQ_MOE_CHUNK_TOKENS", str(c))
        out = empty(T * H, torch.float32)
        idx = empty(T * 8, torch.int32)
        w = empty(T * 8, torch.float32)
        print("moe chunks mode", mode, "T=", T, "chunk", c, flush=True)
        tb.moe_forward(L, T, dev(xn), dev(resid), out, idx, w, workspace=ws, mode=mode)
        assert not host(ws[:COUNTER_BYTES]).any()
        outs.append((host(out).reshape(T, H), host(idx).reshape(T, 8), host(w).reshape(T, 8)))
    monkeypatch.delenv("TBQ_MOE_CHUNK_TOKENS")
    tol = TOL if mode == tb.TBQ_MOE_FP32 else 1e-2
    sample = np.arange(0, T, 13 if T > 64 else 1)
    ref, ridx, rw = oracle.moe(xn[sample], resid[sample], router, gate, up, down, F=F, top_k=k, qtype=fm.Q4_K,
                               bias=bias)
    for out, idx, w in outs:
        assert np.array_equal(idx[sample], ridx)
        assert bits_equal(w[sample], rw)
        assert rel_l2(out[sample] - resid[sample], ref - resid[sample]) <= tol
    assert np.array_equal(outs[0][1], outs[1][1])
