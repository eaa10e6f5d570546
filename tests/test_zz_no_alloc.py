"""tbq_moe_forward_noalloc (the MoE layer on the library's static per-GPU
workspace) against tbq_moe_forward with a caller workspace, through the
C-ABI: two calls in a row on one stream, the second with fewer tokens, in
the decode mode (bit-identical: the same kernels on the same inputs) and
the prefill MFMA mode; the workspace limit is reported as an error.  Run
alone in a fresh process or after the other tests."""
import numpy as np
import pytest

import trailblaze_amd as tb
from conftest import bits_equal, rel_l2
from gpu_util import dev, empty, host
from trailblaze_amd import formats as fm
from trailblaze_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _init():
    print("device:", tb.init(), flush=True)


def _run(fn, L, xn, resid, mode, **kw):
    import torch
    T, H = xn.shape
    out = empty(T * H, torch.float32)
    idx = empty(T * 8, torch.int32)
    w = empty(T * 8, torch.float32)
    fn(L, T, dev(xn), dev(resid), out, idx, w, mode=mode, **kw)
    return host(out).reshape(T, H), host(idx).reshape(T, 8), host(w).reshape(T, 8)


def _with_workspace(L, T, xn, resid, mode):
    import torch
    ws = torch.zeros(tb.moe_workspace_size(L, T, mode), dtype=torch.uint8, device="cuda")
    return _run(tb.moe_forward, L, xn, resid, mode, workspace=ws)


@pytest.mark.parametrize("mode,Ts", [(tb.TBQ_MOE_FP32, (16, 1)), (tb.TBQ_MOE_BF16, (40, 3)),
                                     (tb.TBQ_MOE_I8, (40, 3)), (tb.TBQ_MOE_FP32, (5, 2))])
def test_noalloc_matches_workspace_entry_point(oracle, mode, Ts):
    H, F, E, k = 2048, 768, 128, 8
    router, gate, up, down = synth.moe_layer(H, F, E, fm.Q4_K, seed=77)
    d = lambda a: dev(a)
    L = tb.moe_layer(H, F, E, k, fm.Q4_K, d(router), d(gate), d(up), d(down))
    for i, T in enumerate(Ts):
        print(f"noalloc mode={mode} call {i} T={T}", flush=True)
        rng = np.random.default_rng(300 + 10 * T + mode)
        xn = synth.activations((T, H), rng)
        resid = synth.activations((T, H), rng)
        o1, i1, w1 = _run(tb.moe_forward_noalloc, L, xn, resid, mode)
        o2, i2, w2 = _with_workspace(L, T, xn, resid, mode)
        assert np.array_equal(i1, i2) and bits_equal(w1, w2)
        assert bits_equal(o1, o2), rel_l2(o1, o2)
        if i == len(Ts) - 1:
            ref, ridx, _ = oracle.moe(xn, resid, router, gate, up, down, F=F, top_k=k, qtype=fm.Q4_K)
            assert np.array_equal(i1, ridx)
            tol = 1e-5 if mode == tb.TBQ_MOE_FP32 else 1e-2
            assert rel_l2(o1 - resid, ref - resid) <= tol


def test_noalloc_rejects_workspace_beyond_limit():
    import torch
    H, F, E, k = 2048, 768, 128, 8
    L = tb.moe_layer(H, F, E, k, fm.Q4_K, *(empty(16, torch.float32) for _ in range(4)))
    T = 183   # the first T whose decode workspace exceeds 16 MiB at this shape
    assert tb.moe_workspace_size(L, T, tb.TBQ_MOE_FP32) > (16 << 20) >= tb.moe_workspace_size(L, T - 1,
                                                                                              tb.TBQ_MOE_FP32)
    x = empty(T * H, torch.float32)
    with pytest.raises(tb.TbqError, match="static"):
        tb.moe_forward_noalloc(L, T, x, x, x)


@pytest.mark.parametrize("mode,T", [(tb.TBQ_MOE_FP32, 1), (tb.TBQ_MOE_FP32, 16), (tb.TBQ_MOE_BF16, 40)])
def test_noalloc_under_graph_capture(mode, T):
    """The property the entry point exists for: after one warm-up call (which
    sets up the device's static workspace), the call is captured into a HIP
    graph (torch's global capture mode, under which an allocation fails the
    capture) and replayed; each replay, with new inputs copied in and eager
    work and synchronisations between replays, is bit-identical to the
    workspace entry point on the same inputs."""
    import torch
    H, F, E, k = 2048, 768, 128, 8
    router, gate, up, down = synth.moe_layer(H, F, E, fm.Q4_K, seed=78)
    L = tb.moe_layer(H, F, E, k, fm.Q4_K, dev(router), dev(gate), dev(up), dev(down))
    xn_d = torch.zeros(T * H, dtype=torch.float32, device="cuda")
    rs_d = torch.zeros(T * H, dtype=torch.float32, device="cuda")
    out = torch.empty(T * H, dtype=torch.float32, device="cuda")
    idx = torch.empty(T * 8, dtype=torch.int32, device="cuda")
    w = torch.empty(T * 8, dtype=torch.float32, device="cuda")
    print(f"noalloc graph mode={mode} T={T}: warm-up", flush=True)
    tb.moe_forward_noalloc(L, T, xn_d, rs_d, out, idx, w, mode=mode)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        tb.moe_forward_noalloc(L, T, xn_d, rs_d, out, idx, w, mode=mode)
    torch.cuda.synchronize()
    for r in range(3):
        rng = np.random.default_rng(500 + 7 * r + T + mode)
        xn = synth.activations((T, H), rng)
        resid = synth.activations((T, H), rng)
        xn_d.copy_(torch.from_numpy(xn.reshape(-1)))
        rs_d.copy_(torch.from_numpy(resid.reshape(-1)))
        torch.cuda.synchronize()
        print(f"noalloc graph mode={mode} T={T}: replay {r}", flush=True)
        g.replay()
        o1, i1, w1 = host(out).reshape(T, H), host(idx).reshape(T, 8), host(w).reshape(T, 8)
        o2, i2, w2 = _with_workspace(L, T, xn, resid, mode)
        assert np.array_equal(i1, i2) and bits_equal(w1, w2)
        assert bits_equal(o1, o2), rel_l2(o1, o2)
    del g
