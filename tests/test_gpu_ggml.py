"""GPU parity of libtbq's ggml-layout kernels (TBQ_GGML qtype ids) against
the oracle's ggml decoders (oracle/ggml_layout.c), through the C-ABI:
  * dequant bit-exact, on random blocks and on packer-made blocks with
    subnormal fp16 scales;
  * the int-dot matvec and the fma matvec within rel-L2 1e-5 at every
    row-length class of the int-dot kernel;
  * a dense decode step on ggml-layout weights (norm prologue and SwiGLU
    epilogue kernels included) within the dense tolerance;
  * a MoE layer of ggml-layout experts (routing bit-exact);
  * a ggml-layout GGUF file read with tbq_gguf_set_layout(TBQ_GGML).
ggml's own output is not available here: parity is against the oracle's
restatement of ggml's decoders, which tests/test_ggml_layout.py pins."""
import numpy as np
import pytest

import trailblaze_amd as tb
from conftest import bits_equal, rel_l2
from ggml_pack import GEOM, QTYPE, pack, random_fields
from gpu_util import dev, empty, host
from trailblaze_amd import formats as fm
from trailblaze_amd import synth

pytestmark = pytest.mark.gpu
MATVEC_TOL = 1e-5
DENSE_TOL = 1e-4
PREFILL_TOL = 1e-2
G = fm.GGML
FORMATS = [G | fm.Q2_K, G | fm.Q3_K, G | fm.Q4_K, G | fm.Q5_K, G | fm.Q6_K, G | fm.Q8_0, G | fm.Q4_0]


@pytest.fixture(scope="module", autouse=True)
def _init():
    print("device:", tb.init(), flush=True)


def gpu_dequant(W, qt, M, K):
    import torch
    out = empty(M * K, torch.float32)
    tb.dequant(dev(W), qt, M, K, out)
    return host(out).reshape(M, K)


def gpu_matvec(W, qt, M, K, x, variant=tb.TBQ_MV_AUTO):
    import torch
    y = empty(M, torch.float32)
    tb.matvec(dev(W), qt, M, K, dev(x), y, variant=variant)
    return host(y)


@pytest.mark.parametrize("qt", FORMATS + [G | fm.F16])
def test_ggml_dequant_random_bit_exact(oracle, qt):
    print("ggml dequant", fm.NAMES[qt], flush=True)
    rng = np.random.default_rng(qt)
    M, K = 67, 2048
    W = synth.kquant_matrix(qt, M, K, rng)
    assert bits_equal(gpu_dequant(W, qt, M, K), oracle.dequant_rows(W, qt, M, K))


@pytest.mark.parametrize("fmt", sorted(GEOM))
def test_ggml_dequant_packed_subnormal_scales(oracle, fmt):
    print("ggml dequant packed", fmt, flush=True)
    rng = np.random.default_rng(len(fmt) * 31 + ord(fmt[1]))
    bw = GEOM[fmt][0]
    M, nbr = 9, 2048 // bw
    blk = pack(fmt, random_fields(fmt, M * nbr, rng))
    qt = G | QTYPE[fmt]
    W = blk.reshape(M, -1)
    assert bits_equal(gpu_dequant(W, qt, M, 2048), oracle.dequant_rows(W, qt, M, 2048))


# one shape per row-length class of the int-dot kernel (units of 64 weights:
# <= 4, 8, 16, 32, 64, 128, 192, 256) plus ragged row counts
SHAPES = [(1, 256), (5, 512), (200, 768), (1000, 2048), (4096, 4096), (333, 8192), (64, 12288), (40, 16384)]


@pytest.mark.parametrize("qt", FORMATS)
@pytest.mark.parametrize("M,K", SHAPES)
def test_ggml_matvec_kq(oracle, qt, M, K):
    print("ggml matvec", fm.NAMES[qt], M, K, flush=True)
    rng = np.random.default_rng(M + K + qt)
    W = synth.kquant_matrix(qt, M, K, rng)
    x = synth.activations(K, rng)
    got = gpu_matvec(W, qt, M, K, x, tb.TBQ_MV_KQ)
    assert rel_l2(got, oracle.matvec(W, qt, M, K, x)) <= MATVEC_TOL


@pytest.mark.parametrize("qt", [fm.Q6_K, G | fm.Q6_K])
def test_matvec_q6k_tall(oracle, qt):
    """Q6_K rows of 4096 above 65536 rows take their own launch shape
    (8-wave workgroups, several per CU): a ragged row count, sampled rows."""
    M, K = 70001, 4096
    print("matvec tall", fm.NAMES[qt], M, K, flush=True)
    rng = np.random.default_rng(qt + 5)
    W = synth.kquant_matrix(qt, M, K, rng)
    x = synth.activations(K, rng)
    y = gpu_matvec(W, qt, M, K, x, tb.TBQ_MV_KQ)
    rows = np.sort(np.concatenate([rng.choice(M - 64, 2048, replace=False), np.arange(M - 64, M)]))
    assert rel_l2(y[rows], oracle.matvec(np.ascontiguousarray(W[rows]), qt, len(rows), K, x)) <= MATVEC_TOL


@pytest.mark.parametrize("qt", FORMATS + [G | fm.F16])
@pytest.mark.parametrize("M,K", [(3, 256), (300, 4096)])
def test_ggml_matvec_fma(oracle, qt, M, K):
    print("ggml matvec fma", fm.NAMES[qt], M, K, flush=True)
    rng = np.random.default_rng(7 * M + K + qt)
    W = synth.kquant_matrix(qt, M, K, rng)
    x = synth.activations(K, rng)
    got = gpu_matvec(W, qt, M, K, x, tb.TBQ_MV_FMA)
    assert rel_l2(got, oracle.matvec(W, qt, M, K, x)) <= MATVEC_TOL


@pytest.mark.parametrize("M,K", SHAPES[1:])
def test_ggml_matvec_q4k_intdot(oracle, M, K):
    """The Q4_K-specialised kernels (register-x for K <= 4096, the
    LDS-x kernel above) in ggml's layout."""
    qt = G | fm.Q4_K
    print("ggml matvec q4k intdot", M, K, flush=True)
    rng = np.random.default_rng(3 * M + K)
    W = synth.kquant_matrix(qt, M, K, rng)
    x = synth.activations(K, rng)
    got = gpu_matvec(W, qt, M, K, x, tb.TBQ_MV_INTDOT)
    assert rel_l2(got, oracle.matvec(W, qt, M, K, x)) <= MATVEC_TOL


def test_ggml_matvec_auto_q4k_headline(oracle):
    """The default variant at the headline shape (the register-x Q4_K
    kernel in ggml's layout)."""
    qt, M, K = G | fm.Q4_K, 4096, 4096
    rng = np.random.default_rng(44)
    W = synth.kquant_matrix(qt, M, K, rng)
    x = synth.activations(K, rng)
    assert rel_l2(gpu_matvec(W, qt, M, K, x), oracle.matvec(W, qt, M, K, x)) <= MATVEC_TOL


@pytest.mark.parametrize("ql,qe", [(G | fm.Q4_K, G | fm.Q6_K), (G | fm.Q8_0, G | fm.Q8_0),
                                   (G | fm.Q5_K, G | fm.Q4_K), (G | fm.Q6_K, G | fm.Q3_K)])
def test_ggml_dense_decode(oracle, ql, qe):
    import torch
    from oracle.dense import DenseOracle
    from trailblaze_amd.dense import DenseConfig, SyntheticDense
    cfg = DenseConfig(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=256,
                      max_ctx=64, qtype_layers=ql, qtype_embd=qe)
    m = SyntheticDense(cfg, 12, keep_host=True)
    ref = DenseOracle(oracle, cfg, m.host)
    logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    for pos, tok in enumerate([9, 255, 0]):
        print("ggml dense", fm.NAMES[ql], fm.NAMES[qe], "step", pos, flush=True)
        m.decode(tok, pos, logits)
        assert rel_l2(host(logits), ref.decode(tok, pos)) <= DENSE_TOL, pos


@pytest.mark.parametrize("qt", [G | fm.Q4_K, G | fm.Q6_K, G | fm.Q8_0])
def test_ggml_moe_decode(oracle, qt):
    import torch
    H, F, E, k, T = 512, 256, 16, 4, 3
    print("ggml moe", fm.NAMES[qt], flush=True)
    router, gate, up, down = synth.moe_layer(H, F, E, qt, seed=qt & 0xFF)
    rng = np.random.default_rng(qt)
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    L = tb.moe_layer(H, F, E, k, qt, dev(router), dev(gate), dev(up), dev(down), None)
    out, idx, w = empty(T * H, torch.float32), empty(T * 8, torch.int32), empty(T * 8, torch.float32)
    ws = torch.zeros(tb.moe_workspace_size(L, T), dtype=torch.uint8, device="cuda")
    tb.moe_forward(L, T, dev(xn), dev(resid), out, idx, w, workspace=ws)
    ref, ridx, rw = oracle.moe(xn, resid, router, gate, up, down, F=F, top_k=k, qtype=qt)
    assert np.array_equal(host(idx).reshape(T, 8), ridx)
    assert bits_equal(host(w).reshape(T, 8), rw)
    assert rel_l2(host(out).reshape(T, H) - resid, ref - resid) <= MATVEC_TOL
    if qt != G | fm.Q4_K:   # the fp16 MFMA prefill decodes Q4_K only
        with pytest.raises(tb.TbqError, match="prefill"):
            tb.moe_forward(L, T, dev(xn), dev(resid), out, idx, w, workspace=ws, mode=tb.TBQ_MOE_BF16)
    else:
        assert not tb.moe_mode_supported(L, tb.TBQ_MOE_I8)
        ws16 = torch.zeros(tb.moe_workspace_size(L, T, tb.TBQ_MOE_BF16), dtype=torch.uint8, device="cuda")
        tb.moe_forward(L, T, dev(xn), dev(resid), out, idx, w, workspace=ws16, mode=tb.TBQ_MOE_BF16)
        assert np.array_equal(host(idx).reshape(T, 8), ridx)
        assert rel_l2(host(out).reshape(T, H) - resid, ref - resid) <= PREFILL_TOL


@pytest.mark.parametrize("T", [1, 5])
def test_ggml_moe_decode_config(oracle, T):
    """The Q4_K expert kernels in ggml's layout at the Qwen3-30B-A3B layer
    shape (H 2048, F 768, 128 experts, top-8)."""
    import torch
    H, F, E, k = 2048, 768, 128, 8
    qt = G | fm.Q4_K
    router, gate, up, down = synth.moe_layer(H, F, E, qt, seed=31)
    rng = np.random.default_rng(200 + T)
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    print("ggml moe config T=", T, flush=True)
    L = tb.moe_layer(H, F, E, k, qt, dev(router), dev(gate), dev(up), dev(down), None)
    out, idx, w = empty(T * H, torch.float32), empty(T * 8, torch.int32), empty(T * 8, torch.float32)
    ws = torch.zeros(tb.moe_workspace_size(L, T), dtype=torch.uint8, device="cuda")
    tb.moe_forward(L, T, dev(xn), dev(resid), out, idx, w, workspace=ws)
    ref, ridx, rw = oracle.moe(xn, resid, router, gate, up, down, F=F, top_k=k, qtype=qt)
    assert np.array_equal(host(idx).reshape(T, 8), ridx)
    assert bits_equal(host(w).reshape(T, 8), rw)
    assert rel_l2(host(out).reshape(T, H) - resid, ref - resid) <= MATVEC_TOL


@pytest.mark.parametrize("T", [40, 512])
def test_ggml_moe_prefill_mfma(oracle, T):
    """The fp16 MFMA prefill reading ggml's Q4_K layout (as llama.cpp files
    hold the experts) at the Qwen3-30B-A3B shape with a Zipf(1.1)-skewed
    router: every token routed exactly, outputs within 1e-2 of the oracle on
    a sample of tokens (tokens are independent)."""
    import torch
    H, F, E, k = 2048, 768, 128, 8
    qt = G | fm.Q4_K
    router, gate, up, down = synth.moe_layer(H, F, E, qt, seed=33)
    rng = np.random.default_rng(300 + T)
    bias = synth.zipf_router_bias(E, 1.1, 1.0, rng)
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    L = tb.moe_layer(H, F, E, k, qt, dev(router), dev(gate), dev(up), dev(down), dev(bias))
    assert tb.moe_mode_supported(L, tb.TBQ_MOE_BF16)
    out, idx, w = empty(T * H, torch.float32), empty(T * 8, torch.int32), empty(T * 8, torch.float32)
    ws = torch.zeros(tb.moe_workspace_size(L, T, tb.TBQ_MOE_BF16), dtype=torch.uint8, device="cuda")
    print("ggml moe prefill T=", T, flush=True)
    tb.moe_forward(L, T, dev(xn), dev(resid), out, idx, w, workspace=ws, mode=tb.TBQ_MOE_BF16)
    out, idx, w = host(out).reshape(T, H), host(idx).reshape(T, 8), host(w).reshape(T, 8)
    lg = oracle.router_logits(xn, router, bias)
    for t in range(T):
        ri, rw = oracle.route(lg[t], k)
        assert np.array_equal(idx[t], ri), t
        assert bits_equal(w[t], rw), t
    sample = np.sort(rng.choice(T, min(T, 32), replace=False))
    ref, _, _ = oracle.moe(xn[sample], resid[sample], router, gate, up, down, F=F, top_k=k, qtype=qt, bias=bias)
    assert rel_l2(out[sample] - resid[sample], ref - resid[sample]) <= PREFILL_TOL


def test_ggml_gguf_dense_file(tmp_path, oracle):
    """A GGUF file holds ggml type ids; read with the ggml layout, the
    assembled model decodes bit-identically to the same weights handed to
    tbq_dense_decode with TBQ_GGML qtypes, and within the dense tolerance
    of the oracle."""
    import torch
    from gguf_write import dense_gguf_tensors, write_gguf
    from oracle.dense import DenseOracle
    from trailblaze_amd.dense import DenseConfig, SyntheticDense
    from trailblaze_amd.gguf import GgufFile, dense_decode
    cfg = DenseConfig(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=256,
                      max_ctx=32, qtype_layers=G | fm.Q4_K, qtype_embd=G | fm.Q6_K)
    syn = SyntheticDense(cfg, 13, keep_host=True)
    kv, ts = dense_gguf_tensors(cfg, syn.host)
    assert all(t[1] < 0x100 for t in ts)   # files carry plain ggml ids
    path = tmp_path / "ggml.gguf"
    write_gguf(path, kv, ts)
    ref = DenseOracle(oracle, cfg, syn.host)
    with GgufFile(path) as g:
        g.set_layout(fm.GGML)
        m, ws = g.dense_model(cfg.max_ctx)
        assert (m.qtype_layers, m.qtype_embd) == (G | fm.Q4_K, G | fm.Q6_K)
        assert g.info("blk.0.attn_q.weight")[0] == fm.Q4_K   # the file's own id
        a = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
        b = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
        for pos, tok in enumerate([4, 100, 255]):
            print("ggml gguf dense step", pos, flush=True)
            dense_decode(m, ws, tok, pos, a)
            syn.decode(tok, pos, b)
            la = host(a)
            assert bits_equal(la, host(b)), pos
            assert rel_l2(la, ref.decode(tok, pos)) <= DENSE_TOL, pos
        with pytest.raises(tb.TbqError, match="layout"):
            g.set_layout(3)
