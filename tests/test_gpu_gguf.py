"""GPU tests of the GGUF loader (include/tbq_gguf.h): every tensor of every
format libtbq knows (F32/F16/BF16 norms and routers included) uploaded bit
for bit; a dense model assembled from a file decodes to the same logits, bit
for bit, as the same weights handed to tbq_dense_decode directly, and within
the dense tolerance of the float64 oracle; a MoE layer from a file routes and
combines as the oracle does."""
import ctypes as C

import numpy as np
import pytest

import trailblaze_amd as tb
from conftest import bits_equal, rel_l2
from gguf_write import dense_gguf_tensors, write_gguf
from gpu_util import dev, empty, host
from test_gguf import KV, sample_tensors
from trailblaze_amd import formats as fm
from trailblaze_amd import synth
from trailblaze_amd.gguf import GgufFile, dense_decode

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _init():
    print("device:", tb.init(), flush=True)


def test_gguf_upload_all_bit_exact(tmp_path):
    ts = sample_tensors(np.random.default_rng(9))
    path = tmp_path / "all.gguf"
    write_gguf(path, KV, ts, alignment=64)
    with GgufFile(path) as g:
        n = g.upload_all()
        assert n == len(ts) - 1   # all but the unknown qtype
        for name, qt, dims, data in ts:
            p = g.device_ptr(name)
            if name == "unknown":
                assert p == 0
                continue
            raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
            back = np.empty_like(raw)
            assert tb.lib().tbq_memcpy_d2h(back.ctypes.data_as(C.c_void_p), C.c_void_p(p), raw.size, None)
            assert tb.lib().tbq_stream_sync(None)
            assert np.array_equal(back, raw), name
        assert g.upload_all() == n   # idempotent


def test_gguf_dense_model_decode(tmp_path, oracle):
    import torch
    from oracle.dense import DenseOracle
    from trailblaze_amd.dense import DenseConfig, SyntheticDense
    cfg = DenseConfig(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=512, max_ctx=64)
    syn = SyntheticDense(cfg, 11, keep_host=True)
    kv, ts = dense_gguf_tensors(cfg, syn.host)
    path = tmp_path / "dense.gguf"
    write_gguf(path, kv, ts)
    ref = DenseOracle(oracle, cfg, syn.host)
    with GgufFile(path) as g:
        m, ws = g.dense_model(cfg.max_ctx)
        assert (m.n_layers, m.hidden, m.n_heads, m.n_kv_heads, m.head_dim, m.ffn, m.vocab) == \
               (2, 256, 4, 2, 64, 512, 512)
        assert m.qtype_layers == cfg.qtype_layers and m.qtype_embd == cfg.qtype_embd
        assert m.lm_head == m.tok_embd   # no output.weight: tied
        a = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
        b = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
        for pos, tok in enumerate([5, 300, 511]):
            print("gguf dense step", pos, flush=True)
            dense_decode(m, ws, tok, pos, a)
            syn.decode(tok, pos, b)
            la, lb = host(a), host(b)
            assert bits_equal(la, lb), pos
            assert rel_l2(la, ref.decode(tok, pos)) <= 1e-4, pos


def test_gguf_dense_model_mixed_qtypes(tmp_path, oracle):
    """A mixed-quant file (as llama.cpp's Q4_K_M recipes write them): layer 0
    has a Q6_K attn_v and gate / up of different formats, layer 1 a Q6_K
    ffn_down and a Q5_K attn_output; q|k|v and gate|up then stay separate
    matrices, each with its own qtype."""
    import torch
    from oracle.dense import DenseOracle
    from trailblaze_amd.dense import DenseConfig
    cfg = DenseConfig(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=256, max_ctx=32)
    c, rng = cfg, np.random.default_rng(31)
    D, NQ, NKV = c.head_dim, c.n_heads, c.n_kv_heads
    norm = lambda n: (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    mat = lambda qt, M, K: synth.kquant_matrix(qt, M, K, rng)
    l0 = {"attn_norm": norm(256), "q_norm": norm(64), "k_norm": norm(64), "ffn_norm": norm(256),
          "wq": mat(fm.Q4_K, NQ * D, 256), "wk": mat(fm.Q4_K, NKV * D, 256), "wv": mat(fm.Q6_K, NKV * D, 256),
          "qt_wq": fm.Q4_K, "qt_wk": fm.Q4_K, "qt_wv": fm.Q6_K,
          "wo": mat(fm.Q4_K, 256, NQ * D), "wgate": mat(fm.Q4_K, 512, 256), "wup": mat(fm.Q5_K, 512, 256),
          "qt_wgate": fm.Q4_K, "qt_wup": fm.Q5_K, "wdown": mat(fm.Q4_K, 256, 512)}
    l1 = {"attn_norm": norm(256), "q_norm": norm(64), "k_norm": norm(64), "ffn_norm": norm(256),
          "wqkv": mat(fm.Q4_K, (NQ + 2 * NKV) * D, 256), "wo": mat(fm.Q5_K, 256, NQ * D), "qt_wo": fm.Q5_K,
          "wgu": mat(fm.Q4_K, 1024, 256), "wdown": mat(fm.Q6_K, 256, 512), "qt_wdown": fm.Q6_K}
    hostd = {"layers": [l0, l1], "lm_head": mat(fm.Q6_K, 256, 256), "output_norm": norm(256)}
    kv, ts = dense_gguf_tensors(cfg, hostd)
    path = tmp_path / "mixed.gguf"
    write_gguf(path, kv, ts)
    ref = DenseOracle(oracle, cfg, hostd)
    with GgufFile(path) as g:
        m, ws = g.dense_model(cfg.max_ctx)
        L0, L1 = m.layers[0], m.layers[1]
        assert not L0.wqkv and L0.wq and (L0.qt_q, L0.qt_k, L0.qt_v) == (fm.Q4_K, fm.Q4_K, fm.Q6_K)
        assert not L0.wgu and (L0.qt_gate, L0.qt_up) == (fm.Q4_K, fm.Q5_K)
        assert L1.wqkv and L1.wgu and (L1.qt_o, L1.qt_down) == (fm.Q5_K, fm.Q6_K)
        logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
        for pos, tok in enumerate([1, 77, 255, 3]):
            print("gguf mixed-quant step", pos, flush=True)
            dense_decode(m, ws, tok, pos, logits)
            assert rel_l2(host(logits), ref.decode(tok, pos)) <= 1e-4, pos


def test_gguf_moe_layer(tmp_path, oracle):
    import torch
    H, F, E, k = 512, 256, 16, 4
    router, gate, up, down = synth.moe_layer(H, F, E, fm.Q4_K, seed=21)
    kv = [("general.architecture", "str", "qwen3moe"), ("qwen3moe.embedding_length", "u32", H),
          ("qwen3moe.expert_count", "u32", E), ("qwen3moe.expert_used_count", "u32", k),
          ("qwen3moe.expert_feed_forward_length", "u32", F)]
    ts = [("blk.0.ffn_gate_inp.weight", fm.F32, (H, E), router),
          ("blk.0.ffn_gate_exps.weight", fm.Q4_K, (H, F, E), gate),
          ("blk.0.ffn_up_exps.weight", fm.Q4_K, (H, F, E), up),
          ("blk.0.ffn_down_exps.weight", fm.Q4_K, (F, H, E), down)]
    path = tmp_path / "moe.gguf"
    write_gguf(path, kv, ts)
    rng = np.random.default_rng(21)
    T = 3
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    with GgufFile(path) as g:
        L = g.moe_layer(0)
        assert (L.H, L.F, L.E, L.top_k, L.qtype) == (H, F, E, k, fm.Q4_K)
        out = empty(T * H, torch.float32)
        idx = empty(T * 8, torch.int32)
        w = empty(T * 8, torch.float32)
        ws = torch.zeros(tb.moe_workspace_size(L, T), dtype=torch.uint8, device="cuda")
        tb.moe_forward(L, T, dev(xn), dev(resid), out, idx, w, workspace=ws)
        ref, ridx, rw = oracle.moe(xn, resid, router, gate, up, down, F=F, top_k=k, qtype=fm.Q4_K)
        assert np.array_equal(host(idx).reshape(T, 8), ridx)
        assert bits_equal(host(w).reshape(T, 8), rw)
        assert rel_l2(host(out).reshape(T, H) - resid, ref - resid) <= 1e-5


@pytest.mark.parametrize("split", [False, True])
def test_gguf_moe_layer_mixed_and_split(tmp_path, oracle, split):
    """A K-quant mix (Q4_K gate, Q5_K up, Q6_K down) read from the file with
    each tensor's own qtype, in the packed blk.N.ffn_*_exps form and in the
    reference's split fallback blk.N.ffn_{gate,up,down}.<e>.weight
    (layer4/tb_infer.c:783-791), which the loader packs on the device."""
    import torch
    H, F, E, k = 512, 256, 16, 4
    qg, qu, qd = fm.Q4_K, fm.Q5_K, fm.Q6_K
    router, gate, up, down = synth.moe_layer(H, F, E, qg, seed=22, qt_up=qu, qt_down=qd)
    kv = [("general.architecture", "str", "qwen3moe"), ("qwen3moe.embedding_length", "u32", H),
          ("qwen3moe.expert_count", "u32", E), ("qwen3moe.expert_used_count", "u32", k),
          ("qwen3moe.expert_feed_forward_length", "u32", F)]
    ts = [("blk.0.ffn_gate_inp.weight", fm.F32, (H, E), router)]
    if split:
        for name, qt, t, d0, d1 in (("gate", qg, gate, H, F), ("up", qu, up, H, F), ("down", qd, down, F, H)):
            per = t.reshape(E, -1)
            ts += [(f"blk.0.ffn_{name}.{e}.weight", qt, (d0, d1), per[e]) for e in range(E)]
    else:
        ts += [("blk.0.ffn_gate_exps.weight", qg, (H, F, E), gate),
               ("blk.0.ffn_up_exps.weight", qu, (H, F, E), up),
               ("blk.0.ffn_down_exps.weight", qd, (F, H, E), down)]
    path = tmp_path / "moe_mixed.gguf"
    write_gguf(path, kv, ts)
    rng = np.random.default_rng(23)
    T = 3
    xn = synth.activations((T, H), rng)
    resid = synth.activations((T, H), rng)
    print("gguf moe mixed split=", split, flush=True)
    with GgufFile(path) as g:
        L = g.moe_layer(0)
        assert (L.H, L.F, L.E, L.top_k) == (H, F, E, k)
        assert (L.qt_gate, L.qt_up, L.qt_down) == (qg, qu, qd)
        out = empty(T * H, torch.float32)
        idx = empty(T * 8, torch.int32)
        w = empty(T * 8, torch.float32)
        ws = torch.zeros(tb.moe_workspace_size(L, T), dtype=torch.uint8, device="cuda")
        tb.moe_forward(L, T, dev(xn), dev(resid), out, idx, w, workspace=ws)
        ref, ridx, rw = oracle.moe(xn, resid, router, gate, up, down, F=F, top_k=k, qtype=qg, qt_up=qu,
                                   qt_down=qd)
        assert np.array_equal(host(idx).reshape(T, 8), ridx)
        assert bits_equal(host(w).reshape(T, 8), rw)
        assert rel_l2(host(out).reshape(T, H) - resid, ref - resid) <= 1e-5
