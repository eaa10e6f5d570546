"""GPU parity of tbq_dense_prefill, the batched prefill of a dense
Qwen3-style model (T prompt tokens per layer pass; the reference prefills
token by token, layer4/tb_infer.c:1068-1075), through the C-ABI:
  * batched path (any format or layout; fused or separate matrices): the
    last token's logits and the K/V cache
    rows of every prompt position within PREFILL_TOL of the float64 oracle
    run token by token, and of libtbq's own decode steps; prompts of 1, 7,
    130 and 300 tokens (one, two and three 128-token GEMM tiles), from an
    empty cache and after decoded tokens, head_dim 64 and 128, GQA 2, 4, 8;
  * a one-token prefill is the decode step itself (bit-identical);
  * argument checks."""
import numpy as np
import pytest

import trailblaze_amd as tb
from conftest import bits_equal, rel_l2
from gpu_util import host
from trailblaze_amd import formats as fm

pytestmark = pytest.mark.gpu
# fp16-operand MFMA GEMMs (fp32 accumulate) against float64
PREFILL_TOL = 1e-2


@pytest.fixture(scope="module", autouse=True)
def _init():
    print("device:", tb.init(), flush=True)


def _cfg(**kw):
    from trailblaze_amd.dense import DenseConfig
    base = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=512, max_ctx=512)
    base.update(kw)
    return DenseConfig(**base)


def _check_prefill(oracle, cfg, seed, tokens, pre=()):
    """Decode `pre` token by token, then prefill `tokens`; compare with the
    oracle over pre + tokens and with libtbq's decode steps."""
    import torch
    from oracle.dense import DenseOracle
    from trailblaze_amd.dense import SyntheticDense
    m = SyntheticDense(cfg, seed, keep_host=True)
    seq = SyntheticDense(cfg, seed)
    assert m.prefill_batched()
    ref = DenseOracle(oracle, cfg, m.host)
    logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    for pos, tok in enumerate(pre):
        m.decode(tok, pos, logits)
    print("prefill T=", len(tokens), "pos0=", len(pre), flush=True)
    m.prefill(tokens, len(pre), logits)
    got = host(logits)
    want = None
    for pos, tok in enumerate(list(pre) + list(tokens)):
        want = ref.decode(tok, pos)
    for pos, tok in enumerate(list(pre) + list(tokens)):
        seq.decode(tok, pos, logits)
    assert rel_l2(got, want) <= PREFILL_TOL
    assert rel_l2(got, host(logits)) <= PREFILL_TOL
    n = len(pre) + len(tokens)
    kc = host(m.k_cache).reshape(ref.kc.shape)
    vc = host(m.v_cache).reshape(ref.vc.shape)
    assert rel_l2(kc[:, :, :n], ref.kc[:, :, :n]) <= PREFILL_TOL
    assert rel_l2(vc[:, :, :n], ref.vc[:, :, :n]) <= PREFILL_TOL
    assert not np.any(kc[:, :, n:])


@pytest.mark.parametrize("T", [1, 7, 130])
def test_prefill_from_empty_cache(oracle, T):
    rng = np.random.default_rng(T)
    _check_prefill(oracle, _cfg(), 41, rng.integers(0, 512, T))


def test_prefill_after_decoded_tokens(oracle):
    rng = np.random.default_rng(9)
    _check_prefill(oracle, _cfg(), 42, rng.integers(0, 512, 40), pre=[3, 99, 511, 0, 17])


@pytest.mark.parametrize("G", [4, 8])
def test_prefill_head_dim_128(oracle, G):
    rng = np.random.default_rng(G)
    cfg = _cfg(n_layers=1, hidden=512, n_heads=8, n_kv_heads=8 // G, head_dim=128, ffn=768, vocab=256)
    _check_prefill(oracle, cfg, 43, rng.integers(0, 256, 300))


@pytest.mark.parametrize("G", [1, 2])
def test_prefill_long_context_many_splits(oracle, G):
    """A 100-token prompt after 1100 cached positions (N(0,1) K/V in the
    cache and in the oracle): the attention runs over 8 position splits of
    more than 128 positions each, then merges them."""
    import torch
    from oracle.dense import DenseOracle
    from trailblaze_amd.dense import SyntheticDense
    cfg = _cfg(n_layers=1, n_heads=4, n_kv_heads=4 // G, max_ctx=1536, vocab=256)
    m = SyntheticDense(cfg, 46, keep_host=True)
    ref = DenseOracle(oracle, cfg, m.host)
    rng = np.random.default_rng(12)
    P = 1100
    kc = np.zeros(ref.kc.shape, np.float32)
    vc = np.zeros(ref.vc.shape, np.float32)
    kc[:, :, :P] = rng.standard_normal(kc[:, :, :P].shape)
    vc[:, :, :P] = rng.standard_normal(vc[:, :, :P].shape)
    m.k_cache.copy_(torch.from_numpy(kc))
    m.v_cache.copy_(torch.from_numpy(vc))
    ref.kc[:] = kc
    ref.vc[:] = vc
    toks = rng.integers(0, 256, 100)
    logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    print("prefill long context G=", G, flush=True)
    m.prefill(toks, P, logits)
    for i, tok in enumerate(toks):
        want = ref.decode(tok, P + i)
    assert rel_l2(host(logits), want) <= PREFILL_TOL
    kcg = host(m.k_cache).reshape(ref.kc.shape)
    assert rel_l2(kcg[:, :, P:P + 100], ref.kc[:, :, P:P + 100]) <= PREFILL_TOL


@pytest.mark.parametrize("ql,qe", [(fm.Q8_0, fm.Q6_K), (fm.Q5_K, fm.Q8_0), (fm.GGML | fm.Q4_K, fm.GGML | fm.Q6_K),
                                   (fm.GGML | fm.Q3_K, fm.Q4_K)])
def test_prefill_other_formats(oracle, ql, qe):
    """Layer matrices of every format and either layout take the batched
    path (each matrix dequantised to fp16 before its GEMM)."""
    rng = np.random.default_rng(ql)
    _check_prefill(oracle, _cfg(qtype_layers=ql, qtype_embd=qe, vocab=256), 47, rng.integers(0, 256, 70))


def test_prefill_separate_matrices(oracle):
    """A mixed-quant layer (separate q, k, v and gate, up matrices of
    different formats, as a GGUF file assembles them) on the batched path."""
    import torch
    from gguf_write import dense_gguf_tensors, write_gguf
    from oracle.dense import DenseOracle
    from trailblaze_amd import synth
    from trailblaze_amd.gguf import GgufFile, dense_prefill
    cfg = _cfg(n_layers=1, vocab=256, max_ctx=128)
    r = np.random.default_rng(48)
    norm = lambda n: (1.0 + 0.1 * r.standard_normal(n)).astype(np.float32)
    mat = lambda qt, M, K: synth.kquant_matrix(qt, M, K, r)
    l0 = {"attn_norm": norm(256), "q_norm": norm(64), "k_norm": norm(64), "ffn_norm": norm(256),
          "wq": mat(fm.Q4_K, 256, 256), "wk": mat(fm.Q4_K, 128, 256), "wv": mat(fm.Q6_K, 128, 256),
          "qt_wq": fm.Q4_K, "qt_wk": fm.Q4_K, "qt_wv": fm.Q6_K, "wo": mat(fm.Q5_K, 256, 256), "qt_wo": fm.Q5_K,
          "wgate": mat(fm.Q4_K, 512, 256), "wup": mat(fm.Q8_0, 512, 256), "qt_wgate": fm.Q4_K, "qt_wup": fm.Q8_0,
          "wdown": mat(fm.Q6_K, 256, 512), "qt_wdown": fm.Q6_K}
    hostd = {"layers": [l0], "lm_head": mat(fm.Q6_K, 256, 256), "output_norm": norm(256)}
    kv, ts = dense_gguf_tensors(cfg, hostd)
    import tempfile, os
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "mixed.gguf")
        write_gguf(path, kv, ts)
        ref = DenseOracle(oracle, cfg, hostd)
        with GgufFile(path) as g:
            m, ws = g.dense_model(cfg.max_ctx)
            assert not m.layers[0].wqkv and not m.layers[0].wgu
            toks = r.integers(0, 256, 50)
            logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
            print("prefill separate matrices", flush=True)
            dense_prefill(m, toks, 0, logits)
            for pos, tok in enumerate(toks):
                want = ref.decode(tok, pos)
            assert rel_l2(host(logits), want) <= PREFILL_TOL


def test_prefill_one_token_is_the_decode_step():
    """T = 1 runs the decode step itself: the same logits and cache bits."""
    import torch
    from trailblaze_amd.dense import SyntheticDense
    cfg = _cfg(max_ctx=64)
    a, b = SyntheticDense(cfg, 44), SyntheticDense(cfg, 44)
    la = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    lb = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    a.decode(7, 0, la)
    b.decode(7, 0, lb)
    a.prefill([500], 1, la)
    b.decode(500, 1, lb)
    assert bits_equal(host(la), host(lb))
    assert bits_equal(host(a.k_cache), host(b.k_cache)) and bits_equal(host(a.v_cache), host(b.v_cache))


def test_prefill_rejects_bad_arguments():
    import torch
    from trailblaze_amd.dense import SyntheticDense
    m = SyntheticDense(_cfg(max_ctx=32), 45)
    logits = torch.empty(512, dtype=torch.float32, device="cuda")
    for toks, pos0, what in (([], 0, "T="), ([1] * 30, 3, "positions"), ([1, 512], 0, "out of range"),
                             ([1, -1], 0, "out of range")):
        with pytest.raises(tb.TbqError, match=what):
            m.prefill(toks, pos0, logits)
