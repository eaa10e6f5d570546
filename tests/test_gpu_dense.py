"""GPU parity of tbq_dense_decode (one-token decode of a dense Qwen3-style
model, BASELINE configs[2]'s forward) against the float64 oracle in
oracle/dense.py, through the C-ABI: logits within rel-L2 DENSE_TOL of the
oracle at every step, and the K/V appended to the cache.  Cases: GQA group
sizes 2 and 4, head_dim 64 and 128, a context that spans several attention
chunks, and a second layer format."""
import numpy as np
import pytest

import trailblaze_amd as tb
from conftest import rel_l2
from gpu_util import host
from trailblaze_amd import formats as fm

pytestmark = pytest.mark.gpu
# fp32 kernels (int-dot matvecs, fp32 norms and attention) against float64
DENSE_TOL = 1e-4


@pytest.fixture(scope="module", autouse=True)
def _init():
    print("device:", tb.init(), flush=True)


def _model(cfg, seed):
    from trailblaze_amd.dense import SyntheticDense
    return SyntheticDense(cfg, seed, keep_host=True)


def test_dense_decode_steps(oracle):
    """Five consecutive tokens from an empty cache (GQA 2, head_dim 64)."""
    import torch
    from oracle.dense import DenseOracle
    from trailblaze_amd.dense import DenseConfig
    cfg = DenseConfig(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=512,
                      max_ctx=256)
    m = _model(cfg, 1)
    ref = DenseOracle(oracle, cfg, m.host)
    logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    for pos, tok in enumerate([3, 200, 17, 511, 0]):
        print("dense step", pos, flush=True)
        m.decode(tok, pos, logits)
        want = ref.decode(tok, pos)
        err = rel_l2(host(logits), want)
        assert err <= DENSE_TOL, (pos, err)
    kc = host(m.k_cache).reshape(ref.kc.shape)
    vc = host(m.v_cache).reshape(ref.vc.shape)
    assert rel_l2(kc[:, :, :5], ref.kc[:, :, :5]) <= DENSE_TOL
    assert rel_l2(vc[:, :, :5], ref.vc[:, :, :5]) <= DENSE_TOL
    assert not np.any(kc[:, :, 5:])   # nothing written past pos


@pytest.mark.parametrize("qt", [fm.Q4_K, fm.Q8_0])
def test_dense_decode_long_context(oracle, qt):
    """GQA 4, head_dim 128, a cache pre-filled to position 299 (three
    attention chunks), decode at 300 and 301."""
    import torch
    from oracle.dense import DenseOracle
    from trailblaze_amd.dense import DenseConfig
    cfg = DenseConfig(n_layers=1, hidden=512, n_heads=8, n_kv_heads=2, head_dim=128, ffn=768, vocab=256,
                      max_ctx=512, qtype_layers=qt)
    m = _model(cfg, 2)
    ref = DenseOracle(oracle, cfg, m.host)
    rng = np.random.default_rng(5)
    P = 300
    kc = np.zeros(ref.kc.shape, np.float32)
    vc = np.zeros(ref.vc.shape, np.float32)
    kc[:, :, :P] = rng.standard_normal(kc[:, :, :P].shape)
    vc[:, :, :P] = rng.standard_normal(vc[:, :, :P].shape)
    m.k_cache.copy_(torch.from_numpy(kc))
    m.v_cache.copy_(torch.from_numpy(vc))
    ref.kc[:] = kc
    ref.vc[:] = vc
    logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    for pos, tok in ((P, 7), (P + 1, 255)):
        print("dense long-context step", pos, flush=True)
        m.decode(tok, pos, logits)
        err = rel_l2(host(logits), ref.decode(tok, pos))
        assert err <= DENSE_TOL, (pos, err)


def test_dense_decode_bit_reproducible(oracle):
    """The same token decoded twice at the same position (the second call
    rewrites the same K/V row) gives bit-identical logits: every reduction
    of the step (the RMSNorm sums formed in each workgroup, the attention
    merge, the matvec row sums) runs in a fixed order, and the in-place
    residual updates do not race.  Qwen3-4B widths, one layer, a cache
    filled to position 1000."""
    import torch
    from trailblaze_amd.dense import DenseConfig
    cfg = DenseConfig(n_layers=1, hidden=2560, n_heads=32, n_kv_heads=8, head_dim=128, ffn=9728, vocab=1024,
                      max_ctx=1024)
    m = _model(cfg, 13)
    m.k_cache.normal_()
    m.v_cache.normal_()
    a = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    m.decode(77, 1000, a)
    m.decode(77, 1000, b)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert torch.isfinite(a).all()


@pytest.mark.parametrize("qt,qe", [(fm.F16, fm.Q6_K), (fm.BF16, fm.F16)])
def test_dense_decode_unfused_formats(oracle, qt, qe):
    """Layers (and, with F16 embeddings, the lm_head) in formats the fused
    matvec kernels do not take: the RMSNorm, the SwiGLU and the residual add
    run as launches of their own around tbq_matvec.  Three steps from an
    empty cache."""
    import torch
    from oracle.dense import DenseOracle
    from trailblaze_amd.dense import DenseConfig
    cfg = DenseConfig(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=512,
                      max_ctx=256, qtype_layers=qt, qtype_embd=qe)
    m = _model(cfg, 9)
    ref = DenseOracle(oracle, cfg, m.host)
    logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    for pos, tok in enumerate([11, 400, 3]):
        print("dense unfused-format step", fm.NAMES[qt], pos, flush=True)
        m.decode(tok, pos, logits)
        err = rel_l2(host(logits), ref.decode(tok, pos))
        assert err <= DENSE_TOL, (pos, err)


@pytest.mark.parametrize("nq,nkv,D", [(4, 4, 64), (8, 1, 64), (8, 1, 128), (4, 2, 128)])
def test_dense_decode_gqa_groups(oracle, nq, nkv, D):
    """Every query-heads-per-kv-head group the attention kernel is built for
    (1 = multi-head, 2, 4, 8) at both head dims, over two chunks of cache."""
    import torch
    from oracle.dense import DenseOracle
    from trailblaze_amd.dense import DenseConfig
    H = max(256, nq * D)
    cfg = DenseConfig(n_layers=1, hidden=H, n_heads=nq, n_kv_heads=nkv, head_dim=D, ffn=256, vocab=256,
                      max_ctx=320)
    m = _model(cfg, 7)
    ref = DenseOracle(oracle, cfg, m.host)
    rng = np.random.default_rng(11)
    P = 140   # positions 0..139 cached: the step attends over two 128-position chunks
    kc = np.zeros(ref.kc.shape, np.float32)
    vc = np.zeros(ref.vc.shape, np.float32)
    kc[:, :, :P] = rng.standard_normal(kc[:, :, :P].shape)
    vc[:, :, :P] = rng.standard_normal(vc[:, :, :P].shape)
    m.k_cache.copy_(torch.from_numpy(kc))
    m.v_cache.copy_(torch.from_numpy(vc))
    ref.kc[:] = kc
    ref.vc[:] = vc
    logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    print("dense gqa", nq, nkv, D, flush=True)
    m.decode(9, P, logits)
    assert rel_l2(host(logits), ref.decode(9, P)) <= DENSE_TOL


def test_dense_decode_qwen3_4b_layer(oracle):
    """One layer at the Qwen3-4B widths (hidden 2560, 32/8 heads of 128, ffn
    9728), so every matvec runs the kernel and staging prologue the full
    model uses: add+RMSNorm into the q|k|v (register-x Q4_K kernel) and
    gate|up (K-quant kernel, 19456 rows) stagings, SwiGLU into the down
    staging (K = 9728 over three slices), the final norm into a Q6_K lm_head."""
    import torch
    from oracle.dense import DenseOracle
    from trailblaze_amd.dense import DenseConfig
    cfg = DenseConfig(n_layers=1, hidden=2560, n_heads=32, n_kv_heads=8, head_dim=128, ffn=9728, vocab=1024,
                      max_ctx=64)
    m = _model(cfg, 4)
    ref = DenseOracle(oracle, cfg, m.host)
    logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    for pos, tok in enumerate([11, 1000, 5]):
        print("dense qwen3-4b-width step", pos, flush=True)
        m.decode(tok, pos, logits)
        err = rel_l2(host(logits), ref.decode(tok, pos))
        assert err <= DENSE_TOL, (pos, err)


@pytest.mark.parametrize("qt", [fm.Q4_K, fm.Q8_0])
def test_dense_decode_wide_hidden(oracle, qt):
    """hidden 4608 (72 units per row): the q|k|v, gate|up and lm_head
    matvecs run the K-quant kernel with rows split over two waves, with the
    add+RMSNorm prologue and the SwiGLU epilogue on that split."""
    import torch
    from oracle.dense import DenseOracle
    from trailblaze_amd.dense import DenseConfig
    cfg = DenseConfig(n_layers=1, hidden=4608, n_heads=32, n_kv_heads=4, head_dim=128, ffn=512, vocab=256,
                      max_ctx=64, qtype_layers=qt)
    m = _model(cfg, 8)
    ref = DenseOracle(oracle, cfg, m.host)
    logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    for pos, tok in enumerate([4, 200]):
        print("dense wide-hidden step", pos, flush=True)
        m.decode(tok, pos, logits)
        assert rel_l2(host(logits), ref.decode(tok, pos)) <= DENSE_TOL, pos


@pytest.mark.parametrize("qt", [fm.Q3_K, fm.Q5_K, fm.Q6_K])
def test_dense_decode_segmented_hidden(oracle, qt):
    """hidden 2304 (36 units per row): the q|k|v and gate|up matvecs run the
    segmented K-quant kernel (lanes over consecutive units of consecutive
    rows) with the add+RMSNorm prologue and, for gate|up, the SwiGLU
    epilogue."""
    import torch
    from oracle.dense import DenseOracle
    from trailblaze_amd.dense import DenseConfig
    cfg = DenseConfig(n_layers=1, hidden=2304, n_heads=8, n_kv_heads=2, head_dim=128, ffn=1536, vocab=256,
                      max_ctx=64, qtype_layers=qt)
    m = _model(cfg, 9)
    ref = DenseOracle(oracle, cfg, m.host)
    logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    for pos, tok in enumerate([7, 130]):
        print("dense segmented-hidden step", qt, pos, flush=True)
        m.decode(tok, pos, logits)
        assert rel_l2(host(logits), ref.decode(tok, pos)) <= DENSE_TOL, pos


def test_dense_decode_configs2_context_4096(oracle):
    """BASELINE configs[2] at its context: two layers at the Qwen3-4B widths
    (hidden 2560, 32 query / 8 kv heads of 128, ffn 9728, max_ctx 4096)
    with every layer's cache filled N(0,1) up to position 4094; the step at
    position 4095 attends over all 4096 positions, i.e. 32 attention chunks
    merged by the combine kernel, in both layers (the cache's layer stride
    at max_ctx 4096)."""
    import torch
    from oracle.dense import DenseOracle
    from trailblaze_amd.dense import DenseConfig
    cfg = DenseConfig(n_layers=2, hidden=2560, n_heads=32, n_kv_heads=8, head_dim=128, ffn=9728, vocab=1024,
                      max_ctx=4096)
    m = _model(cfg, 40)
    ref = DenseOracle(oracle, cfg, m.host)
    rng = np.random.default_rng(4096)
    P = 4095
    kc = np.zeros(ref.kc.shape, np.float32)
    vc = np.zeros(ref.vc.shape, np.float32)
    kc[:, :, :P] = rng.standard_normal(kc[:, :, :P].shape, dtype=np.float32)
    vc[:, :, :P] = rng.standard_normal(vc[:, :, :P].shape, dtype=np.float32)
    m.k_cache.copy_(torch.from_numpy(kc))
    m.v_cache.copy_(torch.from_numpy(vc))
    ref.kc[:] = kc
    ref.vc[:] = vc
    del kc, vc
    logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    print("dense configs[2] step at position", P, flush=True)
    m.decode(123, P, logits)
    err = rel_l2(host(logits), ref.decode(123, P))
    assert err <= DENSE_TOL, err
    # the appended K/V rows of both layers
    kcg = host(m.k_cache).reshape(ref.kc.shape)
    vcg = host(m.v_cache).reshape(ref.vc.shape)
    assert rel_l2(kcg[:, :, P], ref.kc[:, :, P]) <= DENSE_TOL
    assert rel_l2(vcg[:, :, P], ref.vc[:, :, P]) <= DENSE_TOL


def test_dense_decode_qwen3_4b_all_layers(oracle):
    """BASELINE configs[2]'s model at full depth and vocabulary: all 36
    layers at the Qwen3-4B widths and the 151936-row Q6_K lm_head (tied
    embedding), two steps from an empty cache, against the float64 oracle
    run layer by layer (decode_layer_major: one layer's weights dequantised
    at a time).  The context is short (max_ctx 8); the 4096-position
    attention is covered at these widths by the two-layer test above."""
    import dataclasses
    import torch
    from oracle.dense import decode_layer_major
    from trailblaze_amd.dense import QWEN3_4B
    cfg = dataclasses.replace(QWEN3_4B, max_ctx=8)
    print("dense Qwen3-4B full depth: building the model", flush=True)
    m = _model(cfg, 36)
    tokens = [151935, 4096]
    outs = []
    for pos, tok in enumerate(tokens):
        logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
        print("dense Qwen3-4B full depth: step", pos, flush=True)
        m.decode(tok, pos, logits)
        outs.append(host(logits))
    print("dense Qwen3-4B full depth: oracle", flush=True)
    want = decode_layer_major(oracle, cfg, m.host, tokens)
    for pos in range(len(tokens)):
        err = rel_l2(outs[pos], want[pos])
        assert err <= DENSE_TOL, (pos, err)


@pytest.mark.parametrize("qt", [fm.Q4_K, fm.Q6_K])
def test_dense_decode_ffn_beyond_16384(oracle, qt):
    """ffn 17408 (Qwen3-14B's): the down matvec's rows are longer than 16384
    weights, which the fused kernels do not stage; the step runs SwiGLU and
    the down matvec (x over 6 wave slices) as launches of their own."""
    import torch
    from oracle.dense import DenseOracle
    from trailblaze_amd.dense import DenseConfig
    cfg = DenseConfig(n_layers=1, hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, ffn=17408, vocab=256,
                      max_ctx=32, qtype_layers=qt)
    m = _model(cfg, 17)
    ref = DenseOracle(oracle, cfg, m.host)
    logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    for pos, tok in enumerate([3, 250]):
        print("dense ffn 17408 step", pos, flush=True)
        m.decode(tok, pos, logits)
        assert rel_l2(host(logits), ref.decode(tok, pos)) <= DENSE_TOL, pos


def test_dense_decode_rejects_bad_position():
    import torch
    from trailblaze_amd.dense import DenseConfig
    cfg = DenseConfig(n_layers=1, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=256, vocab=256,
                      max_ctx=16)
    m = _model(cfg, 3)
    logits = torch.empty(cfg.vocab, dtype=torch.float32, device="cuda")
    with pytest.raises(tb.TbqError, match="pos"):
        m.decode(0, 16, logits)
    with pytest.raises(tb.TbqError, match="token"):
        m.decode(256, 0, logits)
