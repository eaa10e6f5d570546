"""GPU parity for the K-quant path, through the C-ABI (libtbq.so):
  * dequant: bit-exact against the reference's golden vectors and against
    the oracle on random matrices (NaN payloads aside);
  * matvec: relative L2 <= 1e-5 against the oracle (the reference's
    sequential fp32 dot, layer4/tb_gguf.c:376-419) at the BASELINE.json
    shapes and at ragged/edge shapes; exact on exactly-representable inputs;
  * the reference ABI tb_cuda_matvec_device on host buffers;
  * the router's device expf bit-identical to glibc's on a large sample."""
import ctypes as C

import numpy as np
import pytest

import trailblaze_amd as tb
from conftest import bits_equal, golden_names, load_golden, rel_l2
from gpu_util import dev, empty, host
from trailblaze_amd import formats as fm
from trailblaze_amd import synth

pytestmark = pytest.mark.gpu
MATVEC_TOL = 1e-5


@pytest.fixture(scope="module", autouse=True)
def _init():
    import torch
    assert torch.cuda.is_available()
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


@pytest.mark.parametrize("name", golden_names("dequant_"))
def test_dequant_golden_bit_exact(name):
    g = load_golden(name)
    print(name, flush=True)
    got = gpu_dequant(g["W"], int(g["qtype"]), int(g["M"]), int(g["K"]))
    assert bits_equal(got, g["out"])


@pytest.mark.parametrize("qt", [fm.Q2_K, fm.Q3_K, fm.Q4_K, fm.Q5_K, fm.Q6_K, fm.Q8_0, fm.Q4_0, fm.Q8_K])
def test_dequant_random_bit_exact(oracle, qt):
    rng = np.random.default_rng(1000 + qt)
    M, K = 257, 4096
    W = synth.kquant_matrix(qt, M, K, rng)
    assert bits_equal(gpu_dequant(W, qt, M, K), oracle.dequant_rows(W, qt, M, K))


@pytest.mark.parametrize("name", golden_names("matvec_"))
def test_matvec_golden(name):
    g = load_golden(name)
    print(name, flush=True)
    got = gpu_matvec(g["W"], int(g["qtype"]), int(g["M"]), int(g["K"]), g["x"])
    assert rel_l2(got, g["out"]) <= MATVEC_TOL


# BASELINE.json configs[0] and configs[1] shapes (Q6_K lm_head covered by
# test_matvec_lm_head below)
SHAPES = [(fm.Q4_K, 4096, 4096)] + [(qt, M, K) for qt in (fm.Q2_K, fm.Q3_K, fm.Q5_K, fm.Q8_0)
                                    for (M, K) in ((12288, 4096), (4096, 12288))]


@pytest.mark.parametrize("qt,M,K", SHAPES)
def test_matvec_config_shapes(oracle, qt, M, K):
    print(fm.NAMES[qt], M, K, flush=True)
    rng = np.random.default_rng(M * 7 + K + qt)
    W = synth.kquant_matrix(qt, M, K, rng)
    x = synth.activations(K, rng)
    assert rel_l2(gpu_matvec(W, qt, M, K, x), oracle.matvec(W, qt, M, K, x)) <= MATVEC_TOL


def test_matvec_lm_head(oracle):
    qt, M, K = fm.Q6_K, 151936, 4096
    rng = np.random.default_rng(42)
    W = synth.kquant_matrix(qt, M, K, rng)
    x = synth.activations(K, rng)
    y = gpu_matvec(W, qt, M, K, x)
    rows = rng.choice(M, 4096, replace=False)
    rows.sort()
    ref = oracle.matvec(np.ascontiguousarray(W[rows]), qt, len(rows), K, x)
    assert rel_l2(y[rows], ref) <= MATVEC_TOL


@pytest.mark.parametrize("qt", [fm.Q2_K, fm.Q3_K, fm.Q4_K, fm.Q5_K, fm.Q6_K, fm.Q8_0, fm.Q4_0, fm.Q8_K,
                                fm.F16, fm.BF16, fm.F32])
@pytest.mark.parametrize("M,K", [(1, 256), (3, 768), (131, 2048), (517, 512), (64, 12288)])
def test_matvec_edge_shapes(oracle, qt, M, K):
    rng = np.random.default_rng(M + K + qt)
    W = synth.kquant_matrix(qt, M, K, rng)
    x = synth.activations(K, rng)
    assert rel_l2(gpu_matvec(W, qt, M, K, x), oracle.matvec(W, qt, M, K, x)) <= MATVEC_TOL


@pytest.mark.parametrize("variant", [tb.TBQ_MV_FMA, tb.TBQ_MV_INTDOT])
@pytest.mark.parametrize("M,K", [(1, 256), (7, 512), (200, 768), (1000, 2048), (4096, 4096), (6144, 4096),
                                 (2560, 4096), (2049, 4096), (5000, 2560), (333, 8192),
                                 (4096, 12288), (65, 16384)])
def test_matvec_q4k_kernels(oracle, variant, M, K):
    if variant == tb.TBQ_MV_FMA and K > 15360:
        pytest.skip("x does not fit the fma kernel's LDS staging at this K")
    rng = np.random.default_rng(M * 31 + K)
    W = synth.kquant_matrix(fm.Q4_K, M, K, rng)
    x = synth.activations(K, rng)
    assert rel_l2(gpu_matvec(W, fm.Q4_K, M, K, x, variant), oracle.matvec(W, fm.Q4_K, M, K, x)) <= MATVEC_TOL


@pytest.mark.parametrize("scale", [1e-30, 1e-3, 1e3, 1e30])
def test_matvec_q4k_activation_range(oracle, scale):
    """Per-sub-block exponents keep the int-dot kernel in tolerance for tiny
    and huge activations and for LLM-style outlier channels (1000x)."""
    rng = np.random.default_rng(17)
    M, K = 512, 4096
    W = synth.kquant_matrix(fm.Q4_K, M, K, rng)
    x = (synth.activations(K, rng) * np.float32(scale)).astype(np.float32)
    x[rng.choice(K, 12, replace=False)] *= np.float32(1000.0)
    ref = oracle.matvec(W, fm.Q4_K, M, K, x)
    assert rel_l2(gpu_matvec(W, fm.Q4_K, M, K, x, tb.TBQ_MV_INTDOT), ref) <= MATVEC_TOL
    x0 = np.zeros(K, np.float32)
    assert np.all(gpu_matvec(W, fm.Q4_K, M, K, x0, tb.TBQ_MV_INTDOT) == 0.0)


KQ_FORMATS = [fm.Q2_K, fm.Q3_K, fm.Q4_K, fm.Q5_K, fm.Q6_K, fm.Q8_0, fm.Q4_0, fm.Q8_K]


@pytest.mark.parametrize("qt", KQ_FORMATS)
@pytest.mark.parametrize("M,K", [(1, 256), (5, 512), (200, 768), (1000, 2048), (4096, 4096), (333, 8192),
                                 (700, 12288), (65, 16384), (2560, 9728), (1281, 10240)])
def test_matvec_kq_kernel(oracle, qt, M, K):
    """The shared integer-dot kernel for every block format: row slices of
    4..64 units, rows split over 2..4 waves (K > 4096), ragged M; 2560x9728
    and 1281x10240 take five row groups of three slices."""
    rng = np.random.default_rng(M * 13 + K + 7 * qt)
    W = synth.kquant_matrix(qt, M, K, rng)
    x = synth.activations(K, rng)
    assert rel_l2(gpu_matvec(W, qt, M, K, x, tb.TBQ_MV_KQ), oracle.matvec(W, qt, M, K, x)) <= MATVEC_TOL


@pytest.mark.parametrize("qt", KQ_FORMATS)
@pytest.mark.parametrize("M,K", [(5, 2560), (26, 2304), (777, 3072), (2000, 3840), (6144, 2560), (300, 1280),
                                 (8960, 1536), (43, 1792)])
def test_matvec_kq_segmented_rows(oracle, qt, M, K):
    """Rows of 20..60 units (K = 1280 .. 3840, Qwen3-4B's hidden 2560): the
    segmented mapping, a workgroup's lanes over consecutive units of
    consecutive rows, partial sums meeting in LDS; ragged last row block.
    No single-row case: one output of a 2560-term sum can cancel by 10^3
    (sum |w x| = 2740 for a result of 1.2), where the oracle's own fp32 sum
    is already 1.3e-5 from the exact value."""
    rng = np.random.default_rng(M * 11 + K + 5 * qt)
    W = synth.kquant_matrix(qt, M, K, rng)
    x = synth.activations(K, rng)
    assert rel_l2(gpu_matvec(W, qt, M, K, x, tb.TBQ_MV_KQ), oracle.matvec(W, qt, M, K, x)) <= MATVEC_TOL


@pytest.mark.parametrize("qt", KQ_FORMATS)
def test_matvec_tall_64_unit_rows(oracle, qt):
    """Matrices of 64-unit rows (K = 4096) above 32768 rows: the default
    dispatch takes the segmented mapping (16 rows per workgroup pass) for
    every format but Q6_K; 32769 rows leave a last block of one row."""
    M, K = 32769, 4096
    print(f"tall rows qt={qt} M={M} K={K}", flush=True)
    rng = np.random.default_rng(qt + 17)
    W = synth.kquant_matrix(qt, M, K, rng)
    x = synth.activations(K, rng)
    assert rel_l2(gpu_matvec(W, qt, M, K, x), oracle.matvec(W, qt, M, K, x)) <= MATVEC_TOL


def test_matvec_q3k_segmented_from_8193_rows(oracle):
    """Q3_K takes the segmented mapping for 64-unit rows above 8192 rows
    (the other formats above 32768); 12289 rows leave a last block of one."""
    M, K = 12289, 4096
    rng = np.random.default_rng(12289)
    W = synth.kquant_matrix(fm.Q3_K, M, K, rng)
    x = synth.activations(K, rng)
    assert rel_l2(gpu_matvec(W, fm.Q3_K, M, K, x), oracle.matvec(W, fm.Q3_K, M, K, x)) <= MATVEC_TOL


@pytest.mark.parametrize("M,K", [(8193, 2560), (20001, 2560), (9001, 1536)])
def test_matvec_q4k_tall_segmented(oracle, M, K):
    """Q4_K rows of 24 or 40 units taller than 8192 rows: the default
    dispatch takes the K-quant kernel's segmented mapping instead of the
    persistent Q4_K kernel; the last row block is ragged."""
    rng = np.random.default_rng(M + 3)
    W = synth.kquant_matrix(fm.Q4_K, M, K, rng)
    x = synth.activations(K, rng)
    assert rel_l2(gpu_matvec(W, fm.Q4_K, M, K, x), oracle.matvec(W, fm.Q4_K, M, K, x)) <= MATVEC_TOL


@pytest.mark.parametrize("qt", KQ_FORMATS)
@pytest.mark.parametrize("M,K", [(70, 17408), (129, 24576), (33, 32768)])
def test_matvec_long_rows(oracle, qt, M, K):
    """Rows longer than 16384 weights (FFN-down of models with FFN 17408 ..
    32768): x staged over 6 or 8 wave slices with more than 64 KiB of LDS."""
    print(f"long rows qt={qt} M={M} K={K}", flush=True)
    rng = np.random.default_rng(M * 7 + K + qt)
    W = synth.kquant_matrix(qt, M, K, rng)
    x = synth.activations(K, rng)
    assert rel_l2(gpu_matvec(W, qt, M, K, x), oracle.matvec(W, qt, M, K, x)) <= MATVEC_TOL


@pytest.mark.parametrize("qt", [fm.Q4_K, fm.Q6_K, fm.Q3_K, fm.Q8_0, fm.GGML | fm.Q4_K])
@pytest.mark.parametrize("M,K", [(4, 32768 + 256), (300, 53248), (17, 98304)])
def test_matvec_rows_beyond_32768(oracle, qt, M, K):
    """Rows longer than the LDS-staged x (53248 is a 405B-class FFN-down row):
    column slices of 32768 weights with the full row stride, their partial
    products added in slice order; the reference's CUDA entry point has no
    row limit (layer4/tb_gguf_dequant.cu:422-472)."""
    print(f"rows beyond 32768 qt={qt} M={M} K={K}", flush=True)
    rng = np.random.default_rng(M + K + qt)
    W = synth.kquant_matrix(qt, M, K, rng)
    x = synth.activations(K, rng)
    assert rel_l2(gpu_matvec(W, qt, M, K, x), oracle.matvec(W, qt, M, K, x)) <= MATVEC_TOL


def test_matvec_rejects_fma_rows_beyond_limit():
    """F32/F16/BF16 rows stay within the fma kernel's LDS-resident x."""
    import torch
    W = empty(16 * 16384 * 4, torch.uint8)
    x = empty(16384, torch.float32)
    y = empty(4, torch.float32)
    with pytest.raises(tb.TbqError):
        tb.matvec(W, fm.F32, 4, 16384, x, y)


@pytest.mark.parametrize("qt", [fm.Q8_0, fm.Q4_0])
@pytest.mark.parametrize("K", [64, 128, 192])
def test_matvec_kq_short_rows(oracle, qt, K):
    """32-weight block formats at K below one 256-weight super-block."""
    M = 300
    rng = np.random.default_rng(K + qt)
    W = synth.kquant_matrix(qt, M, K, rng)
    x = synth.activations(K, rng)
    assert rel_l2(gpu_matvec(W, qt, M, K, x, tb.TBQ_MV_KQ), oracle.matvec(W, qt, M, K, x)) <= MATVEC_TOL


@pytest.mark.parametrize("qt", KQ_FORMATS)
@pytest.mark.parametrize("scale", [1e-30, 1e-3, 1e3, 1e30])
def test_matvec_kq_activation_range(oracle, qt, scale):
    """One power-of-two exponent per 64 elements keeps the shared kernel in
    tolerance for tiny and huge activations and for 1000x outlier channels;
    x = 0 gives exact zeros."""
    rng = np.random.default_rng(23 + qt)
    M, K = 256, 4096
    W = synth.kquant_matrix(qt, M, K, rng)
    x = (synth.activations(K, rng) * np.float32(scale)).astype(np.float32)
    x[rng.choice(K, 12, replace=False)] *= np.float32(1000.0)
    ref = oracle.matvec(W, qt, M, K, x)
    assert rel_l2(gpu_matvec(W, qt, M, K, x, tb.TBQ_MV_KQ), ref) <= MATVEC_TOL
    x0 = np.zeros(K, np.float32)
    assert np.all(gpu_matvec(W, qt, M, K, x0, tb.TBQ_MV_KQ) == 0.0)


def test_matvec_kq_rejects_uncovered_shapes():
    import torch
    W = empty(4096, torch.uint8)
    x = empty(4096, torch.float32)
    y = empty(4, torch.float32)
    with pytest.raises(tb.TbqError):
        tb.matvec(W, fm.Q8_0, 4, 96, x, y, variant=tb.TBQ_MV_KQ)     # K not a multiple of 64
    with pytest.raises(tb.TbqError):
        tb.matvec(W, fm.F16, 4, 256, x, y, variant=tb.TBQ_MV_KQ)     # no integer form


def test_matvec_exact_one_hot():
    # Q8_0 weights in {0, 1} with d = 1: every output of the fp32 kernel is
    # one x value exactly (the integer-dot kernels round x to 2^-23 of a
    # unit's max |x| and are checked to tolerance elsewhere)
    M, K = 300, 1024
    rng = np.random.default_rng(3)
    W = np.zeros((M, K // 32, 34), np.uint8)
    W[:, :, 0:2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    cols = rng.integers(0, K, M)
    for m, j in enumerate(cols):
        W[m, j // 32, 2 + j % 32] = 1
    x = rng.standard_normal(K).astype(np.float32)
    assert np.array_equal(gpu_matvec(W.reshape(M, -1), fm.Q8_0, M, K, x, tb.TBQ_MV_FMA), x[cols])


def test_matvec_rejects_bad_input():
    import torch
    W = empty(4096, torch.uint8)
    x = empty(300, torch.float32)
    y = empty(4, torch.float32)
    with pytest.raises(tb.TbqError):
        tb.matvec(W, fm.Q4_K, 4, 300, x, y)        # K not a multiple of 256
    with pytest.raises(tb.TbqError):
        tb.matvec(W, 21, 4, 256, x, y)            # qtype without a CPU decoder


def test_reference_abi_matvec_device(oracle):
    L = tb.lib()
    assert L.tb_cuda_init() == 1
    rng = np.random.default_rng(9)
    for qt, M, K in ((fm.Q4_K, 1000, 4096), (fm.Q2_K, 64, 768), (fm.Q6_K, 33, 2048), (fm.Q4_K, 40, 17408)):
        W = synth.kquant_matrix(qt, M, K, rng)
        x = synth.activations(K, rng)
        d = L.tb_cuda_upload_tensor(W.ctypes.data, W.nbytes)
        assert d
        out = np.zeros(M, np.float32)
        assert L.tb_cuda_matvec_device(d, qt, M, K, x.ctypes.data, out.ctypes.data) == 1
        assert rel_l2(out, oracle.matvec(W, qt, M, K, x)) <= MATVEC_TOL
        assert L.tb_cuda_matvec_device(d, 21, M, K, x.ctypes.data, out.ctypes.data) == 0
        L.tb_cuda_free_tensor(d)
    assert L.tb_cuda_upload_x(x.ctypes.data, K) == 1
    L.tb_cuda_sync_all()
    L.tb_cuda_cleanup()


def test_device_expf_matches_glibc(oracle):
    import torch
    rng = np.random.default_rng(12)
    xs = [rng.integers(0, 2 ** 32, 1 << 24, dtype=np.uint64).astype(np.uint32).view(np.float32),
          np.linspace(-20, 0, 1 << 22, dtype=np.float32),
          np.arange(0xBF800000, 0xBF800000 + (1 << 22), dtype=np.uint32).view(np.float32)]
    for x in xs:
        out = empty(x.size, torch.float32)
        tb.expf_device(dev(x), out)
        assert bits_equal(host(out), oracle.expf(x))
