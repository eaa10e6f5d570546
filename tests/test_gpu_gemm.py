"""The batched prefill's GEMM (tbq_gemm, csrc/tbq_gemm.hip): a hand-written
fp16 MFMA kernel with fp32 accumulation, for W as fp16 halves or as Q4_K
rows dequantised inside the kernel.

* fp16 W: against a torch fp32 product of the same fp16 values (only the
  summation order differs), over tile edges (T and N not multiples of the
  128 x 128 tile), a row stride ldc > N and the split-K shapes (partial sums
  added in slice order).
* Q4_K W: close to the fp16 path on the fp16 values of the oracle's
  dequantised weights (the kernel's packed fp16 decode rounds 16 S, M and
  S q - M to fp16, about one fp16 ulp per weight), and to the fp64 product
  of the exact weights.
"""
import numpy as np
import pytest

import trailblaze_amd as tb
from trailblaze_amd import formats as fm, synth

from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _x16(T, K, rng):
    return (rng.standard_normal((T, K)) * 4).astype(np.float16)


@pytest.mark.parametrize("T,N,K,ldc", [
    (2, 128, 256, 0),
    (37, 200, 512, 0),          # partial tiles in t and n
    (300, 640, 2560, 0),
    (512, 2560, 4096, 0),       # split K (80 tiles)
    (512, 2560, 9728, 2688),    # split K, row stride above N
    (130, 6144, 2560, 0),
])
def test_gemm_f16_matches_torch(T, N, K, ldc):
    import torch
    rng = np.random.default_rng(T + N + K)
    X = _x16(T, K, rng)
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float16)
    print("gemm f16", T, N, K, ldc, flush=True)
    ld = ldc or N
    C = torch.full((T, ld), 7.0, dtype=torch.float32, device="cuda")
    tb.gemm(_dev(W), 1, _dev(X), T, N, K, C, ldc=ld)
    got = C.cpu().numpy()
    ref = (torch.from_numpy(X.astype(np.float32)).double() @ torch.from_numpy(W.astype(np.float32)).double().T).numpy()
    assert rel_l2(got[:, :N], ref) <= 1e-6
    if ld > N:   # columns past N untouched
        assert np.all(got[:, N:] == 7.0)


@pytest.mark.parametrize("T,N,K", [(3, 256, 512), (512, 2560, 2560), (200, 768, 4096)])
def test_gemm_q4k_fused_matches_f16_path(oracle, T, N, K):
    import torch
    rng = np.random.default_rng(N + K)
    Wq = synth.kquant_matrix(fm.Q4_K, N, K, rng)
    X = _x16(T, K, rng)
    wf = oracle.dequant_rows(Wq, fm.Q4_K, N, K)              # the reference's fp32 weights
    w16 = wf.astype(np.float16)                              # rounded once, as the prefill's fp16 weights
    print("gemm q4k", T, N, K, flush=True)
    Cq = torch.empty((T, N), dtype=torch.float32, device="cuda")
    Cf = torch.empty((T, N), dtype=torch.float32, device="cuda")
    tb.gemm(_dev(Wq), fm.Q4_K, _dev(X), T, N, K, Cq)
    tb.gemm(_dev(w16), 1, _dev(X), T, N, K, Cf)
    a, b = Cq.cpu().numpy(), Cf.cpu().numpy()
    assert rel_l2(a, b) <= 1e-3
    ref = X.astype(np.float64) @ wf.astype(np.float64).T
    assert rel_l2(a, ref) <= 1e-3   # fp16 rounding of the weights
    assert rel_l2(b, ref) <= 1e-3


def test_gemm_rejects_bad_shapes():
    import torch
    X = torch.zeros((4, 256), dtype=torch.float16, device="cuda")
    W = torch.zeros((8, 256), dtype=torch.float16, device="cuda")
    C = torch.zeros((4, 8), dtype=torch.float32, device="cuda")
    with pytest.raises(tb.TbqError):
        tb.gemm(W, 1, X, 4, 6, 256, C)      # N not a multiple of 4
    with pytest.raises(tb.TbqError):
        tb.gemm(W, 1, X, 4, 8, 200, C)      # K not a multiple of 256
    with pytest.raises(tb.TbqError):
        tb.gemm(W, 10, X, 4, 8, 256, C)     # Q2_K weights: not this kernel's
