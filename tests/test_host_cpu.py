"""CPU checks of libtbq's C11 host layer and of the drop-in contract, with
no GPU:

* tbq_moe_block_host (trailblaze_amd/host/tbq_moe_host.c) compiled against a
  host-memory stand-in for the device API (tests/host_mock.c): across calls
  whose T and mode change, the MoE workspace always starts at the cached
  buffer's first byte and its counter area is zero on entry to every call,
  including right after the buffer is regrown from non-zeroed memory.
* TBQ_FORCE_NO_DEVICE=1 (the fault-injection switch): tb_cuda_init returns 0,
  uploads return NULL and tb_cuda_matvec_device returns 0, the contract the
  reference's CPU fallback relies on (layer4/tb_gguf.c:444-451, :505-514).
* Where /root/reference exists: the reference's own sources built with
  -DTB_CUDA link against libtbq.so unchanged (its tb_infer test binary), and
  its tb_gguf_tensor_matvec falls back to a bit-identical CPU result for no
  device, an unsupported qtype and a NULL device pointer (oracle/ref_fallback.c).
"""
import ctypes as C
import os
import subprocess
import sys
import tempfile

import numpy as np
import pytest

import trailblaze_amd as tb

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.environ.get("TBQ_REFERENCE", "/root/reference")


class MoeLayer(C.Structure):
    _fields_ = [("H", C.c_int), ("F", C.c_int), ("E", C.c_int), ("top_k", C.c_int), ("qtype", C.c_int),
                ("router", C.c_void_p), ("bias", C.c_void_p), ("gate", C.c_void_p), ("up", C.c_void_p),
                ("down", C.c_void_p), ("qt_gate", C.c_int), ("qt_up", C.c_int), ("qt_down", C.c_int)]


@pytest.fixture(scope="module")
def host_block():
    d = tempfile.mkdtemp(prefix="tbq_host_")
    so = os.path.join(d, "libhostmock.so")
    subprocess.run(["gcc", "-std=c11", "-O1", "-fPIC", "-shared", "-Wall", "-Wextra", "-Werror",
                    "-I", os.path.join(ROOT, "include"), "-o", so,
                    os.path.join(ROOT, "trailblaze_amd", "host", "tbq_moe_host.c"),
                    os.path.join(ROOT, "tests", "host_mock.c"), "-lpthread"], check=True)
    lib = C.CDLL(so)
    lib.tbq_moe_block_host.restype = C.c_int
    lib.tbq_moe_block_host.argtypes = [C.c_void_p, C.c_int] + [C.c_void_p] * 5 + [C.c_int]
    for n in ("mock_last_alloc", "mock_last_ws"):
        getattr(lib, n).restype = C.c_void_p
    return lib


def test_moe_host_block_workspace_is_fixed_and_zeroed(host_block):
    lib = host_block
    H, F, E, k = 512, 256, 16, 4
    L = MoeLayer(H, F, E, k, 12, 0x1000, 0, 0x2000, 0x3000, 0x4000)
    allocs = 0
    for i, (T, mode) in enumerate([(5, 0), (1, 0), (16, 0), (1, 0), (40, 1), (1, 0), (3, 1), (2, 0)]):
        rng = np.random.default_rng(i)
        xn = rng.standard_normal((T, H), dtype=np.float32)
        resid = rng.standard_normal((T, H), dtype=np.float32)
        out = np.zeros((T, H), np.float32)
        idx = np.zeros((T, 8), np.int32)
        w = np.zeros((T, 8), np.float32)
        assert lib.tbq_moe_block_host(C.byref(L), T, xn.ctypes.data, resid.ctypes.data, out.ctypes.data,
                                      idx.ctypes.data, w.ctypes.data, mode) == 1
        # the workspace starts at the cached buffer's first byte, whatever T
        assert lib.mock_last_ws() == lib.mock_last_alloc(), (T, mode)
        assert lib.mock_bad_counters() == 0, f"counters not zero on entry at call {i} (T={T})"
        np.testing.assert_array_equal(out, resid + 2 * xn)
        assert (idx[:, :k] >= 0).all() and (idx[:, k:] == -1).all()
        allocs = lib.mock_allocs()
    assert lib.mock_calls() == 8
    assert allocs >= 3   # T=5, then regrown for T=16 and for the prefill mode


def test_moe_host_block_mixed_qtypes_fall_back_to_fp32(host_block):
    """A prefill mode that does not take the layer (a Q6_K down tensor under
    Q4_K gate/up, as llama.cpp's K-quant mixes write) runs in TBQ_MOE_FP32;
    an all-Q4_K layer keeps the mode it asked for."""
    lib = host_block
    H, F, E, k, T = 512, 256, 16, 4, 3
    xn = np.ones((T, H), np.float32)
    resid = np.zeros((T, H), np.float32)
    out = np.zeros((T, H), np.float32)
    idx = np.zeros((T, 8), np.int32)
    w = np.zeros((T, 8), np.float32)
    for qts, mode, ran in [((0, 0, 14), 1, 0), ((0, 0, 0), 1, 1), ((11, 11, 12), 2, 0), ((12, 12, 12), 2, 2),
                           ((0, 0, 14), 0, 0)]:
        L = MoeLayer(H, F, E, k, 12, 0x1000, 0, 0x2000, 0x3000, 0x4000, *qts)
        assert lib.tbq_moe_block_host(C.byref(L), T, xn.ctypes.data, resid.ctypes.data, out.ctypes.data,
                                      idx.ctypes.data, w.ctypes.data, mode) == 1
        assert lib.mock_last_mode() == ran, (qts, mode)


def _run_forced(code):
    env = dict(os.environ, TBQ_FORCE_NO_DEVICE="1")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, cwd=ROOT, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


def test_forced_no_device_fallback_contract():
    out = _run_forced(
        "import ctypes as C, numpy as np\n"
        "import trailblaze_amd as tb\n"
        "L = tb.lib()\n"
        "assert L.tb_cuda_init() == 0\n"
        "assert L.tbq_init() == 0\n"
        "assert b'TBQ_FORCE_NO_DEVICE' in L.tbq_last_error()\n"
        "buf = np.arange(4096, dtype=np.uint8)\n"
        "assert not L.tb_cuda_upload_tensor(buf.ctypes.data, buf.nbytes)\n"
        "x = np.ones(256, np.float32); y = np.zeros(4, np.float32)\n"
        "assert L.tb_cuda_matvec_device(C.c_void_p(0x1000), 12, 4, 256, x.ctypes.data, y.ctypes.data) == 0\n"
        "assert L.tb_cuda_matvec_device(C.c_void_p(0x1000), 21, 4, 256, x.ctypes.data, y.ctypes.data) == 0\n"
        "assert L.tb_cuda_matvec_device(None, 12, 4, 256, x.ctypes.data, y.ctypes.data) == 0\n"
        "assert L.tb_cuda_upload_x(x.ctypes.data, 256) == 0\n"
        "L.tb_cuda_sync_all(); L.tb_cuda_cleanup()\n"
        "assert not L.tbq_malloc(64)\n"
        "print('forced fallback ok')\n")
    assert "forced fallback ok" in out


needs_ref = pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "layer4")),
                               reason="reference sources not present on this host")


@needs_ref
def test_reference_links_against_libtbq_and_falls_back_on_cpu():
    tb.lib()   # libtbq.so is built
    odir = os.path.join(ROOT, "oracle")
    r = subprocess.run(["make", "-s", "-C", odir, f"REF={REF}", "ref-tbcuda"], capture_output=True, text=True,
                       timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert os.path.exists(os.path.join(odir, "_ref", "tb_infer_tbq"))
    env = dict(os.environ, TBQ_FORCE_NO_DEVICE="1")
    r = subprocess.run([os.path.join(odir, "_ref", "ref_fallback")], env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("bit-identical") == 3 and "PASS" in r.stdout, r.stdout
