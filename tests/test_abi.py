"""CPU checks of the boundary: libtbq.so loads without a GPU, exports every
function that include/*.h declares (and nothing in SYMBOLS is undeclared),
and the host-compiled copy of the router's expf equals glibc's expf on all
2^32 inputs."""
import ctypes as C
import os
import re
import subprocess

import pytest

import trailblaze_amd as tb

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not h.endswith(".h"):
            continue
        src = open(os.path.join(ROOT, "include", h)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(t(?:bq|b_cuda)_\w+)\s*\(", src, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    lib = tb.lib()
    decl = declared_functions()
    assert len(decl) >= 42
    assert decl == set(tb.SYMBOLS), decl ^ set(tb.SYMBOLS)
    out = subprocess.run(["nm", "-D", "--defined-only", tb.LIB_PATH], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    for name in decl:
        assert name in exported, name
        getattr(lib, name)


def test_host_side_calls_without_device():
    lib = tb.lib()
    assert lib.tbq_row_bytes(12, 4096) == 16 * 144
    assert lib.tbq_row_bytes(14, 4096) == 16 * 210
    assert lib.tbq_row_bytes(8, 4096) == 128 * 34
    assert lib.tbq_row_bytes(99, 4096) == 0
    for qt in (0, 1, 2, 8, 10, 11, 12, 13, 14, 15, 30):
        assert lib.tbq_qtype_supported(qt) == 1
    assert lib.tbq_qtype_supported(21) == 0
    assert tb.formats.row_bytes(12, 768) == lib.tbq_row_bytes(12, 768)


def test_router_expf_matches_glibc_on_all_inputs(oracle):
    fn = C.cast(tb.lib().tbq_expf_host, C.c_void_p).value
    bad = oracle.lib.tbo_expf_exhaustive_mismatches(fn, os.cpu_count() or 8)
    assert bad == 0


def test_dense_prefill_workspace_host_side():
    """tbq_dense_prefill_workspace_size / _batched are host-only: which
    path a model takes (hidden <= 8192 and ffn <= 16384 batched) and that
    the batched workspace grows with the prompt while the per-token one is
    the decode workspace plus the token ids.  Fake, aligned device
    pointers: nothing is dereferenced."""
    import ctypes as C
    from trailblaze_amd.dense import DenseLayer, DenseModel
    from trailblaze_amd import formats as fm
    lib = tb.lib()
    fake = 1 << 20

    def model(hidden, ffn, n_layers=2):
        layers = (DenseLayer * n_layers)()
        for L in layers:
            for name in ("attn_norm", "q_norm", "k_norm", "ffn_norm", "wqkv", "wo", "wgu", "wdown"):
                setattr(L, name, fake)
        m = DenseModel(n_layers, hidden, 8, 2, 128, ffn, 1024, 4096, 1e-6, 1e6, fm.Q4_K, fm.Q6_K,
                       fake, fake, fake, layers, fake, fake)
        m._layers = layers
        return m

    small, wide = model(2560, 9728), model(8448, 9728)
    assert lib.tbq_dense_prefill_batched(C.byref(small)) == 1
    assert lib.tbq_dense_prefill_batched(C.byref(wide)) == 0
    dec = lib.tbq_dense_workspace_size(C.byref(small))
    w1, w2 = (lib.tbq_dense_prefill_workspace_size(C.byref(small), T) for T in (16, 512))
    assert dec > 0 and w2 > w1 > dec
    # T = 1 runs the decode step: its workspace plus the token ids
    assert dec < lib.tbq_dense_prefill_workspace_size(C.byref(small), 1) <= dec + 256
    dw = lib.tbq_dense_workspace_size(C.byref(wide))
    assert dw < lib.tbq_dense_prefill_workspace_size(C.byref(wide), 512) <= dw + 512 * 4 + 256
    assert lib.tbq_dense_prefill_workspace_size(C.byref(small), 0) == 0
