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
