"""CPU tests of libtbq's GGUF loader (include/tbq_gguf.h): metadata of every
GGUF value type, the tensor table and each tensor's bytes for every format
libtbq knows (and an unknown one), both alignments and GGUF versions 2 and
3, and rejection of malformed files (bad magic or version, truncation at
every point of the header, a tensor past the end, a bad alignment)."""
import numpy as np
import pytest

import trailblaze_amd as tb
from gguf_write import gguf_bytes, write_gguf
from trailblaze_amd import formats as fm
from trailblaze_amd import synth
from trailblaze_amd.gguf import GgufFile

KV = [("general.architecture", "str", "testarch"), ("a.u8", "u8", 200), ("a.i8", "i8", -5), ("a.u16", "u16", 65000),
      ("a.i16", "i16", -30000), ("a.u32", "u32", 4000000000), ("a.i32", "i32", -2000000000), ("a.f32", "f32", 0.25),
      ("a.bool", "bool", True), ("a.arr_u32", "arr", ("u32", [1, 2, 3])),
      ("a.arr_str", "arr", ("str", ["x", "yy", "zzz"])), ("a.u64", "u64", 2 ** 40 + 3), ("a.i64", "i64", -2 ** 40),
      ("a.f64", "f64", -1.5e-7), ("a.after_arrays", "str", "still parsed")]


def sample_tensors(rng):
    ts = [("f32", fm.F32, (12, 3), rng.standard_normal(36).astype(np.float32)),
          ("f16", fm.F16, (64,), rng.standard_normal(64).astype(np.float16)),
          ("bf16", fm.BF16, (32, 2), rng.integers(0, 2 ** 16, 64, dtype=np.uint16))]
    for qt in (fm.Q4_0, fm.Q8_0, fm.Q2_K, fm.Q3_K, fm.Q4_K, fm.Q5_K, fm.Q6_K, fm.Q8_K):
        K = 512 if fm.GEOMETRY[qt][0] == 256 else 128
        ts.append((f"q{qt}", qt, (K, 3), synth.kquant_matrix(qt, 3, K, rng)))
    ts.append(("unknown", 16, (256, 2), rng.integers(0, 256, 132, dtype=np.uint8)))   # a type libtbq does not know
    return ts


@pytest.mark.parametrize("alignment,version", [(None, 3), (64, 3), (None, 2)])
def test_gguf_parse(tmp_path, alignment, version):
    rng = np.random.default_rng(7)
    ts = sample_tensors(rng)
    path = tmp_path / "m.gguf"
    write_gguf(path, KV, ts, alignment=alignment, version=version)
    with GgufFile(path) as g:
        assert g.names() == [t[0] for t in ts]
        assert g.get_str("general.architecture") == "testarch"
        assert g.get_int("a.u8") == 200 and g.get_int("a.i8") == -5
        assert g.get_int("a.u16") == 65000 and g.get_int("a.i16") == -30000
        assert g.get_int("a.u32") == 4000000000 and g.get_int("a.i32") == -2000000000
        assert g.get_int("a.u64") == 2 ** 40 + 3 and g.get_int("a.i64") == -2 ** 40
        assert g.get_int("a.bool") == 1
        assert g.get_float("a.f32") == 0.25 and g.get_float("a.f64") == -1.5e-7
        assert g.get_float("a.u32") == 4000000000.0
        assert g.get_str("a.after_arrays") == "still parsed"
        if alignment:
            assert g.get_int("general.alignment") == alignment
        for key, getter in (("a.missing", g.get_int), ("a.f32", g.get_int), ("a.u8", g.get_str),
                            ("a.arr_u32", g.get_float)):
            with pytest.raises(tb.TbqError):
                getter(key)
        for name, qt, dims, data in ts:
            q, d, nb = g.info(name)
            assert (q, d) == (qt, dims), name
            raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
            if name == "unknown":
                assert nb == 0
                with pytest.raises(tb.TbqError):
                    g.host_bytes(name)
                continue
            assert nb == raw.size == tb.lib().tbq_row_bytes(qt, dims[0]) * int(np.prod(dims[1:])), name
            assert np.array_equal(g.host_bytes(name), raw), name
            assert g.device_ptr(name) == 0   # nothing uploaded
        with pytest.raises(KeyError):
            g.index("nope")


def test_gguf_rejects_malformed(tmp_path):
    rng = np.random.default_rng(8)
    ts = sample_tensors(rng)[:4]
    good = gguf_bytes(KV[:3], ts)
    p = tmp_path / "bad.gguf"

    def rejects(data, what):
        p.write_bytes(data)
        with pytest.raises(tb.TbqError, match=what):
            GgufFile(p)

    rejects(b"GGUX" + good[4:], "magic")
    rejects(good[:4] + (1).to_bytes(4, "little") + good[8:], "version")
    rejects(good[:20], "short|truncated|implausible")
    # truncation anywhere in the header or the data is reported, never read past
    hdr_end = len(gguf_bytes(KV[:3], []))
    for cut in sorted(set(np.linspace(24, len(good) - 1, 60).astype(int)) | set(range(hdr_end - 4, hdr_end + 8))):
        rejects(good[:cut], "truncated|past the end|implausible|bad header")
    # a tensor offset beyond the file
    big = gguf_bytes(KV[:3], ts[:1])
    i = big.index(b"f32") + 3 + 4 + 16 + 4   # name, n_dims, two dims, qtype -> offset
    rejects(big[:i] + (1 << 40).to_bytes(8, "little") + big[i + 8:], "past the end")
    rejects(gguf_bytes(KV[:3], ts, alignment=48), "power of two")
    with pytest.raises(tb.TbqError, match="cannot open"):
        GgufFile(tmp_path / "missing.gguf")
