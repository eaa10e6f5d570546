"""Writes GGUF v2/v3 files for the loader tests (test infrastructure).

Layout per the GGUF specification: magic "GGUF", version (u32), tensor and
metadata counts (u64), metadata (key string, value type u32, value), tensor
infos (name, n_dims u32, dims u64 in ggml order, ggml type u32, offset u64
from the data section), padding to the alignment, then each tensor's bytes
at its offset (each offset a multiple of the alignment).
"""
from __future__ import annotations

import struct

import numpy as np

GT = dict(u8=0, i8=1, u16=2, i16=3, u32=4, i32=5, f32=6, bool=7, str=8, arr=9, u64=10, i64=11, f64=12)
_FMT = dict(u8="<B", i8="<b", u16="<H", i16="<h", u32="<I", i32="<i", f32="<f", bool="<?", u64="<Q", i64="<q",
            f64="<d")


def _s(b) -> bytes:
    b = b.encode() if isinstance(b, str) else bytes(b)
    return struct.pack("<Q", len(b)) + b


def _scalar(t: str, v) -> bytes:
    return _s(v) if t == "str" else struct.pack(_FMT[t], v)


def gguf_bytes(kv, tensors, alignment=None, version=3) -> bytes:
    """kv: [(key, type, value)] with type a GT name, or (key, "arr",
    (elem type, [values])); tensors: [(name, qtype, dims, uint8 array)]."""
    items = list(kv) + ([("general.alignment", "u32", alignment)] if alignment is not None else [])
    out = bytearray(b"GGUF") + struct.pack("<IQQ", version, len(tensors), len(items))
    for key, typ, val in items:
        out += _s(key) + struct.pack("<I", GT[typ])
        if typ == "arr":
            et, vals = val
            out += struct.pack("<IQ", GT[et], len(vals)) + b"".join(_scalar(et, v) for v in vals)
        else:
            out += _scalar(typ, val)
    align = alignment or 32
    blobs = [np.ascontiguousarray(data).view(np.uint8).tobytes() for _, _, _, data in tensors]
    offs, off = [], 0
    for b in blobs:
        off = (off + align - 1) // align * align
        offs.append(off)
        off += len(b)
    for (name, qt, dims, _), o in zip(tensors, offs):
        out += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", qt, o)
    out += b"\0" * ((-len(out)) % align)
    base = len(out)
    for b, o in zip(blobs, offs):
        out += b"\0" * (base + o - len(out))
        out += b
    return bytes(out)


def write_gguf(path, kv, tensors, alignment=None, version=3):
    with open(path, "wb") as f:
        f.write(gguf_bytes(kv, tensors, alignment, version))


def dense_gguf_tensors(cfg, host, arch="qwen3"):
    """Metadata and tensors of a dense model from SyntheticDense's host copy:
    the fused q|k|v and gate|up matrices split back into the separate GGUF
    tensors (rows are contiguous, so the split is by rows)."""
    from trailblaze_amd import formats as fm
    c = cfg
    D, NQ, NKV = c.head_dim, c.n_heads, c.n_kv_heads
    kv = [("general.architecture", "str", arch), (f"{arch}.block_count", "u32", c.n_layers),
          (f"{arch}.embedding_length", "u32", c.hidden), (f"{arch}.attention.head_count", "u32", NQ),
          (f"{arch}.attention.head_count_kv", "u32", NKV), (f"{arch}.attention.key_length", "u32", D),
          (f"{arch}.feed_forward_length", "u32", c.ffn), (f"{arch}.context_length", "u32", c.max_ctx),
          (f"{arch}.attention.layer_norm_rms_epsilon", "f32", c.norm_eps),
          (f"{arch}.rope.freq_base", "f32", c.rope_theta),
          ("tokenizer.ggml.tokens", "arr", ("str", [f"t{i}" for i in range(8)]))]
    f32 = lambda a: np.asarray(a, np.float32)
    c_embd = c.qtype_embd & 0xFF   # a file holds plain ggml ids, whatever layout reads it
    ts = [("token_embd.weight", c_embd, (c.hidden, c.vocab), host["lm_head"]),
          ("output_norm.weight", fm.F32, (c.hidden,), f32(host["output_norm"]))]
    for l, t in enumerate(host["layers"]):
        qt = lambda name: t.get("qt_" + name, c.qtype_layers) & 0xFF
        if "wqkv" in t:
            qkv = t["wqkv"]
            q, k, v = qkv[:NQ * D], qkv[NQ * D:(NQ + NKV) * D], qkv[(NQ + NKV) * D:]
            qq = qk = qv = qt("wqkv")
        else:
            q, k, v, qq, qk, qv = t["wq"], t["wk"], t["wv"], qt("wq"), qt("wk"), qt("wv")
        if "wgu" in t:
            gate, up, qg, qu = t["wgu"][:c.ffn], t["wgu"][c.ffn:], qt("wgu"), qt("wgu")
        else:
            gate, up, qg, qu = t["wgate"], t["wup"], qt("wgate"), qt("wup")
        p = f"blk.{l}."
        ts += [(p + "attn_norm.weight", fm.F32, (c.hidden,), f32(t["attn_norm"])),
               (p + "attn_q.weight", qq, (c.hidden, NQ * D), q),
               (p + "attn_k.weight", qk, (c.hidden, NKV * D), k),
               (p + "attn_v.weight", qv, (c.hidden, NKV * D), v),
               (p + "attn_q_norm.weight", fm.F32, (D,), f32(t["q_norm"])),
               (p + "attn_k_norm.weight", fm.F32, (D,), f32(t["k_norm"])),
               (p + "attn_output.weight", qt("wo"), (NQ * D, c.hidden), t["wo"]),
               (p + "ffn_norm.weight", fm.F32, (c.hidden,), f32(t["ffn_norm"])),
               (p + "ffn_gate.weight", qg, (c.hidden, c.ffn), gate),
               (p + "ffn_up.weight", qu, (c.hidden, c.ffn), up),
               (p + "ffn_down.weight", qt("wdown"), (c.ffn, c.hidden), t["wdown"])]
    return kv, ts
