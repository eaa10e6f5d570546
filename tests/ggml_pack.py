"""Block packer for ggml's own on-disk layouts (test infrastructure).

Written from the block struct descriptions of ggml-common.h (field order,
widths and which bits of which byte hold which weight), not from its
dequantize loops: each format gives, for every weight index e of a block,
the byte and bit position of each of its fields, and the packer scatters
random integers to those positions with numpy.  values() gives each weight's
closed-form value from the same integers, rounded one operation at a time
in float32, so a decoder that reads any bit from the wrong place fails.

Field positions per weight e of a 256-weight block (n = e // 128 the half,
k = (e % 128) // 32 the 2-bit slot, l = e % 32):
  Q4_K  qs[32*(e//64) + l], nibble (e//32) % 2; sub-block j = e//32 has a
        6-bit scale and min: j < 4 in the low 6 bits of scales[j] and
        scales[j+4]; j >= 4 their low 4 bits in the low / high nibble of
        scales[j+4] and their top 2 bits in bits 6-7 of scales[j-4] / scales[j]
  Q5_K  Q4_K's, plus the 5th bit in bit e//32 of qh[l]
  Q6_K  low 4 bits: ql[64n + (e%128)%64], nibble (e%128)//64; top 2 bits:
        bits 2k of qh[32n + l]; int8 scale scales[e//16]
  Q3_K  low 2 bits: bits 2k of qs[32n + l]; 3rd bit: bit e//32 of hmask[l];
        6-bit scale i = e//16: low 4 bits in nibble i//8 of scales[i%8], top
        2 bits in bits 2*(i//4) of scales[8 + i%4]; value (q - 4)(s - 32)
  Q2_K  2 bits as Q3_K's low bits; scales[e//16]: scale low nibble, min high
  Q4_0  (32 weights) qs[e % 16], nibble e // 16
Byte offsets: Q4_K d 0, dmin 2, scales 4, qs 16; Q5_K qh 16, qs 48; Q6_K ql
0, qh 128, scales 192, d 208; Q3_K hmask 0, qs 32, scales 96, d 108; Q2_K
scales 0, qs 16, d 80, dmin 82; Q4_0 / Q8_0 d 0, qs 2.
"""
from __future__ import annotations

import numpy as np

GEOM = {"q4_0": (32, 18), "q8_0": (32, 34), "q2_k": (256, 84), "q3_k": (256, 110), "q4_k": (256, 144),
        "q5_k": (256, 176), "q6_k": (256, 210)}
QTYPE = {"q4_0": 2, "q8_0": 8, "q2_k": 10, "q3_k": 11, "q4_k": 12, "q5_k": 13, "q6_k": 14}
QBITS = {"q4_0": 4, "q8_0": 8, "q2_k": 2, "q3_k": 3, "q4_k": 4, "q5_k": 5, "q6_k": 6}


def _halves(rng, n, subnormal_frac=0.1):
    """fp16 bit patterns: mostly normal values of moderate size, some
    subnormals (which ggml decodes as IEEE)."""
    v = rng.uniform(1e-3, 1e-2, n).astype(np.float16).view(np.uint16)
    sub = rng.random(n) < subnormal_frac
    v[sub] = rng.integers(1, 1024, int(sub.sum()), dtype=np.uint16)   # exponent 0
    return v


def random_fields(fmt: str, nb: int, rng) -> dict:
    """Random integer fields of nb blocks."""
    bw, _ = GEOM[fmt]
    f = {"q": rng.integers(0, 1 << QBITS[fmt], (nb, bw)).astype(np.int64), "d": _halves(rng, nb)}
    if fmt == "q8_0":
        f["q"] = rng.integers(-128, 128, (nb, bw)).astype(np.int64)
    if fmt in ("q4_k", "q5_k"):
        f["sc"] = rng.integers(0, 64, (nb, 8))
        f["mn"] = rng.integers(0, 64, (nb, 8))
        f["dmin"] = _halves(rng, nb)
    elif fmt == "q2_k":
        f["sc"] = rng.integers(0, 16, (nb, 16))
        f["mn"] = rng.integers(0, 16, (nb, 16))
        f["dmin"] = _halves(rng, nb)
    elif fmt == "q3_k":
        f["sc"] = rng.integers(0, 64, (nb, 16))
    elif fmt == "q6_k":
        f["sc"] = rng.integers(-128, 128, (nb, 16))
    return f


def _put_bits(blk, byte_idx, shift, vals):
    """OR vals << shift into blk[:, byte_idx] (byte_idx, shift per weight)."""
    nb = blk.shape[0]
    rows = np.repeat(np.arange(nb), byte_idx.size).reshape(nb, -1)
    cols = np.broadcast_to(byte_idx, (nb, byte_idx.size))
    np.bitwise_or.at(blk, (rows, cols), (vals << shift).astype(np.uint8))


def _half_bytes(blk, off, h):
    blk[:, off:off + 2] = h.astype("<u2").view(np.uint8).reshape(-1, 2)


def pack(fmt: str, f: dict) -> np.ndarray:
    """[nb, block bytes] uint8 blocks holding the fields f."""
    bw, bb = GEOM[fmt]
    q = f["q"]
    nb = q.shape[0]
    blk = np.zeros((nb, bb), np.uint8)
    e = np.arange(bw)
    n, k, l = e // 128, (e % 128) // 32, e % 32
    if fmt == "q4_0":
        _half_bytes(blk, 0, f["d"])
        _put_bits(blk, 2 + e % 16, 4 * (e // 16), q)
    elif fmt == "q8_0":
        _half_bytes(blk, 0, f["d"])
        blk[:, 2:34] = q.astype(np.int8).view(np.uint8)
    elif fmt in ("q4_k", "q5_k"):
        _half_bytes(blk, 0, f["d"])
        _half_bytes(blk, 2, f["dmin"])
        qs0 = 16 if fmt == "q4_k" else 48
        _put_bits(blk, qs0 + 32 * (e // 64) + l, 4 * ((e // 32) % 2), q & 15)
        if fmt == "q5_k":
            _put_bits(blk, 16 + l, e // 32, q >> 4)
        sc, mn = f["sc"], f["mn"]
        j = np.arange(4)
        _put_bits(blk, 4 + j, 0, sc[:, :4])                  # scales 0-3
        _put_bits(blk, 4 + j + 4, 0, mn[:, :4])              # mins 0-3
        _put_bits(blk, 4 + j + 8, 0, sc[:, 4:] & 15)         # scales 4-7, low 4 bits
        _put_bits(blk, 4 + j + 8, 4, mn[:, 4:] & 15)         # mins 4-7, low 4 bits
        _put_bits(blk, 4 + j, 6, sc[:, 4:] >> 4)             # scales 4-7, top 2 bits
        _put_bits(blk, 4 + j + 4, 6, mn[:, 4:] >> 4)         # mins 4-7, top 2 bits
    elif fmt == "q6_k":
        _put_bits(blk, 64 * n + (e % 128) % 64, 4 * ((e % 128) // 64), q & 15)
        _put_bits(blk, 128 + 32 * n + l, 2 * k, q >> 4)
        blk[:, 192:208] = f["sc"].astype(np.int8).view(np.uint8)
        _half_bytes(blk, 208, f["d"])
    elif fmt == "q3_k":
        _put_bits(blk, 32 + 32 * n + l, 2 * k, q & 3)
        _put_bits(blk, l, e // 32, q >> 2)
        i = np.arange(16)
        _put_bits(blk, 96 + i % 8, 4 * (i // 8), f["sc"] & 15)
        _put_bits(blk, 96 + 8 + i % 4, 2 * (i // 4), f["sc"] >> 4)
        _half_bytes(blk, 108, f["d"])
    elif fmt == "q2_k":
        _put_bits(blk, 16 + 32 * n + l, 2 * k, q)
        blk[:, :16] = (f["sc"] | (f["mn"] << 4)).astype(np.uint8)
        _half_bytes(blk, 80, f["d"])
        _half_bytes(blk, 82, f["dmin"])
    return blk


def values(fmt: str, f: dict) -> np.ndarray:
    """[nb, block weights] float32: each weight's value from the fields."""
    f32 = np.float32
    half = lambda h: h.astype(np.uint16).view(np.float16).astype(f32)[:, None]
    q = f["q"].astype(f32)
    d = half(f["d"])
    bw = GEOM[fmt][0]
    if fmt == "q4_0":
        return (q - f32(8)) * d
    if fmt == "q8_0":
        return q * d
    if fmt in ("q4_k", "q5_k", "q2_k"):
        grp = 32 if fmt != "q2_k" else 16
        s = np.repeat(f["sc"], grp, axis=1).astype(f32)
        m = np.repeat(f["mn"], grp, axis=1).astype(f32)
        return (d * s) * q - half(f["dmin"]) * m
    if fmt == "q3_k":
        s = np.repeat(f["sc"] - 32, 16, axis=1).astype(f32)
        return (d * s) * (q - f32(4))
    if fmt == "q6_k":
        s = np.repeat(f["sc"], 16, axis=1).astype(f32)
        return (d * s) * (q - f32(32))
    raise ValueError(fmt)
