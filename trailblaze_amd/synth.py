"""Seeded synthetic inputs for the benchmark configurations.

One generator (numpy PCG64, ``numpy.random.default_rng(seed)``) produces every
value of a configuration.  K-quant blocks are uniform random bytes with their
fp16 scale fields overwritten by fp16(U(1e-3, 1e-2)) (round-to-nearest-even),
so every 6-bit scale/min, every quant and every Q6_K int8 scale is uniform.
Q8_K blocks get an f32 scale U(1e-3, 1e-2).  Activations are fp32 N(0, 1).
"""
from __future__ import annotations

import numpy as np

from . import formats as fm


def kquant_matrix(qtype: int, M: int, K: int, rng: np.random.Generator) -> np.ndarray:
    """[M, row_bytes] uint8 matrix of random blocks (random quant and scale
    bytes, fp16 scale fields in [1e-3, 1e-2]); the fields sit at the same
    offsets in the reference's layouts and ggml's, so it serves both."""
    bw, bb = fm.GEOMETRY[qtype]
    qtype = fm.base(qtype)
    if qtype in (fm.F32, fm.F16, fm.BF16):
        if qtype == fm.F32:
            return rng.standard_normal((M, K), dtype=np.float32).view(np.uint8).reshape(M, K * 4)
        v = rng.standard_normal((M, K), dtype=np.float32)
        if qtype == fm.F16:
            return v.astype(np.float16).view(np.uint8).reshape(M, K * 2)
        return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(M, K * 2)
    nb = M * (K // bw)
    blocks = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    if qtype == fm.Q8_K:
        d = rng.uniform(1e-3, 1e-2, size=nb).astype(np.float32)
        blocks[:, 0:4] = d.view(np.uint8).reshape(nb, 4)
    else:
        for off in fm.SCALE_FIELDS[qtype]:
            d = rng.uniform(1e-3, 1e-2, size=nb).astype(np.float16)
            blocks[:, off:off + 2] = d.view(np.uint8).reshape(nb, 2)
    return blocks.reshape(M, (K // bw) * bb)


def activations(shape, rng: np.random.Generator) -> np.ndarray:
    return rng.standard_normal(shape, dtype=np.float32)


def router_weights(E: int, H: int, rng: np.random.Generator) -> np.ndarray:
    return (rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)


def zipf_router_bias(E: int, s: float, c: float, rng: np.random.Generator) -> np.ndarray:
    """Per-expert logit bias c*ln(p_r(e)) with p_r proportional to r^-s over a
    seeded rank permutation r(e) (rank 1 = most loaded)."""
    ranks = rng.permutation(E) + 1
    p = ranks.astype(np.float64) ** (-s)
    p /= p.sum()
    return (c * np.log(p)).astype(np.float32)


def moe_layer(H: int, F: int, E: int, qtype: int, seed: int, qt_gate: int = 0, qt_up: int = 0, qt_down: int = 0):
    """Expert tensors in the reference's packed layout: gate/up [E*F rows, H],
    down [E*H rows, F] (layer4/tb_infer.c:780-806), plus the fp32 router.
    qt_gate/qt_up/qt_down give a tensor its own format (0 = qtype)."""
    rng = np.random.default_rng(seed)
    router = router_weights(E, H, rng)
    gate = kquant_matrix(qt_gate or qtype, E * F, H, rng)
    up = kquant_matrix(qt_up or qtype, E * F, H, rng)
    down = kquant_matrix(qt_down or qtype, E * H, F, rng)
    return router, gate, up, down
