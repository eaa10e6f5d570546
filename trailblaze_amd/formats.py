"""GGUF block formats on the hot path (ggml type ids as used by the reference,
layer4/tb_gguf.h:24 and the geometry table layer4/tb_gguf.c:380-394)."""
from __future__ import annotations

F32, F16, Q4_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K, BF16 = 0, 1, 2, 8, 10, 11, 12, 13, 14, 15, 30

NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K",
         Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", Q8_K: "Q8_K", BF16: "BF16"}
BY_NAME = {v: k for k, v in NAMES.items()}

# qtype -> (weights per block, bytes per block)
GEOMETRY = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q8_0: (32, 34),
            Q2_K: (256, 84), Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176),
            Q6_K: (256, 210), Q8_K: (256, 292)}

# Byte offsets of the fp16 scale fields inside one block (d first, then dmin).
SCALE_FIELDS = {Q4_0: (0,), Q8_0: (0,), Q2_K: (80, 82), Q3_K: (108,), Q4_K: (0, 2),
                Q5_K: (0, 2), Q6_K: (208,)}

KQUANTS = (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0)

# GGML | id: ggml's own on-disk layout of the format (TBQ_GGML in
# include/tbq.h).  Same geometry and field offsets; the quant bits, 6-bit
# scales and fp16 fields are read as ggml reads them.  F32, BF16 and Q8_K
# read the same in both layouts.
GGML = 0x100
for _q in list(GEOMETRY):
    GEOMETRY[GGML | _q] = GEOMETRY[_q]
    NAMES[GGML | _q] = "ggml " + NAMES[_q]
for _q in list(SCALE_FIELDS):
    SCALE_FIELDS[GGML | _q] = SCALE_FIELDS[_q]
GGML_FORMATS = tuple(GGML | q for q in (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, Q4_0, F16))


def base(qtype: int) -> int:
    """The ggml type id of a qtype (the layout flag removed)."""
    return qtype & 0xFF


def row_bytes(qtype: int, K: int) -> int:
    bw, bb = GEOMETRY[qtype]
    return (K + bw - 1) // bw * bb


def weight_bytes(qtype: int, M: int, K: int) -> int:
    return M * row_bytes(qtype, K)
