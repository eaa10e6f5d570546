"""ctypes bindings for the parity oracle (oracle/liboracle*.so) and, when it
was built, the compiled reference (oracle/_ref/libtbref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg.  The product package never imports it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_SO = os.path.join(HERE, "_ref", "libtbref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")


def host_has_avx512() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    fl = set(line.split(":", 1)[1].split())
                    need = {"avx512f", "avx512bw", "avx512dq", "avx512vl", "avx512cd", "avx512_vnni"}
                    return need <= fl
    except OSError:
        pass
    return False


def _load(path):
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} missing: run `make -C oracle` (or __graft_entry__.build())")
    return C.CDLL(path)


class Oracle:
    """The C11 restatement of the reference CPU path."""

    def __init__(self, avx512: bool | None = None):
        if avx512 is None:
            avx512 = host_has_avx512()
        name = "liboracle_avx512.so" if avx512 else "liboracle.so"
        self.path = os.path.join(HERE, name)
        L = self.lib = _load(self.path)
        L.tbo_f16_to_f32.restype = C.c_float
        L.tbo_f16_to_f32.argtypes = [C.c_uint16]
        L.tbo_bf16_to_f32.restype = C.c_float
        L.tbo_bf16_to_f32.argtypes = [C.c_uint16]
        L.tbo_f16_ieee.restype = C.c_float
        L.tbo_f16_ieee.argtypes = [C.c_uint16]
        L.tbo_row_bytes.restype = C.c_size_t
        L.tbo_row_bytes.argtypes = [C.c_int, C.c_int]
        L.tbo_dequant_row.argtypes = [_u8p, C.c_int, C.c_int, _f32p]
        L.tbo_dequant_rows.argtypes = [_u8p, C.c_int, C.c_int, C.c_int, _f32p]
        L.tbo_dequant_matvec.argtypes = [_u8p, C.c_int, C.c_int, C.c_int, _f32p, _f32p]
        L.tbo_swiglu.argtypes = [_f32p, _f32p, _f32p, C.c_int]
        L.tbo_route_experts.restype = C.c_int
        L.tbo_route_experts.argtypes = [_f32p, C.c_int, C.c_int, _i32p, _f32p]
        L.tbo_router_logits.argtypes = [C.c_int, C.c_int, C.c_int, _f32p, _f32p, C.c_void_p, _f32p]
        L.tbo_moe_forward.argtypes = [C.c_int] * 8 + [_f32p, _f32p, _f32p, C.c_void_p,
                                                      _u8p, _u8p, _u8p, _f32p, C.c_void_p, C.c_void_p]
        L.tbo_quantize_q8k.argtypes = [_f32p, C.c_int, _u8p]
        L.tbo_expf_batch.argtypes = [_f32p, _f32p, C.c_size_t]
        L.tbo_expf_exhaustive_mismatches.restype = C.c_longlong
        L.tbo_expf_exhaustive_mismatches.argtypes = [C.c_void_p, C.c_int]
        L.tbo_matvec_q4k_avx512s.argtypes = [_u8p, C.c_int, C.c_int, _f32p, _f32p]
        L.tbo_have_avx512.restype = C.c_int

    def f16(self, h: int) -> float:
        return self.lib.tbo_f16_to_f32(h)

    def f16_ieee(self, h: int) -> float:
        """ggml's fp16 decode (IEEE binary16, subnormals included)."""
        return self.lib.tbo_f16_ieee(h)

    def row_bytes(self, qtype: int, K: int) -> int:
        return int(self.lib.tbo_row_bytes(qtype, K))

    def dequant_rows(self, W: np.ndarray, qtype: int, M: int, K: int) -> np.ndarray:
        out = np.empty((M, K), np.float32)
        self.lib.tbo_dequant_rows(np.ascontiguousarray(W).reshape(-1), qtype, M, K, out.reshape(-1))
        return out

    def matvec(self, W: np.ndarray, qtype: int, M: int, K: int, x: np.ndarray) -> np.ndarray:
        out = np.empty(M, np.float32)
        self.lib.tbo_dequant_matvec(np.ascontiguousarray(W).reshape(-1), qtype, M, K,
                                    np.ascontiguousarray(x, np.float32), out)
        return out

    def swiglu(self, g: np.ndarray, u: np.ndarray) -> np.ndarray:
        out = np.empty_like(g, np.float32)
        self.lib.tbo_swiglu(np.ascontiguousarray(g, np.float32), np.ascontiguousarray(u, np.float32),
                            out, g.size)
        return out

    def route(self, logits: np.ndarray, top_k: int):
        idx = np.zeros(8, np.int32)
        w = np.zeros(8, np.float32)
        k = self.lib.tbo_route_experts(np.ascontiguousarray(logits, np.float32), logits.size, top_k, idx, w)
        return idx[:k].copy(), w[:k].copy()

    def router_logits(self, xn, router, bias=None):
        T, H = xn.shape
        E = router.shape[0]
        out = np.empty((T, E), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self.lib.tbo_router_logits(T, H, E, np.ascontiguousarray(xn, np.float32).reshape(-1),
                                   np.ascontiguousarray(router, np.float32).reshape(-1),
                                   None if b is None else b.ctypes.data, out.reshape(-1))
        return out

    def moe(self, xn, resid, router, gate, up, down, *, F, top_k, qtype, bias=None, qt_gate=0, qt_up=0,
            qt_down=0):
        """The MoE block per token; qt_gate/qt_up/qt_down give a tensor its
        own qtype (0 = qtype)."""
        T, H = xn.shape
        E = router.shape[0]
        out = np.empty((T, H), np.float32)
        idx = np.empty((T, 8), np.int32)
        w = np.empty((T, 8), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self.lib.tbo_moe_forward(T, H, F, E, top_k, qt_gate or qtype, qt_up or qtype, qt_down or qtype,
                                 np.ascontiguousarray(xn, np.float32).reshape(-1),
                                 np.ascontiguousarray(resid, np.float32).reshape(-1),
                                 np.ascontiguousarray(router, np.float32).reshape(-1),
                                 None if b is None else b.ctypes.data,
                                 np.ascontiguousarray(gate).reshape(-1), np.ascontiguousarray(up).reshape(-1),
                                 np.ascontiguousarray(down).reshape(-1), out.reshape(-1),
                                 idx.ctypes.data, w.ctypes.data)
        return out, idx, w

    def quantize_q8k(self, x: np.ndarray) -> np.ndarray:
        K = x.size
        out = np.zeros(K // 256 * 292, np.uint8)
        self.lib.tbo_quantize_q8k(np.ascontiguousarray(x, np.float32).reshape(-1), K, out)
        return out

    def expf(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        self.lib.tbo_expf_batch(x.reshape(-1), out.reshape(-1), x.size)
        return out

    def matvec_q4k_avx512s(self, W, M, K, x):
        out = np.empty(M, np.float32)
        self.lib.tbo_matvec_q4k_avx512s(np.ascontiguousarray(W).reshape(-1), M, K,
                                        np.ascontiguousarray(x, np.float32), out)
        return out


class Reference:
    """The reference's own C sources compiled by oracle/Makefile (`make ref`)."""

    @staticmethod
    def available() -> bool:
        return os.path.exists(REF_SO)

    def __init__(self):
        L = self.lib = _load(REF_SO)
        L.tb_gguf_dequant_row.argtypes = [_u8p, C.c_int, C.c_int, _f32p]
        L.tb_gguf_dequant_matvec.argtypes = [_u8p, C.c_int, C.c_int, C.c_int, _f32p, _f32p]
        L.tbref_route.restype = C.c_int
        L.tbref_route.argtypes = [_f32p, C.c_int, C.c_int, _i32p, _f32p]
        L.tbref_swiglu.argtypes = [_f32p, _f32p, _f32p, C.c_int]
        L.tbref_dispatch_matvec_avx512.argtypes = [_u8p, C.c_int, C.c_int, C.c_int, _f32p, _f32p]
        L.tbref_moe_block.argtypes = [C.c_int] * 8 + [_f32p, _f32p, _f32p, _u8p, _u8p, _u8p, _f32p]

    def dequant_rows(self, W, qtype, M, K, row_bytes):
        out = np.empty((M, K), np.float32)
        Wf = np.ascontiguousarray(W).reshape(-1)
        for m in range(M):
            o = np.empty(K, np.float32)
            self.lib.tb_gguf_dequant_row(np.ascontiguousarray(Wf[m * row_bytes:(m + 1) * row_bytes]), qtype, K, o)
            out[m] = o
        return out

    def matvec(self, W, qtype, M, K, x):
        out = np.empty(M, np.float32)
        self.lib.tb_gguf_dequant_matvec(np.ascontiguousarray(W).reshape(-1), qtype, M, K,
                                        np.ascontiguousarray(x, np.float32), out)
        return out

    def dispatch_matvec_avx512(self, W, qtype, M, K, x):
        out = np.empty(M, np.float32)
        self.lib.tbref_dispatch_matvec_avx512(np.ascontiguousarray(W).reshape(-1), qtype, M, K,
                                              np.ascontiguousarray(x, np.float32), out)
        return out

    def moe_block(self, xn, resid, router, gate, up, down, *, F, top_k, qtype, qt_gate=0, qt_up=0, qt_down=0):
        """The reference's MoE branch (layer4/tb_infer.c:753-833,876) composed
        of its own functions, per token (no router bias); each expert tensor
        in its own qtype (0 = qtype)."""
        T, H = xn.shape
        E = router.shape[0]
        out = np.empty((T, H), np.float32)
        self.lib.tbref_moe_block(T, H, F, E, top_k, qt_gate or qtype, qt_up or qtype, qt_down or qtype,
                                 np.ascontiguousarray(xn, np.float32).reshape(-1),
                                 np.ascontiguousarray(resid, np.float32).reshape(-1),
                                 np.ascontiguousarray(router, np.float32).reshape(-1),
                                 np.ascontiguousarray(gate).reshape(-1), np.ascontiguousarray(up).reshape(-1),
                                 np.ascontiguousarray(down).reshape(-1), out.reshape(-1))
        return out

    def route(self, logits, top_k):
        idx = np.zeros(8, np.int32)
        w = np.zeros(8, np.float32)
        k = self.lib.tbref_route(np.ascontiguousarray(logits, np.float32), logits.size, top_k, idx, w)
        return idx[:k].copy(), w[:k].copy()

    def swiglu(self, g, u):
        out = np.empty_like(g, np.float32)
        self.lib.tbref_swiglu(np.ascontiguousarray(g, np.float32), np.ascontiguousarray(u, np.float32),
                              out, g.size)
        return out
