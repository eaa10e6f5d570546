"""Dense Qwen3-style decode on libtbq (tbq_dense_decode, include/tbq.h).

``DenseModel``/``DenseLayer`` mirror the C structs; ``SyntheticDense`` builds a
random-init model of a given shape on the device (the seeded recipe of
``synth``: K-quant blocks with fp16(U(1e-3, 1e-2)) scale fields, fp32 norm
weights around 1) and keeps the host copies of small models for the tests.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _check, _ptr, _stream, formats as fm, lib, synth

_vp, _i, _f = C.c_void_p, C.c_int, C.c_float


class DenseLayer(C.Structure):
    _fields_ = [("attn_norm", _vp), ("q_norm", _vp), ("k_norm", _vp), ("ffn_norm", _vp),
                ("wqkv", _vp), ("wo", _vp), ("wgu", _vp), ("wdown", _vp),
                ("wq", _vp), ("wk", _vp), ("wv", _vp), ("wgate", _vp), ("wup", _vp),
                ("qt_qkv", _i), ("qt_o", _i), ("qt_gu", _i), ("qt_down", _i), ("qt_q", _i), ("qt_k", _i),
                ("qt_v", _i), ("qt_gate", _i), ("qt_up", _i)]


class DenseModel(C.Structure):
    _fields_ = [("n_layers", _i), ("hidden", _i), ("n_heads", _i), ("n_kv_heads", _i), ("head_dim", _i),
                ("ffn", _i), ("vocab", _i), ("max_ctx", _i), ("norm_eps", _f), ("rope_theta", _f),
                ("qtype_layers", _i), ("qtype_embd", _i), ("tok_embd", _vp), ("lm_head", _vp),
                ("output_norm", _vp), ("layers", C.POINTER(DenseLayer)), ("k_cache", _vp), ("v_cache", _vp)]


@dataclass
class DenseConfig:
    n_layers: int
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    max_ctx: int
    norm_eps: float = 1e-6
    rope_theta: float = 1e6
    qtype_layers: int = fm.Q4_K
    qtype_embd: int = fm.Q6_K


# Qwen3-4B shape, context 4096
QWEN3_4B = DenseConfig(n_layers=36, hidden=2560, n_heads=32, n_kv_heads=8, head_dim=128, ffn=9728,
                       vocab=151936, max_ctx=4096)


class SyntheticDense:
    """A random-init model on the device.  keep_host=True also keeps every
    tensor on the host (``self.host``) for the oracle."""

    def __init__(self, cfg: DenseConfig, seed: int, keep_host: bool = False):
        import torch
        self.cfg = c = cfg
        rng = np.random.default_rng(seed)
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
        QR = (c.n_heads + 2 * c.n_kv_heads) * c.head_dim
        norm = lambda n: (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        self.host = {"layers": []} if keep_host else None
        self._keep = []
        layers = (DenseLayer * c.n_layers)()
        for l in range(c.n_layers):
            t = {"attn_norm": norm(c.hidden), "q_norm": norm(c.head_dim), "k_norm": norm(c.head_dim),
                 "ffn_norm": norm(c.hidden),
                 "wqkv": synth.kquant_matrix(c.qtype_layers, QR, c.hidden, rng),
                 "wo": synth.kquant_matrix(c.qtype_layers, c.hidden, c.n_heads * c.head_dim, rng),
                 "wgu": synth.kquant_matrix(c.qtype_layers, 2 * c.ffn, c.hidden, rng),
                 "wdown": synth.kquant_matrix(c.qtype_layers, c.hidden, c.ffn, rng)}
            d = {k: dev(v) for k, v in t.items()}
            self._keep.append(d)
            for k, v in d.items():
                setattr(layers[l], k, v.data_ptr())
            if keep_host:
                self.host["layers"].append(t)
        lm = synth.kquant_matrix(c.qtype_embd, c.vocab, c.hidden, rng)
        on = norm(c.hidden)
        self.lm_head = dev(lm)
        self.output_norm = dev(on)
        if keep_host:
            self.host["lm_head"] = lm
            self.host["output_norm"] = on
        del lm
        kv = (c.n_layers, c.n_kv_heads, c.max_ctx, c.head_dim)
        self.k_cache = torch.zeros(kv, dtype=torch.float32, device="cuda")
        self.v_cache = torch.zeros(kv, dtype=torch.float32, device="cuda")
        self.layers = layers
        self.model = DenseModel(c.n_layers, c.hidden, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn, c.vocab,
                                c.max_ctx, c.norm_eps, c.rope_theta, c.qtype_layers, c.qtype_embd,
                                self.lm_head.data_ptr(), self.lm_head.data_ptr(), self.output_norm.data_ptr(),
                                layers, self.k_cache.data_ptr(), self.v_cache.data_ptr())
        ws = int(lib().tbq_dense_workspace_size(C.byref(self.model)))
        _check(ws > 0, "tbq_dense_workspace_size")
        self.workspace = torch.empty(ws, dtype=torch.uint8, device="cuda")

    def decode(self, token: int, pos: int, logits, stream=None):
        """logits[vocab] (device fp32) for `token` at `pos`; appends K/V at pos."""
        _check(lib().tbq_dense_decode(C.byref(self.model), token, pos, _ptr(logits), _ptr(self.workspace),
                                      self.workspace.numel(), _stream(stream)), "tbq_dense_decode")
        return logits

    def prefill(self, tokens, pos0: int, logits, stream=None):
        """tbq_dense_prefill of `tokens` at positions pos0.. : the last
        token's logits into `logits`, K/V of every position appended."""
        import torch
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        n = int(lib().tbq_dense_prefill_workspace_size(C.byref(self.model), len(toks)))
        ws = getattr(self, "_pf_ws", None)
        if n > 0 and (ws is None or ws.numel() < n):
            ws = self._pf_ws = torch.empty(n, dtype=torch.uint8, device="cuda")
        self._pf_tokens = toks   # read by an asynchronous copy on the stream
        # (n == 0: bad arguments, which the call itself reports)
        _check(lib().tbq_dense_prefill(C.byref(self.model), toks.ctypes.data, len(toks), pos0, _ptr(logits),
                                       _ptr(ws), 0 if ws is None else ws.numel(), _stream(stream)),
               "tbq_dense_prefill")
        return logits

    def prefill_batched(self) -> bool:
        return bool(lib().tbq_dense_prefill_batched(C.byref(self.model)))

    def matvec_shapes(self):
        """(qtype, M, K, weight tensor) of every matvec one decode step runs."""
        c = self.cfg
        QR = (c.n_heads + 2 * c.n_kv_heads) * c.head_dim
        out = []
        for d in self._keep:
            out += [(c.qtype_layers, QR, c.hidden, d["wqkv"]),
                    (c.qtype_layers, c.hidden, c.n_heads * c.head_dim, d["wo"]),
                    (c.qtype_layers, 2 * c.ffn, c.hidden, d["wgu"]),
                    (c.qtype_layers, c.hidden, c.ffn, d["wdown"])]
        out.append((c.qtype_embd, c.vocab, c.hidden, self.lm_head))
        return out
