"""GGUF file to HBM through libtbq's loader (include/tbq_gguf.h).

``GgufFile`` wraps the C handle: metadata and tensor-table lookups, the
mapped bytes of a tensor, upload of every tensor, and the assembly of a
dense model (for ``tbq_dense_decode``) or a MoE layer (for
``tbq_moe_forward``) from the file.  The handle owns every device buffer it
creates; they are freed by ``close()``.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import MoeLayer, TbqError, _check, _ptr, _stream, lib


class GgufFile:
    def __init__(self, path: str):
        self.h = lib().tbq_gguf_open(str(path).encode())
        if not self.h:
            raise TbqError(f"tbq_gguf_open failed: {lib().tbq_last_error().decode()}")
        self.path = str(path)
        self._models = []

    def close(self):
        if self.h:
            lib().tbq_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- tensor table ---------------------------------------------------
    def names(self):
        return [lib().tbq_gguf_tensor_name(self.h, i).decode() for i in range(lib().tbq_gguf_n_tensors(self.h))]

    def index(self, name: str) -> int:
        i = lib().tbq_gguf_find(self.h, name.encode())
        if i < 0:
            raise KeyError(name)
        return i

    def info(self, name: str):
        """(qtype, dims in ggml order, bytes)."""
        qt, nd = C.c_int(), C.c_int()
        dims = (C.c_longlong * 4)()
        nb = C.c_size_t()
        _check(lib().tbq_gguf_tensor_info(self.h, self.index(name), C.byref(qt), C.byref(nd), dims, C.byref(nb)),
               "tbq_gguf_tensor_info")
        return qt.value, tuple(dims[:nd.value]), nb.value

    def host_bytes(self, name: str) -> np.ndarray:
        """A copy of the tensor's bytes in the file."""
        _, _, nb = self.info(name)
        p = lib().tbq_gguf_tensor_host(self.h, self.index(name))
        if not p:
            raise TbqError(f"tensor {name} has no known size")
        return np.ctypeslib.as_array((C.c_uint8 * nb).from_address(p)).copy()

    def device_ptr(self, name: str) -> int:
        return lib().tbq_gguf_tensor_device(self.h, self.index(name)) or 0

    # ---- metadata -------------------------------------------------------
    def get_int(self, key: str) -> int:
        v = C.c_longlong()
        _check(lib().tbq_gguf_get_int(self.h, key.encode(), C.byref(v)), "tbq_gguf_get_int")
        return v.value

    def get_float(self, key: str) -> float:
        v = C.c_double()
        _check(lib().tbq_gguf_get_float(self.h, key.encode(), C.byref(v)), "tbq_gguf_get_float")
        return v.value

    def get_str(self, key: str) -> str:
        buf = C.create_string_buffer(1024)
        _check(lib().tbq_gguf_get_str(self.h, key.encode(), buf, len(buf)), "tbq_gguf_get_str")
        return buf.value.decode()

    def set_layout(self, layout: int) -> None:
        """0 = the reference's block layouts (default), formats.GGML = ggml's:
        the qtypes of models and layers assembled afterwards carry the flag."""
        _check(lib().tbq_gguf_set_layout(self.h, layout), "tbq_gguf_set_layout")

    # ---- device residency ------------------------------------------------
    def upload_all(self) -> int:
        n = lib().tbq_gguf_upload_all(self.h)
        _check(n >= 0, "tbq_gguf_upload_all")
        return n

    def dense_model(self, max_ctx: int):
        """(DenseModel, workspace tensor) assembled from the file."""
        import torch
        from .dense import DenseLayer, DenseModel
        arch = self.get_str("general.architecture")
        n = self.get_int(f"{arch}.block_count")
        layers = (DenseLayer * n)()
        m = DenseModel()
        _check(lib().tbq_gguf_dense_model(self.h, max_ctx, C.byref(m), layers, n), "tbq_gguf_dense_model")
        ws = torch.empty(int(lib().tbq_dense_workspace_size(C.byref(m))), dtype=torch.uint8, device="cuda")
        self._models.append((m, layers, ws))
        return m, ws

    def moe_layer(self, layer: int) -> MoeLayer:
        L = MoeLayer()
        _check(lib().tbq_gguf_moe_layer(self.h, layer, C.byref(L)), "tbq_gguf_moe_layer")
        L._keep = (self,)
        return L


def dense_decode(m, ws, token: int, pos: int, logits, stream=None):
    """tbq_dense_decode on a model from ``GgufFile.dense_model``."""
    _check(lib().tbq_dense_decode(C.byref(m), token, pos, _ptr(logits), _ptr(ws), ws.numel(), _stream(stream)),
           "tbq_dense_decode")
    return logits


def dense_prefill(m, tokens, pos0: int, logits, stream=None):
    """tbq_dense_prefill on a model from ``GgufFile.dense_model``: the last
    token's logits; the workspace is allocated per call."""
    import numpy as np
    import torch
    toks = np.ascontiguousarray(tokens, dtype=np.int32)
    n = int(lib().tbq_dense_prefill_workspace_size(C.byref(m), len(toks)))
    _check(n > 0, "tbq_dense_prefill_workspace_size")
    ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    _check(lib().tbq_dense_prefill(C.byref(m), toks.ctypes.data, len(toks), pos0, _ptr(logits), _ptr(ws), n,
                                   _stream(stream)), "tbq_dense_prefill")
    torch.cuda.synchronize()   # the token copy has run before `toks` goes away
    return logits

