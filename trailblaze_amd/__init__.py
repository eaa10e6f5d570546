"""trailblaze_amd -- MI355X (gfx950) K-quant dequant-matvec and MoE block for
Trailblaze, behind the reference's C call surface.

The product is the shared library ``libtbq.so`` (HIP kernels + C-ABI shim +
C11 host layer, headers in include/).  This package only loads it and offers
thin Python entry points over the same C functions, taking torch tensors as
device-memory handles and torch's current stream as the HIP stream.  There is
no CPU fallback: if the library is missing or the device refuses a call, the
call raises.
"""
from __future__ import annotations

import ctypes as C
import os

from . import formats
from .formats import row_bytes

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtbq.so")

TBQ_MOE_FP32 = 0
TBQ_MOE_BF16 = 1
TBQ_MOE_I8 = 2
TBQ_MV_AUTO, TBQ_MV_FMA, TBQ_MV_INTDOT, TBQ_MV_KQ = 0, 1, 2, 3

# (name, restype, argtypes) for every symbol declared in include/tbq.h,
# include/tbq_gguf.h and include/tb_gguf_dequant.h.
_vp, _i, _sz, _f = C.c_void_p, C.c_int, C.c_size_t, C.c_float
SYMBOLS = {
    # include/tbq.h
    "tbq_init": (_i, []),
    "tbq_last_error": (C.c_char_p, []),
    "tbq_device_name": (C.c_char_p, []),
    "tbq_cu_count": (_i, []),
    "tbq_malloc": (_vp, [_sz]),
    "tbq_free": (_i, [_vp]),
    "tbq_memcpy_h2d": (_i, [_vp, _vp, _sz, _vp]),
    "tbq_memcpy_d2h": (_i, [_vp, _vp, _sz, _vp]),
    "tbq_stream_sync": (_i, [_vp]),
    "tbq_device_sync": (_i, []),
    "tbq_row_bytes": (_sz, [_i, _i]),
    "tbq_qtype_supported": (_i, [_i]),
    "tbq_dequant": (_i, [_vp, _i, _i, _i, _vp, _vp]),
    "tbq_matvec": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp]),
    "tbq_matvec_variant": (_i, [_vp, _i, _i, _i, _vp, _vp, _i, _vp]),
    "tbq_route": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp]),
    "tbq_moe_workspace_size": (_sz, [_vp, _i, _i]),
    "tbq_moe_mode_supported": (_i, [_vp, _i]),
    "tbq_moe_forward": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i, _vp]),
    "tbq_moe_block_host": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _i]),
    "tbq_moe_forward_noalloc": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _i, _vp]),
    "tbq_dense_workspace_size": (_sz, [_vp]),
    "tbq_dense_decode": (_i, [_vp, _i, _i, _vp, _vp, _sz, _vp]),
    "tbq_dense_prefill_workspace_size": (_sz, [_vp, _i]),
    "tbq_dense_prefill": (_i, [_vp, _vp, _i, _i, _vp, _vp, _sz, _vp]),
    "tbq_dense_prefill_batched": (_i, [_vp]),
    "tbq_quantize_q8k": (_i, [_vp, C.c_longlong, _vp, _vp]),
    "tbq_gemm_workspace_size": (_sz, [_i, _i, _i]),
    "tbq_gemm": (_i, [_i, _vp, _vp, _i, _i, _i, _vp, _i, _vp, _sz, _vp]),
    "tbq_expf_device": (_i, [_vp, _vp, _sz, _vp]),
    "tbq_expf_host": (_f, [_f]),
    # include/tbq_gguf.h
    "tbq_gguf_open": (_vp, [C.c_char_p]),
    "tbq_gguf_close": (None, [_vp]),
    "tbq_gguf_n_tensors": (_i, [_vp]),
    "tbq_gguf_find": (_i, [_vp, C.c_char_p]),
    "tbq_gguf_tensor_name": (C.c_char_p, [_vp, _i]),
    "tbq_gguf_tensor_info": (_i, [_vp, _i, _vp, _vp, _vp, _vp]),
    "tbq_gguf_tensor_host": (_vp, [_vp, _i]),
    "tbq_gguf_get_int": (_i, [_vp, C.c_char_p, _vp]),
    "tbq_gguf_get_float": (_i, [_vp, C.c_char_p, _vp]),
    "tbq_gguf_get_str": (_i, [_vp, C.c_char_p, _vp, _sz]),
    "tbq_gguf_upload_all": (_i, [_vp]),
    "tbq_gguf_tensor_device": (_vp, [_vp, _i]),
    "tbq_gguf_dense_model": (_i, [_vp, _i, _vp, _vp, _i]),
    "tbq_gguf_moe_layer": (_i, [_vp, _i, _vp]),
    "tbq_gguf_set_layout": (_i, [_vp, _i]),
    # include/tb_gguf_dequant.h (the reference ABI)
    "tb_cuda_init": (_i, []),
    "tb_cuda_upload_tensor": (_vp, [_vp, _sz]),
    "tb_cuda_free_tensor": (None, [_vp]),
    "tb_cuda_upload_x": (_i, [_vp, _i]),
    "tb_cuda_set_snap": (None, [_vp]),
    "tb_cuda_matvec_device": (_i, [_vp, _i, _i, _i, _vp, _vp]),
    "tb_cuda_sync_all": (None, []),
    "tb_cuda_cleanup": (None, []),
}


class TbqError(RuntimeError):
    pass


class MoeLayer(C.Structure):
    """Mirror of ``tbq_moe_layer`` (include/tbq.h)."""
    _fields_ = [("H", C.c_int), ("F", C.c_int), ("E", C.c_int), ("top_k", C.c_int), ("qtype", C.c_int),
                ("router", C.c_void_p), ("bias", C.c_void_p), ("gate", C.c_void_p), ("up", C.c_void_p),
                ("down", C.c_void_p), ("qt_gate", C.c_int), ("qt_up", C.c_int), ("qt_down", C.c_int)]


_lib = None


def lib():
    """Load libtbq.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise TbqError(f"{LIB_PATH} is missing: build it with `python -m trailblaze_amd.build`")
        # torch ships its own libamdhip64.so.7; loading torch first makes
        # libtbq bind to that same HIP runtime (one runtime per process, so
        # torch's device pointers and streams are valid in libtbq)
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SYMBOLS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(ok, what):
    if not ok:
        raise TbqError(f"{what} failed: {lib().tbq_last_error().decode()}")


def init() -> str:
    _check(lib().tbq_init(), "tbq_init")
    return lib().tbq_device_name().decode()


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(stream=None):
    import torch
    s = torch.cuda.current_stream() if stream is None else stream
    return C.c_void_p(s.cuda_stream)


def dequant(W, qtype: int, nrows: int, K: int, out, stream=None):
    """out[nrows*K] (fp32 device tensor) = bit-exact dequantised weights."""
    _check(lib().tbq_dequant(_ptr(W), qtype, nrows, K, _ptr(out), _stream(stream)), "tbq_dequant")
    return out


def matvec(W, qtype: int, M: int, K: int, x, y, stream=None, variant: int = TBQ_MV_AUTO):
    """y[M] = dequant(W) . x on the device (all arguments device tensors)."""
    _check(lib().tbq_matvec_variant(_ptr(W), qtype, M, K, _ptr(x), _ptr(y), variant, _stream(stream)),
           "tbq_matvec")
    return y


def route(xn, router, bias, T, H, E, top_k, sel_idx, sel_w, stream=None):
    _check(lib().tbq_route(_ptr(xn), _ptr(router), _ptr(bias), T, H, E, top_k, _ptr(sel_idx), _ptr(sel_w),
                           _stream(stream)), "tbq_route")


def moe_layer(H, F, E, top_k, qtype, router, gate, up, down, bias=None, qt_gate=0, qt_up=0,
              qt_down=0) -> MoeLayer:
    """A ``tbq_moe_layer`` over device tensors; qt_gate/qt_up/qt_down give a
    tensor its own qtype (0 = qtype)."""
    L = MoeLayer(H, F, E, top_k, qtype, router.data_ptr(), 0 if bias is None else bias.data_ptr(),
                 gate.data_ptr(), up.data_ptr(), down.data_ptr(), qt_gate, qt_up, qt_down)
    L._keep = (router, gate, up, down, bias)   # keep the tensors alive
    return L


def moe_mode_supported(L: MoeLayer, mode: int) -> bool:
    """Whether tbq_moe_forward takes layer L in ``mode``."""
    return bool(lib().tbq_moe_mode_supported(C.byref(L), mode))


def moe_workspace_size(L: MoeLayer, T: int, mode: int = TBQ_MOE_FP32) -> int:
    return int(lib().tbq_moe_workspace_size(C.byref(L), T, mode))


def moe_forward(L: MoeLayer, T, xn, resid, out, sel_idx=None, sel_w=None, workspace=None,
                mode: int = TBQ_MOE_FP32, stream=None):
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _check(lib().tbq_moe_forward(C.byref(L), T, _ptr(xn), _ptr(resid), _ptr(out), _ptr(sel_idx), _ptr(sel_w),
                                 _ptr(workspace), ws_bytes, mode, _stream(stream)), "tbq_moe_forward")
    return out


def moe_forward_noalloc(L: MoeLayer, T, xn, resid, out, sel_idx=None, sel_w=None, mode: int = TBQ_MOE_FP32,
                        stream=None):
    """tbq_moe_forward with the library's static per-GPU workspace (no
    allocation anywhere on the call's path)."""
    _check(lib().tbq_moe_forward_noalloc(C.byref(L), T, _ptr(xn), _ptr(resid), _ptr(out), _ptr(sel_idx),
                                         _ptr(sel_w), mode, _stream(stream)), "tbq_moe_forward_noalloc")
    return out


def gemm(W, wqt: int, X16, T: int, N: int, K: int, C_out, ldc: int = 0, workspace=None, stream=None):
    """C_out[T][ldc or N] = X16[T][K] . W[N][K]^T with the batched prefill's
    GEMM (W fp16 halves, wqt = 1, or Q4_K rows, wqt = 12)."""
    import torch
    if workspace is None:
        nb = int(lib().tbq_gemm_workspace_size(T, N, K))
        workspace = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda") if nb else None
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _check(lib().tbq_gemm(wqt, _ptr(W), _ptr(X16), T, N, K, _ptr(C_out), ldc or N, _ptr(workspace), ws_bytes,
                          _stream(stream)), "tbq_gemm")
    return C_out


def expf_device(x, out, stream=None):
    _check(lib().tbq_expf_device(_ptr(x), _ptr(out), x.numel(), _stream(stream)), "tbq_expf_device")
    return out


__all__ = ["formats", "row_bytes", "lib", "init", "dequant", "matvec", "route", "moe_layer", "moe_forward",
           "moe_forward_noalloc", "moe_workspace_size", "moe_mode_supported", "gemm", "expf_device", "MoeLayer", "TbqError", "SYMBOLS", "TBQ_MOE_FP32", "TBQ_MOE_BF16",
           "TBQ_MOE_I8"]
