"""ctypes binding of libhynomas_hip.so (the gfx950 kernels behind include/hynomas.h).

The library is loaded lazily on first use, after torch (whose HIP runtime it binds to).  There is no
fallback: if the library is missing or a call fails, a RuntimeError says why.
"""
import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libhynomas_hip.so")

# enums of include/hynomas.h
DTYPE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
KIND = {"int8": 0, "fp8": 1}
ROUND = {"half_away": 0, "half_even": 1}
EPI_ACC32 = 3
NORM = {"layer": 0, "rms": 1}

_lib = None
_lock = threading.Lock()

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i = ctypes.c_int
_f = ctypes.c_float

SIGNATURES = {
    "hn_version": ([], _i),
    "hn_last_error": ([], ctypes.c_char_p),
    "hn_quantize_act": ([_p, _i, _i64, _i64, _i64, _i64, _i, _i, _p, _i64, _p, _i64, _p], _i),
    "hn_block_gemm": ([_p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _p, _i, _i64, _i64, _i64, _i64, _i, _i, _p, _i,
                       _i64, _p, _i64, _p], _i),
    "hn_block_linear_workspace_bytes": ([_i64, _i64, _i64], _i64),
    "hn_block_linear": ([_p, _i, _i64, _i64, _i64, _i64, _i, _i, _p, _i64, _p, _i64, _i64, _p, _i, _i64, _p, _i, _i64,
                         _p, _i64, _p], _i),
    "hn_block_linear_noalloc": ([_p, _i, _i64, _i64, _i64, _i64, _i, _i, _p, _i64, _p, _i64, _i64, _p, _i, _i64, _p,
                                 _i, _i64, _p], _i),
    "hn_attention": ([_p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64,
                      _i64, _i64, _i64, _i64, _f, _p], _i),
    "hn_adaln": ([_p, _p, _p, _i, _i64, _i64, _i64, _f, _i, _p, _p], _i),
    "hn_adaln_quant": ([_p, _p, _p, _i, _i64, _i64, _i64, _f, _i, _i, _i64, _p, _p, _p], _i),
    "hn_gated_residual": ([_p, _p, _p, _i, _i64, _i64, _i64, _p, _p], _i),
    "hn_gated_residual_frames": ([_p, _p, _p, _p, _i, _i64, _i64, _i64, _i64, _p, _p], _i),
    "hn_qkv_heads": ([_p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _p, _i, _i64, _i64, _i64, _i64, _i64, _i, _p, _p,
                      _p, _p, _f, _p, _i64, _i64, _p], _i),
    "hn_qkv_heads_vt": ([_p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _p, _i, _i64, _i64, _i64, _i64, _i64, _i, _p,
                         _p, _p, _p, _f, _p, _i64, _i64, _p, _i64, _i64, _i64, _p], _i),
    "hn_dequantize_rows": ([_p, _i64, _p, _i64, _i64, _i64, _p, _i, _i64, _p], _i),
    "hn_qk_norm_rope": ([_p, _i64, _p, _p, _p, _i64, _i64, _i64, _i64, _f, _p, _p], _i),
    "hn_pixelumm_qk": ([_p, _i64, _p, _p, _p, _p, _i64, _i64, _i64, _f, _p, _p], _i),
}


def lib():
    """The loaded library (raises RuntimeError if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(f"Hy-Nomas HIP kernels are not built ({LIB_PATH} missing); run "
                                   "`python comfyui-hy-nomas_amd/build.py` or __graft_entry__.build()")
            l = ctypes.CDLL(LIB_PATH)
            for name, (args, res) in SIGNATURES.items():
                fn = getattr(l, name)
                fn.argtypes = args
                fn.restype = res
            _lib = l
    return _lib


def call(name, *args):
    """Call an entry point; a non-zero status raises RuntimeError with the library's message."""
    l = lib()
    rc = getattr(l, name)(*args)
    if rc != 0:
        msg = l.hn_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (status {rc}): {msg}")


def require_device(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("Hy-Nomas HIP kernels take device tensors; got a tensor on " + str(t.device))


def stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t):
    return t.data_ptr() if t is not None else None


def dtype_code(t):
    try:
        return DTYPE[t.dtype]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {t.dtype}") from None
