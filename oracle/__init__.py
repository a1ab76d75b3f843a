"""CPU parity oracle for the quantized DiT linear path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
package, and only to check the product's results (or, for the baseline, as the timed CPU restatement).  The product
package never imports it.

The arithmetic lives in ``hn_oracle.c`` (compiled by ``oracle/build.py`` into ``liboracle.so``).  This
module converts numpy / torch CPU arrays to the C calling convention.  All inputs are float32 arrays
holding the exact values of the bf16 tensors; outputs are float32 before the final bf16 cast, which the
caller performs with torch (round to nearest even, the same rule as the device store).

Reference functions restated (reference-tree file:line):
  quantize          hy_nomas/kernels.py:22-54, hy_nomas/ops.py:41-52
  dequantize_g128   hy_nomas/ops.py:55-62
  block_gemm        hy_nomas/kernels.py:80-170
  adaln/adaln_quant hy_nomas/fused.py:37-62, hy_nomas/kernels.py:173-207
  gated_residual    hy_nomas/fused.py:108-128
  qk_norm_rope      hy_nomas/fused.py:65-105
  pixelumm_qk       hy_nomas/fused.py:131-186
  fp8 weight blocks hy_nomas/pixelumm.py:60-82
  dequant_linear    hy_nomas/ops.py:167-176 (the reference's CPU fallback: dequantize + F.linear)
  swiglu            hy_nomas/pixelumm.py:314-323 (the decoder MLP's silu(gate) * up on bf16 tensors)
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

KIND = {"int8": 0, "fp8": 1}
ROUND = {"half_away": 0, "half_even": 1}
EPILOGUE = {None: 0, "gelu": 1, "gelu_quant": 2}
NORM = {"layer": 0, "rms": 1}

_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i64 = ctypes.c_int64


def lib():
    """Load liboracle.so, building it from hn_oracle.c if it is not there yet."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        from . import build
        build.build()
    l = ctypes.CDLL(LIB_PATH)
    l.hno_quantize.argtypes = [ctypes.c_void_p, _i64, _i64, _i64, _i64, ctypes.c_int, ctypes.c_int,
                               ctypes.c_void_p, ctypes.c_void_p]
    l.hno_block_gemm.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                 ctypes.c_void_p, _i64, _i64, _i64, _i64, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    l.hno_adaln.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, _i64, _i64, _i64, ctypes.c_float,
                            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                            ctypes.c_void_p]
    l.hno_gated_residual.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, _i64, _i64, _i64,
                                     ctypes.c_void_p]
    l.hno_qk_norm_rope.argtypes = [ctypes.c_void_p, _i64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                   _i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
    l.hno_pixelumm_qk.argtypes = [ctypes.c_void_p, _i64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                  ctypes.c_void_p, _i64, _i64, _i64, ctypes.c_float, ctypes.c_void_p]
    l.hno_e4m3_encode.argtypes = [ctypes.c_float]
    l.hno_e4m3_encode.restype = ctypes.c_uint8
    l.hno_e4m3_encode_array.argtypes = [ctypes.c_void_p, _i64, ctypes.c_void_p]
    l.hno_e4m3_decode.argtypes = [ctypes.c_uint8]
    l.hno_e4m3_decode.restype = ctypes.c_float
    l.hno_gelu_tanh.argtypes = [ctypes.c_float]
    l.hno_gelu_tanh.restype = ctypes.c_float
    l.hno_silu.argtypes = [ctypes.c_float]
    l.hno_silu.restype = ctypes.c_float
    l.hno_swiglu.argtypes = [ctypes.c_void_p, ctypes.c_void_p, _i64, ctypes.c_void_p]
    l.hno_check_fast_division.argtypes = [ctypes.c_int, _i64, _i64]
    l.hno_check_fast_division.restype = ctypes.c_int64
    l.hno_check_fast_division2.argtypes = [_i64, _i64, ctypes.c_int]
    l.hno_check_fast_division2.restype = ctypes.c_int64
    l.hno_check_scale_division.argtypes = []
    l.hno_check_scale_division.restype = ctypes.c_int64
    l.hno_check_reciprocal_refinement.argtypes = []
    l.hno_check_reciprocal_refinement.restype = ctypes.c_int64
    _lib = l
    return l


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def to_f32(t):
    """torch tensor (any dtype, CPU or device) or array -> contiguous float32 numpy array."""
    if hasattr(t, "detach"):
        return np.ascontiguousarray(t.detach().float().cpu().numpy())
    return _f32(t)


def rbf16(a):
    """fp32 -> nearest bf16 (ties to even), kept as fp32 (hy_nomas/kernels.py:67-71)."""
    a = _f32(a)
    b = a.view(np.uint32).astype(np.uint64)
    b = (b + (((b >> 16) & 1) + 0x7FFF)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32)


def e4m3_encode(a):
    """fp32 -> OCP e4m3fn code bits, round to nearest even, overflow to the NaN code 0x7F."""
    return e4m3_encode_fast(a)


def e4m3_decode_table():
    l = lib()
    return np.array([l.hno_e4m3_decode(i) for i in range(256)], dtype=np.float32)


def quantize(x, group=128, kind="int8", rounding="half_away"):
    """x [M, K] -> (codes [M, K] int8 or uint8 e4m3 bits, scales [M, K / group] fp32)."""
    x = to_f32(x)
    m, k = x.shape
    if group is None:
        group = k
    assert k % group == 0
    q = np.empty((m, k), dtype=np.int8 if kind == "int8" else np.uint8)
    s = np.empty((m, k // group), dtype=np.float32)
    lib().hno_quantize(_p(x), k, m, k, group, KIND[kind], ROUND[rounding], _p(q), _p(s))
    return q, s


def quantize_kv(x):
    """hy_nomas/world.py:83-90: x [L, H, D] -> (int8 [L, H, D], fp32 [L, H, 1]), one group per (token, head)."""
    x = to_f32(x)
    l, h, d = x.shape
    q, s = quantize(x.reshape(l * h, d), d)
    return q.reshape(l, h, d), s.reshape(l, h, 1)


def dequantize_kv(q, s):
    """hy_nomas/world.py:93-94 to bf16: fp32 product of code and scale, rounded once, then to bf16."""
    return rbf16(np.asarray(q, dtype=np.float32) * _f32(s))


def quantize_g128(w):
    """hy_nomas/ops.py:41-52 weight quantization (K padded up to a multiple of 128 with zeros)."""
    w = to_f32(w)
    n, k = w.shape
    groups = (k + 127) // 128
    padded = np.zeros((n, groups * 128), dtype=np.float32)
    padded[:, :k] = w
    q, s = quantize(padded, 128, "int8", "half_away")
    return np.ascontiguousarray(q[:, :k]), s


def dequantize_g128(q, s):
    """hy_nomas/ops.py:55-62: fp32 product of code and group scale (before the cast to the model dtype)."""
    q = np.asarray(q)
    n, k = q.shape
    rep = np.repeat(np.asarray(s, dtype=np.float32), 128, axis=1)[:, :k]
    return q.astype(np.float32) * rep


def block_gemm(qa, sa, qw, sw, bias=None, kind="int8", epilogue=None, want_acc32=False):
    """hy_nomas/kernels.py:80-170.  Returns out fp32 [M, N] (pre-cast), or (codes, qs, h) for gelu_quant;
    with want_acc32 also the full-K int32 dot products."""
    qa = np.ascontiguousarray(qa)
    qw = np.ascontiguousarray(qw)
    sa = _f32(sa)
    sw = _f32(sw)
    m, k = qa.shape
    n = qw.shape[0]
    group = k // sa.shape[1]
    assert sw.shape[1] == sa.shape[1]
    b = _f32(bias) if bias is not None else None
    out = np.empty((m, n), dtype=np.float32)
    qout = np.empty((m, n), dtype=np.int8) if epilogue == "gelu_quant" else None
    qs = np.empty((m, n // 128), dtype=np.float32) if epilogue == "gelu_quant" else None
    acc = np.empty((m, n), dtype=np.int32) if want_acc32 else None
    lib().hno_block_gemm(_p(qa), _p(sa), _p(qw), _p(sw), _p(b), m, n, k, group, KIND[kind], EPILOGUE[epilogue],
                         _p(out), _p(qout), _p(qs), _p(acc))
    res = (qout, qs, out) if epilogue == "gelu_quant" else out
    return (res, acc) if want_acc32 else res


def swiglu(g, u):
    """h = rbf16(rbf16(silu(g)) * u) for bf16-valued g, u (hy_nomas/pixelumm.py:322): the down_proj input of
    the decoder MLP.  Returns fp32 arrays holding bf16 values."""
    g = _f32(g)
    u = _f32(u)
    assert g.shape == u.shape
    h = np.empty_like(g)
    lib().hno_swiglu(_p(g), _p(u), g.size, _p(h))
    return h


def swiglu_quant(g, u, kind="fp8"):
    """The swiglu product quantized per row and 128 columns, as the down projection's activation
    quantizer does (pixelumm.py:152 -> kernels.py:22-54): (codes, scales, h)."""
    h = swiglu(g, u)
    q, s = quantize(h, 128, kind)
    return q, s, h


def adaln(x, shift, scale, eps=1e-6, norm="layer", quant=False, rounding="half_away"):
    """x [B, L, D], shift/scale [B, D] -> y fp32 [B*L, D] (pre-cast), or (q, s, y) with quant."""
    x = to_f32(x)
    b, l, d = x.shape
    shift = to_f32(shift)
    scale = to_f32(scale)
    y = np.empty((b * l, d), dtype=np.float32)
    q = np.empty((b * l, d), dtype=np.int8) if quant else None
    s = np.empty((b * l, d // 128), dtype=np.float32) if quant else None
    lib().hno_adaln(_p(x), _p(shift), _p(scale), b, l, d, eps, NORM[norm], int(quant), ROUND[rounding],
                    _p(y), _p(q), _p(s))
    return (q, s, y) if quant else y


def gated_residual(x, y, gate):
    x = to_f32(x)
    b, l, d = x.shape
    y = to_f32(y)
    gate = to_f32(gate)
    out = np.empty((b, l, d), dtype=np.float32)
    lib().hno_gated_residual(_p(x), _p(y), _p(gate), b, l, d, _p(out))
    return out


def qk_norm_rope(x, weight, rope=None, eps=1e-6):
    """x [B, L, H, D] -> fp32 [B, L, H, D] before the bf16 cast."""
    x = to_f32(x)
    b, l, h, d = x.shape
    w = to_f32(weight)
    if rope is not None:
        c, s = to_f32(rope[0]), to_f32(rope[1])
    else:
        c = s = np.zeros((1, d), dtype=np.float32)
    out = np.empty((b, l, h, d), dtype=np.float32)
    lib().hno_qk_norm_rope(_p(x), h * d, _p(w), _p(c), _p(s), b, l, h, d, eps, int(rope is not None), _p(out))
    return out


def pixelumm_qk(x, weight_t, weight_hw, cos, sin, eps=1e-6):
    """x [1, N, H, D] -> fp32 [1, N, H, D] before the bf16 cast."""
    x = to_f32(x)
    _, n, h, d = x.shape
    out = np.empty((1, n, h, d), dtype=np.float32)
    lib().hno_pixelumm_qk(_p(x), h * d, _p(to_f32(weight_t)), _p(to_f32(weight_hw)), _p(to_f32(cos)),
                          _p(to_f32(sin)), n, h, d, eps, _p(out))
    return out


def fp8_block_quantize(w):
    """hy_nomas/pixelumm.py:77-82: e4m3 codes with one fp32 scale per 128x128 block (absmax clamped at 1e-4)."""
    w = to_f32(w)
    n, k = w.shape
    blocks = w.reshape(n // 128, 128, k // 128, 128)
    s = (np.maximum(np.abs(blocks).max(axis=(1, 3)), np.float32(1e-4)) / np.float32(448.0)).astype(np.float32)
    q = e4m3_encode_fast(blocks / s[:, None, :, None]).reshape(n, k)
    return q, s


def e4m3_encode_fast(a):
    """Array form of hno_e4m3_encode (one C call for the whole array)."""
    a = _f32(a)
    out = np.empty(a.shape, dtype=np.uint8)
    lib().hno_e4m3_encode_array(_p(a), a.size, _p(out))
    return out


def dequantize_fp8_block(q, s):
    """hy_nomas/pixelumm.py:60-63, fp32 (before the cast to the model dtype)."""
    table = e4m3_decode_table()
    n, k = q.shape
    w = table[np.asarray(q, dtype=np.uint8)].reshape(n // 128, 128, k // 128, 128) * s[:, None, :, None]
    return w.reshape(n, k).astype(np.float32)


def dequant_linear(x, qw, sw, bias=None):
    """The reference's CPU fallback (hy_nomas/ops.py:172-176 with ops.py:55-62 and kernels.py:216-218):
    dequantize the int8 g128 weight to the activation dtype and run F.linear.  torch CPU tensors in/out."""
    import torch
    n, k = qw.shape
    w = (qw.view(n, k // 128, 128).float() * sw.float().unsqueeze(-1)).view(n, k).to(x.dtype)
    return torch.nn.functional.linear(x, w, bias)
