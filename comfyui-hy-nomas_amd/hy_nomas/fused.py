"""Fused elementwise kernels for the DiT block (gfx950 HIP), rounding where the reference rounds.

Drop-in for the reference's `hy_nomas/fused.py` (same names and arguments):

* `adaln`: LayerNorm (fp32), `* (1 + scale)` with `1 + scale` rounded to bf16, `+ shift`, one bf16 rounding.
* `qk_norm_rope`: RMSNorm in fp32, rounded to bf16, times the bf16 weight (rounded), interleaved RoPE in
  fp32, rounded.
* `gated_residual`: `x + y * gate`, the product and the sum each rounded to bf16 (bit-exact with torch).
* `pixelumm_qk`: PixelUMM's split-half RMSNorm + sectioned rotate-half MRoPE, one bf16 rounding.

Each is one HBM pass.  `HY_NOMAS_FUSED=0` makes `available()` false so callers use torch arithmetic.
"""
import os

import torch

from . import _lib

ENABLED = os.environ.get("HY_NOMAS_FUSED", "1") != "0"


def available(x):
    return ENABLED and x.is_cuda and x.dtype == torch.bfloat16


def adaln(x, shift, scale, eps=1e-6, norm="layer"):
    """x [B, L, D] bf16, shift/scale [B, D] bf16 -> modulate(layer_norm(x), shift, scale) in bf16
    (hy_nomas/fused.py:55-62).  `norm="rms"` uses RMSNorm."""
    _lib.require_device(x, shift, scale)
    b, l, d = x.shape
    if shift.numel() != b * d or scale.numel() != b * d:
        raise RuntimeError(f"adaln: shift/scale must be [B, D] = {(b, d)}")
    x = x.contiguous()
    y = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    if b * l == 0:
        return y
    shift = shift.to(x.dtype).contiguous()
    scale = scale.to(x.dtype).contiguous()
    _lib.call("hn_adaln", x.data_ptr(), shift.data_ptr(), scale.data_ptr(), _lib.dtype_code(x), b, l, d, eps,
              _lib.NORM[norm], y.data_ptr(), _lib.stream(x))
    return y


def qk_norm_rope(x, weight, rope=None, eps=1e-6):
    """x [B, L, H, D] bf16 (rows may be strided, heads contiguous), weight [D] -> RMSNorm(x) * weight, then
    RoPE with (cos, sin) [L, D] fp32 when given.  Returns a contiguous [B, L, H, D] bf16 tensor
    (hy_nomas/fused.py:94-105)."""
    if x.dtype != torch.bfloat16:
        raise RuntimeError(f"qk_norm_rope: x must be bfloat16 (the projection output), got {x.dtype}")
    _lib.require_device(x, weight)
    b, l, h, d = x.shape
    if weight.numel() != d:
        raise RuntimeError(f"qk_norm_rope: weight must have the head dim's {d} values")
    if x.stride(3) != 1 or x.stride(2) != d or x.stride(0) != l * x.stride(1) or x.data_ptr() % 16 \
            or x.stride(1) % 8:
        x = x.contiguous()
    y = torch.empty((b, l, h, d), device=x.device, dtype=torch.bfloat16)
    if b * l * h == 0:
        return y
    w = weight.to(torch.bfloat16).float().contiguous()
    if rope is not None:
        cos, sin = rope[0].float().contiguous(), rope[1].float().contiguous()
        if tuple(cos.shape) != (l, d) or tuple(sin.shape) != (l, d):
            raise RuntimeError(f"rope tables must be [L, D] = {(l, d)}, got {tuple(cos.shape)} / {tuple(sin.shape)}")
        cp, sp = cos.data_ptr(), sin.data_ptr()
    else:
        cp = sp = None
    _lib.call("hn_qk_norm_rope", x.data_ptr(), x.stride(1), w.data_ptr(), cp, sp, b, l, h, d, eps, y.data_ptr(),
              _lib.stream(x))
    return y


def gated_residual(x, y, gate):
    """x + y * gate[:, None] with bf16 rounding of the product and the sum; x, y [B, L, D], gate [B, D]
    (hy_nomas/fused.py:121-128)."""
    _lib.require_device(x, y, gate)
    b, l, d = x.shape
    if tuple(y.shape) != (b, l, d) or gate.numel() != b * d:
        raise RuntimeError(f"gated_residual: y must be [B, L, D] = {(b, l, d)} and gate [B, D]")
    x = x.contiguous()
    y = y.contiguous()
    gate = gate.to(x.dtype).contiguous()
    out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    if b * l == 0:
        return out
    _lib.call("hn_gated_residual", x.data_ptr(), y.data_ptr(), gate.data_ptr(), _lib.dtype_code(x), b, l, d,
              out.data_ptr(), _lib.stream(x))
    return out


def gated_residual_frames(x, y, gate, frame):
    """gated_residual(x, y, gate) followed by the camera module's per-frame add in one pass
    (hy_nomas/model.py:518-520): x, y [B, T * P, D], gate [B, D], frame [B, T, D] (or [1, T, D], broadcast
    over the batch) -> (gated_residual(x, y, gate).view(B, T, P, D) + frame[:, :, None]).view(B, T * P, D),
    with the same two roundings."""
    _lib.require_device(x, y, gate, frame)
    b, l, d = x.shape
    if tuple(y.shape) != (b, l, d) or gate.numel() != b * d or frame.dim() != 3:
        raise RuntimeError(f"gated_residual_frames: y must be [B, L, D] = {(b, l, d)}, gate [B, D], frame 3-D")
    t = frame.shape[1]
    if frame.shape[0] not in (1, b) or frame.shape[2] != d or t == 0 or l % t:
        raise RuntimeError(f"gated_residual_frames: frame {tuple(frame.shape)} does not tile x {tuple(x.shape)}")
    x = x.contiguous()
    y = y.contiguous()
    gate = gate.to(x.dtype).contiguous()
    frame = frame.to(x.dtype).expand(b, t, d).contiguous()
    out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    if b * l == 0:
        return out
    _lib.call("hn_gated_residual_frames", x.data_ptr(), y.data_ptr(), gate.data_ptr(), frame.data_ptr(),
              _lib.dtype_code(x), b, t, l // t, d, out.data_ptr(), _lib.stream(x))
    return out


def pixelumm_qk(x, weight_t, weight_hw, cos, sin, eps=1e-6):
    """x [1, N, H, D] (a projection's output, heads contiguous), cos/sin [N, D] fp32 -> bf16 [1, N, H, D]
    (hy_nomas/fused.py:178-186)."""
    if x.dtype != torch.bfloat16:
        raise RuntimeError(f"pixelumm_qk: x must be bfloat16 (the projection output), got {x.dtype}")
    _lib.require_device(x, weight_t, weight_hw, cos, sin)
    b, n, h, d = x.shape
    if b != 1:
        raise RuntimeError(f"pixelumm_qk takes one sequence (x [1, N, H, D]); got batch {b}")
    if x.stride(3) != 1 or x.stride(2) != d or x.data_ptr() % 16 or x.stride(1) % 8:
        x = x.contiguous()
    y = torch.empty((b, n, h, d), device=x.device, dtype=torch.bfloat16)
    if b * n * h == 0:
        return y
    if tuple(cos.shape) != (n, d) or tuple(sin.shape) != (n, d):
        raise RuntimeError(f"cos/sin must be [N, D] = {(n, d)}, got {tuple(cos.shape)} / {tuple(sin.shape)}")
    if weight_t.numel() != d // 2 or weight_hw.numel() != d // 2:
        raise RuntimeError("weight_t / weight_hw must hold D / 2 values")
    wt = weight_t.float().contiguous()
    whw = weight_hw.float().contiguous()
    cos = cos.float().contiguous()
    sin = sin.float().contiguous()
    _lib.call("hn_pixelumm_qk", x.data_ptr(), x.stride(1), wt.data_ptr(), whw.data_ptr(), cos.data_ptr(),
              sin.data_ptr(), b * n, h, d, eps, y.data_ptr(), _lib.stream(x))
    return y
