"""int8 K/V history: absmax per token and head, round half away from zero (hy_nomas/world.py:80-94).

Same functions, arguments and results as the reference's `world.quantize_kv` / `world.dequantize_kv`, on the
gfx950 kernels: the activation quantizer with one group per (token, head) row, and a fused row-scaled
dequantization (one read of the codes, one write of the output, no fp32 intermediate tensor).
"""
import torch

from . import _lib, kernels


def _quantize_rows_torch(x):
    """Absmax per row (last dim) / 127 (1 for an all-zero row), IEEE quotient, half away from zero, clamp
    +-127, in torch steps on x's device: the path for host tensors and head dims the device quantizer does
    not take (multiples of 128 only)."""
    xf = x.float()
    peak = xf.abs().amax(dim=-1, keepdim=True)
    scale = torch.where(peak > 0, peak / 127.0, torch.ones_like(peak))
    y = xf / scale
    codes = torch.trunc(y + torch.copysign(torch.full_like(y, 0.5), y)).clamp_(-127, 127)
    return codes.to(torch.int8), scale


def quantize_kv(x):
    """x [L, H, D] -> (int8 [L, H, D], fp32 scale [L, H, 1]) (hy_nomas/world.py:83-90), on any device.
    Device tensors with D % 128 == 0 take the gfx950 quantizer; host tensors and other head dims take the
    same arithmetic in torch steps."""
    l, h, d = x.shape
    if not x.is_cuda or d % kernels.GROUP or x.numel() == 0:
        return _quantize_rows_torch(x)
    x2 = x.reshape(l * h, d)
    # one group per row: the g128 kernel when a row is one 128-channel group, else the per-row kernel
    q, s = kernels.quantize_activations(x2, "int8", kernels.GROUP if d == kernels.GROUP else None)
    return q.view(l, h, d), s.view(l, h, 1)


def dequantize_kv(q, scale, dtype=torch.bfloat16):
    """(q.float() * scale).to(dtype) in one pass (hy_nomas/world.py:93-94): q [..., D] int8, scale [..., 1].
    Host tensors, and head dims the device kernel does not take (D % 16 != 0), use the same torch steps."""
    d = q.shape[-1]
    if not q.is_cuda or not scale.is_cuda or d % 16 or dtype not in _lib.DTYPE:
        return (q.float() * scale.to(q.device)).to(dtype)
    rows = q.numel() // d if d else 0
    out = torch.empty(q.shape, device=q.device, dtype=dtype)
    if rows == 0:
        return out
    if tuple(scale.shape) != tuple(q.shape[:-1]) + (1,):
        raise RuntimeError(f"dequantize_kv: scale shape {tuple(scale.shape)} does not match codes {tuple(q.shape)}")
    q2 = q.reshape(rows, d)
    if not q2.is_contiguous() or q2.data_ptr() % 16:
        q2 = q2.contiguous()
    s2 = scale.reshape(rows).float().contiguous()
    _lib.call("hn_dequantize_rows", q2.data_ptr(), q2.stride(0), s2.data_ptr(), 1, rows, d, out.data_ptr(),
              _lib.dtype_code(out), d, _lib.stream(q))
    return out
