"""Attention of the double-stream block on the gfx950 bf16 matrix cores (hy_nomas/model.py:145-223).

`attention(q, k, v, transformer_options=None)` has the reference's signature and result: q [B, Lq, H, D],
k / v [B, Lk, H, D] -> softmax attention over all keys, [B, Lq, H, D].  `segment_attention(q, k, v, history,
plan, transformer_options=None)` is the reference's segment-level call: the current tokens attend to the
cached history keys plus the current video keys and, with an action plan, to their own group's text keys.
`transformer_options` (ComfyUI's per-call options, which the reference hands to ComfyUI's attention) is
accepted in the same position and not used.

Two backends, chosen by the keyword `backend`: "sdpa" (torch's scaled-dot-product attention, the default the
reference also reaches through ComfyUI) and "hip" (this package's kernel, `hn_attention`).
`HY_NOMAS_ATTENTION` selects one for every call that does not name it.  The HIP kernel takes head dim 128 in
bf16; other inputs use SDPA.
"""
import os

import torch
import torch.nn.functional as F

from . import _lib

BACKEND_ENV = "HY_NOMAS_ATTENTION"
KEY_TILE = 64          # keys per tile of the kernel; V^T rows are padded to a multiple of it


def choose_backend(name=None):
    """The attention backend of a call: `name`, else HY_NOMAS_ATTENTION, else "sdpa"."""
    name = name or os.environ.get(BACKEND_ENV, "sdpa")
    if name not in ("sdpa", "hip"):
        raise ValueError(f"attention backend must be 'sdpa' or 'hip', got {name!r}")
    return name


def _hip_ok(q, k, v):
    return (q.is_cuda and q.dtype == k.dtype == v.dtype == torch.bfloat16 and q.shape[-1] == 128
            and k.shape[-1] == 128 and v.shape[-1] == 128)


def transpose_values(vh):
    """vh [B, H, Lk, D] -> V^T [B, H, D, Lk_pad] bf16: the layout `hn_attention` reads V in.  Keys run along the
    last dim, padded with zero keys up to a multiple of the kernel's key tile, and the keys of each 16-key group
    are stored in the order 0-3, 8-11, 4-7, 12-15 (key 16 g + 8 a + 4 b + c at position 16 g + 8 b + 4 a + c),
    the order in which the kernel's matrix-core operands hold them."""
    b, h, lk, d = vh.shape
    pad = -(-lk // KEY_TILE) * KEY_TILE
    vt = torch.empty((b, h, d, pad), device=vh.device, dtype=torch.bfloat16)
    full = lk // 16 * 16

    def put(dst, src):  # src [B, H, n, D] (n % 16 == 0) -> dst [B, H, D, n] in the grouped key order
        n = src.shape[2]
        dst.unflatten(3, (n // 16, 2, 2, 4)).copy_(src.unflatten(2, (n // 16, 2, 2, 4)).permute(0, 1, 6, 2, 4, 3, 5))

    if full:
        put(vt[..., :full], vh[:, :, :full])
    if pad > full:
        tail = torch.zeros((b, h, pad - full, d), device=vh.device, dtype=torch.bfloat16)
        tail[:, :, :lk - full] = vh[:, :, full:]
        put(vt[..., full:], tail)
    return vt


def values_buffer(b, h, lk, device, d=128):
    """An empty V^T buffer [B, H, D, Lk padded to the key tile] for writers of the layout (`kernels.qkv_heads`
    with `vt`): the padding keys past Lk are zeroed here, the keys themselves are left to the writer.

    Keys are permuted within each 16-key group, so when Lk % 16 != 0 some padding keys of the last partial
    group sit at physical positions below Lk.  The zeroing therefore starts at that group's first position;
    the writer then overwrites the group's real keys.  (The kernel gives padding keys zero weight, but a
    zero weight times uninitialised NaN bits would still be NaN.)"""
    pad = -(-lk // KEY_TILE) * KEY_TILE
    vt = torch.empty((b, h, d, pad), device=device, dtype=torch.bfloat16)
    start = lk // 16 * 16
    if pad > start:
        vt[..., start:].zero_()
    return vt


def _rows16(t):
    """t with a contiguous last dim and 16-byte aligned rows (a copy only when needed)."""
    if t.stride(-1) != 1 or t.data_ptr() % 16 or any(st % 8 for st in t.stride()[:-1]):
        t = t.contiguous()
    return t


def attention_hip(q, k, vt, lk, out=None, scale=None):
    """The kernel on explicit layouts.  q [B, Lq, H, 128] or any strided view with the dims contiguous (rows
    16-byte aligned); k likewise [B, Lk, H, 128]; vt = transpose_values(v head-major) [B, H, 128, >= Lk padded].
    Returns out [B, Lq, H, 128] bf16 (token-major: out.view(B, Lq, H * 128) feeds the out-projection)."""
    _lib.require_device(q, k, vt)
    b, lq, h, d = q.shape
    if k.shape[0] != b or k.shape[2] != h or k.shape[3] != d or k.shape[1] != lk:
        raise RuntimeError(f"attention: k {tuple(k.shape)} does not match q {tuple(q.shape)} with Lk={lk}")
    if tuple(vt.shape[:3]) != (b, h, d) or vt.shape[3] < -(-lk // KEY_TILE) * KEY_TILE or vt.stride(3) != 1:
        raise RuntimeError(f"attention: V^T {tuple(vt.shape)} is not [B, H, D, Lk padded to {KEY_TILE}]")
    q, k = _rows16(q), _rows16(k)
    if out is None:
        out = torch.empty((b, lq, h, d), device=q.device, dtype=torch.bfloat16)
    if out.stride(3) != 1 or out.data_ptr() % 8 or any(st % 4 for st in out.stride()[:3]):
        raise RuntimeError("attention: out must have a contiguous head dim and 8-byte aligned rows")
    if b * lq == 0:
        return out
    if lk == 0:
        raise RuntimeError("attention: no keys")
    scale = d ** -0.5 if scale is None else scale
    _lib.call("hn_attention", q.data_ptr(), q.stride(0), q.stride(2), q.stride(1), k.data_ptr(), k.stride(0), k.stride(2),
              k.stride(1), vt.data_ptr(), vt.stride(0), vt.stride(1), vt.stride(2), out.data_ptr(), out.stride(0),
              out.stride(2), out.stride(1), b, h, lq, lk, d, float(scale), _lib.stream(q))
    return out


def attention(q, k, v, transformer_options=None, *, backend=None):
    """q [B, Lq, H, D], k / v [B, Lk, H, D] -> [B, Lq, H, D] (hy_nomas/model.py:145-150)."""
    if choose_backend(backend) == "hip" and _hip_ok(q, k, v):
        vt = transpose_values(v.transpose(1, 2))
        return attention_hip(q, k, vt, k.shape[1])
    return sdpa(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)).transpose(1, 2)


def attention_heads(qh, kh, vh, backend=None):
    """`attention` on head-major operands qh [B, H, Lq, D], kh / vh [B, H, Lk, D] (as the QKV epilogue writes
    them).  Returns [B, Lq, H, D] (a view for SDPA, a contiguous tensor for the HIP kernel)."""
    if choose_backend(backend) == "hip" and _hip_ok(qh, kh, vh):
        return attention_hip(qh.transpose(1, 2), kh.transpose(1, 2), transpose_values(vh), kh.shape[2])
    return sdpa(qh, kh, vh).transpose(1, 2)


def sdpa(qh, kh, vh):
    """torch's SDPA on head-major operands, with only the flash / memory-efficient kernels allowed: at video
    lengths the math fallback would materialize an [L, L] score matrix per head, so an unsupported case raises.
    The operands are made contiguous first (torch's batched bf16 products misbehave on transposed views)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    qh, kh, vh = (t if t.is_contiguous() else t.contiguous() for t in (qh, kh, vh))
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        return F.scaled_dot_product_attention(qh, kh, vh)


def _keys(parts):
    """Keys and values of one attention call: the (k, v) pairs of `parts` joined along the token axis."""
    parts = [p for p in parts if p is not None and p[0].shape[1]]
    if len(parts) == 1:
        return parts[0]
    return torch.cat([p[0] for p in parts], dim=1), torch.cat([p[1] for p in parts], dim=1)


def segment_attention(q, k, v, history, plan, transformer_options=None, *, backend=None):
    """The current tokens' attention of one segment (hy_nomas/model.py:199-223): q / k / v [B, Lv + Lt, H, D] (video
    tokens first), history (hk, hv) [1 or B, Lh, H, D] or None, plan with `groups` (None: every current token
    queries every key) and `video_tokens`.  Each group's queries attend to the history, every current video key
    and the group's own text keys (indices into the text part)."""
    batch = q.shape[0]
    hist = None
    if history is not None:
        hist = tuple(t if t.shape[0] == batch else t.expand(batch, -1, -1, -1) for t in history)
    groups = getattr(plan, "groups", None)
    if groups is None:
        return attention(q, *_keys([hist, (k, v)]), backend=backend)
    lv = plan.video_tokens
    video = (k[:, :lv], v[:, :lv])
    out = torch.empty_like(q)
    for q_idx, text_idx in groups:
        text = (k[:, lv + text_idx], v[:, lv + text_idx]) if text_idx.numel() else None
        out[:, q_idx] = attention(q[:, q_idx], *_keys([hist, video, text]), backend=backend)
    return out
