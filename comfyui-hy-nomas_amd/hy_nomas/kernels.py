"""Block-scaled W8A8 linears on the MI355X int8 / fp8 matrix cores (gfx950 HIP kernels).

Drop-in for the reference's `hy_nomas/kernels.py` (same names, arguments and return values):

    y[m, n] = sum_g  a_scale[m, g] * w_scale[n, g] * sum_{k in g} qa[m, k] * qw[n, k]   (+ bias[n])

int8: absmax / 127, round half away from zero, exact int32 products per group.
fp8:  absmax / 448 (OCP e4m3fn), fp32 accumulation.

The group is 128 channels (the reference's layout: scales [rows, K / 128]).  A scale tensor with a single
column selects one scale per token (activations) or per output channel (weights); the GEMM then
accumulates the whole K in int32 and dequantizes once.  Weights are used as stored.
"""
import weakref

import torch

from . import _lib

GROUP = 128
EPILOGUES = {None: 0, "gelu": 1, "gelu_quant": 2, "swiglu_quant": 4}
# int8 whole-K accumulation keeps the exact dot product in int32: |sum| <= 128 * 128 * K < 2^31 needs
# K < 131072.  Longer K takes the per-group fold with the single scale repeated per group.
WHOLE_K_INT32_LIMIT = 131072

# Scale tensors known to be positive and finite (or not), by tensor identity and in-place version:
# {id: (weakref, version, ok)}.  The fp8 GEMM with 128 x 128 block weight scales keeps its running sum in units
# of the current group's scale product, which needs every activation and weight scale positive and finite.
# Dispatch only looks the verdict up: it never reads a scale tensor, so it never waits for the device and
# can be captured into a graph.  Scales with no verdict take the per-group fold on scales repeated per
# channel, which is exact for any values.
_SCALES_CHECKED = {}


def _remember_scales(t, ok):
    key = id(t)
    _SCALES_CHECKED[key] = (weakref.ref(t, lambda _r, key=key: _SCALES_CHECKED.pop(key, None)), t._version, ok)


def _verdict(t):
    """The recorded verdict for `t` as it is now: True, False, or None if there is none (no device access)."""
    hit = _SCALES_CHECKED.get(id(t))
    if hit is not None and hit[0]() is t and hit[1] == t._version:
        return hit[2]
    return None


def _known_positive_finite(t):
    """True if `t`, as it is now, is recorded as positive and finite (no device access)."""
    return _verdict(t) is True


def trust_scales(*tensors):
    """Record scale tensors made by this package's quantizers (absmax / 127 or 1, max(absmax, 1e-12) / 448,
    clamped block scales): positive, and finite for finite inputs, so the GEMM needs no check of them."""
    for t in tensors:
        if t is not None:
            _remember_scales(t, True)


def validate_scales(*tensors):
    """Check scale tensors from elsewhere (a checkpoint's fp8 block scales) once and remember the verdict, so
    that block_gemm / block_linear read fp8 block scales as stored.  Meant for load time: on a device tensor
    the check waits for the device, once per tensor and in-place version; on a host tensor it does not touch
    the device.  Returns True if every value of every tensor is positive and finite."""
    ok_all = True
    for t in tensors:
        if t is None:
            continue
        ok = _verdict(t)
        if ok is None:
            ok = bool(torch.all((t > 0) & torch.isfinite(t)))
            _remember_scales(t, ok)
        ok_all = ok_all and ok
    return ok_all


def _aligned(t, bytes_):
    return t.data_ptr() % bytes_ == 0


def _rows(x):
    """x with unit column stride, 16-byte aligned rows (copy only if needed)."""
    if x.stride(-1) != 1 or not _aligned(x, 16) or (x.stride(0) * x.element_size()) % 16:
        x = x.contiguous()
    return x


def quantize_activations(x, kind="int8", group=GROUP, rounding="half_away"):
    """x [M, K] (K % 128 == 0) -> codes [M, K] and fp32 scales [M, K / group] (hy_nomas/kernels.py:45-54).

    `group=None` (or K) gives one scale per token; `rounding="half_even"` switches the int8 rounding."""
    _lib.require_device(x)
    m, k = x.shape
    g = k if group is None else group
    dtype = torch.int8 if kind == "int8" else torch.float8_e4m3fn
    q = torch.empty((m, k), device=x.device, dtype=dtype)
    s = torch.empty((m, k // g), device=x.device, dtype=torch.float32)
    if m == 0:
        return q, s
    x = _rows(x)
    _lib.call("hn_quantize_act", x.data_ptr(), _lib.dtype_code(x), x.stride(0), m, k, g, _lib.KIND[kind],
              _lib.ROUND[rounding], q.data_ptr(), q.stride(0), s.data_ptr(), s.stride(0), _lib.stream(x))
    trust_scales(s)
    return q, s


_CODE_DTYPES = {"int8": (torch.int8,), "fp8": (torch.float8_e4m3fn, torch.uint8)}


def _check_weights(qw, sw, bias, kind, k, who="block_gemm"):
    """The weight side of a GEMM: codes of the kind with K columns, weight-scale rows for every output channel
    (one per channel or one per 128), a bias of N values.  Raises RuntimeError."""
    if kind not in _CODE_DTYPES:
        raise RuntimeError(f"kind must be 'int8' or 'fp8', got {kind!r}")
    if qw.dim() != 2 or sw.dim() != 2:
        raise RuntimeError(f"{who}: weight codes and scales must be 2-D")
    if qw.dtype not in _CODE_DTYPES[kind]:
        raise RuntimeError(f"{who}: {kind} weight codes expected, got {qw.dtype}")
    n = qw.shape[0]
    if qw.shape[1] != k:
        raise RuntimeError(f"{who}: activations have K={k}, weights K={qw.shape[1]}")
    if sw.shape[0] not in (n, (n + GROUP - 1) // GROUP):
        raise RuntimeError(f"{who}: {sw.shape[0]} weight-scale rows for {n} output channels")
    if bias is not None and (bias.dim() != 1 or bias.shape[0] != n):
        raise RuntimeError(f"{who}: bias of shape {tuple(bias.shape)} for {n} output channels")


def _check_gemm(qa, sa, qw, sw, bias, kind):
    """Shapes and dtypes the kernels rely on (the C ABI sees only pointers and strides): codes of the kind,
    matching K, one activation-scale row per token, and the weight side (`_check_weights`)."""
    if kind not in _CODE_DTYPES:
        raise RuntimeError(f"kind must be 'int8' or 'fp8', got {kind!r}")
    if qa.dim() != 2 or sa.dim() != 2:
        raise RuntimeError("block_gemm: codes and scales must be 2-D")
    if qa.dtype not in _CODE_DTYPES[kind]:
        raise RuntimeError(f"block_gemm: {kind} codes expected, got {qa.dtype}")
    m, k = qa.shape
    if sa.shape[0] != m:
        raise RuntimeError(f"block_gemm: {sa.shape[0]} activation-scale rows for {m} tokens")
    _check_weights(qw, sw, bias, kind, k)


def _layout(sw, n, k, kind, sa_cols, sa=None, swiglu=False):
    """How the GEMM reads the scales: (sw, sw_rows, group, groups).  `sa_cols`: activation-scale columns
    (1 or K / 128); `sa`: the activation scales when they are not this call's own quantizer output.

    sw_rows = 128: one weight-scale row per 128 output channels (the fp8 block layout), read as stored by
    the per-group fold.  With fp8 codes that fold keeps its running sum in units of the current group's
    scale product, which needs every activation and weight scale positive and finite: scales made by this
    package's quantizers, or passed through `validate_scales`.  Other scales are repeated per channel
    instead (the reference's own layout, pixelumm.py:153), whose fold has no such condition.  The swiglu
    epilogue has no such fallback: it checks unknown scales once (`validate_scales`).  group = K: one scale
    per token and per channel, accumulated over the whole K (int8 only while the int32 sum cannot
    overflow)."""
    sw_rows = 1 if sw.shape[0] == n else GROUP
    if sw_rows == GROUP and sw.shape[0] != (n + GROUP - 1) // GROUP:
        raise RuntimeError(f"weight scales with {sw.shape[0]} rows for {n} output channels")
    if sw_rows == GROUP and kind == "fp8":
        if swiglu:
            if not validate_scales(*(t for t in (sa, sw) if t is not None)):
                raise RuntimeError("swiglu_quant: fp8 block scales must be positive and finite")
        elif not ((sa is None or _known_positive_finite(sa)) and _known_positive_finite(sw)):
            # each block row repeated for its 128 channels (expand + copy: no device synchronization)
            sw = sw.float()[:, None, :].expand(-1, GROUP, -1).reshape(-1, sw.shape[1])[:n]
            sw_rows = 1
    if sw_rows == 1 and sa_cols == 1 and sw.shape[1] == 1 and (kind == "fp8" or k < WHOLE_K_INT32_LIMIT):
        return sw, sw_rows, k, 1
    return sw, sw_rows, GROUP, k // GROUP


def _scales(s, rows, groups):
    """fp32 [rows, groups] with unit column stride; a single column is broadcast to `groups` columns."""
    s = s.float()
    if s.shape[1] != groups:
        if s.shape[1] != 1:
            raise RuntimeError(f"scale tensor with {s.shape[1]} columns, expected {groups} or 1")
        s = s.expand(rows, groups)
    if s.stride(1) != 1:
        s = s.contiguous()
    return s


def block_gemm(qa, sa, qw, sw, bias=None, out_dtype=torch.bfloat16, kind="int8", epilogue=None):
    """Block-scaled GEMM on quantized activations (hy_nomas/kernels.py:152-170).  With epilogue
    "gelu_quant" returns (int8 [M, N], scales [M, N / 128]) ready for the next int8 linear; otherwise
    [M, N] in `out_dtype`.  Weight scales are [N, K/128] or [N, 1] (one row per output channel), or
    [ceil(N/128), K/128]: one row per 128 output channels (the fp8 128 x 128 block layout).

    "swiglu_quant" (the decoder MLP, hy_nomas/pixelumm.py:314-323): qw holds the gate and up weights
    interleaved in 128-row blocks (`pixelumm.interleave_gate_up`); returns the codes of
    bf16(silu(gate) * up) in this GEMM's kind, [M, N / 2], and their scales [M, N / 256], ready for the
    down projection.  Needs per-token scales, or fp8 with block weight scales."""
    _lib.require_device(qa, sa, qw, sw, bias)
    _check_gemm(qa, sa, qw, sw, bias, kind)
    m, k = qa.shape
    n = qw.shape[0]
    mode = EPILOGUES[epilogue]
    quantized = mode in (2, 4)
    if mode == 2:
        out = torch.empty((m, n), device=qa.device, dtype=torch.int8)
        qs = torch.empty((m, n // GROUP), device=qa.device, dtype=torch.float32)
    elif mode == 4:
        if n % (2 * GROUP):
            raise RuntimeError(f"swiglu_quant: {n} weight rows are not whole gate/up block pairs of {2 * GROUP}")
        out = torch.empty((m, n // 2), device=qa.device, dtype=torch.int8 if kind == "int8" else torch.float8_e4m3fn)
        qs = torch.empty((m, n // (2 * GROUP)), device=qa.device, dtype=torch.float32)
    else:
        out = torch.empty((m, n), device=qa.device, dtype=out_dtype)
        qs = None
    if m == 0:
        return (out, qs) if quantized else out
    sw, sw_rows, group, groups = _layout(sw, n, k, kind, sa.shape[1], sa, swiglu=mode == 4)
    sa = _scales(sa, m, groups)
    sw = _scales(sw, sw.shape[0], groups)
    qa = _rows(qa)
    qw = _rows(qw)
    if bias is not None and not bias.is_contiguous():
        bias = bias.contiguous()
    _lib.call("hn_block_gemm", qa.data_ptr(), qa.stride(0), sa.data_ptr(), sa.stride(0), qw.data_ptr(), qw.stride(0),
              sw.data_ptr(), sw.stride(0), sw_rows, _lib.ptr(bias), _lib.dtype_code(bias) if bias is not None else 0,
              m, n, k, group, _lib.KIND[kind], mode, out.data_ptr(), 0 if quantized else _lib.dtype_code(out),
              out.stride(0), _lib.ptr(qs), qs.stride(0) if qs is not None else 0, _lib.stream(qa))
    if quantized:
        trust_scales(qs)
        return out, qs
    return out


def qkv_heads(qa, sa, qw, sw, bias, q_norm_w, k_norm_w, batch, rope=None, kind="int8", eps=1e-6, out=None,
              l_offset=0, vt=None):
    """The q/k/v projection with QK RMSNorm and RoPE in the GEMM epilogue, written head-major for attention
    (hy_nomas/model.py:253-267 with fused.py:65-105): qa [batch * L, K] codes (scales sa), qw [3 * hidden, K]
    the stacked q, k, v weights (scales sw, bias [3 * hidden] or None), norm weights [128], rope (cos, sin)
    [L, 128] or None.  Returns `out` bf16 [3, batch, hidden / 128, L_total, 128] (allocated with
    L_total = L when not given); tokens land at rows l_offset .. l_offset + L, so the image and text streams
    can share one buffer.  q = out[0], k = out[1], v = out[2] are contiguous [B, H, L_total, 128].

    vt: a V^T buffer [batch, hidden / 128, 128, >= l_offset + L] bf16 (the HIP attention's V layout,
    `attention.values_buffer`): v goes there instead, token l at key l_offset + l, and `out` holds only q and k
    ([2, ...] is enough).  Needs L % 32 == 0 and l_offset % 16 == 0 (`vt_direct_ok`)."""
    _lib.require_device(qa, sa, qw, sw, bias, q_norm_w, k_norm_w)
    _check_gemm(qa, sa, qw, sw, bias, kind)
    if q_norm_w.numel() != 128 or k_norm_w.numel() != 128:
        raise RuntimeError("qkv_heads: QK-norm weights must have the head dim's 128 values")
    m, k = qa.shape
    n = qw.shape[0]
    if n % 3 or (n // 3) % 128:
        raise RuntimeError(f"qkv_heads: {n} weight rows are not q, k, v of whole 128-channel heads")
    hidden = n // 3
    if batch <= 0 or m % batch:
        raise RuntimeError(f"qkv_heads: {m} token rows do not split into batch {batch}")
    length = m // batch
    parts = 3 if vt is None else 2
    if out is None:
        out = torch.empty((parts, batch, hidden // 128, length, 128), device=qa.device, dtype=torch.bfloat16)
    if (out.dtype != torch.bfloat16 or out.dim() != 5 or out.shape[0] < parts
            or tuple(out.shape[1:3]) != (batch, hidden // 128) or out.shape[4] != 128 or not out.is_contiguous()
            or out.shape[3] < l_offset + length):
        raise RuntimeError(f"qkv_heads: out must be contiguous bf16 [{parts}, {batch}, {hidden // 128}, "
                           f">= {l_offset + length}, 128]")
    if vt is not None:
        _lib.require_device(vt)
        if not vt_direct_ok(length, l_offset):
            raise RuntimeError(f"qkv_heads: V^T output needs L % 32 == 0 and l_offset % 16 == 0 (L={length}, "
                               f"l_offset={l_offset})")
        if (vt.dtype != torch.bfloat16 or vt.dim() != 4 or tuple(vt.shape[:3]) != (batch, hidden // 128, 128)
                or vt.stride(3) != 1 or vt.shape[3] < l_offset + length):
            raise RuntimeError(f"qkv_heads: vt must be bf16 [{batch}, {hidden // 128}, 128, >= {l_offset + length}] "
                               "with contiguous keys")
    if m == 0:
        return out
    sw, sw_rows, group, groups = _layout(sw, n, k, kind, sa.shape[1], sa)
    sa = _scales(sa, m, groups)
    sw = _scales(sw, sw.shape[0], groups)
    qa, qw = _rows(qa), _rows(qw)
    if bias is not None and not bias.is_contiguous():
        bias = bias.contiguous()
    wq = q_norm_w.to(torch.bfloat16).float().contiguous()
    wk = k_norm_w.to(torch.bfloat16).float().contiguous()
    if rope is not None:
        cos, sin = rope[0].float().contiguous(), rope[1].float().contiguous()
        if tuple(cos.shape) != (length, 128) or tuple(sin.shape) != (length, 128):
            raise RuntimeError(f"rope tables must be [L, 128] = {(length, 128)}, got {tuple(cos.shape)}")
        cp, sp = cos.data_ptr(), sin.data_ptr()
    else:
        cp = sp = None
    args = (qa.data_ptr(), qa.stride(0), sa.data_ptr(), sa.stride(0), qw.data_ptr(), qw.stride(0),
            sw.data_ptr(), sw.stride(0), sw_rows, _lib.ptr(bias), _lib.dtype_code(bias) if bias is not None else 0,
            batch, length, hidden, k, group, _lib.KIND[kind], wq.data_ptr(), wk.data_ptr(), cp, sp, eps,
            out.data_ptr(), out.shape[3], l_offset)
    if vt is None:
        _lib.call("hn_qkv_heads", *args, _lib.stream(qa))
    else:
        _lib.call("hn_qkv_heads_vt", *args, vt.data_ptr(), vt.stride(0), vt.stride(1), vt.stride(2), _lib.stream(qa))
    return out


def vt_direct_ok(length, l_offset):
    """Whether qkv_heads can write v of `length` tokens at key `l_offset` straight into V^T."""
    return length % 32 == 0 and l_offset % 16 == 0


def block_gemm_acc32(qa, qw):
    """Full-K int32 dot products qa @ qw^T of int8 codes (a test hook: the exact integer accumulator)."""
    _lib.require_device(qa, qw)
    m, k = qa.shape
    n = qw.shape[0]
    if qa.dtype != torch.int8 or qw.dtype != torch.int8 or qw.shape[1] != k:
        raise RuntimeError("block_gemm_acc32: int8 codes with matching K expected")
    if k >= WHOLE_K_INT32_LIMIT:
        raise RuntimeError(f"block_gemm_acc32: K={k} could overflow the int32 accumulator (K < {WHOLE_K_INT32_LIMIT})")
    out = torch.empty((m, n), device=qa.device, dtype=torch.int32)
    if m == 0:
        return out
    qa = _rows(qa)
    qw = _rows(qw)
    _lib.call("hn_block_gemm", qa.data_ptr(), qa.stride(0), None, 0, qw.data_ptr(), qw.stride(0), None, 0, 1, None, 0,
              m, n, k, k, _lib.KIND["int8"], _lib.EPI_ACC32, out.data_ptr(), 0, out.stride(0), None, 0,
              _lib.stream(qa))
    return out


def adaln_quant(x, shift, scale, eps=1e-6, norm="layer", rounding="half_away", group=GROUP):
    """x [B, L, D] bf16, shift/scale [B, D] -> int8 codes [B * L, D] and scales [B * L, D / 128] of the
    modulated LayerNorm (hy_nomas/kernels.py:198-207).  Any D that is a multiple of 128 (e.g. 3072);
    `norm="rms"` uses RMSNorm instead of LayerNorm; `group=None` gives one scale per token ([B * L, 1],
    D <= 4096)."""
    _lib.require_device(x, shift, scale)
    b, l, d = x.shape
    if shift.numel() != b * d or scale.numel() != b * d:
        raise RuntimeError(f"adaln_quant: shift/scale must be [B, D] = {(b, d)}")
    g = d if group is None else group
    x = x.contiguous()
    shift = shift.to(x.dtype).contiguous()
    scale = scale.to(x.dtype).contiguous()
    q = torch.empty((b * l, d), device=x.device, dtype=torch.int8)
    s = torch.empty((b * l, d // g), device=x.device, dtype=torch.float32)
    if b * l == 0:
        return q, s
    _lib.call("hn_adaln_quant", x.data_ptr(), shift.data_ptr(), scale.data_ptr(), _lib.dtype_code(x), b, l, d, eps,
              _lib.NORM[norm], _lib.ROUND[rounding], g, q.data_ptr(), s.data_ptr(), _lib.stream(x))
    return q, s


def block_linear(x, qw, sw, bias=None, kind="int8", rounding="half_away"):
    """F.linear with block-scaled 8-bit weights: x [..., K] -> [..., N] in x's dtype
    (hy_nomas/kernels.py:210-222).  Weight scales [N, K/128] select per-token-and-group activation
    quantization; per-channel scales [N, 1] select per-token quantization; block scales
    [ceil(N/128), K/128] (one row per 128 output channels) are taken as they are.  One library call
    (hn_block_linear) quantizes into a workspace and runs the GEMM.  `rounding` (an addition to the
    reference's signature): "half_even" rounds the int8 activation codes half to even."""
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    m, k = x2.shape
    if k % GROUP or m == 0:
        from .ops import dequantize_g128
        if sw.shape[0] != qw.shape[0]:
            sw = sw.repeat_interleave(GROUP, dim=0)[: qw.shape[0]]
        return torch.nn.functional.linear(x, dequantize_g128(qw, sw, x.dtype), bias)
    _lib.require_device(x, qw, sw, bias)
    _check_weights(qw, sw, bias, kind, k, "block_linear")
    n = qw.shape[0]
    group = k if sw.shape[1] == 1 else GROUP
    # the activation quantizer's scales are positive (finite for finite x): only the weight scales are checked
    sw, sw_rows, gemm_group, groups = _layout(sw, n, k, kind, k // group)
    if gemm_group != group:
        # per-token scales over a K the int32 sum cannot hold: quantize per token, fold per group
        with torch.cuda.device(x.device):
            qa, sa = quantize_activations(x2, kind, None, rounding)
            out = block_gemm(qa, sa, qw, sw, bias, x.dtype, kind)
        return out.reshape(*shape[:-1], n)
    if x2.dtype not in _lib.DTYPE:
        x2 = x2.float()
    x2 = _rows(x2)
    sw = _scales(sw, sw.shape[0], groups)
    qw = _rows(qw)
    if bias is not None and not bias.is_contiguous():
        bias = bias.contiguous()
    out = torch.empty((m, n), device=x.device, dtype=x.dtype if x.dtype in _lib.DTYPE else torch.float32)
    nbytes = _lib.lib().hn_block_linear_workspace_bytes(m, k, group)
    ws = torch.empty(nbytes, device=x.device, dtype=torch.uint8)
    with torch.cuda.device(x.device):
        _lib.call("hn_block_linear", x2.data_ptr(), _lib.dtype_code(x2), x2.stride(0), m, k, group, _lib.KIND[kind],
                  _lib.ROUND[rounding], qw.data_ptr(), qw.stride(0), sw.data_ptr(), sw.stride(0), sw_rows,
                  _lib.ptr(bias), _lib.dtype_code(bias) if bias is not None else 0, n, out.data_ptr(),
                  _lib.dtype_code(out), out.stride(0), ws.data_ptr(), nbytes, _lib.stream(x2))
    return out.reshape(*shape[:-1], n).to(x.dtype)


def int8_g128_linear(x, qw, sw, bias=None):
    return block_linear(x, qw, sw, bias, kind="int8")
