"""Torch restatements of the reference's DiT block arithmetic -- TEST INFRASTRUCTURE ONLY.

Like the rest of ``oracle/``, only ``tests/`` import this module, to check results; the product package never
does.  These are the reference's non-fused torch forms that its fused kernels replace, and the float32
"exact-matmul" double-stream block the int8 path is compared against:

  layer_norm, modulate        hy_nomas/model.py:103-111
  RMSNorm                     hy_nomas/model.py:89-100
  rope_freqs, apply_rope      hy_nomas/model.py:114-138
  reference_double_stream     hy_nomas/model.py:230-303 with the exact Linear (ops.py:172-176)
  double_stream_rows          the same block for sampled query rows, at any length
"""
import torch
import torch.nn.functional as F


def layer_norm(x, eps=1e-6):
    """LayerNorm without affine, in fp32 (hy_nomas/model.py:103-106)."""
    return F.layer_norm(x.float(), (x.shape[-1],), eps=eps)


def modulate(x, shift, scale):
    """x * (1 + scale) + shift with [B, D] factors broadcast over tokens (hy_nomas/model.py:109-111)."""
    return x * (1 + scale.unsqueeze(1)) + shift.unsqueeze(1)


class RMSNorm(torch.nn.Module):
    """Normalize in fp32, cast back to the input dtype, then scale in that dtype (hy_nomas/model.py:89-100)."""

    def __init__(self, dim, eps=1e-6, dtype=None, device=None):
        super().__init__()
        self.eps = eps
        self.weight = torch.nn.Parameter(torch.ones(dim, dtype=dtype, device=device))

    def forward(self, x):
        xf = x.float()
        n = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)).type_as(x)
        return n * self.weight.to(dtype=n.dtype, device=n.device)


def rope_freqs(rope_dims, theta, t, h, w, t_offset=0, device=None):
    """3-D RoPE tables (cos, sin) [t*h*w, sum(rope_dims)] fp32 on the grid [t_offset, t_offset + t) x [0, h) x
    [0, w), each angle repeated for its interleaved pair (hy_nomas/model.py:114-128)."""
    spans = ((t_offset, t), (0, h), (0, w))
    axes = [torch.linspace(start, start + n, n + 1, dtype=torch.float32, device=device)[:n] for start, n in spans]
    grid = torch.meshgrid(*axes, indexing="ij")
    cos, sin = [], []
    for dim, pos in zip(rope_dims, grid):
        inv = 1.0 / (theta ** (torch.arange(0, dim, 2, device=device)[: dim // 2].float() / dim))
        ang = torch.outer(pos.reshape(-1), inv)
        cos.append(ang.cos().repeat_interleave(2, dim=1))
        sin.append(ang.sin().repeat_interleave(2, dim=1))
    return torch.cat(cos, dim=1), torch.cat(sin, dim=1)


def apply_rope(x, cos, sin):
    """Interleaved-pair rotation in fp32, cast back (hy_nomas/model.py:131-138).  x [B, L, H, D]."""
    xf = x.float()
    even, odd = xf.reshape(*x.shape[:-1], -1, 2).unbind(-1)
    turned = torch.stack([-odd, even], dim=-1).flatten(3)
    return (xf * cos[None, :, None, :] + turned * sin[None, :, None, :]).type_as(x)


def _dequantized(lin):
    """fp32 weight of an int8 linear (codes times their per-channel or per-128-group scales)."""
    reps = lin.qw.shape[1] // lin.sw.shape[1]
    return lin.qw.float() * lin.sw.float().repeat_interleave(reps, dim=1)


def _linear(x, lin, w=None):
    w = _dequantized(lin) if w is None else w
    return F.linear(x, w, None if lin.bias is None else lin.bias.float())


def _rms(z, w, eps):
    return z * torch.rsqrt(z.pow(2).mean(-1, keepdim=True) + eps) * w.float()


def _qkv(blk, x, mods, rope, eps):
    """fp32 q, k, v [B, L, H, D] of one stream: adaLN output rounded to bf16 (the fused kernel's output
    dtype), exact linear on the dequantized weight, QK RMSNorm, RoPE."""
    shift1, scale1 = mods[0].float(), mods[1].float()
    xm = modulate(layer_norm(x, eps), shift1, scale1).to(torch.bfloat16).float()
    b, n, d = x.shape
    t = _linear(xm, blk.qkv).view(b, n, 3, blk.heads, d // blk.heads)
    q, k, v = t[:, :, 0], t[:, :, 1], t[:, :, 2]
    q, k = _rms(q, blk.q_norm_w, eps), _rms(k, blk.k_norm_w, eps)
    if rope is not None:
        q, k = apply_rope(q, *rope), apply_rope(k, *rope)
    return q, k, v


def _post(blk, x, attn, mods, eps):
    """Out-projection, gated residual, adaLN, GELU-tanh MLP, gated residual, all fp32 (row-local)."""
    gate1, shift2, scale2, gate2 = (m.float() for m in mods[2:])
    x = x + _linear(attn, blk.proj) * gate1.unsqueeze(1)
    h = F.gelu(_linear(modulate(layer_norm(x, eps), shift2, scale2), blk.fc1), approximate="tanh")
    return x + _linear(h, blk.fc2) * gate2.unsqueeze(1)


def softmax_attention(q, k, v):
    """float32 softmax(q k^T / sqrt(D)) v on token-major q [B, Lq, H, D], k / v [B, Lk, H, D] -> [B, Lq, H, D]."""
    qh, kh, vh = (t.float().transpose(1, 2) for t in (q, k, v))
    p = torch.softmax(qh @ kh.transpose(-1, -2).contiguous() / qh.shape[-1] ** 0.5, dim=-1)
    return (p @ vh.contiguous()).transpose(1, 2)


def segment_attention(q, k, v, history=None, groups=None, video_tokens=None):
    """The segment's attention of hy_nomas/model.py:199-223 in float32: q / k / v [B, Lv + Lt, H, D] are the
    current tokens (video first); history (hk, hv) [1 or B, Lh, H, D] or None.  Without groups every current
    token attends to [history | all current keys]; with groups [(query indices, text key indices)] each group's
    queries attend to [history | the current video keys | the group's text keys]."""
    b = q.shape[0]
    hist = None
    if history is not None:
        hist = tuple(t.float().expand(b, -1, -1, -1) for t in history)
    if groups is None:
        keys = k if hist is None else torch.cat([hist[0], k.float()], dim=1)
        vals = v if hist is None else torch.cat([hist[1], v.float()], dim=1)
        return softmax_attention(q, keys, vals)
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    for q_idx, t_idx in groups:
        ks, vs = [k[:, :video_tokens].float()], [v[:, :video_tokens].float()]
        if hist is not None:
            ks.insert(0, hist[0])
            vs.insert(0, hist[1])
        if t_idx.numel():
            ks.append(k[:, video_tokens + t_idx].float())
            vs.append(v[:, video_tokens + t_idx].float())
        out[:, q_idx] = softmax_attention(q[:, q_idx], torch.cat(ks, dim=1), torch.cat(vs, dim=1))
    return out


def reference_double_stream(img_blk, txt_blk, img, txt, img_mods, txt_mods, rope=None, eps=1e-6, history=None,
                            groups=None):
    """The double-stream block in float32 torch arithmetic with dequantized weights and unquantized
    activations (the reference's exact-matmul path).  img_blk / txt_blk carry `qkv, proj, fc1, fc2` (int8 codes
    `qw`, scales `sw`, `bias`), `q_norm_w`, `k_norm_w`, `heads`.  history / groups: as `segment_attention`.
    Returns (img, txt) float32."""
    img, txt = img.float(), txt.float()
    iq, ik, iv = _qkv(img_blk, img, img_mods, rope, eps)
    tq, tk, tv = _qkv(txt_blk, txt, txt_mods, None, eps)
    q, k, v = (torch.cat(p, dim=1) for p in ((iq, tq), (ik, tk), (iv, tv)))
    lv = img.shape[1]
    att = segment_attention(q, k, v, history, groups, lv).reshape(img.shape[0], -1, img.shape[2])
    return _post(img_blk, img, att[:, :lv], img_mods, eps), _post(txt_blk, txt, att[:, lv:], txt_mods, eps)


def double_stream_rows(img_blk, txt_blk, img, txt, img_mods, txt_mods, rope, img_rows, txt_rows, eps=1e-6):
    """`reference_double_stream` evaluated only at sampled token rows, for lengths where the full [L, L]
    attention does not fit: q/k/v of every token (fp32), the joint softmax attention of the sampled query
    rows only, then the row-local rest of the block for those rows.  Batch 1.  img_rows / txt_rows index the
    image and text tokens.  Returns (img [len(img_rows), D], txt [len(txt_rows), D]) float32."""
    img, txt = img.float(), txt.float()
    iq, ik, iv = _qkv(img_blk, img, img_mods, rope, eps)
    tq, tk, tv = _qkv(txt_blk, txt, txt_mods, None, eps)
    k = torch.cat((ik, tk), dim=1)[0].transpose(0, 1)       # [H, L, D]
    v = torch.cat((iv, tv), dim=1)[0].transpose(0, 1)
    del ik, tk, iv, tv
    out = []
    for blk, x, q, rows, mods in ((img_blk, img, iq, img_rows, img_mods), (txt_blk, txt, tq, txt_rows, txt_mods)):
        r = torch.as_tensor(rows, device=x.device, dtype=torch.long)
        qs = q[0, r].transpose(0, 1)                            # [H, S, D]
        p = torch.softmax(qs @ k.transpose(-1, -2) / qs.shape[-1] ** 0.5, dim=-1)
        att = (p @ v).transpose(0, 1).reshape(1, len(rows), -1)  # [1, S, D]
        out.append(_post(blk, x[:, r], att, mods, eps)[0])
    return out[0], out[1]
