"""The DiT double-stream block half on the quantized path, and the torch helpers it is checked against.

Helpers (hy_nomas/model.py:89-138): `layer_norm`, `modulate`, `RMSNorm`, `rope_freqs`, `apply_rope` -- the
torch arithmetic the fused kernels replace.

`DiTBlockInt8` wires one stream of `DoubleStreamBlock` (hy_nomas/model.py:246-286) through this package's
kernels: fused LayerNorm/modulate/int8 quantization -> int8 QKV GEMM (q, k, v weights concatenated along
N, which is column-for-column identical to three GEMMs on the same codes) -> QK-RMSNorm + RoPE -> torch
SDPA -> int8 out-projection -> gated residual -> fused norm/quant -> int8 FFN-up with the GELU + int8
requantization epilogue -> int8 FFN-down -> gated residual.
"""
import torch
import torch.nn.functional as F

from . import fused, kernels


def layer_norm(x, eps=1e-6):
    """LayerNorm without affine in fp32 (hy_nomas/model.py:103-106)."""
    return F.layer_norm(x.float(), (x.shape[-1],), eps=eps)


def modulate(x, shift, scale):
    """hy_nomas/model.py:109-111 (fp32 when x is an fp32 norm)."""
    return x * (1 + scale.unsqueeze(1)) + shift.unsqueeze(1)


class RMSNorm(torch.nn.Module):
    """Normalize in fp32, cast back, then scale in the input dtype (hy_nomas/model.py:89-100)."""

    def __init__(self, dim, eps=1e-6, dtype=None, device=None):
        super().__init__()
        self.eps = eps
        self.weight = torch.nn.Parameter(torch.ones(dim, dtype=dtype, device=device))

    def forward(self, x):
        out = x.float()
        out = (out * torch.rsqrt(out.pow(2).mean(-1, keepdim=True) + self.eps)).type_as(x)
        return out * self.weight.to(dtype=out.dtype, device=out.device)


def rope_freqs(rope_dims, theta, t, h, w, t_offset=0, device=None):
    """3-D RoPE tables (cos, sin) [t*h*w, sum(rope_dims)] on the grid [t_offset, t_offset + t) x [0, h) x [0, w),
    fp32, each angle repeated for its interleaved pair (hy_nomas/model.py:114-128)."""
    axes = []
    for start, n in ((t_offset, t), (0, h), (0, w)):
        axes.append(torch.linspace(start, start + n, n + 1, dtype=torch.float32, device=device)[:n])
    grid = torch.meshgrid(*axes, indexing="ij")
    cos, sin = [], []
    for dim, pos in zip(rope_dims, grid):
        freqs = 1.0 / (theta ** (torch.arange(0, dim, 2, device=device)[: dim // 2].float() / dim))
        angles = torch.outer(pos.reshape(-1), freqs)
        cos.append(angles.cos().repeat_interleave(2, dim=1))
        sin.append(angles.sin().repeat_interleave(2, dim=1))
    return torch.cat(cos, dim=1), torch.cat(sin, dim=1)


def apply_rope(x, cos, sin):
    """Interleaved-pair rotation in fp32, cast back (hy_nomas/model.py:131-138).  x [B, L, H, D]."""
    xf = x.float()
    real, imag = xf.reshape(*x.shape[:-1], -1, 2).unbind(-1)
    rotated = torch.stack([-imag, real], dim=-1).flatten(3)
    return (xf * cos[None, :, None, :] + rotated * sin[None, :, None, :]).type_as(x)


class Int8Linear:
    """Device-resident int8 weight codes, fp32 scales ([N, K/128] g128 or [N, 1] per channel) and bias."""

    def __init__(self, qw, sw, bias=None):
        self.qw, self.sw, self.bias = qw, sw, bias

    @staticmethod
    def cat(linears):
        """Concatenate along N (e.g. q, k, v -> one QKV GEMM)."""
        bias = None if linears[0].bias is None else torch.cat([l.bias for l in linears])
        return Int8Linear(torch.cat([l.qw for l in linears]), torch.cat([l.sw for l in linears]), bias)


class DiTBlockInt8:
    """One stream of the double-stream block on the int8 path (hy_nomas/model.py:246-286).

    qkv, proj, fc1, fc2: Int8Linear.  q_norm_w / k_norm_w: [head_dim] bf16.
    per_token=False: the reference's layout -- activations quantized per token and 128 channels (adaLN
    quantization, the FFN-up GELU + requantization epilogue), weights per 128-channel group or per channel.
    per_token=True: one scale per token for every activation and per-channel weights ([N, 1] scales), so every
    GEMM accumulates the whole K in int32; FFN-up then writes bf16 GELU outputs that are quantized per token
    (a per-token requantization needs the whole row, which no GEMM tile holds)."""

    def __init__(self, qkv, proj, fc1, fc2, q_norm_w, k_norm_w, heads, per_token=False):
        self.qkv, self.proj, self.fc1, self.fc2 = qkv, proj, fc1, fc2
        self.q_norm_w, self.k_norm_w = q_norm_w, k_norm_w
        self.heads = heads
        self.per_token = per_token
        self.group = None if per_token else kernels.GROUP

    def attention_inputs(self, x, shift1, scale1, rope=None):
        """adaLN + int8 quantization shared by q/k/v -> one QKV GEMM -> QK-norm (+RoPE).  x [B, L, D]."""
        b, n, d = x.shape
        qa, sa = kernels.adaln_quant(x, shift1, scale1, group=self.group)
        qkv = kernels.block_gemm(qa, sa, self.qkv.qw, self.qkv.sw, self.qkv.bias, out_dtype=x.dtype)
        qkv = qkv.view(b, n, 3, self.heads, d // self.heads)
        q = fused.qk_norm_rope(qkv[:, :, 0], self.q_norm_w, rope)
        k = fused.qk_norm_rope(qkv[:, :, 1], self.k_norm_w, rope)
        v = qkv[:, :, 2]
        return q, k, v

    def attention_heads(self, x, shift1, scale1, rope=None, out=None, l_offset=0):
        """adaLN + int8 quantization -> one QKV GEMM whose epilogue applies QK-norm (+RoPE) and writes q, k, v
        head-major: out [3, B, H, L_total, D] (tokens at l_offset ..).  x [B, L, D]."""
        b, n, d = x.shape
        qa, sa = kernels.adaln_quant(x, shift1, scale1, group=self.group)
        return kernels.qkv_heads(qa, sa, self.qkv.qw, self.qkv.sw, self.qkv.bias, self.q_norm_w, self.k_norm_w, b,
                                 rope, out=out, l_offset=l_offset)

    def post(self, x, attn, gate1, shift2, scale2, gate2):
        """Out-projection + gated residual, then the MLP half with its gated residual.  attn [B, L, D]."""
        x = fused.gated_residual(x, kernels.block_linear(attn, self.proj.qw, self.proj.sw, self.proj.bias), gate1)
        qa, sa = kernels.adaln_quant(x, shift2, scale2, group=self.group)
        if self.per_token:
            g = kernels.block_gemm(qa, sa, self.fc1.qw, self.fc1.sw, self.fc1.bias, out_dtype=x.dtype, epilogue="gelu")
            qh, sh = kernels.quantize_activations(g, group=None)
            del g
        else:
            qh, sh = kernels.block_gemm(qa, sa, self.fc1.qw, self.fc1.sw, self.fc1.bias, epilogue="gelu_quant")
        h = kernels.block_gemm(qh, sh, self.fc2.qw, self.fc2.sw, self.fc2.bias, out_dtype=x.dtype)
        return fused.gated_residual(x, h.view_as(x), gate2)

    def forward(self, x, mods, rope=None):
        """Self-attention over this stream only (torch SDPA, unchanged), then `post`."""
        shift1, scale1, gate1, shift2, scale2, gate2 = mods
        hm = self.attention_heads(x, shift1, scale1, rope)
        attn = attention_heads(hm[0], hm[1], hm[2]).reshape(x.shape)
        return self.post(x, attn, gate1, shift2, scale2, gate2)


def attention(q, k, v):
    """Joint softmax attention over the token axis with torch SDPA: q, k, v [B, L, H, D] -> [B, L, H, D].

    The operands are made contiguous in [B, H, L, D] first (torch's batched bf16 products misbehave on
    transposed views), and only the flash / memory-efficient kernels are allowed: at video lengths the
    math fallback would materialize an [L, L] score matrix per head, so an unsupported case raises."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    qh, kh, vh = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        out = F.scaled_dot_product_attention(qh, kh, vh)
    return out.transpose(1, 2)


def attention_heads(qh, kh, vh):
    """`attention` on head-major operands qh, kh, vh [B, H, L, D] (contiguous, as the QKV epilogue writes
    them): no layout copies before SDPA.  Returns [B, L, H, D] (a view of SDPA's output)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        out = F.scaled_dot_product_attention(qh, kh, vh)
    return out.transpose(1, 2)


class DoubleStreamBlockInt8:
    """The double-stream DiT block on the int8 path (hy_nomas/model.py:230-286): image and text streams with
    their own weights and modulations, one joint attention over the concatenated tokens (image first), then
    each stream's out-projection, gated residuals and MLP.  The image stream gets RoPE; the text stream none.

    img / txt: DiTBlockInt8 halves.  forward(img, txt, img_mods, txt_mods, rope) -> (img, txt)."""

    def __init__(self, img, txt):
        self.img, self.txt = img, txt

    def forward(self, img, txt, img_mods, txt_mods, rope=None):
        shift1, scale1, gate1, shift2, scale2, gate2 = img_mods
        tshift1, tscale1, tgate1, tshift2, tscale2, tgate2 = txt_mods
        b, lv = img.shape[0], img.shape[1]
        # both streams' q, k, v land head-major in one buffer, image tokens first (the reference's
        # torch.cat order), so attention runs on it without concatenation or layout copies
        hm = torch.empty((3, b, self.img.heads, lv + txt.shape[1], img.shape[2] // self.img.heads),
                         device=img.device, dtype=torch.bfloat16)
        self.img.attention_heads(img, shift1, scale1, rope, out=hm, l_offset=0)
        self.txt.attention_heads(txt, tshift1, tscale1, None, out=hm, l_offset=lv)
        attn = attention_heads(hm[0], hm[1], hm[2])
        del hm
        attn = attn.reshape(b, attn.shape[1], -1)
        img = self.img.post(img, attn[:, :lv], gate1, shift2, scale2, gate2)
        txt = self.txt.post(txt, attn[:, lv:], tgate1, tshift2, tscale2, tgate2)
        return img, txt


def reference_double_stream(img_blk, txt_blk, img, txt, img_mods, txt_mods, rope=None, eps=1e-6):
    """The same double-stream block in float32 torch arithmetic with dequantized weights and unquantized
    activations (the reference's exact-matmul path, hy_nomas/model.py:246-286 with ops.py:172-176); tensors may
    live on any device.  Returns (img, txt) float32."""
    def lin(x, l):
        w = l.qw.float() * l.sw.float().repeat_interleave(l.qw.shape[1] // l.sw.shape[1], dim=1)
        return F.linear(x, w, None if l.bias is None else l.bias.float())

    def qkv(blk, x, mods, rope):
        shift1, scale1 = mods[0].float(), mods[1].float()
        xm = modulate(layer_norm(x, eps), shift1, scale1).to(torch.bfloat16).float()
        b, n, d = x.shape
        t = lin(xm, blk.qkv).view(b, n, 3, blk.heads, d // blk.heads)
        q, k, v = t[:, :, 0], t[:, :, 1], t[:, :, 2]

        def rms(z, w):
            return z * torch.rsqrt(z.pow(2).mean(-1, keepdim=True) + eps) * w.float()
        q, k = rms(q, blk.q_norm_w), rms(k, blk.k_norm_w)
        if rope is not None:
            q, k = apply_rope(q, *rope), apply_rope(k, *rope)
        return q, k, v

    def post(blk, x, attn, mods):
        gate1, shift2, scale2, gate2 = (m.float() for m in mods[2:])
        x = x + lin(attn, blk.proj) * gate1.unsqueeze(1)
        h = lin(modulate(layer_norm(x, eps), shift2, scale2), blk.fc1)
        h = F.gelu(h, approximate="tanh")
        return x + lin(h, blk.fc2) * gate2.unsqueeze(1)

    img, txt = img.float(), txt.float()
    iq, ik, iv = qkv(img_blk, img, img_mods, rope)
    tq, tk, tv = qkv(txt_blk, txt, txt_mods, None)
    q, k, v = (torch.cat(p, dim=1).transpose(1, 2) for p in ((iq, tq), (ik, tk), (iv, tv)))
    att = torch.softmax(q @ k.transpose(-1, -2) / q.shape[-1] ** 0.5, dim=-1) @ v
    att = att.transpose(1, 2).reshape(img.shape[0], -1, img.shape[2])
    lv = img.shape[1]
    return post(img_blk, img, att[:, :lv], img_mods), post(txt_blk, txt, att[:, lv:], txt_mods)
