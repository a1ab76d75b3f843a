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

    qkv, proj, fc1, fc2: Int8Linear.  q_norm_w / k_norm_w: [head_dim] bf16."""

    def __init__(self, qkv, proj, fc1, fc2, q_norm_w, k_norm_w, heads):
        self.qkv, self.proj, self.fc1, self.fc2 = qkv, proj, fc1, fc2
        self.q_norm_w, self.k_norm_w = q_norm_w, k_norm_w
        self.heads = heads

    def attention_inputs(self, x, shift1, scale1, rope=None):
        """adaLN + int8 quantization shared by q/k/v -> one QKV GEMM -> QK-norm (+RoPE).  x [B, L, D]."""
        b, n, d = x.shape
        qa, sa = kernels.adaln_quant(x, shift1, scale1)
        qkv = kernels.block_gemm(qa, sa, self.qkv.qw, self.qkv.sw, self.qkv.bias, out_dtype=x.dtype)
        qkv = qkv.view(b, n, 3, self.heads, d // self.heads)
        q = fused.qk_norm_rope(qkv[:, :, 0], self.q_norm_w, rope)
        k = fused.qk_norm_rope(qkv[:, :, 1], self.k_norm_w, rope)
        v = qkv[:, :, 2]
        return q, k, v

    def post(self, x, attn, gate1, shift2, scale2, gate2):
        """Out-projection + gated residual, then the MLP half with its gated residual.  attn [B, L, D]."""
        x = fused.gated_residual(x, kernels.block_linear(attn, self.proj.qw, self.proj.sw, self.proj.bias), gate1)
        qa, sa = kernels.adaln_quant(x, shift2, scale2)
        qh, sh = kernels.block_gemm(qa, sa, self.fc1.qw, self.fc1.sw, self.fc1.bias, epilogue="gelu_quant")
        h = kernels.block_gemm(qh, sh, self.fc2.qw, self.fc2.sw, self.fc2.bias, out_dtype=x.dtype)
        return fused.gated_residual(x, h.view_as(x), gate2)

    def forward(self, x, mods, rope=None):
        """Self-attention over this stream only (torch SDPA, unchanged), then `post`."""
        shift1, scale1, gate1, shift2, scale2, gate2 = mods
        q, k, v = self.attention_inputs(x, shift1, scale1, rope)
        attn = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2),
                                              v.transpose(1, 2).contiguous())
        attn = attn.transpose(1, 2).reshape(x.shape)
        return self.post(x, attn, gate1, shift2, scale2, gate2)
