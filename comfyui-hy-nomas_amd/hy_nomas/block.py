"""The DiT double-stream block on the quantized path.

`DiTBlockInt8` wires one stream of `DoubleStreamBlock` (hy_nomas/model.py:246-286) through this package's
kernels: fused LayerNorm/modulate/int8 quantization -> int8 QKV GEMM (q, k, v weights concatenated along
N, which is column-for-column identical to three GEMMs on the same codes) -> QK-RMSNorm + RoPE -> torch
SDPA -> int8 out-projection -> gated residual -> fused norm/quant -> int8 FFN-up with the GELU + int8
requantization epilogue -> int8 FFN-down -> gated residual.
"""
import torch
import torch.nn.functional as F

from . import attention as attn
from . import fused, kernels


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

    def attention_heads(self, x, shift1, scale1, rope=None, out=None, l_offset=0, vt=None):
        """adaLN + int8 quantization -> one QKV GEMM whose epilogue applies QK-norm (+RoPE) and writes q, k, v
        head-major: out [3, B, H, L_total, D] (tokens at l_offset ..).  x [B, L, D].  With `vt` (a V^T buffer of
        the HIP attention), v goes there and out holds q and k."""
        b, n, d = x.shape
        qa, sa = kernels.adaln_quant(x, shift1, scale1, group=self.group)
        return kernels.qkv_heads(qa, sa, self.qkv.qw, self.qkv.sw, self.qkv.bias, self.q_norm_w, self.k_norm_w, b,
                                 rope, out=out, l_offset=l_offset, vt=vt)

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

    def forward(self, x, mods, rope=None, backend=None):
        """Self-attention over this stream only (`attention.attention_heads`: torch SDPA by default, or the HIP
        kernel), then `post`."""
        shift1, scale1, gate1, shift2, scale2, gate2 = mods
        hm = self.attention_heads(x, shift1, scale1, rope)
        out = attn.attention_heads(hm[0], hm[1], hm[2], backend).reshape(x.shape)
        return self.post(x, out, gate1, shift2, scale2, gate2)


class DoubleStreamBlockInt8:
    """The double-stream DiT block on the int8 path (hy_nomas/model.py:230-286): image and text streams with
    their own weights and modulations, one joint attention over the concatenated tokens (image first), then
    each stream's out-projection, gated residuals and MLP.  The image stream gets RoPE; the text stream none.

    img / txt: DiTBlockInt8 halves.  forward(img, txt, img_mods, txt_mods, rope) -> (img, txt)."""

    def __init__(self, img, txt):
        self.img, self.txt = img, txt

    def forward(self, img, txt, img_mods, txt_mods, rope=None, backend=None, history=None, plan=None,
                capture=None):
        """`backend`: the attention backend ("sdpa", "hip"; None: HY_NOMAS_ATTENTION, else "sdpa").
        As the reference's block (hy_nomas/model.py:288-297): `history` is the cached (keys, values) of earlier
        segments, [1 or B, Lh, H, D], or None; `plan` the segment's attention plan (`groups`, `video_tokens`;
        model.py:154-196), or None for every current token attending to every key; `capture(k, v)` is called
        with the current tokens' keys and values [B, L, H, D] (views of the QKV buffer), as the reference hands
        them to the history cache."""
        shift1, scale1, gate1, shift2, scale2, gate2 = img_mods
        tshift1, tscale1, tgate1, tshift2, tscale2, tgate2 = txt_mods
        b, lv = img.shape[0], img.shape[1]
        heads, ltot = self.img.heads, lv + txt.shape[1]
        whole = history is None and getattr(plan, "groups", None) is None
        if (whole and capture is None and attn.choose_backend(backend) == "hip" and img.shape[2] == heads * 128
                and kernels.vt_direct_ok(lv, 0) and kernels.vt_direct_ok(txt.shape[1], lv)):
            # the HIP kernel's operands straight from the QKV epilogues: q and k head-major, v as V^T
            hm = torch.empty((2, b, heads, ltot, 128), device=img.device, dtype=torch.bfloat16)
            vt = attn.values_buffer(b, heads, ltot, img.device)
            self.img.attention_heads(img, shift1, scale1, rope, out=hm, l_offset=0, vt=vt)
            self.txt.attention_heads(txt, tshift1, tscale1, None, out=hm, l_offset=lv, vt=vt)
            out = attn.attention_hip(hm[0].transpose(1, 2), hm[1].transpose(1, 2), vt, ltot)
            del hm, vt
            out = out.reshape(b, ltot, -1)
            img = self.img.post(img, out[:, :lv], gate1, shift2, scale2, gate2)
            txt = self.txt.post(txt, out[:, lv:], tgate1, tshift2, tscale2, tgate2)
            return img, txt
        # both streams' q, k, v land head-major in one buffer, image tokens first (the reference's
        # torch.cat order), so attention runs on it without concatenation or layout copies
        hm = torch.empty((3, b, heads, ltot, img.shape[2] // heads), device=img.device, dtype=torch.bfloat16)
        self.img.attention_heads(img, shift1, scale1, rope, out=hm, l_offset=0)
        self.txt.attention_heads(txt, tshift1, tscale1, None, out=hm, l_offset=lv)
        if capture is not None:
            capture(hm[1].transpose(1, 2), hm[2].transpose(1, 2))
        if whole:
            out = attn.attention_heads(hm[0], hm[1], hm[2], backend)
        else:
            q, k, v = (t.transpose(1, 2) for t in hm)
            out = attn.segment_attention(q, k, v, history, plan, backend=backend)
        del hm
        out = out.reshape(b, out.shape[1], -1)
        img = self.img.post(img, out[:, :lv], gate1, shift2, scale2, gate2)
        txt = self.txt.post(txt, out[:, lv:], tgate1, tshift2, tscale2, tgate2)
        return img, txt
