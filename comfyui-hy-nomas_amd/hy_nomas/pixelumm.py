"""PixelUMM decoder FP8 weights: e4m3fn codes with one fp32 scale per 128x128 block, the Linear that
runs them on the gfx950 fp8 matrix cores, the decoder's SwiGLU MLP with its gate and up projections in one
GEMM, and the checkpoint reader (the FP8 layout, dispatch, MLP and loader of the reference's
`hy_nomas/pixelumm.py:35-158, 314-323, 470-485`; the rest of the decoder model is not part of this
package).
"""
import dataclasses

import torch
import torch.nn.functional as F

from . import kernels

FP8_FORMAT = "pixelumm_fp8_bf16_single_v1"
FP8_LAYOUT = "NomasFP8Block128Layout"


@dataclasses.dataclass(frozen=True)
class Arch:
    """The decoder's shape (hy_nomas/pixelumm.py:40-52)."""
    hidden_size: int = 4096
    intermediate_size: int = 12288
    num_layers: int = 36
    num_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta_t: float = 1_000_000.0
    rope_theta_hw: float = 10_000.0

    @property
    def rope_sections(self):
        return self.head_dim // 2, self.head_dim // 4, self.head_dim // 4


def quantize_fp8_block(tensor):
    """w [N, K] (multiples of 128) -> (e4m3fn codes [N, K], fp32 scales [N/128, K/128]): absmax per block,
    clamped at 1e-4, over 448 (hy_nomas/pixelumm.py:77-82)."""
    n, k = tensor.shape
    blocks = tensor.float().view(n // 128, 128, k // 128, 128)
    s = blocks.abs().amax(dim=(1, 3)).clamp_min(1e-4) / 448.0
    q = (blocks / s[:, None, :, None]).to(torch.float8_e4m3fn).view(n, k)
    kernels.trust_scales(s)
    return q, s


def dequantize_fp8_block(qdata, scale, dtype=torch.bfloat16):
    """hy_nomas/pixelumm.py:60-63: fp32 product of code and block scale, one cast to `dtype`."""
    n, k = qdata.shape
    w = qdata.float().view(n // 128, 128, k // 128, 128) * scale[:, None, :, None]
    return w.view(n, k).to(dtype)


def fp8_block_linear(x, qdata, scale, bias=None):
    """F.linear with fp8 block weights on the fp8 matrix cores, activations quantized to e4m3 per token
    and 128 channels (hy_nomas/pixelumm.py:147-155).  The reference expands the block scales to one row
    per output channel; here the GEMM reads the [N/128, K/128] block scales directly, one scale product
    per token and 128-block in the group fold."""
    return kernels.block_linear(x, qdata, scale, bias, kind="fp8")


class DecoderOps:
    """Linear with `fp8_weight` / `fp8_scale` pairs.  `matmul`: "dequant" runs bf16 GEMMs on dequantized
    weights, "fp8" runs the fp8 matrix-core GEMM."""

    @classmethod
    def with_matmul(cls, matmul):
        linear = type("Linear", (cls.Linear,), {"matmul": matmul})
        return type(f"DecoderOps_{matmul}", (cls,), {"Linear": linear})

    class Linear(torch.nn.Module):
        matmul = "dequant"

        def __init__(self, in_features, out_features, bias=True, device=None, dtype=None):
            super().__init__()
            self.in_features, self.out_features = in_features, out_features
            self.weight = None
            self.scale = None
            self.bias = None
            self._has_bias = bias
            self._dtype = dtype

        def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                                  unexpected_keys, error_msgs):
            q = state_dict.pop(prefix + "fp8_weight", None)
            s = state_dict.pop(prefix + "fp8_scale", None)
            w = state_dict.pop(prefix + "weight", None)
            b = state_dict.pop(prefix + "bias", None)
            if q is not None:
                self.weight, self.scale = q, s.float()
            elif w is not None:
                self.weight = w.to(self._dtype) if self._dtype is not None else w
            else:
                missing_keys.append(prefix + "weight")
                return
            if b is not None:
                self.bias = b.to(self._dtype) if self._dtype is not None else b
            elif self._has_bias:
                missing_keys.append(prefix + "bias")

        def forward(self, input):
            weight = self.weight.to(input.device)
            bias = self.bias.to(device=input.device, dtype=input.dtype) if self.bias is not None else None
            if self.scale is not None:
                scale = self.scale.to(input.device)
                if self.matmul == "fp8" and input.is_cuda:
                    return fp8_block_linear(input, weight, scale, bias)
                weight = dequantize_fp8_block(weight, scale, input.dtype)
            return F.linear(input, weight.to(input.dtype), bias)


def interleave_gate_up(gate, up):
    """(codes, block scales) of gate_proj and up_proj, [I, K] + [I/128, K/128] each -> the weight of the
    fused SwiGLU GEMM: 128-row blocks alternating gate, up ([2I, K], [2I/128, K/128]).  A GEMM tile of 256
    weight rows then holds the gate and up rows of the same 128 MLP channels."""
    (qg, sg), (qu, su) = gate, up
    i, k = qg.shape
    if qu.shape != qg.shape or su.shape != sg.shape or i % 128 or sg.shape[0] != i // 128:
        raise RuntimeError(f"interleave_gate_up: gate {tuple(qg.shape)}/{tuple(sg.shape)} and up "
                           f"{tuple(qu.shape)}/{tuple(su.shape)} are not matching 128x128 block weights")
    as_bytes = (lambda t: t.view(torch.uint8)) if qg.element_size() == 1 else (lambda t: t)
    q = torch.stack((as_bytes(qg).reshape(i // 128, 128, k), as_bytes(qu).reshape(i // 128, 128, k)), dim=1)
    q = q.reshape(2 * i, k).view(qg.dtype)
    s = torch.stack((sg.float(), su.float()), dim=1).reshape(2 * i // 128, sg.shape[1]).contiguous()
    return q, s


def swiglu_mlp(x, gate_up, down, bias=None):
    """down_proj(silu(gate_proj(x)) * up_proj(x)) on fp8 block weights (hy_nomas/pixelumm.py:314-323):
    x quantized to e4m3 once, one GEMM over the interleaved gate/up weight whose epilogue forms
    bf16(bf16(silu(gate)) * up) and quantizes it per token and 128 channels, then the down GEMM.
    The same roundings as the reference's three fp8 linears and torch's bf16 silu and product.
    `gate_up` = interleave_gate_up(...), `down` = (codes [H, I], block scales [H/128, I/128])."""
    q_gu, s_gu = gate_up
    q_d, s_d = down
    lead, k = x.shape[:-1], x.shape[-1]
    x2 = x.reshape(-1, k)
    if x2.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        x2 = x2.to(torch.bfloat16)
    with torch.cuda.device(x.device):
        qa, sa = kernels.quantize_activations(x2, "fp8")
        hq, hs = kernels.block_gemm(qa, sa, q_gu, s_gu, kind="fp8", epilogue="swiglu_quant")
        y = kernels.block_gemm(hq, hs, q_d, s_d, bias, out_dtype=x.dtype, kind="fp8")
    return y.view(*lead, q_d.shape[0])


class MLP(torch.nn.Module):
    """The decoder MLP (hy_nomas/pixelumm.py:314-323) over `ops.Linear`s.  With fp8 weights on all three
    projections, `matmul == "fp8"` and a device input, the forward is `swiglu_mlp` (gate and up in one
    GEMM); otherwise it is the reference's expression."""

    def __init__(self, arch, ops, dtype=None, device=None):
        super().__init__()
        kw = dict(dtype=dtype, device=device)
        self.gate_proj = ops.Linear(arch.hidden_size, arch.intermediate_size, bias=False, **kw)
        self.up_proj = ops.Linear(arch.hidden_size, arch.intermediate_size, bias=False, **kw)
        self.down_proj = ops.Linear(arch.intermediate_size, arch.hidden_size, bias=False, **kw)
        self._fused = None

    def _fused_weights(self, device):
        key = (device, self.gate_proj.weight.data_ptr(), self.up_proj.weight.data_ptr())
        if self._fused is None or self._fused[0] != key:
            gate = (self.gate_proj.weight.to(device), self.gate_proj.scale.to(device))
            up = (self.up_proj.weight.to(device), self.up_proj.scale.to(device))
            self._fused = (key, interleave_gate_up(gate, up))
        return self._fused[1]

    def forward(self, x):
        lins = (self.gate_proj, self.up_proj, self.down_proj)
        if (x.is_cuda and all(getattr(l, "matmul", None) == "fp8" and getattr(l, "scale", None) is not None
                              for l in lins)):
            down = (self.down_proj.weight.to(x.device), self.down_proj.scale.to(x.device))
            return swiglu_mlp(x, self._fused_weights(x.device), down)
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


DECODER_PREFIX = "decoder."


def load_state_dict(path):
    """(state dict, holds FP8 block-128 weights) of a PixelUMM checkpoint: its ``decoder.*`` tensors with the
    prefix removed (the reference's pixelumm.py:470-485).  The tensor names and the metadata come from the
    safetensors header, the tensors from safetensors; nothing in the file executes.  A file without decoder
    tensors raises ValueError."""
    from safetensors import safe_open

    from .loader import read_header

    table, metadata = read_header(path)
    names = [name for name in table if name.startswith(DECODER_PREFIX)]
    if not names:
        raise ValueError(f"{path}: no {DECODER_PREFIX}* tensors, so not a PixelUMM checkpoint")
    with safe_open(path, framework="pt", device="cpu") as handle:
        state = {name[len(DECODER_PREFIX):]: handle.get_tensor(name) for name in names}
    fp8 = metadata.get("format") == FP8_FORMAT or any(name.endswith(".fp8_weight") for name in state)
    return state, fp8


def fp8_state_dict(state, dtype=torch.bfloat16):
    """A float decoder state dict with each 2-D Linear weight whose sides are multiples of 128 replaced by
    its `fp8_weight` / `fp8_scale` pair (the FP8 layout's state_dict_tensors, pixelumm.py:77-94); other
    tensors cast to `dtype`.  Saved with metadata {"format": FP8_FORMAT}, it is the single-file FP8
    format that `load_state_dict` reads."""
    out = {}
    for key, value in state.items():
        if key.endswith(".weight") and value.ndim == 2 and value.shape[0] % 128 == 0 and value.shape[1] % 128 == 0:
            q, s = quantize_fp8_block(value)
            out[key[:-len("weight")] + "fp8_weight"] = q
            out[key[:-len("weight")] + "fp8_scale"] = s
        else:
            out[key] = value.to(dtype) if value.is_floating_point() else value
    return out
