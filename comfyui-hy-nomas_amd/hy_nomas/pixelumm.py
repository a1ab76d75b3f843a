"""PixelUMM decoder FP8 weights: e4m3fn codes with one fp32 scale per 128x128 block, and the Linear that
runs them on the gfx950 fp8 matrix cores (the FP8 layout and dispatch of the reference's
`hy_nomas/pixelumm.py:56-158`; the decoder model itself is not part of this package).
"""
import torch
import torch.nn.functional as F

from . import kernels

FP8_FORMAT = "pixelumm_fp8_bf16_single_v1"
FP8_LAYOUT = "NomasFP8Block128Layout"


def quantize_fp8_block(tensor):
    """w [N, K] (multiples of 128) -> (e4m3fn codes [N, K], fp32 scales [N/128, K/128]): absmax per block,
    clamped at 1e-4, over 448 (hy_nomas/pixelumm.py:77-82)."""
    n, k = tensor.shape
    blocks = tensor.float().view(n // 128, 128, k // 128, 128)
    s = blocks.abs().amax(dim=(1, 3)).clamp_min(1e-4) / 448.0
    q = (blocks / s[:, None, :, None]).to(torch.float8_e4m3fn).view(n, k)
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
