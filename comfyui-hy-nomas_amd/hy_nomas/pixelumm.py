"""PixelUMM decoder FP8 weights: e4m3fn codes with one fp32 scale per 128x128 block, the Linear that
runs them on the gfx950 fp8 matrix cores, the decoder's SwiGLU MLP with its gate and up projections in one
GEMM, and the checkpoint reader (the FP8 layout, dispatch, MLP and loader of the reference's
`hy_nomas/pixelumm.py:35-158, 314-323, 470-485`; the rest of the decoder model is not part of this
package).

With ComfyUI importable, `DecoderOps` extends `comfy.ops.manual_cast` as the reference's does, and its fp8
weights are `QuantizedTensor`s of the registered `NomasFP8Block128Layout` (when comfy-kitchen is present).
Without it, `DecoderOps` is a plain torch module family with the same interface.  Either way the fp8 matmul
reads the [N/128, K/128] block scales as stored; the reference expands them per output channel
(`scale.repeat_interleave(128, 0)`, pixelumm.py:153), which makes the GEMM fold every channel's scale
separately.  Block scales are checked once, when a Linear loads them (positive and finite, on the host
tensor), and the per-call device copies inherit that verdict, so no forward waits for the device.
"""
import dataclasses

import torch
import torch.nn.functional as F

from . import kernels

try:
    import comfy.model_management  # noqa: F401
    import comfy.ops
    from comfy.quant_ops import QuantizedTensor
    _COMFY = True
except ImportError:
    _COMFY = False

try:
    from comfy_kitchen.tensor import BaseLayoutParams, QuantizedLayout, register_layout_class
    _CK = True
except ImportError:
    _CK = False

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


if _CK:
    class NomasFP8Block128Layout(QuantizedLayout):
        """The decoder's FP8 weights as a comfy-kitchen layout (hy_nomas/pixelumm.py:65-96): e4m3fn codes with
        one fp32 scale per 128 x 128 block, saved as `<name>.fp8_weight` / `<name>.fp8_scale`."""
        MIN_SM_VERSION = None

        @dataclasses.dataclass(frozen=True)
        class Params(BaseLayoutParams):
            pass

        @classmethod
        def quantize(cls, tensor, scale=None, **kwargs):
            q, s = quantize_fp8_block(tensor)
            return q, cls.Params(scale=s, orig_dtype=tensor.dtype, orig_shape=tuple(tensor.shape))

        @classmethod
        def dequantize(cls, qdata, params):
            return dequantize_fp8_block(qdata, params.scale, params.orig_dtype)

        @classmethod
        def get_plain_tensors(cls, qtensor):
            return qtensor._qdata, qtensor._params.scale

        @classmethod
        def state_dict_tensors(cls, qdata, params):
            return {".fp8_weight": qdata, ".fp8_scale": params.scale}

    register_layout_class(FP8_LAYOUT, NomasFP8Block128Layout)
else:
    NomasFP8Block128Layout = None


def _scales_ok(lin, scale):
    """Whether the linear's stored block scales are positive and finite: decided once per stored tensor and
    in-place version (`kernels.validate_scales`; at load time the tensor is the checkpoint's host copy, so the
    check does not touch the device)."""
    if lin._scale_src is not scale or lin._scale_version != scale._version:
        lin._scale_ok = kernels.validate_scales(scale)
        lin._scale_src, lin._scale_version = scale, scale._version
    return lin._scale_ok


def _load_fp8_pair(lin, state_dict, prefix, missing_keys):
    """(codes, fp32 block scales, plain weight, bias) from `fp8_weight` / `fp8_scale` or `weight`, and `bias`
    (hy_nomas/pixelumm.py:128-143); the plain weight and the bias in the layer dtype.  None for a missing
    weight (reported in `missing_keys`)."""
    q = state_dict.pop(prefix + "fp8_weight", None)
    s = state_dict.pop(prefix + "fp8_scale", None)
    w = state_dict.pop(prefix + "weight", None)
    b = state_dict.pop(prefix + "bias", None)
    if q is None and w is None:
        missing_keys.append(prefix + "weight")
        return None
    if q is not None and s is None:
        missing_keys.append(prefix + "fp8_scale")
        return None
    if q is not None:
        s = s.float()
        _scales_ok(lin, s)
        w = None
    elif lin._dtype is not None:
        w = w.to(lin._dtype)
    if b is not None:
        b = b.to(lin._dtype) if lin._dtype is not None else b
    elif lin._has_bias:
        missing_keys.append(prefix + "bias")
    return q, s, w, b


def _fp8_forward(lin, input, qdata, scale, stored_scale, bias):
    """F.linear on fp8 block weights: the fp8 matrix-core GEMM with the block scales as stored (a device
    copy of checked scales inherits their verdict), or dequantize + F.linear (pixelumm.py:147-155)."""
    if lin.matmul == "fp8" and input.is_cuda:
        if _scales_ok(lin, stored_scale):
            kernels.trust_scales(scale)
        return fp8_block_linear(input, qdata, scale, bias)
    return F.linear(input, dequantize_fp8_block(qdata, scale, input.dtype), bias)


def _init_linear(lin, in_features, out_features, bias, dtype):
    lin.in_features, lin.out_features = in_features, out_features
    lin.weight = None
    lin.bias = None
    lin._has_bias = bias
    lin._dtype = dtype
    lin._scale_src, lin._scale_version, lin._scale_ok = None, None, False


if _COMFY:
    class DecoderOps(comfy.ops.manual_cast):
        """ComfyUI's cast-on-use ops with a Linear that also loads `fp8_weight` / `fp8_scale` pairs into
        `QuantizedTensor`s of the FP8 block-128 layout.  `matmul`: "dequant" runs bf16 GEMMs on dequantized
        weights, "fp8" the fp8 matrix-core GEMM (activations quantized per token and 128 channels)."""

        @classmethod
        def with_matmul(cls, matmul):
            linear = type("Linear", (cls.Linear,), {"matmul": matmul})
            return type(f"DecoderOps_{matmul}", (cls,), {"Linear": linear})

        class Linear(comfy.ops.manual_cast.Linear):
            matmul = "dequant"

            def __init__(self, in_features, out_features, bias=True, device=None, dtype=None):
                torch.nn.Module.__init__(self)
                _init_linear(self, in_features, out_features, bias, dtype)

            def reset_parameters(self):
                return None

            def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs):
                got = _load_fp8_pair(self, state_dict, prefix, missing_keys)
                if got is None:
                    return
                q, s, w, b = got
                if q is not None:
                    if NomasFP8Block128Layout is None:
                        raise RuntimeError("PixelUMM FP8 weights need comfy-kitchen (it ships with ComfyUI)")
                    params = NomasFP8Block128Layout.Params(scale=s, orig_dtype=self._dtype or torch.bfloat16,
                                                           orig_shape=tuple(q.shape))
                    w = QuantizedTensor(q, FP8_LAYOUT, params)
                self.weight = torch.nn.Parameter(w, requires_grad=False)
                if b is not None:
                    self.bias = torch.nn.Parameter(b, requires_grad=False)

            def forward_comfy_cast_weights(self, input):
                with comfy.ops.CastBiasWeightContext(self, input, offloadable=True) as (weight, bias):
                    if isinstance(weight, QuantizedTensor):
                        return _fp8_forward(self, input, weight._qdata, weight._params.scale,
                                            self.weight._params.scale, bias)
                    return F.linear(input, weight, bias)

            def forward(self, *args, **kwargs):
                return self.forward_comfy_cast_weights(*args, **kwargs)

            def fp8_parts(self):
                """(codes, block scales) as stored, or None for a plain weight."""
                if isinstance(self.weight, QuantizedTensor):
                    return self.weight._qdata, self.weight._params.scale
                return None
else:
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
                _init_linear(self, in_features, out_features, bias, dtype)
                self.scale = None

            def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs):
                got = _load_fp8_pair(self, state_dict, prefix, missing_keys)
                if got is None:
                    return
                q, s, w, b = got
                self.weight, self.scale = (q, s) if q is not None else (w, None)
                if b is not None:
                    self.bias = b

            def forward(self, input):
                weight = self.weight.to(input.device)
                bias = self.bias.to(device=input.device, dtype=input.dtype) if self.bias is not None else None
                if self.scale is not None:
                    return _fp8_forward(self, input, weight, self.scale.to(input.device), self.scale, bias)
                return F.linear(input, weight.to(input.dtype), bias)

            def fp8_parts(self):
                """(codes, block scales) as stored, or None for a plain weight."""
                return (self.weight, self.scale) if self.scale is not None else None


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
    if kernels._known_positive_finite(sg) and kernels._known_positive_finite(su):
        kernels.trust_scales(s)  # the same values, rearranged
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
    projections, `matmul == "fp8"`, scales that passed the load-time check, no ComfyUI weight or bias patches
    (LoRA hooks) and a device input, the forward is `swiglu_mlp` (gate and up in one GEMM); otherwise it is
    the reference's expression."""

    def __init__(self, arch, ops, dtype=None, device=None):
        super().__init__()
        kw = dict(dtype=dtype, device=device)
        self.gate_proj = ops.Linear(arch.hidden_size, arch.intermediate_size, bias=False, **kw)
        self.up_proj = ops.Linear(arch.hidden_size, arch.intermediate_size, bias=False, **kw)
        self.down_proj = ops.Linear(arch.intermediate_size, arch.hidden_size, bias=False, **kw)
        self._fused = None

    @staticmethod
    def _fusable(lin):
        parts = lin.fp8_parts() if getattr(lin, "matmul", None) == "fp8" and hasattr(lin, "fp8_parts") else None
        if parts is None or getattr(lin, "weight_function", None) or getattr(lin, "bias_function", None):
            return None
        return parts if _scales_ok(lin, parts[1]) else None

    def _fused_weights(self, device, gate, up):
        key = (device, gate[0].data_ptr(), up[0].data_ptr(), gate[0]._version, up[0]._version, gate[1]._version,
               up[1]._version)
        if self._fused is None or self._fused[0] != key:
            q, s = interleave_gate_up((gate[0].to(device), gate[1].to(device)), (up[0].to(device), up[1].to(device)))
            kernels.trust_scales(s)  # both sources passed the check
            self._fused = (key, (q, s))
        return self._fused[1]

    def forward(self, x):
        parts = [self._fusable(l) for l in (self.gate_proj, self.up_proj, self.down_proj)]
        if x.is_cuda and all(p is not None for p in parts):
            down = (parts[2][0].to(x.device), parts[2][1].to(x.device))
            kernels.trust_scales(down[1])
            return swiglu_mlp(x, self._fused_weights(x.device, parts[0], parts[1]), down)
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
