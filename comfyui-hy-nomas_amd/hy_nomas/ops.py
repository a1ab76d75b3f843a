"""Tencent's INT8 DiT weight layout and the Linear that runs it on the MI355X int8 matrix cores.

Drop-in for the reference's `hy_nomas/ops.py`.  Each Linear stores `weight_q` (int8 [N, K]) and
`weight_scale` (fp32 [N, ceil(K / 128)]): symmetric absmax per output row and 128-wide input group.
The Linear picks the matmul:

* `exact`: dequantize to the activation dtype, `F.linear` (the reference's arithmetic).
* `int8`: W8A8 on the int8 matrix cores (`kernels.int8_g128_linear`), activations quantized per token and
  per 128-group so the weight groups stay intact.

With ComfyUI importable, `NomasOps` extends `comfy.ops.manual_cast` exactly like the reference (quantized
weights are `QuantizedTensor`s of the registered layout).  Without it, `NomasOps` is a plain torch
module family with the same interface (`with_matmul`, `Linear.forward`, `fast_int8`, `int8_weights`), and
the quantized weight is a small `Int8G128Weight` holder with the same `_qdata` / `_params.scale` fields.
"""
import contextlib
import dataclasses
import json
import logging
import os

import torch
import torch.nn.functional as F

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

GROUP = 128
LAYOUT = "NomasInt8G128Layout"
# "exact" | "int8"; the loader sets it per model, the env var overrides for benchmarks
MATMUL_ENV = "HY_NOMAS_MATMUL"


def quantize_g128(weight):
    """Symmetric per-row, per-128-column-group int8, half away from zero (hy_nomas/ops.py:41-52).

    Device tensors with K % 128 == 0 run the activation quantization kernel (the same rule); other
    inputs use torch arithmetic with the same fp32 steps."""
    n, k = weight.shape
    if weight.is_cuda and k % GROUP == 0 and weight.dtype in (torch.bfloat16, torch.float16, torch.float32) and n:
        from .kernels import quantize_activations
        return quantize_activations(weight, "int8", GROUP)
    groups = (k + GROUP - 1) // GROUP
    padded = F.pad(weight.float(), (0, groups * GROUP - k))
    rows = padded.reshape(n, groups, GROUP)
    peak = rows.abs().amax(dim=-1)
    scale = torch.where(peak > 0, peak / 127.0, torch.ones_like(peak))
    y = rows / scale.unsqueeze(-1)
    q = torch.where(y >= 0, torch.floor(y + 0.5), torch.ceil(y - 0.5)).clamp_(-127, 127)
    return q.to(torch.int8).reshape(n, -1)[:, :k].contiguous(), scale.contiguous()


def dequantize_g128(qdata, scale, dtype=torch.bfloat16):
    """fp32 product of code and group scale, one cast to `dtype` (hy_nomas/ops.py:55-62)."""
    n, k = qdata.shape
    scale = scale.float()
    if k % GROUP == 0 and scale.shape[1] == k // GROUP:
        weight = (qdata.view(n, k // GROUP, GROUP).float() * scale.unsqueeze(-1)).view(n, k)
    else:
        weight = qdata.float() * scale.repeat_interleave(GROUP, dim=1)[:, :k]
    return weight.to(dtype)


@dataclasses.dataclass(frozen=True)
class _Params:
    scale: torch.Tensor
    orig_dtype: torch.dtype
    orig_shape: tuple


class Int8G128Weight:
    """A quantized weight without ComfyUI: int8 codes `_qdata` [N, K] and `_params.scale` [N, K/128]."""

    def __init__(self, qdata, scale, dtype=torch.bfloat16):
        self._qdata = qdata
        self._params = _Params(scale=scale, orig_dtype=dtype, orig_shape=tuple(qdata.shape))

    @property
    def shape(self):
        return self._qdata.shape

    @property
    def device(self):
        return self._qdata.device

    def to(self, device=None, **kwargs):
        return Int8G128Weight(self._qdata.to(device), self._params.scale.to(device), self._params.orig_dtype)

    def dequantize(self):
        return dequantize_g128(self._qdata, self._params.scale, self._params.orig_dtype)


if _CK:
    class NomasInt8G128Layout(QuantizedLayout):
        MIN_SM_VERSION = None

        @dataclasses.dataclass(frozen=True)
        class Params(BaseLayoutParams):
            pass

        @classmethod
        def quantize(cls, tensor, scale=None, **kwargs):
            q, s = quantize_g128(tensor)
            return q, cls.Params(scale=s, orig_dtype=tensor.dtype, orig_shape=tuple(tensor.shape))

        @classmethod
        def dequantize(cls, qdata, params):
            return dequantize_g128(qdata, params.scale, params.orig_dtype)

        @classmethod
        def get_plain_tensors(cls, qtensor):
            return qtensor._qdata, qtensor._params.scale

        @classmethod
        def state_dict_tensors(cls, qdata, params):
            return {"_q": qdata, "_scale": params.scale}

    register_layout_class(LAYOUT, NomasInt8G128Layout)


def make_weight(qdata, scale, dtype=torch.bfloat16):
    """The quantized weight object a Linear holds (a ComfyUI QuantizedTensor when ComfyUI is present)."""
    if _COMFY and _CK:
        params = NomasInt8G128Layout.Params(scale=scale, orig_dtype=dtype, orig_shape=tuple(qdata.shape))
        return QuantizedTensor(qdata, LAYOUT, params)
    if _COMFY:
        raise RuntimeError("Hy-Nomas INT8 weights need comfy-kitchen (it ships with ComfyUI)")
    return Int8G128Weight(qdata, scale, dtype)


def is_quantized(weight):
    if _COMFY:
        return isinstance(weight, QuantizedTensor)
    return isinstance(weight, Int8G128Weight)


def matmul_mode(default="exact"):
    return os.environ.get(MATMUL_ENV, default)


def _load_linear(self, state_dict, prefix, missing_keys, error_msgs):
    """Shared state-dict loading of `weight_q` + `weight_scale` (or a plain `weight`) and `bias`
    (hy_nomas/ops.py:129-154)."""
    q = state_dict.pop(prefix + "weight_q", None)
    scale = state_dict.pop(prefix + "weight_scale", None)
    plain = state_dict.pop(prefix + "weight", None)
    bias = state_dict.pop(prefix + "bias", None)
    if q is not None:
        if scale is None:
            error_msgs.append(f"{prefix}weight_q without {prefix}weight_scale")
            return None, None, False
        if tuple(q.shape) != (self.out_features, self.in_features):
            error_msgs.append(f"{prefix}weight_q has shape {tuple(q.shape)}, expected "
                              f"{(self.out_features, self.in_features)}")
            return None, None, False
        weight = make_weight(q, scale.float(), self._dtype or torch.bfloat16)
    elif plain is not None:
        weight = plain if self._dtype is None else plain.to(self._dtype)
    else:
        missing_keys.append(prefix + "weight")
        return None, None, False
    if bias is not None:
        bias = bias if self._dtype is None else bias.to(self._dtype)
    elif self._has_bias:
        missing_keys.append(prefix + "bias")
    return weight, bias, True


def _linear_forward(self, input, weight, bias):
    """int8 matrix-core path or the exact dequantize + F.linear path (hy_nomas/ops.py:167-176)."""
    if is_quantized(weight):
        mode = self.matmul or matmul_mode(self.default_matmul)
        qdata, scale = weight._qdata, weight._params.scale
        if mode == "int8" and input.is_cuda:
            from .kernels import int8_g128_linear
            return int8_g128_linear(input, qdata, scale, bias)
        weight = dequantize_g128(qdata, scale, input.dtype)
    return F.linear(input, weight, bias)


if _COMFY:
    class NomasOps(comfy.ops.manual_cast):
        """ComfyUI's cast-on-use ops with a Linear that also loads `weight_q`/`weight_scale` pairs."""

        @classmethod
        def with_matmul(cls, matmul):
            linear = type("Linear", (cls.Linear,), {"default_matmul": matmul})
            return type(f"NomasOps_{matmul}", (cls,), {"Linear": linear})

        class Linear(comfy.ops.manual_cast.Linear):
            default_matmul = "exact"

            def __init__(self, in_features, out_features, bias=True, device=None, dtype=None):
                torch.nn.Module.__init__(self)
                self.in_features = in_features
                self.out_features = out_features
                self.weight = None
                self.bias = None
                self._has_bias = bias
                self._dtype = dtype
                self.matmul = None

            def reset_parameters(self):
                return None

            def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs):
                weight, bias, ok = _load_linear(self, state_dict, prefix, missing_keys, error_msgs)
                if not ok:
                    return
                self.weight = torch.nn.Parameter(weight, requires_grad=False)
                if bias is not None:
                    self.bias = torch.nn.Parameter(bias, requires_grad=False)

            def convert_weight(self, weight, inplace=False, **kwargs):
                return weight.dequantize() if isinstance(weight, QuantizedTensor) else weight

            def set_weight(self, weight, inplace_update=False, seed=None, return_weight=False, **kwargs):
                if isinstance(self.weight, QuantizedTensor):
                    q, s = quantize_g128(weight)
                    weight = make_weight(q, s, self.weight._params.orig_dtype)
                if return_weight:
                    return weight
                self.weight = torch.nn.Parameter(weight, requires_grad=False)

            def forward_comfy_cast_weights(self, input):
                with comfy.ops.CastBiasWeightContext(self, input, offloadable=True) as (weight, bias):
                    return _linear_forward(self, input, weight, bias)

            def forward(self, *args, **kwargs):
                return self.forward_comfy_cast_weights(*args, **kwargs)

            def fast_int8(self, input):
                """Whether this linear can take pre-quantized int8 activations (`int8_weights`)."""
                return (isinstance(self.weight, QuantizedTensor) and input.is_cuda
                        and (self.matmul or matmul_mode(self.default_matmul)) == "int8"
                        and not self.weight_function and not self.bias_function)

            @contextlib.contextmanager
            def int8_weights(self, input):
                """(int8 codes, scales, bias) on the input's device, cast the way the rest of ComfyUI casts."""
                with comfy.ops.CastBiasWeightContext(self, input, offloadable=True) as (weight, bias):
                    yield weight._qdata, weight._params.scale, bias
else:
    class NomasOps:
        """Standalone op family (no ComfyUI): `NomasOps.Linear`, `with_matmul`, same Linear interface."""

        @classmethod
        def with_matmul(cls, matmul):
            linear = type("Linear", (cls.Linear,), {"default_matmul": matmul})
            return type(f"NomasOps_{matmul}", (cls,), {"Linear": linear})

        class Linear(torch.nn.Module):
            default_matmul = "exact"

            def __init__(self, in_features, out_features, bias=True, device=None, dtype=None):
                super().__init__()
                self.in_features = in_features
                self.out_features = out_features
                self.weight = None
                self.bias = None
                self._has_bias = bias
                self._dtype = dtype
                self.matmul = None

            def reset_parameters(self):
                return None

            def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs):
                weight, bias, ok = _load_linear(self, state_dict, prefix, missing_keys, error_msgs)
                if not ok:
                    return
                self.weight = weight if is_quantized(weight) else torch.nn.Parameter(weight, requires_grad=False)
                if bias is not None:
                    self.bias = torch.nn.Parameter(bias, requires_grad=False)

            def to(self, *args, **kwargs):
                super().to(*args, **kwargs)
                if is_quantized(self.weight):
                    device = torch._C._nn._parse_to(*args, **kwargs)[0]
                    if device is not None:
                        self.weight = self.weight.to(device)
                return self

            def set_weight(self, weight, return_weight=False, **kwargs):
                if is_quantized(self.weight):
                    q, s = quantize_g128(weight)
                    weight = make_weight(q, s, self.weight._params.orig_dtype)
                if return_weight:
                    return weight
                self.weight = weight if is_quantized(weight) else torch.nn.Parameter(weight, requires_grad=False)

            def _on_device(self, input):
                weight = self.weight
                if is_quantized(weight) and weight.device != input.device:
                    weight = weight.to(input.device)
                elif not is_quantized(weight):
                    weight = weight.to(device=input.device, dtype=input.dtype)
                bias = self.bias.to(device=input.device, dtype=input.dtype) if self.bias is not None else None
                return weight, bias

            def forward(self, input):
                weight, bias = self._on_device(input)
                return _linear_forward(self, input, weight, bias)

            def fast_int8(self, input):
                return (is_quantized(self.weight) and input.is_cuda
                        and (self.matmul or matmul_mode(self.default_matmul)) == "int8")

            @contextlib.contextmanager
            def int8_weights(self, input):
                weight, bias = self._on_device(input)
                yield weight._qdata, weight._params.scale, bias


def quantized_linears(module):
    return [m for m in module.modules() if isinstance(m, NomasOps.Linear) and is_quantized(m.weight)]


def describe(module):
    linears = quantized_linears(module)
    size = sum(m.weight._qdata.numel() for m in linears)
    logging.info("Hy-Nomas: %d int8 g128 linears (%.2f G weights)", len(linears), size / 1e9)
    return json.dumps({"int8_linears": len(linears)})
