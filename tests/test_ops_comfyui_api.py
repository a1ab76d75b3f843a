"""`ops.NomasOps` on the ComfyUI side of the module (hy_nomas/ops.py:104-191), which needs ComfyUI and
comfy-kitchen to import.  Neither is installed here, so this test supplies a stand-in of exactly the names the
module uses:
- `comfy.model_management`;
- `comfy.ops.manual_cast` with its `Linear`, and `comfy.ops.CastBiasWeightContext`;
- `comfy.quant_ops.QuantizedTensor`: a tensor subclass holding `_qdata`, `_layout` and `_params`, which
  dequantizes through its registered layout;
- `comfy_kitchen.tensor`: `BaseLayoutParams`, `QuantizedLayout`, `register_layout_class`.

It then loads a fresh `hy_nomas.ops` against them and runs the subclass on the CPU.  The stand-in is test
infrastructure: it pins the logic of the ComfyUI branch (state-dict loading into the registered layout, the
cast context, exact forward, weight conversion and re-quantization, the matmul variants), not ComfyUI's own
behaviour."""
import dataclasses
import importlib
import sys
import types

import pytest
import torch
import torch.nn.functional as F

LAYOUTS = {}
CASTS = []


@dataclasses.dataclass(frozen=True)
class BaseLayoutParams:
    scale: torch.Tensor
    orig_dtype: torch.dtype
    orig_shape: tuple


class QuantizedLayout:
    pass


def register_layout_class(name, cls):
    LAYOUTS[name] = cls


class QuantizedTensor(torch.Tensor):
    """Codes + layout parameters behind a tensor of the original shape and dtype (no data of its own)."""

    @staticmethod
    def __new__(cls, qdata, layout, params):
        t = torch.Tensor._make_wrapper_subclass(cls, qdata.shape, dtype=params.orig_dtype, device=qdata.device,
                                                requires_grad=False)
        t._qdata, t._layout, t._params = qdata, layout, params
        return t

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        if func is torch.ops.aten.detach.default:
            x = args[0]
            return QuantizedTensor(x._qdata, x._layout, x._params)
        raise NotImplementedError(f"{func} is not part of the stand-in")

    def dequantize(self):
        return LAYOUTS[self._layout].dequantize(self._qdata, self._params)


class CastBiasWeightContext:
    """The module's weight and bias for this input: quantized weights as they are, others in its dtype."""

    def __init__(self, module, input, offloadable=False):
        self.module, self.input = module, input

    def __enter__(self):
        CASTS.append(type(self.module).__name__)
        w, b = self.module.weight, self.module.bias
        if not isinstance(w, QuantizedTensor):
            w = w.to(self.input.dtype)
        return w, (b.to(self.input.dtype) if b is not None else None)

    def __exit__(self, *exc):
        return False


class _ManualCast:
    class Linear(torch.nn.Linear):
        comfy_cast_weights = True
        weight_function = []
        bias_function = []


@pytest.fixture
def comfy_ops(monkeypatch):
    comfy = types.ModuleType("comfy")
    mm = types.ModuleType("comfy.model_management")
    cops = types.ModuleType("comfy.ops")
    cops.manual_cast = _ManualCast
    cops.CastBiasWeightContext = CastBiasWeightContext
    qops = types.ModuleType("comfy.quant_ops")
    qops.QuantizedTensor = QuantizedTensor
    comfy.model_management, comfy.ops, comfy.quant_ops = mm, cops, qops
    ck = types.ModuleType("comfy_kitchen")
    ckt = types.ModuleType("comfy_kitchen.tensor")
    ckt.BaseLayoutParams, ckt.QuantizedLayout, ckt.register_layout_class = (BaseLayoutParams, QuantizedLayout,
                                                                            register_layout_class)
    ck.tensor = ckt
    for name, mod in (("comfy", comfy), ("comfy.model_management", mm), ("comfy.ops", cops),
                      ("comfy.quant_ops", qops), ("comfy_kitchen", ck), ("comfy_kitchen.tensor", ckt)):
        monkeypatch.setitem(sys.modules, name, mod)
    saved = sys.modules.pop("hy_nomas.ops", None)
    import hy_nomas
    saved_attr = getattr(hy_nomas, "ops", None)
    try:
        ops = importlib.import_module("hy_nomas.ops")
        assert ops._COMFY and ops._CK
        LAYOUTS.clear()
        CASTS.clear()
        importlib.reload(ops)  # registers the layout with this test's registry
        yield ops
    finally:
        sys.modules.pop("hy_nomas.ops", None)
        if saved is not None:
            sys.modules["hy_nomas.ops"] = saved
        if saved_attr is not None:
            hy_nomas.ops = saved_attr


def _weights(n, k, seed):
    """A float weight [n, k] and a bf16 bias [n]."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n, k, generator=g) * 0.05
    return w, (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16)


def test_comfyui_linear_loads_the_layout_and_runs_the_exact_path(comfy_ops, monkeypatch):
    ops = comfy_ops
    monkeypatch.delenv(ops.MATMUL_ENV, raising=False)
    n, k = 48, 256
    w, bias = _weights(n, k, 3)
    q, s = ops.quantize_g128(w)
    lin = ops.NomasOps.Linear(k, n, dtype=torch.bfloat16)
    assert isinstance(lin, torch.nn.Linear) and lin.weight is None
    missing, unexpected, errors = [], [], []
    lin._load_from_state_dict({"l.weight_q": q, "l.weight_scale": s, "l.bias": bias}, "l.", {}, True, missing,
                              unexpected, errors)
    assert not missing and not errors
    assert isinstance(lin.weight, QuantizedTensor) and lin.weight._layout == ops.LAYOUT
    assert isinstance(lin.weight, torch.nn.Parameter) and not lin.weight.requires_grad
    assert LAYOUTS[ops.LAYOUT] is ops.NomasInt8G128Layout
    assert torch.equal(lin.weight._qdata, q) and torch.equal(lin.weight._params.scale, s.float())
    assert lin.weight._params.orig_dtype == torch.bfloat16 and lin.weight.shape == (n, k)

    x = torch.randn(5, k, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    CASTS.clear()
    y = lin(x)
    assert CASTS == ["Linear"]  # forward goes through ComfyUI's cast context
    assert torch.equal(y, F.linear(x, ops.dequantize_g128(q, s, torch.bfloat16), bias))
    # the int8 variant on a host tensor also takes the exact path (the matrix cores need device tensors)
    lin8 = ops.NomasOps.with_matmul("int8").Linear(k, n, dtype=torch.bfloat16)
    assert lin8.default_matmul == "int8" and issubclass(ops.NomasOps.with_matmul("int8"), ops.NomasOps)
    lin8._load_from_state_dict({"weight_q": q, "weight_scale": s, "bias": bias}, "", {}, True, [], [], [])
    assert not lin8.fast_int8(x)
    assert torch.equal(lin8(x), y)


def test_comfyui_linear_weight_conversion_and_requantization(comfy_ops):
    ops = comfy_ops
    n, k = 32, 384
    w, bias = _weights(n, k, 5)
    q, s = ops.quantize_g128(w)
    lin = ops.NomasOps.Linear(k, n, dtype=torch.bfloat16)
    lin._load_from_state_dict({"weight_q": q, "weight_scale": s, "bias": bias}, "", {}, True, [], [], [])
    plain = lin.convert_weight(lin.weight)
    assert torch.equal(plain, ops.dequantize_g128(q, s, torch.bfloat16))
    assert lin.convert_weight(plain) is plain
    # a patched weight (e.g. a LoRA merge) is re-quantized into the same layout
    w2 = w + 0.01
    ret = lin.set_weight(w2, return_weight=True)
    q2, s2 = ops.quantize_g128(w2)
    assert isinstance(ret, QuantizedTensor) and torch.equal(ret._qdata, q2) and torch.equal(ret._params.scale, s2)
    assert torch.equal(lin.weight._qdata, q)  # return_weight leaves the module as it was
    lin.set_weight(w2)
    assert isinstance(lin.weight, QuantizedTensor) and torch.equal(lin.weight._qdata, q2)
    assert ops.quantized_linears(torch.nn.Sequential(lin)) == [lin]
    assert '"int8_linears": 1' in ops.describe(torch.nn.Sequential(lin))
    # the layout class round-trips its own quantization
    qq, params = ops.NomasInt8G128Layout.quantize(w)
    assert torch.equal(qq, q) and params.orig_shape == (n, k)
    assert torch.equal(ops.NomasInt8G128Layout.dequantize(qq, params), ops.dequantize_g128(q, s, w.dtype))
    qt = ops.make_weight(q, s)
    assert ops.NomasInt8G128Layout.get_plain_tensors(qt)[0] is q
    assert set(ops.NomasInt8G128Layout.state_dict_tensors(q, params)) == {"_q", "_scale"}


def test_comfyui_linear_plain_weights_and_load_errors(comfy_ops):
    ops = comfy_ops
    n, k = 16, 128
    w, bias = _weights(n, k, 7)
    lin = ops.NomasOps.Linear(k, n, dtype=torch.bfloat16)
    lin._load_from_state_dict({"weight": w, "bias": bias}, "", {}, True, [], [], [])
    assert not isinstance(lin.weight, QuantizedTensor) and lin.weight.dtype == torch.bfloat16
    x = torch.randn(3, k).to(torch.bfloat16)
    assert torch.equal(lin(x), F.linear(x, w.to(torch.bfloat16), bias))
    q, s = ops.quantize_g128(w)
    errors, missing = [], []
    ops.NomasOps.Linear(k, n)._load_from_state_dict({"weight_q": q}, "", {}, True, missing, [], errors)
    assert errors and "weight_scale" in errors[0]
    errors = []
    ops.NomasOps.Linear(k + 128, n)._load_from_state_dict({"weight_q": q, "weight_scale": s}, "", {}, True, [], [],
                                                          errors)
    assert errors and "shape" in errors[0]
    missing = []
    ops.NomasOps.Linear(k, n)._load_from_state_dict({"bias": bias}, "", {}, True, missing, [], [])
    assert missing == ["weight"]
