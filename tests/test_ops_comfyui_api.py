"""`ops.NomasOps` on the ComfyUI side of the module (hy_nomas/ops.py:104-191), which needs ComfyUI and
comfy-kitchen to import.  Neither is installed here, so this test supplies a stand-in of exactly the names the
module uses:
- `comfy.model_management`;
- `comfy.ops.manual_cast` with its `Linear`, and `comfy.ops.CastBiasWeightContext`;
- `comfy.quant_ops.QuantizedTensor`: a tensor subclass holding `_qdata`, `_layout` and `_params`, which
  dequantizes through its registered layout;
- `comfy_kitchen.tensor`: `BaseLayoutParams`, `QuantizedLayout`, `register_layout_class`.

It then loads a fresh `hy_nomas.ops` (and `hy_nomas.pixelumm`, the decoder's FP8 ops) against them and runs
the subclasses on the CPU, and the decoder's fp8 matmul on the GPU.  The stand-in is test infrastructure: it
pins the logic of the ComfyUI branches (state-dict loading into the registered layouts, the cast context,
exact and dequantized forwards, weight conversion and re-quantization, the matmul variants, the block scales
handed to the fp8 GEMM as stored), not ComfyUI's own behaviour."""
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
        dev = self.input.device
        if not isinstance(w, QuantizedTensor):
            w = w.to(device=dev, dtype=self.input.dtype)
        elif w._qdata.device != dev:  # a quantized weight moves as codes + layout parameters
            params = dataclasses.replace(w._params, scale=w._params.scale.to(dev))
            w = QuantizedTensor(w._qdata.to(dev), w._layout, params)
        return w, (b.to(device=dev, dtype=self.input.dtype) if b is not None else None)

    def __exit__(self, *exc):
        return False


class _ManualCast:
    class Linear(torch.nn.Linear):
        comfy_cast_weights = True
        weight_function = []
        bias_function = []


def _install_comfy(monkeypatch):
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


def _fresh_module(monkeypatch, name):
    """A fresh import of hy_nomas.<name> against the stand-in (the package's own module is restored after)."""
    _install_comfy(monkeypatch)
    full = f"hy_nomas.{name}"
    saved = sys.modules.pop(full, None)
    import hy_nomas
    saved_attr = getattr(hy_nomas, name, None)
    try:
        mod = importlib.import_module(full)
        assert mod._COMFY and mod._CK
        LAYOUTS.clear()
        CASTS.clear()
        importlib.reload(mod)  # registers the layout with this test's registry
        yield mod
    finally:
        sys.modules.pop(full, None)
        if saved is not None:
            sys.modules[full] = saved
        if saved_attr is not None:
            setattr(hy_nomas, name, saved_attr)


@pytest.fixture
def comfy_ops(monkeypatch):
    yield from _fresh_module(monkeypatch, "ops")


@pytest.fixture
def comfy_pixelumm(monkeypatch):
    yield from _fresh_module(monkeypatch, "pixelumm")


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


def _fp8_state(n, k, seed, device="cpu"):
    """fp8_weight / fp8_scale / bias of one decoder linear, as the FP8 checkpoint holds them."""
    from hy_nomas import pixelumm

    w, bias = _weights(n, k, seed)
    q, sblk = pixelumm.quantize_fp8_block(w)
    return {"fp8_weight": q.to(device), "fp8_scale": sblk.clone().to(device), "bias": bias.to(device)}


def test_comfyui_decoder_linear_loads_the_fp8_layout_and_dequantizes(comfy_pixelumm):
    """The decoder's Linear on the ComfyUI side (hy_nomas/pixelumm.py:99-158): fp8_weight / fp8_scale load into a
    QuantizedTensor of the registered NomasFP8Block128Layout; the dequant path (and the fp8 variant on a host
    input) is F.linear on the dequantized weight through ComfyUI's cast context; the block scales are checked
    on the host at load; plain weights and missing keys behave as the reference's."""
    px = comfy_pixelumm
    n, k = 256, 384
    sd = _fp8_state(n, k, 11)
    q, sblk, bias = sd["fp8_weight"], sd["fp8_scale"], sd["bias"]
    lin = px.DecoderOps.Linear(k, n, dtype=torch.bfloat16)
    assert isinstance(lin, torch.nn.Linear) and lin.weight is None
    missing = []
    lin._load_from_state_dict({"d.fp8_weight": q, "d.fp8_scale": sblk, "d.bias": bias}, "d.", {}, True, missing,
                              [], [])
    assert not missing
    assert isinstance(lin.weight, QuantizedTensor) and lin.weight._layout == px.FP8_LAYOUT
    assert LAYOUTS[px.FP8_LAYOUT] is px.NomasFP8Block128Layout
    assert torch.equal(lin.weight._qdata.view(torch.uint8), q.view(torch.uint8))
    assert torch.equal(lin.weight._params.scale, sblk)
    assert lin.weight._params.scale.shape == (n // 128, k // 128)  # stored per block, not per channel
    assert lin._scale_ok and px.kernels._known_positive_finite(lin.weight._params.scale)
    x = torch.randn(7, k, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)
    CASTS.clear()
    y = lin(x)
    assert CASTS == ["Linear"]
    assert torch.equal(y, F.linear(x, px.dequantize_fp8_block(q, sblk, torch.bfloat16), bias))
    fp8 = px.DecoderOps.with_matmul("fp8").Linear(k, n, dtype=torch.bfloat16)
    assert issubclass(px.DecoderOps.with_matmul("fp8"), px.DecoderOps) and fp8.matmul == "fp8"
    fp8._load_from_state_dict(dict(sd), "", {}, True, [], [], [])
    assert torch.equal(fp8(x), y)  # a host input takes the dequant path
    # the layout class: its quantization is quantize_fp8_block, and it saves the checkpoint's key names
    w, _ = _weights(n, k, 11)
    qq, params = px.NomasFP8Block128Layout.quantize(w)
    assert torch.equal(qq.view(torch.uint8), q.view(torch.uint8)) and torch.equal(params.scale, sblk)
    assert torch.equal(px.NomasFP8Block128Layout.dequantize(qq, params), px.dequantize_fp8_block(q, sblk, w.dtype))
    assert set(px.NomasFP8Block128Layout.state_dict_tensors(qq, params)) == {".fp8_weight", ".fp8_scale"}
    assert px.NomasFP8Block128Layout.get_plain_tensors(lin.weight)[1] is lin.weight._params.scale
    # a zero block scale is recorded as failing the check (the fp8 GEMM then folds scales per channel)
    bad = dict(_fp8_state(n, k, 13))
    bad["fp8_scale"][1, 2] = 0.0
    lin_bad = px.DecoderOps.Linear(k, n)
    lin_bad._load_from_state_dict(bad, "", {}, True, [], [], [])
    assert not lin_bad._scale_ok
    # plain weights, a missing bias, a missing weight
    plain = px.DecoderOps.Linear(k, n, dtype=torch.bfloat16)
    missing = []
    plain._load_from_state_dict({"weight": w}, "", {}, True, missing, [], [])
    assert missing == ["bias"] and plain.weight.dtype == torch.bfloat16
    assert not isinstance(plain.weight, QuantizedTensor) and plain.fp8_parts() is None
    assert torch.equal(plain(x), F.linear(x, w.to(torch.bfloat16)))
    missing = []
    px.DecoderOps.Linear(k, n)._load_from_state_dict({}, "p.", {}, True, missing, [], [])
    assert missing == ["p.weight"]
    # codes without their block scales are reported, not loaded
    missing, no_scale = [], px.DecoderOps.Linear(k, n)
    no_scale._load_from_state_dict({"p.fp8_weight": q}, "p.", {}, True, missing, [], [])
    assert missing == ["p.fp8_scale"] and no_scale.weight is None


@pytest.mark.gpu
def test_comfyui_decoder_fp8_path_reads_block_scales_as_stored(comfy_pixelumm, dev, monkeypatch):
    """The fp8 matmul through the ComfyUI branch: the GEMM receives the [N/128, K/128] block scales as stored
    (sw_rows = 128 at the C ABI; the reference passes them repeated per channel, pixelumm.py:153), the result is
    bit-identical to pixelumm.fp8_block_linear, the per-call device copy of the host-checked scales needs no
    device check, and weights resident on the device run without any synchronization.  The fused SwiGLU MLP
    takes the ComfyUI weights too."""
    px = comfy_pixelumm
    from hy_nomas import _lib

    print("ComfyUI decoder fp8 path", flush=True)
    n, k = 512, 1024
    calls = []
    real_call = _lib.call

    def spy(name, *args):
        calls.append((name, args))
        return real_call(name, *args)

    monkeypatch.setattr(_lib, "call", spy)
    sd = _fp8_state(n, k, 21)
    x = (torch.randn(3, 50, k, generator=torch.Generator().manual_seed(22)) * 2).to(torch.bfloat16).to(dev)
    for resident in (False, True):
        lin = px.DecoderOps.with_matmul("fp8").Linear(k, n, dtype=torch.bfloat16)
        state = {key: v.to(dev) for key, v in sd.items()} if resident else dict(sd)
        lin._load_from_state_dict(state, "", {}, True, [], [], [])
        torch.cuda.synchronize()
        calls.clear()
        if resident:
            torch.cuda.set_sync_debug_mode("error")
        try:
            y = lin(x)
        finally:
            torch.cuda.set_sync_debug_mode(0)
        lin_calls = [a for name, a in calls if name == "hn_block_linear"]
        assert len(lin_calls) == 1 and lin_calls[0][12] == 128, "block scales must reach the GEMM as stored"
        s_ref = sd["fp8_scale"].to(dev)
        assert px.kernels.validate_scales(s_ref)  # the same block-scale path as the module's call
        ref = px.fp8_block_linear(x, sd["fp8_weight"].to(dev), s_ref, sd["bias"].to(dev))
        assert torch.equal(y, ref)
        want = F.linear(x.float(), px.dequantize_fp8_block(sd["fp8_weight"], sd["fp8_scale"], torch.float32).to(dev),
                        sd["bias"].float().to(dev))
        assert ((y.float() - want).abs().max() / want.abs().max()).item() < 3e-2
    # the decoder MLP on ComfyUI weights: gate and up in one SwiGLU GEMM, then down
    arch = px.Arch(hidden_size=k, intermediate_size=n)
    mlp = px.MLP(arch, px.DecoderOps.with_matmul("fp8"), dtype=torch.bfloat16)
    for i, name in enumerate(("gate_proj", "up_proj", "down_proj")):
        o, kk = (k, n) if name == "down_proj" else (n, k)
        q, s = px.quantize_fp8_block(torch.randn(o, kk, generator=torch.Generator().manual_seed(30 + i)) * 0.03)
        getattr(mlp, name)._load_from_state_dict({f"{name}.fp8_weight": q, f"{name}.fp8_scale": s.clone()},
                                                  f"{name}.", {}, True, [], [], [])
    calls.clear()
    y = mlp(x)
    names = [name for name, _ in calls]
    assert names.count("hn_block_gemm") == 2 and "hn_block_linear" not in names  # the fused pair of GEMMs
    unfused = mlp.down_proj(F.silu(mlp.gate_proj(x)) * mlp.up_proj(x))
    assert torch.equal(y, unfused)
