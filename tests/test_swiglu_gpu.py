"""The decoder MLP's SwiGLU with gate and up in one GEMM (hy_nomas/pixelumm.py:314-323) against the unfused
sequence the reference runs: gate and up as separate block GEMMs with bf16 outputs, torch's bf16 silu and
product, then the down projection's activation quantizer.  The fused epilogue reads the same accumulators,
so its codes and scales must equal the unfused ones bit for bit; the oracle checks the silu product on the
CPU from the GEMMs' bf16 outputs."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from conftest import seeded

pytestmark = pytest.mark.gpu


def fp8_block_weight(g, rows, cols, dev, scale=0.02):
    from hy_nomas import pixelumm

    from hy_nomas import kernels

    q, s = pixelumm.quantize_fp8_block(torch.randn(rows, cols, generator=g) * scale)
    q, s = q.to(dev), s.to(dev)
    assert kernels.validate_scales(s)  # the device copy: read as stored by every GEMM of the comparison
    return q, s


def unfused(x, gate, up, kind="fp8", group=128):
    """The reference's order: quantize x, gate / up GEMMs to bf16, F.silu(gate) * up in bf16, quantize."""
    from hy_nomas import kernels

    qa, sa = kernels.quantize_activations(x, kind, group)
    gt = kernels.block_gemm(qa, sa, gate[0], gate[1], kind=kind)
    ut = kernels.block_gemm(qa, sa, up[0], up[1], kind=kind)
    h = F.silu(gt) * ut
    hq, hs = kernels.quantize_activations(h, kind, 128)
    return hq, hs, gt, ut, h


@pytest.mark.parametrize("m,k,i", [(300, 256, 384), (1000, 512, 1024), (129, 4096, 128), (2048, 1024, 256)])
def test_swiglu_quant_fp8_block_matches_unfused(dev, m, k, i):
    from hy_nomas import kernels, pixelumm

    print(f"swiglu_quant fp8 m={m} k={k} i={i}", flush=True)
    g = seeded(m + k + i)
    x = (torch.randn(m, k, generator=g) * 1.5).to(torch.bfloat16).to(dev)
    gate = fp8_block_weight(g, i, k, dev)
    up = fp8_block_weight(g, i, k, dev)
    hq_ref, hs_ref, gt, ut, h = unfused(x, gate, up)
    qa, sa = kernels.quantize_activations(x, "fp8")
    q_gu, s_gu = pixelumm.interleave_gate_up(gate, up)
    assert q_gu.shape == (2 * i, k) and s_gu.shape == (2 * i // 128, k // 128)
    hq, hs = kernels.block_gemm(qa, sa, q_gu, s_gu, kind="fp8", epilogue="swiglu_quant")
    assert hq.dtype == torch.float8_e4m3fn and hq.shape == (m, i) and hs.shape == (m, i // 128)
    assert torch.equal(hs, hs_ref)
    assert torch.equal(hq.view(torch.uint8), hq_ref.view(torch.uint8))
    # the oracle's silu product of the GEMMs' bf16 outputs, then its quantizer
    q_o, s_o, h_o = oracle.swiglu_quant(gt.float().cpu().numpy(), ut.float().cpu().numpy(), "fp8")
    assert np.array_equal(h_o, h.float().cpu().numpy())
    assert np.array_equal(hs.cpu().numpy(), s_o)
    assert np.array_equal(hq.view(torch.uint8).cpu().numpy(), q_o)


def test_swiglu_quant_int8_per_token_matches_unfused(dev):
    """The per-token x per-channel int8 layout: the same epilogue with int8 codes, half away from zero."""
    from hy_nomas import kernels, ops

    print("swiglu_quant int8 per token", flush=True)
    g = seeded(77)
    m, k, i = 515, 768, 512
    x = (torch.randn(m, k, generator=g) * 2).to(torch.bfloat16).to(dev)
    wg = torch.randn(i, k, generator=g) * 0.03
    wu = torch.randn(i, k, generator=g) * 0.03
    # per-channel int8 weights: group = K
    gate = kernels.quantize_activations(wg.to(dev), "int8", None)
    up = kernels.quantize_activations(wu.to(dev), "int8", None)
    hq_ref, hs_ref, *_ = unfused(x, gate, up, "int8", None)
    qa, sa = kernels.quantize_activations(x, "int8", None)
    q_gu = torch.stack((gate[0].view(i // 128, 128, k), up[0].view(i // 128, 128, k)), 1).reshape(2 * i, k)
    s_gu = torch.stack((gate[1].view(i // 128, 128, 1), up[1].view(i // 128, 128, 1)), 1).reshape(2 * i, 1)
    hq, hs = kernels.block_gemm(qa, sa, q_gu, s_gu, kind="int8", epilogue="swiglu_quant")
    assert hq.dtype == torch.int8 and hq.shape == (m, i)
    assert torch.equal(hs, hs_ref)
    assert torch.equal(hq, hq_ref)
    del ops


def test_swiglu_mlp_module_matches_reference_expression(dev):
    """pixelumm.MLP with fp8 weights: the fused forward equals the reference's
    down_proj(F.silu(gate_proj(x)) * up_proj(x)) through three fp8 linears, bit for bit."""
    from hy_nomas import pixelumm

    print("decoder MLP fused vs unfused", flush=True)
    g = seeded(5)
    arch = pixelumm.Arch(hidden_size=512, intermediate_size=1536)
    ops = pixelumm.DecoderOps.with_matmul("fp8")
    mlp = pixelumm.MLP(arch, ops)
    sd = {}
    for name, (o, k) in {"gate_proj": (1536, 512), "up_proj": (1536, 512), "down_proj": (512, 1536)}.items():
        q, s = pixelumm.quantize_fp8_block(torch.randn(o, k, generator=g) * 0.03)
        sd[f"{name}.fp8_weight"], sd[f"{name}.fp8_scale"] = q.to(dev), s.to(dev)
    res = mlp.load_state_dict(sd, strict=False)
    assert not res.unexpected_keys
    x = (torch.randn(2, 333, 512, generator=g)).to(torch.bfloat16).to(dev)
    got = mlp(x)
    ref = mlp.down_proj(F.silu(mlp.gate_proj(x)) * mlp.up_proj(x))
    assert got.shape == (2, 333, 512) and got.dtype == torch.bfloat16
    assert torch.equal(got, ref)
    # and close to the float product on the dequantized weights
    wd = {n: pixelumm.dequantize_fp8_block(getattr(mlp, n).weight, getattr(mlp, n).scale, torch.float32)
          for n in ("gate_proj", "up_proj", "down_proj")}
    xf = x.float()
    hf = F.silu(xf @ wd["gate_proj"].t()) * (xf @ wd["up_proj"].t())
    yf = hf @ wd["down_proj"].t()
    assert ((got.float() - yf).norm() / yf.norm()).item() < 5e-2


def test_swiglu_quant_rejects_bad_layouts(dev):
    from hy_nomas import kernels

    g = seeded(9)
    x = torch.randn(64, 256, generator=g).to(torch.bfloat16).to(dev)
    qa, sa = kernels.quantize_activations(x, "fp8")
    q, s = fp8_block_weight(g, 384, 256, dev)       # 384 rows: not whole gate/up pairs of 256
    with pytest.raises(RuntimeError):
        kernels.block_gemm(qa, sa, q, s, kind="fp8", epilogue="swiglu_quant")
    qi, si = kernels.quantize_activations(x, "int8")
    w = kernels.quantize_activations(torch.randn(256, 256, generator=g).to(dev), "int8")
    with pytest.raises(RuntimeError):                # int8 g128: no two-token-block tile for the split
        kernels.block_gemm(qi, si, w[0], w[1], kind="int8", epilogue="swiglu_quant")


def test_fast_silu_equals_the_reference_for_every_bf16_value(dev):
    """The SwiGLU epilogue's silu of a bf16 value (hardware exponential and reciprocal, the library form near
    bf16 rounding midpoints and for g < -16), one value at a time and in pairs rounded by the hardware pack,
    against the fp32 form rounded to bf16, for all 65536 bf16 bit patterns in each slot
    (libhynomas_probes.so: hnp_silu_mismatches), and against torch's silu of the bf16 values on the CPU
    (the reference's F.silu), NaNs compared as NaNs."""
    import ctypes
    import os

    path = os.path.join(os.path.dirname(__file__), "..", "comfyui-hy-nomas_amd", "hy_nomas", "libhynomas_probes.so")
    lib = ctypes.CDLL(path)
    lib.hnp_silu_mismatches.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    value = torch.empty(65536, dtype=torch.int32, device=dev)
    bad = torch.empty(65536, dtype=torch.int32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.hnp_silu_mismatches(value.data_ptr(), bad.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert int(bad.sum().item()) == 0
    g = (torch.arange(65536, dtype=torch.int32) << 16).view(torch.float32).to(torch.bfloat16)
    ref = torch.nn.functional.silu(g).float()
    got = value.cpu().view(torch.float32)
    both_nan = torch.isnan(ref) & torch.isnan(got)
    assert torch.equal(got[~both_nan], ref[~both_nan])
