"""Activation quantization on the GPU vs the CPU oracle: bit-exact codes and scales
(hy_nomas/kernels.py:22-54)."""
import numpy as np
import pytest
import torch

import oracle
from conftest import seeded

pytestmark = pytest.mark.gpu


def outlier_input(m, k, seed=0, dtype=torch.bfloat16):
    """~N(0, 1) with 1% of channels scaled x20 (the benchmark's activation distribution)."""
    g = seeded(seed)
    x = torch.randn(m, k, generator=g)
    ch = torch.randperm(k, generator=g)[: max(1, k // 100)]
    x[:, ch] *= 20
    return x.to(dtype)


def check_quant(x, dev, kind="int8", group=128, rounding="half_away"):
    from hy_nomas import kernels

    print(f"quant case kind={kind} group={group} rounding={rounding} shape={tuple(x.shape)} dtype={x.dtype}",
          flush=True)
    q, s = kernels.quantize_activations(x.to(dev), kind, group, rounding)
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.quantize(x, group or x.shape[1], kind, rounding)
    got_q = q.cpu().view(torch.uint8 if kind == "fp8" else torch.int8).numpy()
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32)), "scales differ"
    bad = np.argwhere(got_q != q_ref)
    assert bad.size == 0, f"{len(bad)} codes differ, first at {bad[:3].tolist()}"


@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("m,k", [(1, 128), (7, 256), (300, 2048), (1024, 3072), (33, 12288)])
def test_quant_g128(dev, kind, m, k):
    check_quant(outlier_input(m, k, seed=m + k), dev, kind, 128)


@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("m,k", [(1, 128), (5, 384), (300, 2048), (1024, 3072), (65, 12288)])
def test_quant_per_token(dev, kind, m, k):
    check_quant(outlier_input(m, k, seed=m * k), dev, kind, None)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_quant_input_dtypes(dev, dtype):
    check_quant(outlier_input(129, 1024, seed=3, dtype=dtype), dev, "int8", 128)
    check_quant(outlier_input(129, 1024, seed=4, dtype=dtype), dev, "fp8", None)


def test_quant_half_even(dev):
    check_quant(outlier_input(200, 3072, seed=5), dev, "int8", 128, "half_even")
    check_quant(outlier_input(200, 3072, seed=6), dev, "int8", None, "half_even")


def test_quant_ties_and_zero_groups(dev):
    # peak 127 -> scale exactly 1: every k + 0.5 is a tie that must round away from zero
    k = 256
    x = torch.zeros(4, k)
    ties = torch.arange(-126.5, 127.0, 1.0)[:128]
    x[0, :128] = ties
    x[0, 0] = 127.0
    x[1, 128:] = -ties.flip(0)
    x[1, 200] = -127.0
    x[2] = 0.0                                  # all-zero row: scale 1, codes 0
    x[3, :128] = torch.tensor([2.0 ** -120] * 128)  # tiny values (the division fallback path)
    x[3, 128:] = -1e-38
    x = x.to(torch.bfloat16)
    for group in (128, None):
        check_quant(x, dev, "int8", group)
        check_quant(x, dev, "fp8", group)
        check_quant(x, dev, "int8", group, "half_even")


def test_quant_group_magnitudes_across_the_fast_quotient_range(dev):
    """int8 groups whose absmax lies on both sides of the two-op quotient's range [2^-80, 2^100) and at the
    ends of the float range.  Each first group holds peak * (2k + 1) / 254 rounded to bf16 (next to the
    half-away ties of codes k), each second group random values of the same magnitude.  Both roundings,
    one scale per group and one per token, bit-exact against the oracle."""
    g = seeded(17)
    rows = []
    for e in (-126, -100, -81, -80, -79, -1, 0, 99, 100, 101, 120, 126):
        peak = 1.5 * 2.0 ** e
        ties = torch.tensor([peak * (2 * k + 1) / 254 for k in range(-64, 63)] + [peak])
        rand = torch.randn(128, generator=g) * (peak / 4)
        rand[0] = -peak
        rows.append(torch.cat([ties, rand]))
    x = torch.stack(rows).to(torch.bfloat16)
    assert torch.isfinite(x.float()).all()
    for group in (128, None):
        check_quant(x, dev, "int8", group)
        check_quant(x, dev, "int8", group, "half_even")


def test_quant_strided_rows(dev):
    from hy_nomas import kernels

    big = outlier_input(100, 4096, seed=7)
    x = big.to(dev)[:, 512:512 + 2048]         # row stride 4096, unit column stride
    q, s = kernels.quantize_activations(x)
    q_ref, s_ref = oracle.quantize(big[:, 512:512 + 2048])
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(s.cpu().numpy(), s_ref)


def test_fp8_encoding_every_bf16(dev):
    """Every finite bf16 value quantized with scale 1 (group peak 448) must encode like torch's e4m3fn cast."""
    from hy_nomas import kernels

    bits = torch.arange(0, 0x10000, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    vals = bits.float()
    vals = vals[torch.isfinite(vals) & (vals.abs() <= 448)]
    n = (vals.numel() // 127) * 127
    rows = vals[:n].view(-1, 127)
    x = torch.cat([rows, torch.full((rows.shape[0], 1), 448.0)], dim=1).to(torch.bfloat16)  # peak 448
    q, s = kernels.quantize_activations(x.to(dev), "fp8", 128)
    assert torch.all(s.cpu() == 1.0)
    ref = x.float().to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(q.cpu().view(torch.uint8), ref)


def test_hardware_e4m3_conversion_equals_the_encoder(dev):
    """The hardware OCP e4m3 conversion (v_cvt_pk_fp8_f32) against the software encoder, which the CPU tests pin
    to torch's float8_e4m3fn cast: every fp32 value with |x| < 2^9 (the quotients x / scale of the fp8
    quantizers lie within 448 (1 + 2^-22)), both signs, both byte positions and both half-words of the packed
    result (libhynomas_probes.so: hnp_e4m3_mismatches).  The kernels use the hardware form only for such
    finite quotients."""
    import ctypes
    import os

    path = os.path.join(os.path.dirname(__file__), "..", "comfyui-hy-nomas_amd", "hy_nomas", "libhynomas_probes.so")
    lib = ctypes.CDLL(path)
    u32, ci, vp = ctypes.c_uint32, ctypes.c_int, ctypes.c_void_p
    lib.hnp_e4m3_mismatches.argtypes = [u32, u32, ci, vp, vp, vp]
    blocks = 2048
    count = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
    first = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    hi = 0x44000000  # 2^9
    print(f"e4m3 conversion over fp32 patterns [0, {hi:#x}) and their negatives", flush=True)
    assert lib.hnp_e4m3_mismatches(0, hi, blocks, count.data_ptr(), first.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    bad = int(count.sum().item())
    low = int(first.cpu().numpy().view(np.uint32).min())
    assert bad == 0, (bad, hex(low))
