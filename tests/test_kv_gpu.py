"""int8 K/V history quantization on the GPU vs the oracle (hy_nomas/world.py:80-94): codes and scales bit-exact,
dequantization bit-exact against torch's (q.float() * scale).to(dtype)."""
import numpy as np
import pytest
import torch

import oracle
from conftest import seeded

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("l,h,d", [(1, 1, 128), (333, 24, 128), (70, 8, 256), (0, 4, 128)])
def test_quantize_kv_bit_exact(dev, l, h, d):
    from hy_nomas import kv

    print(f"quantize_kv l={l} h={h} d={d}", flush=True)
    g = seeded(l * 31 + h + d)
    x = (torch.randn(l, h, d, generator=g) * 2).to(torch.bfloat16)
    if l > 3:
        x[2, 0] = 0.0                                   # an all-zero head
        x[3, 0] = 0.0
        x[3, 0, 0] = 127.0                              # scale exactly 1, then exact ties
        x[3, 0, 1:5] = torch.tensor([0.5, -0.5, 2.5, -2.5])
    q, s = kv.quantize_kv(x.to(dev))
    assert q.shape == (l, h, d) and s.shape == (l, h, 1) and q.dtype == torch.int8 and s.dtype == torch.float32
    if l == 0:
        return
    q_ref, s_ref = oracle.quantize_kv(x)
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)
    if l > 3:
        assert q[3, 0, 1:5].cpu().tolist() == [1, -1, 3, -3]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("l,h,d", [(257, 24, 128), (5, 3, 64), (1, 1, 16)])
def test_dequantize_kv_matches_torch(dev, dtype, l, h, d):
    from hy_nomas import kv

    print(f"dequantize_kv {dtype} l={l} h={h} d={d}", flush=True)
    g = seeded(l + h * 7 + d)
    q = torch.randint(-127, 128, (l, h, d), generator=g, dtype=torch.int8)
    s = (torch.rand(l, h, 1, generator=g) * 0.05 + 1e-4).float()
    s[0, 0, 0] = 1.0
    got = kv.dequantize_kv(q.to(dev), s.to(dev), dtype)
    ref = (q.to(dev).float() * s.to(dev)).to(dtype)
    assert got.dtype == dtype and got.shape == q.shape
    assert torch.equal(got.view(torch.int8) if dtype != torch.float32 else got, ref.view(torch.int8) if dtype != torch.float32 else ref)
    if dtype == torch.bfloat16:
        assert np.array_equal(got.float().cpu().numpy(), oracle.dequantize_kv(q.numpy(), s.numpy()))


def test_kv_round_trip_at_history_size(dev):
    """Quantize then dequantize a [57344, 24, 128] K slab (the config-4 history): the round trip error is at most
    half a step of each head's scale plus fp32 rounding (a size-independent property), and every head's codes
    reach +-127."""
    from hy_nomas import kv

    print("kv round trip 57344x24x128", flush=True)
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(57344, 24, 128, generator=g, device=dev).to(torch.bfloat16)
    q, s = kv.quantize_kv(x)
    y = kv.dequantize_kv(q, s, torch.float32)
    err = (y - x.float()).abs()
    # half a step, plus the fp32 roundings of the quotient and of the product (a few ulps of |x|)
    assert bool((err <= s * 0.5 + x.float().abs() * 2.0 ** -21).all())
    assert int(q.abs().amax(dim=-1).min()) == 127
