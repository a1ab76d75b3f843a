"""The fused DiT elementwise kernels at their full benchmark size, x bf16 [1, 32768, 3072] ~N(0, 1) with
per-sample shift / scale / gate [1, 3072] ~N(0, 0.1), against the oracle over every element (the
reference's tolerances, tests/test_fused.py:12-60): adaLN (LayerNorm and RMSNorm), adaLN + int8
quantization (the reference's 128-channel groups, and one scale per token), and the gated residual
(bit-exact)."""
import numpy as np
import pytest
import torch

import oracle
from conftest import seeded

pytestmark = pytest.mark.gpu

L, D = 32768, 3072


@pytest.fixture(scope="module")
def data():
    g = seeded(3072)
    x = torch.randn(1, L, D, generator=g).to(torch.bfloat16)
    y = torch.randn(1, L, D, generator=g).to(torch.bfloat16)
    shift, scale, gate = ((torch.randn(1, D, generator=g) * 0.1).to(torch.bfloat16) for _ in range(3))
    return x, y, shift, scale, gate


@pytest.mark.parametrize("norm", ["layer", "rms"])
def test_adaln_full_size(dev, data, norm):
    from hy_nomas import fused

    print(f"adaln full size [1, {L}, {D}] norm={norm}", flush=True)
    x, _, shift, scale, _ = data
    got = fused.adaln(x.to(dev), shift.to(dev), scale.to(dev), norm=norm).cpu()
    ref = torch.from_numpy(oracle.adaln(x, shift, scale, norm=norm)).view(1, L, D).to(torch.bfloat16)
    mismatch = (got != ref).float().mean().item()
    assert mismatch < 1e-3, mismatch
    assert (got.float() - ref.float()).abs().max().item() < 0.05


@pytest.mark.parametrize("group", [128, None])
def test_adaln_quant_full_size(dev, data, group):
    from hy_nomas import kernels

    print(f"adaln_quant full size [1, {L}, {D}] group={group}", flush=True)
    x, _, shift, scale, _ = data
    q, s = kernels.adaln_quant(x.to(dev), shift.to(dev), scale.to(dev), group=group)
    q_ref, s_ref, y = oracle.adaln(x, shift, scale, quant=True)
    if group is None:
        q_ref, s_ref = oracle.quantize(y, D)
    q, s = q.cpu().numpy(), s.cpu().numpy()
    assert s.shape == s_ref.shape
    mismatch = (q != q_ref).mean()
    assert mismatch < 1e-3, mismatch
    # The modulated values are rounded to bf16 after an fp32 reduction whose order differs from the
    # oracle's, so a few of them differ by one bf16 ulp.  Where such a value is its group's absmax, the
    # scale differs by that ulp (<= 2^-7 relative): rare over 3.1 M groups, never more than one ulp.
    rel = np.abs(s / s_ref - 1)
    assert (rel > 1e-3).mean() < 1e-3, (rel > 1e-3).mean()
    assert rel.max() <= 2 ** -7, rel.max()
    # a code that differs is off by one step (a quotient next to a rounding boundary), never more
    assert np.abs(q.astype(np.int32) - q_ref.astype(np.int32)).max() <= 1


def test_gated_residual_full_size(dev, data):
    from hy_nomas import fused

    print(f"gated_residual full size [1, {L}, {D}]", flush=True)
    x, y, _, _, gate = data
    got = fused.gated_residual(x.to(dev), y.to(dev), gate.to(dev)).cpu()
    ref = torch.from_numpy(oracle.gated_residual(x, y, gate)).to(torch.bfloat16)
    assert torch.equal(got, ref)
