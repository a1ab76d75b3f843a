"""Fused DiT elementwise kernels on the GPU vs the CPU oracle and the torch arithmetic they replace
(hy_nomas/fused.py; tolerances of the reference's tests/test_fused.py)."""
import numpy as np
import pytest
import torch

import oracle
from conftest import seeded

pytestmark = pytest.mark.gpu


def bf(t):
    return t.to(torch.bfloat16)


@pytest.mark.parametrize("b,l,d,norm", [(2, 777, 2048, "layer"), (1, 4096, 3072, "layer"), (1, 300, 3072, "rms"),
                                        (3, 5, 136, "layer")])
def test_adaln(dev, b, l, d, norm):
    from hy_nomas import fused

    print(f"adaln b={b} l={l} d={d} norm={norm}", flush=True)
    g = seeded(b * l + d)
    # strided input like the reference test: transpose of [B, D, L]
    x = bf(torch.randn(b, d, l, generator=g) * 3).transpose(1, 2)
    shift = bf(torch.randn(b, d, generator=g))
    scale = bf(torch.randn(b, d, generator=g))
    got = fused.adaln(x.to(dev), shift.to(dev), scale.to(dev), norm=norm).cpu()
    ref = bf(torch.from_numpy(oracle.adaln(x.contiguous(), shift, scale, norm=norm)).view(b, l, d))
    mismatch = (got != ref).float().mean().item()
    assert mismatch < 1e-3, mismatch
    assert (got.float() - ref.float()).abs().max().item() < 0.05


def test_adaln_matches_torch(dev):
    """hy_nomas tests/test_fused.py:12-21 against torch's F.layer_norm + modulate on the CPU."""
    from hy_nomas import fused
    from oracle import torch_forms

    g = seeded(1)
    x = bf(torch.randn(2, 2048, 777, generator=g) * 3).transpose(1, 2)
    shift = bf(torch.randn(2, 2048, generator=g))
    scale = bf(torch.randn(2, 2048, generator=g))
    ref = bf(torch_forms.modulate(torch_forms.layer_norm(x), shift, scale))
    got = fused.adaln(x.to(dev), shift.to(dev), scale.to(dev)).cpu()
    assert (got != ref).float().mean().item() < 1e-3
    assert (got.float() - ref.float()).abs().max().item() < 0.05


@pytest.mark.parametrize("b,l,d,norm", [(1, 300, 2048, "layer"), (1, 2048, 3072, "layer"), (2, 100, 3072, "rms"),
                                        (1, 64, 12288, "layer")])
def test_adaln_quant(dev, b, l, d, norm):
    from hy_nomas import kernels

    print(f"adaln_quant b={b} l={l} d={d} norm={norm}", flush=True)
    g = seeded(l + d)
    x = bf(torch.randn(b, d, l, generator=g) * 3).transpose(1, 2)
    shift = bf(torch.randn(b, d, generator=g))
    scale = bf(torch.randn(b, d, generator=g))
    q, s = kernels.adaln_quant(x.to(dev), shift.to(dev), scale.to(dev), norm=norm)
    q_ref, s_ref, _ = oracle.adaln(x.contiguous(), shift, scale, norm=norm, quant=True)
    assert (q.cpu().numpy() != q_ref).mean() < 1e-3
    assert np.allclose(s.cpu().numpy(), s_ref, rtol=1e-3)


@pytest.mark.parametrize("d,group,norm", [(128, 128, "layer"), (384, None, "rms"), (640, 128, "rms"),
                                          (640, None, "layer"), (1152, 128, "layer"), (4096, None, "layer")])
def test_adaln_quant_widths(dev, d, group, norm):
    """adaLN + int8 quant at widths off the 512-multiple chunk schedule (one or a few 128-channel groups a
    row) and with one scale per token, against the oracle: codes mismatch < 1e-3 and one step at most, scales
    within one bf16 ulp of the group peak (the reduction order moves a few modulated values by an ulp)."""
    from hy_nomas import kernels

    b, l = 2, 97
    print(f"adaln_quant widths d={d} group={group} norm={norm}", flush=True)
    g = seeded(7 * d + (group is None))
    x = bf(torch.randn(b, d, l, generator=g) * 3).transpose(1, 2)
    shift = bf(torch.randn(b, d, generator=g))
    scale = bf(torch.randn(b, d, generator=g))
    q, s = kernels.adaln_quant(x.to(dev), shift.to(dev), scale.to(dev), norm=norm, group=group)
    q_ref, s_ref, y = oracle.adaln(x.contiguous(), shift, scale, norm=norm, quant=True)
    if group is None:
        q_ref, s_ref = oracle.quantize(y, d)
    q, s = q.cpu().numpy(), s.cpu().numpy()
    assert s.shape == s_ref.shape
    assert (q != q_ref).mean() < 1e-3
    assert np.abs(q.astype(np.int32) - q_ref.astype(np.int32)).max() <= 1
    assert np.abs(s / s_ref - 1).max() <= 2 ** -7


def test_adaln_nonfinite_factors(dev):
    """inf and NaN in the shift / scale factors (the block stages them with the software bf16 rounding): the
    outputs' NaN and inf positions equal the oracle's, NaNs carry torch's code 0x7FC0, and the finite outputs
    keep the usual tolerance."""
    from hy_nomas import fused

    b, l, d = 2, 33, 640
    g = seeded(31)
    x = bf(torch.randn(b, d, l, generator=g) * 3).transpose(1, 2)
    shift = bf(torch.randn(b, d, generator=g))
    scale = bf(torch.randn(b, d, generator=g))
    scale[0, 5] = float("inf")
    scale[1, 100] = -float("inf")
    shift[1, 9] = float("nan")
    got = fused.adaln(x.to(dev), shift.to(dev), scale.to(dev)).cpu()
    ref = bf(torch.from_numpy(oracle.adaln(x.contiguous(), shift, scale)).view(b, l, d))
    assert torch.equal(got.isnan(), ref.isnan()) and torch.equal(got.isinf(), ref.isinf())
    assert got.isnan().any() and got.isinf().any()
    assert (got.view(torch.int16)[got.isnan()] == 0x7FC0).all()
    fin = torch.isfinite(ref)
    assert torch.equal(got[got.isinf()], ref[ref.isinf()])
    assert (got[fin] != ref[fin]).float().mean().item() < 1e-3
    assert (got[fin].float() - ref[fin].float()).abs().max().item() < 0.05


@pytest.mark.parametrize("group", [128, None])
def test_adaln_quant_nonfinite(dev, group):
    """inf and NaN in the factors and in two token rows, quantized: scales against the oracle's quantization of
    its own adaLN output (the peaks skip NaN; an infinite peak gives an infinite scale), finite scales within
    one bf16 ulp, and the codes of every finite value one step at most (zero under an infinite peak).  NaN
    values, and the infinite ones (inf / inf), have no defined code in the reference (its clamp's maximum and
    minimum ignore NaN where it runs, giving -127; the oracle's C conversion gives 0): they are not compared."""
    from hy_nomas import kernels

    print(f"adaln_quant nonfinite group={group}", flush=True)
    b, l, d = 2, 33, 640
    g = seeded(37 + (group is None))
    x = bf(torch.randn(b, l, d, generator=g) * 3)
    x[0, 3, 17] = float("inf")
    x[1, 7, 300] = float("nan")
    shift = bf(torch.randn(b, d, generator=g))
    scale = bf(torch.randn(b, d, generator=g))
    scale[0, 5] = float("inf")
    scale[1, 100] = -float("inf")
    shift[1, 9] = float("nan")
    q, s = kernels.adaln_quant(x.to(dev), shift.to(dev), scale.to(dev), group=group)
    q_ref, s_ref, y = oracle.adaln(x, shift, scale, quant=True)
    if group is None:
        q_ref, s_ref = oracle.quantize(y, d)
    q, s = q.cpu().numpy(), s.cpu().numpy()
    assert np.isinf(s_ref).any() and np.isnan(y).any()
    assert np.array_equal(np.isinf(s), np.isinf(s_ref)) and not np.isnan(s).any()
    fin = np.isfinite(s_ref)
    assert np.abs(s[fin] / s_ref[fin] - 1).max() <= 2 ** -7
    num = np.isfinite(y)
    assert np.abs(q[num].astype(np.int32) - q_ref[num].astype(np.int32)).max() <= 1
    assert (q[num] != q_ref[num]).mean() < 1e-3


def test_adaln_quant_matches_unfused(dev):
    """hy_nomas tests/test_fused.py:52-60."""
    from hy_nomas import fused, kernels

    g = seeded(2)
    x = bf(torch.randn(1, 2048, 300, generator=g) * 3).transpose(1, 2).to(dev)
    shift = bf(torch.randn(1, 2048, generator=g)).to(dev)
    scale = bf(torch.randn(1, 2048, generator=g)).to(dev)
    q, s = kernels.adaln_quant(x, shift, scale)
    q_ref, s_ref = kernels.quantize_activations(fused.adaln(x, shift, scale).view(-1, 2048))
    assert (q != q_ref).float().mean().item() < 1e-3
    assert torch.allclose(s, s_ref, rtol=1e-3)


@pytest.mark.parametrize("b,l,d", [(1, 500, 2048), (2, 1000, 3072), (1, 3, 8)])
def test_gated_residual_bit_exact(dev, b, l, d):
    """hy_nomas tests/test_fused.py:43-49: bit-exact against torch's bf16 arithmetic (and the oracle)."""
    from hy_nomas import fused

    g = seeded(l)
    x = bf(torch.randn(b, d, l, generator=g)).transpose(1, 2)   # strided, like the patch embed
    y = bf(torch.randn(b, l, d, generator=g))
    gate = bf(torch.randn(b, d, generator=g))
    got = fused.gated_residual(x.to(dev), y.to(dev), gate.to(dev))
    ref_gpu = x.to(dev) + y.to(dev) * gate.to(dev).unsqueeze(1)
    assert torch.equal(got, ref_gpu)
    assert torch.equal(got.cpu(), bf(torch.from_numpy(oracle.gated_residual(x, y, gate))))


def test_qk_norm_rope(dev):
    """hy_nomas tests/test_fused.py:24-40 tolerances, against torch RMSNorm + apply_rope and the oracle."""
    from hy_nomas import fused
    from oracle import torch_forms

    b, l, h, d = 2, 96, 16, 128
    g = seeded(3)
    lin = bf(torch.randn(b, l, h * d, generator=g) * 5)
    x = lin.view(b, l, h, d)
    norm = torch_forms.RMSNorm(d).bfloat16()
    with torch.no_grad():
        norm.weight.copy_(torch.rand(d, generator=g) + 0.5)
    rope = torch_forms.rope_freqs([16, 56, 56], 256, 4, 4, 6)
    with torch.no_grad():
        ref = torch_forms.apply_rope(norm(x).to(torch.bfloat16), *rope)
        ref_plain = norm(x).to(torch.bfloat16)
    got = fused.qk_norm_rope(x.to(dev), norm.weight.detach().to(dev), (rope[0].to(dev), rope[1].to(dev))).cpu()
    got_plain = fused.qk_norm_rope(x.to(dev), norm.weight.detach().to(dev), None).cpu()
    assert (got_plain != ref_plain).float().mean().item() < 1e-3
    assert (got != ref).float().mean().item() < 1e-2
    assert ((got.float() - ref.float()).norm() / ref.float().norm()).item() < 1e-3
    ora = bf(torch.from_numpy(oracle.qk_norm_rope(x, norm.weight.detach(), rope)))
    assert (got != ora).float().mean().item() < 1e-2


def test_qk_norm_rope_strided_qkv(dev):
    """q/k as strided views of one QKV GEMM output (token stride 3*H*D), as the block harness calls it."""
    from hy_nomas import fused

    b, l, h, d = 1, 77, 24, 128
    g = seeded(4)
    qkv = bf(torch.randn(b, l, 3, h, d, generator=g) * 2)
    w = bf(torch.rand(d, generator=g) + 0.5)
    got = fused.qk_norm_rope(qkv.to(dev)[:, :, 1], w.to(dev), None).cpu()
    ref = bf(torch.from_numpy(oracle.qk_norm_rope(qkv[:, :, 1].contiguous(), w, None)))
    assert (got != ref).float().mean().item() < 1e-3


def test_pixelumm_qk(dev):
    from hy_nomas import fused

    n, h, d = 200, 8, 128
    g = seeded(5)
    x = bf(torch.randn(1, n, h, d, generator=g) * 3)
    wt = bf(torch.rand(d // 2, generator=g) + 0.5)
    whw = bf(torch.rand(d // 2, generator=g) + 0.5)
    ang = torch.rand(n, d, generator=g) * 6.28
    cos, sin = ang.cos(), ang.sin()
    got = fused.pixelumm_qk(x.to(dev), wt.to(dev), whw.to(dev), cos.to(dev), sin.to(dev)).cpu()
    ref = bf(torch.from_numpy(oracle.pixelumm_qk(x, wt, whw, cos, sin)))
    assert (got != ref).float().mean().item() < 1e-2
    assert ((got.float() - ref.float()).norm() / ref.float().norm()).item() < 1e-3


@pytest.mark.parametrize("b,l,d", [(1, 300, 3072), (2, 77, 2048), (1, 5, 128)])
def test_adaln_quant_per_token(dev, b, l, d):
    """The per-token extension: one scale per row of the modulated norm, the oracle's per-token quantization of
    the oracle's rbf16 adaLN output (codes to the reference test's 1e-3 mismatch, scales to 1e-3)."""
    from hy_nomas import kernels

    print(f"adaln_quant per-token b={b} l={l} d={d}", flush=True)
    g = seeded(l + d + 7)
    x = bf(torch.randn(b, l, d, generator=g) * 3)
    shift = bf(torch.randn(b, d, generator=g))
    scale = bf(torch.randn(b, d, generator=g))
    q, s = kernels.adaln_quant(x.to(dev), shift.to(dev), scale.to(dev), group=None)
    assert tuple(s.shape) == (b * l, 1)
    _, _, y = oracle.adaln(x, shift, scale, quant=True)
    q_ref, s_ref = oracle.quantize(y, d)
    assert (q.cpu().numpy() != q_ref).mean() < 1e-3
    assert np.allclose(s.cpu().numpy(), s_ref, rtol=1e-3)


@pytest.mark.parametrize("d,group,norm", [(3072, 128, "layer"), (3072, None, "layer"), (640, 128, "rms"),
                                          (2048, None, "rms"), (12288, 128, "layer")])
def test_adaln_quant_half_even(dev, d, group, norm):
    """adaLN + int8 quant with half-even codes (the rounding the per-token W8A8 path uses) against the oracle's
    half-even quantization of its own adaLN output: codes mismatch < 1e-3 and one step at most (the statistics'
    reduction order moves a few modulated values by an ulp), scales within one bf16 ulp."""
    from hy_nomas import kernels

    b, l = 2, 129
    print(f"adaln_quant half_even d={d} group={group} norm={norm}", flush=True)
    g = seeded(11 * d + (group is None) + 3 * (norm == "rms"))
    x = bf(torch.randn(b, l, d, generator=g) * 3)
    shift = bf(torch.randn(b, d, generator=g))
    scale = bf(torch.randn(b, d, generator=g))
    q, s = kernels.adaln_quant(x.to(dev), shift.to(dev), scale.to(dev), norm=norm, rounding="half_even", group=group)
    q_ref, s_ref, y = oracle.adaln(x, shift, scale, norm=norm, quant=True, rounding="half_even")
    if group is None:
        q_ref, s_ref = oracle.quantize(y, d, "int8", rounding="half_even")
    q, s = q.cpu().numpy(), s.cpu().numpy()
    assert s.shape == s_ref.shape
    assert (q != q_ref).mean() < 1e-3
    assert np.abs(q.astype(np.int32) - q_ref.astype(np.int32)).max() <= 1
    assert np.abs(s / s_ref - 1).max() <= 2 ** -7


@pytest.mark.parametrize("group", [128, None])
def test_adaln_quant_subnormal_rows(dev, group):
    """Rows of bf16 subnormals (|x| < 2^-126) next to ordinary rows, with zero shift and scale: the outputs are
    the centred values times rstd, so a mean that lost the subnormal terms (a flushed sum) would move every
    code of those rows.  Against the oracle, whose C arithmetic keeps subnormals: codes one step at most."""
    from hy_nomas import kernels

    print(f"adaln_quant subnormal rows group={group}", flush=True)
    g = seeded(4242 + (group is None))
    b, l, d = 1, 64, 3072
    x = torch.randn(b, l, d, generator=g)
    x[:, ::2] *= 2.0 ** -130  # even rows: bf16 subnormals (and zeros)
    x = bf(x)
    assert (x[:, ::2].float().abs().max() < 2.0 ** -126) and (x[:, ::2] != 0).float().mean() > 0.9
    shift = torch.zeros(b, d, dtype=torch.bfloat16)
    scale = torch.zeros(b, d, dtype=torch.bfloat16)
    q, s = kernels.adaln_quant(x.to(dev), shift.to(dev), scale.to(dev), group=group)
    q_ref, s_ref, y = oracle.adaln(x, shift, scale, quant=True)
    if group is None:
        q_ref, s_ref = oracle.quantize(y, d)
    q, s = q.cpu().numpy(), s.cpu().numpy()
    assert np.abs(q.astype(np.int32) - q_ref.astype(np.int32)).max() <= 1
    assert (q != q_ref).mean() < 1e-3
    assert np.abs(s / s_ref - 1).max() <= 2 ** -7


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("b,t,p,d,frame_b", [(1, 3, 5, 3072, 1), (2, 4, 33, 256, 2), (2, 2, 7, 64, 1)])
def test_gated_residual_frames_matches_two_torch_ops(dev, dtype, b, t, p, d, frame_b):
    """The block's last gated residual and the camera module's per-frame add (hy_nomas/model.py:518-520)
    in one pass: bit-exact against gated_residual followed by torch's broadcast add."""
    from hy_nomas import fused

    print(f"gated_residual_frames {dtype} b={b} t={t} p={p} d={d}", flush=True)
    g = seeded(b * 100 + t * 10 + p + d)
    x = (torch.randn(b, t * p, d, generator=g) * 3).to(dtype).to(dev)
    y = torch.randn(b, t * p, d, generator=g).to(dtype).to(dev)
    gate = (torch.randn(b, d, generator=g) * 0.3).to(dtype).to(dev)
    frame = (torch.randn(frame_b, t, d, generator=g) * 0.5).to(dtype).to(dev)
    got = fused.gated_residual_frames(x, y, gate, frame)
    ref = (fused.gated_residual(x, y, gate).view(b, t, p, d) + frame.unsqueeze(2)).view(b, t * p, d)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    with pytest.raises(RuntimeError):
        fused.gated_residual_frames(x, y, gate, frame[:, :1].expand(frame_b, t + 1, d)[:, : t + 1])


@pytest.mark.parametrize("h", [1, 2, 3, 4, 5, 6, 12, 24])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_qk_norm_rope_head_groups(dev, h, d):
    """Each group of lanes normalizes G heads of one token (G = 6, 4, 2 or 1 by the head count): every head
    of a multi-head call equals a one-head call on that head's strided view (always G = 1) bit for bit, and
    the whole agrees with the oracle."""
    from hy_nomas import fused

    print(f"qk_norm_rope head groups h={h} d={d}", flush=True)
    b, l = 2, 37
    g = seeded(100 + h * 7 + d)
    x = bf(torch.randn(b, l, h, d, generator=g) * 3)
    w = bf(torch.rand(d, generator=g) + 0.5)
    ang = torch.rand(l, d, generator=g) * 6.28
    rope = (ang.cos(), ang.sin())
    xd, wd, rd = x.to(dev), w.to(dev), (rope[0].to(dev), rope[1].to(dev))
    for r, rdv in ((None, None), (rope, rd)):
        got = fused.qk_norm_rope(xd, wd, rdv)
        for k in range(h):
            assert torch.equal(got[:, :, k:k + 1], fused.qk_norm_rope(xd[:, :, k:k + 1], wd, rdv))
        ora = bf(torch.from_numpy(oracle.qk_norm_rope(x, w, r)))
        assert (got.cpu() != ora).float().mean().item() < 1e-2


@pytest.mark.parametrize("d", [64, 128, 256])
def test_qk_norm_rope_nonfinite(dev, d):
    """NaN and inf inputs.  A head holding a NaN comes out as torch's NaN code 0x7FC0 in every dim; a head
    holding an inf has r = 0, so its inf dim (and, with the rotation, that dim's pair partner) is NaN and the
    rest zero; a head whose sum of squares overflows comes out as zeros; a NaN weight gives 0x7FC0 in its
    dim (and its pair partner) of every head.  Every other output equals the same call on clean data bit
    for bit."""
    from hy_nomas import fused

    print(f"qk_norm_rope nonfinite d={d}", flush=True)
    b, l, h = 1, 9, 6
    g = seeded(300 + d)
    x = bf(torch.randn(b, l, h, d, generator=g) * 3)
    w = bf(torch.rand(d, generator=g) + 0.5)
    ang = torch.rand(l, d, generator=g) * 6.28
    rope = (ang.cos().to(dev), ang.sin().to(dev))
    clean = x.clone()
    x[0, 1, 2, 5] = float("nan")
    x[0, 3, 0, d - 1] = float("inf")
    x[0, 4, 5, 7] = -float("inf")
    x[0, 6, 3] = 3e38   # the sum of squares overflows: r = 0
    nan_code = 0x7FC0

    def pair(i, rotated):
        return [i & ~1, i | 1] if rotated else [i]

    for rp in (None, rope):
        got = fused.qk_norm_rope(x.to(dev), w.to(dev), rp).cpu()
        ref = fused.qk_norm_rope(clean.to(dev), w.to(dev), rp).cpu()
        bits = got.view(torch.int16)
        assert (bits[0, 1, 2] == nan_code).all()
        for t, k, i in ((3, 0, d - 1), (4, 5, 7)):
            nan_dims = pair(i, rp is not None)
            assert (bits[0, t, k, nan_dims] == nan_code).all()
            zero_dims = [c for c in range(d) if c not in nan_dims]
            assert (got[0, t, k, zero_dims].float() == 0).all()
        assert (got[0, 6, 3].float() == 0).all()
        touched = torch.zeros(l, h, dtype=torch.bool)
        for t, k in ((1, 2), (3, 0), (4, 5), (6, 3)):
            touched[t, k] = True
        assert torch.equal(got[0][~touched], ref[0][~touched])
        ora = torch.from_numpy(oracle.qk_norm_rope(x, w, None if rp is None else (rp[0].cpu(), rp[1].cpu())))
        assert torch.equal(ora.isnan(), got.float().isnan())
        # a NaN weight in dim 5: that dim (and dim 4, its rotation partner) of every head is NaN
        wn = w.clone()
        wn[5] = float("nan")
        got = fused.qk_norm_rope(clean.to(dev), wn.to(dev), rp).cpu()
        bad = pair(5, rp is not None)
        keep = [i for i in range(d) if i not in bad]
        assert (got.view(torch.int16)[..., bad] == nan_code).all()
        assert torch.equal(got[..., keep], ref[..., keep])


def test_pixelumm_qk_nonfinite(dev):
    """A NaN in the T half of a head makes that half torch's NaN code 0x7FC0 (its norm is NaN); the head's HW
    half and every other head equal the same call on clean data bit for bit."""
    from hy_nomas import fused

    n, h, d = 11, 6, 128
    g = seeded(400)
    x = bf(torch.randn(1, n, h, d, generator=g) * 3)
    wt = bf(torch.rand(d // 2, generator=g) + 0.5).to(dev)
    whw = bf(torch.rand(d // 2, generator=g) + 0.5).to(dev)
    ang = torch.rand(n, d, generator=g) * 6.28
    cos, sin = ang.cos().to(dev), ang.sin().to(dev)
    ref = fused.pixelumm_qk(x.to(dev), wt, whw, cos, sin).cpu()
    x[0, 4, 2, 17] = float("nan")
    got = fused.pixelumm_qk(x.to(dev), wt, whw, cos, sin).cpu()
    assert (got.view(torch.int16)[0, 4, 2, :64] == 0x7FC0).all()
    assert torch.equal(got[0, 4, 2, 64:], ref[0, 4, 2, 64:])
    keep = torch.ones(n, h, dtype=torch.bool)
    keep[4, 2] = False
    assert torch.equal(got[0][keep], ref[0][keep])


@pytest.mark.parametrize("h", [1, 2, 3, 6, 24])
def test_pixelumm_qk_head_groups(dev, h):
    """The PixelUMM kernel's head groups: each head of a multi-head call equals a one-head call bit for bit."""
    from hy_nomas import fused

    print(f"pixelumm_qk head groups h={h}", flush=True)
    n, d = 53, 128
    g = seeded(200 + h)
    x = bf(torch.randn(1, n, h, d, generator=g) * 3)
    wt = bf(torch.rand(d // 2, generator=g) + 0.5)
    whw = bf(torch.rand(d // 2, generator=g) + 0.5)
    ang = torch.rand(n, d, generator=g) * 6.28
    cos, sin = ang.cos().to(dev), ang.sin().to(dev)
    xd, wtd, whwd = x.to(dev), wt.to(dev), whw.to(dev)
    got = fused.pixelumm_qk(xd, wtd, whwd, cos, sin)
    for k in range(h):
        assert torch.equal(got[:, :, k:k + 1], fused.pixelumm_qk(xd[:, :, k:k + 1], wtd, whwd, cos, sin))
    ref = bf(torch.from_numpy(oracle.pixelumm_qk(x, wt, whw, cos.cpu(), sin.cpu())))
    assert (got.cpu() != ref).float().mean().item() < 1e-2
