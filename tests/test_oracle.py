"""Pins the CPU oracle (oracle/hn_oracle.c) without trusting its own formulas.

Each oracle function is checked against something independent of its implementation:
  * hand-derived known answers (tests/golden/known_answers.json, made by exact rational arithmetic in
    tests/golden/make_known_answers.py);
  * library routines: torch's float8_e4m3fn cast, F.layer_norm, F.gelu(approximate="tanh"), torch's bf16
    arithmetic, and the reference's own non-fused torch forms of RMSNorm / RoPE / MRoPE restated with torch ops;
  * invariants a plausible mistake breaks: +-127 at the group absmax, |q * s - x| <= s / 2, ties away from
    zero, per-group scale independence, exact integer sums, error bounds against float64 products;
  * an exhaustive check of the division lemma the device quantizers rely on.
"""
import json
import os
from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))


def bf16_values(n, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, generator=g) * scale).to(torch.bfloat16).float().numpy()


# ------------------------------------------------------------------------------------------------
# activation / weight quantization (kernels.py:22-54, ops.py:41-52)

def test_quantize_known_answers():
    ka = json.load(open(os.path.join(HERE, "golden", "known_answers.json")))
    for case in ka["quantize"]:
        x = np.array(case["x"], dtype=np.float32).reshape(case["shape"])
        q, s = oracle.quantize(x, case["group"], case["kind"], case["rounding"])
        assert s.ravel().tolist() == pytest.approx(case["scales"], rel=0, abs=0), case["name"]
        assert q.ravel().astype(int).tolist() == case["codes"], case["name"]


def test_quantize_invariants():
    x = bf16_values(64 * 3072, seed=1).reshape(64, 3072)
    x[:, ::97] *= 20.0
    q, s = oracle.quantize(x)
    xs = x.reshape(64, 24, 128)
    qs = q.reshape(64, 24, 128).astype(np.float64)
    peak = np.abs(xs).max(-1)
    assert np.array_equal(s, (peak.astype(np.float32) / np.float32(127)).astype(np.float32))
    arg = np.abs(xs).argmax(-1)
    at_peak = np.take_along_axis(qs, arg[..., None], -1)[..., 0]
    assert np.all(np.abs(at_peak) == 127)
    err = np.abs(qs * s[..., None] - xs)
    # x / s is rounded to fp32 before the integer rounding: allow half an fp32 ulp of a quotient <= 127
    assert np.all(err <= s[..., None] * (0.5 + 2.0 ** -17))
    # groups are independent: scaling one group leaves the others' codes unchanged
    x2 = xs.copy()
    x2[:, 5] *= 1000.0
    q2, s2 = oracle.quantize(x2.reshape(64, 3072))
    keep = [g for g in range(24) if g != 5]
    assert np.array_equal(q2.reshape(64, 24, 128)[:, keep], q.reshape(64, 24, 128)[:, keep])
    assert np.array_equal(s2[:, keep], s[:, keep])


def test_quantize_per_token_is_one_group():
    x = bf16_values(8 * 1024, seed=2).reshape(8, 1024)
    q, s = oracle.quantize(x, None)
    assert s.shape == (8, 1)
    assert np.array_equal(s[:, 0], (np.abs(x).max(1) / np.float32(127)).astype(np.float32))
    assert np.all(np.abs(q.astype(np.float64) * s - x) <= s * (0.5 + 2.0 ** -17))


def test_quantize_ties_round_away_and_even():
    # scale exactly 1 (peak 127): every k + 0.5 is a tie
    x = np.zeros((1, 128), dtype=np.float32)
    x[0, 0] = 127.0
    ties = np.arange(-63.5, 63.0, 1.0, dtype=np.float32)
    x[0, 1:1 + len(ties)] = ties
    q, _ = oracle.quantize(x)
    away = np.sign(ties) * np.floor(np.abs(ties) + 0.5)
    assert np.array_equal(q[0, 1:1 + len(ties)], away.astype(np.int8))
    qe, _ = oracle.quantize(x, rounding="half_even")
    assert np.array_equal(qe[0, 1:1 + len(ties)], np.round(ties).astype(np.int8))   # numpy rounds half to even


def test_quantize_zero_group_and_g128_weights():
    x = np.zeros((2, 256), dtype=np.float32)
    x[1, 128:] = bf16_values(128, seed=3)
    q, s = oracle.quantize(x)
    assert s[0].tolist() == [1.0, 1.0] and s[1, 0] == 1.0 and np.all(q[0] == 0) and np.all(q[1, :128] == 0)
    # the torch weight quantizer of the package follows the same rule (independent implementation)
    from hy_nomas import ops
    w = torch.from_numpy(bf16_values(64 * 384, seed=4).reshape(64, 384))
    qt, st = ops.quantize_g128(w)
    qo, so = oracle.quantize(w.numpy())
    assert np.array_equal(qt.numpy(), qo) and np.array_equal(st.numpy(), so)
    # K not a multiple of 128: zero padding inside the last group
    w2 = torch.from_numpy(bf16_values(16 * 200, seed=5).reshape(16, 200))
    q2, s2 = ops.quantize_g128(w2)
    qo2, so2 = oracle.quantize_g128(w2.numpy())
    assert np.array_equal(q2.numpy(), qo2) and np.array_equal(s2.numpy(), so2)


def test_kv_quant_matches_reference_torch_form():
    """world.py:83-94 restated with torch ops (absmax per (token, head), IEEE division, floor/ceil half away,
    clamp; dequant as an fp32 product then bf16) against the oracle, with forced ties and an all-zero head."""
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(37, 5, 128, generator=g) * 3).to(torch.bfloat16).float()
    x[3, 2] = 0.0                                     # all-zero head: scale 1, codes 0
    x[4, 1, :] = torch.arange(128, dtype=torch.float32) - 63.5   # peak 64 -> scale 64/127: no tie by design
    x[5, 0, :] = 0.0
    x[5, 0, 0] = 127.0                                # scale exactly 1: the next values are exact ties
    x[5, 0, 1:9] = torch.tensor([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5])
    peak = x.abs().amax(dim=-1, keepdim=True)
    scale = torch.where(peak > 0, peak / 127.0, torch.ones_like(peak))
    scaled = x / scale
    ref_q = torch.where(scaled >= 0, torch.floor(scaled + 0.5), torch.ceil(scaled - 0.5)).clamp_(-127, 127)
    q, s = oracle.quantize_kv(x.numpy())
    assert np.array_equal(q, ref_q.to(torch.int8).numpy()) and np.array_equal(s, scale.numpy())
    assert q[5, 0, 1:9].tolist() == [1, -1, 2, -2, 3, -3, 127, -127]
    ref_dq = (torch.from_numpy(q).float() * torch.from_numpy(s)).to(torch.bfloat16).float().numpy()
    assert np.array_equal(oracle.dequantize_kv(q, s), ref_dq)


def test_fast_division_lemma_exhaustive():
    """Every bf16 absmax >= 2^-80 and every bf16 x with |x| <= absmax, both signs: the device's reciprocal +
    FMA quotient with unclamped rounding gives the same int8 codes (half away from zero and half to even) as
    IEEE x / scale with the reference's clamped rounding, and the same e4m3 codes."""
    lib = oracle.lib()
    assert lib.hno_check_fast_division(0, 1, 0x7F80) == 0
    assert lib.hno_check_fast_division(1, 1, 0x7F80) == 0


def test_two_op_division_lemma_exhaustive():
    """The int8 quantizers' two-operation quotient fma(x, r, x * rl) (r = RN(1 / s), rl = RN(fma(-s, r, 1) * r))
    gives the reference's int8 codes, both roundings, for every bf16 absmax in [2^-80, 2^100) and every bf16
    x with |x| <= absmax, both signs.  A planted error (rl dropped) must be caught: x * r alone changes codes
    next to exact .5 ties."""
    lib = oracle.lib()
    assert lib.hno_check_fast_division2(1, 0x7F80, 0) == 0
    assert lib.hno_check_fast_division2(0x3F00, 0x4380, 1) > 0  # peaks 0.5 .. 256 with the planted error


def test_reciprocal_refinement_exhaustive():
    """The device's 1 / scale: any hardware reciprocal within 2 ulp, refined by one FMA Newton step, is the
    correctly rounded reciprocal for every bf16 peak >= 2^-80 (int8 and fp8 scales)."""
    assert oracle.lib().hno_check_reciprocal_refinement() == 0


def test_half_even_code_by_magic_add():
    """The half-even int8 code as the low byte of fp32(y + 1.5 * 2^23) (the device's one-op form) equals the low
    byte of rint(y), ties to even, for every integer and half-integer in [-128, 128] with its 8 nearest fp32
    neighbours on each side, every fp32 in [125, 128) and its negative (the largest codes), and 4 million
    random quotients in [-127.5, 127.5]."""
    rng = np.random.default_rng(7)
    ties = np.arange(-256, 257, dtype=np.float32) / np.float32(2)
    near, up, down = [ties], ties.copy(), ties.copy()
    for _ in range(8):
        up = np.nextafter(up, np.float32(np.inf))
        down = np.nextafter(down, np.float32(-np.inf))
        near += [up, down]
    lo = np.frombuffer(np.float32(125.0).tobytes(), np.uint32)[0]
    hi = np.frombuffer(np.float32(128.0).tobytes(), np.uint32)[0]
    top = np.arange(lo, hi, dtype=np.uint32).view(np.float32)
    y = np.concatenate(near + [top, -top, rng.uniform(-127.5, 127.5, 4_000_000).astype(np.float32)])
    want = (np.rint(y).astype(np.int32) & 0xFF).astype(np.uint8)
    got = ((y + np.float32(1.5 * 2 ** 23)).view(np.uint32) & 0xFF).astype(np.uint8)
    assert np.array_equal(got, want)
    # a planted error must be caught: with 2^23 the negative quotients fall into the binade below, whose
    # spacing is 1/2, so their low bytes are no longer the codes
    bad = ((y + np.float32(2 ** 23)).view(np.uint32) & 0xFF).astype(np.uint8)
    assert not np.array_equal(bad, want)


def test_fast_scale_division_exhaustive():
    """The device's group scales peak / 127 and max(peak, 1e-12) / 448 from the reciprocal + FMA quotient
    equal IEEE division for every bf16 peak >= 2^-80."""
    assert oracle.lib().hno_check_scale_division() == 0


# ------------------------------------------------------------------------------------------------
# fp8 e4m3fn encoding (kernels.py:39-41, pixelumm.py:77-82)

def test_e4m3_encode_matches_torch_every_bf16_and_edges():
    bits = np.arange(0, 0x10000, dtype=np.uint32) << 16
    vals = bits.view(np.float32)
    vals = vals[np.isfinite(vals)]
    edges = np.array([448.0, 464.0, 464.0001, 479.99, 480.0, 1e-12, 2 ** -9, 2 ** -10, 2 ** -10 * 1.5,
                      2 ** -6, 2 ** -6 * 0.99, 0.0, -0.0, 1.0625, 1.1875], dtype=np.float32)
    rnd = np.random.default_rng(0).standard_normal(200000).astype(np.float32) * 50
    for v in (vals, edges, -edges, rnd):
        mine = oracle.e4m3_encode(v)
        ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(mine, ref)
    table = oracle.e4m3_decode_table()
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(table), np.isnan(ref))
    assert np.array_equal(table[~np.isnan(table)], ref[~np.isnan(ref)])


def test_fp8_block_weights_match_torch_cast():
    w = torch.randn(256, 384, generator=torch.Generator().manual_seed(6)) * 0.02
    q, s = oracle.fp8_block_quantize(w.numpy())
    from hy_nomas import pixelumm
    qt, st = pixelumm.quantize_fp8_block(w)
    assert np.array_equal(q, qt.view(torch.uint8).numpy()) and np.allclose(s, st.numpy(), rtol=0, atol=0)


# ------------------------------------------------------------------------------------------------
# block-scaled GEMM (kernels.py:80-170)

def int8_operands(m, n, k, seed, per_channel=False):
    g = torch.Generator().manual_seed(seed)
    qa = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).numpy()
    qw = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).numpy()
    ng = 1 if per_channel else k // 128
    sa = (torch.rand(m, ng, generator=g) * 1e-2 + 1e-3).numpy()
    sw = (torch.rand(n, ng, generator=g) * 4e-3 + 1e-3).numpy()
    bias = torch.randn(n, generator=g).to(torch.bfloat16).float().numpy() * 0.02
    return qa, sa, qw, sw, bias


def test_gemm_integer_sums_brute_force():
    qa, sa, qw, sw, _ = int8_operands(5, 7, 256, seed=7)
    _, acc = oracle.block_gemm(qa, sa, qw, sw, want_acc32=True)
    for m in range(5):
        for n in range(7):
            assert acc[m, n] == sum(int(a) * int(b) for a, b in zip(qa[m], qw[n]))


def test_gemm_known_answer_permutation():
    """qa = identity codes with unit scales: out[m, n] = code qw[n, m] * sw[n] exactly."""
    k = 128
    qa = np.eye(k, dtype=np.int8)
    qw = torch.randint(-127, 128, (64, k), generator=torch.Generator().manual_seed(8), dtype=torch.int8).numpy()
    sa = np.ones((k, 1), dtype=np.float32)
    sw = np.full((64, 1), 0.5, dtype=np.float32)
    out = oracle.block_gemm(qa, sa, qw, sw)
    assert np.array_equal(out, qw.T.astype(np.float32) * 0.5)


@pytest.mark.parametrize("per_channel", [False, True])
def test_gemm_against_float64_product(per_channel):
    qa, sa, qw, sw, bias = int8_operands(40, 96, 1024, seed=9, per_channel=per_channel)
    out = oracle.block_gemm(qa, sa, qw, sw, bias)
    k = qa.shape[1]
    ra = np.repeat(sa.astype(np.float64), k // sa.shape[1], 1)
    rw = np.repeat(sw.astype(np.float64), k // sw.shape[1], 1)
    exact = (qa * ra) @ (qw * rw).T + bias
    # a handful of fp32 roundings per group: relative error far below 1e-5 of the output scale
    assert np.abs(out - exact).max() <= 1e-5 * np.abs(exact).max()
    # bias enters once, additively
    out_nb = oracle.block_gemm(qa, sa, qw, sw, None)
    assert np.abs((out - out_nb) - bias).max() <= 1e-6 * np.abs(exact).max()


def test_gemm_gelu_epilogues_against_torch():
    qa, sa, qw, sw, bias = int8_operands(64, 256, 512, seed=10)
    plain = oracle.block_gemm(qa, sa, qw, sw, bias)
    gelu = oracle.block_gemm(qa, sa, qw, sw, bias, epilogue="gelu")
    ref = F.gelu(torch.from_numpy(plain).to(torch.bfloat16).float(), approximate="tanh").to(torch.bfloat16).float()
    g = torch.from_numpy(gelu)
    # torch evaluates tanh-GELU through tanh, the reference through a sigmoid: last-bit differences only
    assert (g != ref).float().mean().item() < 1e-2
    assert (g - ref).abs().max().item() <= 2 ** -7 * ref.abs().max().item()
    codes, qs, h = oracle.block_gemm(qa, sa, qw, sw, bias, epilogue="gelu_quant")
    q2, s2 = oracle.quantize(h)
    assert np.array_equal(codes, q2) and np.array_equal(qs, s2) and np.array_equal(h, gelu)


def test_gemm_fp8_against_float64_product():
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(32, 512, generator=g)).to(torch.bfloat16)
    w = torch.randn(128, 512, generator=g) * 0.02
    qa, sa = oracle.quantize(x, 128, "fp8")
    qw, sblk = oracle.fp8_block_quantize(w.numpy())
    sw = np.repeat(sblk, 128, 0)
    out = oracle.block_gemm(qa, sa, qw, sw, kind="fp8")
    table = oracle.e4m3_decode_table().astype(np.float64)
    exact = (table[qa] * np.repeat(sa, 128, 1)) @ (table[qw] * np.repeat(sw, 128, 1)).T
    assert np.abs(out - exact).max() <= 1e-5 * np.abs(exact).max()


# ------------------------------------------------------------------------------------------------
# fused elementwise (fused.py, kernels.py:173-207)

def test_adaln_against_torch_layer_norm():
    g = torch.Generator().manual_seed(12)
    x = (torch.randn(2, 100, 2048, generator=g) * 3).to(torch.bfloat16)
    shift = torch.randn(2, 2048, generator=g).to(torch.bfloat16)
    scale = torch.randn(2, 2048, generator=g).to(torch.bfloat16)
    ref = (F.layer_norm(x.float(), (2048,), eps=1e-6) * (1 + scale.unsqueeze(1)).to(torch.bfloat16).float()
           + shift.unsqueeze(1).float()).to(torch.bfloat16)
    got = torch.from_numpy(oracle.adaln(x, shift, scale)).view(2, 100, 2048).to(torch.bfloat16)
    assert (got != ref).float().mean().item() < 1e-3
    assert (got.float() - ref.float()).abs().max().item() < 0.05
    # a constant row normalizes to 0, so the output is exactly the shift
    xc = torch.full((1, 3, 2048), 1.5).to(torch.bfloat16)
    yc = oracle.adaln(xc, shift[:1], scale[:1])
    assert np.array_equal(torch.from_numpy(yc).to(torch.bfloat16).float().numpy(),
                          np.broadcast_to(shift[:1].float().numpy(), (3, 2048)))


def test_adaln_rms_against_torch():
    g = torch.Generator().manual_seed(13)
    x = (torch.randn(1, 64, 3072, generator=g) * 2).to(torch.bfloat16)
    shift = torch.randn(1, 3072, generator=g).to(torch.bfloat16) * 0.1
    scale = torch.randn(1, 3072, generator=g).to(torch.bfloat16) * 0.1
    xf = x.float()
    n = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    ref = (n * (1 + scale.unsqueeze(1)).to(torch.bfloat16).float() + shift.unsqueeze(1).float()).to(torch.bfloat16)
    got = torch.from_numpy(oracle.adaln(x, shift, scale, norm="rms")).view(1, 64, 3072).to(torch.bfloat16)
    assert (got != ref).float().mean().item() < 1e-3


def test_adaln_quant_is_quantized_adaln():
    g = torch.Generator().manual_seed(14)
    x = (torch.randn(1, 50, 3072, generator=g) * 3).to(torch.bfloat16)
    shift = torch.randn(1, 3072, generator=g).to(torch.bfloat16)
    scale = torch.randn(1, 3072, generator=g).to(torch.bfloat16)
    q, s, y = oracle.adaln(x, shift, scale, quant=True)
    y_plain = oracle.adaln(x, shift, scale)
    assert np.array_equal(y, oracle.rbf16(y_plain))
    q2, s2 = oracle.quantize(y)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_gated_residual_matches_torch_bf16():
    g = torch.Generator().manual_seed(15)
    x = torch.randn(2, 300, 512, generator=g).to(torch.bfloat16)
    y = torch.randn(2, 300, 512, generator=g).to(torch.bfloat16)
    gate = torch.randn(2, 512, generator=g).to(torch.bfloat16)
    ref = x + y * gate.unsqueeze(1)
    got = torch.from_numpy(oracle.gated_residual(x, y, gate)).to(torch.bfloat16)
    assert torch.equal(got, ref)


def test_qk_norm_rope_against_torch_forms():
    from oracle import torch_forms
    b, l, h, d = 1, 96, 4, 128
    g = torch.Generator().manual_seed(16)
    x = (torch.randn(b, l, h, d, generator=g) * 5).to(torch.bfloat16)
    norm = torch_forms.RMSNorm(d).bfloat16()
    with torch.no_grad():
        norm.weight.copy_(torch.rand(d, generator=g) + 0.5)
        plain = norm(x).to(torch.bfloat16)
        rope = torch_forms.rope_freqs([16, 56, 56], 256, 4, 4, 6)
        roped = torch_forms.apply_rope(plain, *rope)
    got_plain = torch.from_numpy(oracle.qk_norm_rope(x, norm.weight.detach(), None)).to(torch.bfloat16)
    got = torch.from_numpy(oracle.qk_norm_rope(x, norm.weight.detach(), rope)).to(torch.bfloat16)
    assert (got_plain != plain).float().mean().item() < 1e-3
    assert (got != roped).float().mean().item() < 1e-2
    assert ((got.float() - roped.float()).norm() / roped.float().norm()).item() < 1e-3
    # zero angles: the rotation is the identity
    zero = (torch.ones(l, d), torch.zeros(l, d))
    assert torch.equal(torch.from_numpy(oracle.qk_norm_rope(x, norm.weight.detach(), zero)).to(torch.bfloat16),
                       got_plain)


def test_pixelumm_qk_against_torch_form():
    """Split-half RMSNorm in fp32 (no intermediate rounding), then rotate-half MRoPE over the sections
    (D/2, D/4, D/4), one bf16 rounding: the reference's non-fused torch path (pixelumm.py:198-200, 279-290)."""
    n, h, d = 40, 3, 128
    g = torch.Generator().manual_seed(17)
    x = (torch.randn(1, n, h, d, generator=g) * 3).to(torch.bfloat16)
    wt = (torch.rand(d // 2, generator=g) + 0.5).to(torch.bfloat16)
    whw = (torch.rand(d // 2, generator=g) + 0.5).to(torch.bfloat16)
    ang = torch.rand(n, d, generator=g) * 6.28
    cos, sin = ang.cos(), ang.sin()

    def rms(v, w):
        return w.float() * (v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + 1e-6))

    def rotate_half(v):
        a, b = v.chunk(2, dim=-1)
        return torch.cat((-b, a), dim=-1)

    xf = x.float()
    t, hw = xf.chunk(2, dim=-1)
    normed = torch.cat((rms(t, wt), rms(hw, whw)), dim=-1)
    rot = torch.cat([rotate_half(p) for p in normed.split((d // 2, d // 4, d // 4), dim=-1)], dim=-1)
    ref = (normed * cos[None, :, None] + rot * sin[None, :, None]).to(torch.bfloat16)
    got = torch.from_numpy(oracle.pixelumm_qk(x, wt, whw, cos, sin)).to(torch.bfloat16)
    assert (got != ref).float().mean().item() < 1e-2
    assert ((got.float() - ref.float()).norm() / ref.float().norm()).item() < 1e-3


def test_dequant_linear_fallback_matches_float64():
    """The reference's CPU fallback restated (dequantize + F.linear) against float64 arithmetic."""
    g = torch.Generator().manual_seed(18)
    x = torch.randn(8, 256, generator=g).to(torch.bfloat16)
    qw = torch.randint(-127, 128, (32, 256), generator=g, dtype=torch.int8)
    sw = torch.rand(32, 2, generator=g) * 4e-3 + 1e-3
    bias = (torch.randn(32, generator=g) * 0.02).to(torch.bfloat16)
    out = oracle.dequant_linear(x, qw, sw, bias)
    w = (qw.double().view(32, 2, 128) * sw.double().unsqueeze(-1)).view(32, 256).to(torch.bfloat16).double()
    exact = x.double() @ w.T + bias.double()
    assert ((out.double() - exact).abs().max() / exact.abs().max()).item() < 1e-2


def test_exact_rational_rounding_agrees_except_fp32_quirk():
    """The oracle's int8 codes equal exact round-half-away-from-zero of the fp32 quotient, except where
    fp32 evaluation of y + 0.5 itself rounds up to the next integer (kernels.py:35 evaluates it in fp32)."""
    x = bf16_values(4 * 1024, seed=19, scale=3.0).reshape(4, 1024)
    q, s = oracle.quantize(x)
    y = (x.reshape(4, 8, 128) / s[..., None]).astype(np.float32).ravel()
    qf = q.ravel()
    quirk = 0
    for yi, qi in zip(y.tolist(), qf.tolist()):
        fy = Fraction(yi)
        mag = abs(fy) + Fraction(1, 2)
        exact = int(mag.numerator // mag.denominator) * (1 if fy >= 0 else -1)
        exact = max(-127, min(127, exact))
        if exact != qi:
            # only allowed when |y| + 0.5 is not representable and fp32 rounding crossed the integer
            assert float(np.float32(abs(yi)) + np.float32(0.5)) == abs(qi)
            quirk += 1
    assert quirk <= 2


def test_swiglu_silu_matches_torch_bf16_and_float64_for_every_bf16():
    """oracle.swiglu's silu (pixelumm.py:322, F.silu on a bf16 tensor): for every finite bf16 g, with u = 1,
    h equals torch's CPU bf16 silu, and equals the float64 silu rounded to bf16 wherever exp(-g) is finite in
    fp32 (below -88.7 the fp32 formula gives -0, as torch's does).  Then the product rounding: h(g, u) for
    random bf16 u equals rbf16(h(g, 1) * u), the exact product rounded once."""
    import torch

    bits = np.arange(65536, dtype=np.uint32)
    g = (bits << 16).view(np.float32)
    g = g[np.isfinite(g)]
    h = oracle.swiglu(g, np.ones_like(g))
    t = torch.nn.functional.silu(torch.from_numpy(g).to(torch.bfloat16)).float().numpy()
    assert np.array_equal(h.view(np.uint32), t.view(np.uint32))
    ok = g > -88.5
    g64 = g[ok].astype(np.float64)
    exact = g64 / (1.0 + np.exp(-g64))
    assert np.array_equal(h[ok], oracle.rbf16(exact.astype(np.float32)))
    rng = np.random.default_rng(3)
    u = oracle.rbf16(rng.standard_normal(g.size).astype(np.float32) * 4)
    h2 = oracle.swiglu(g, u)
    with np.errstate(over="ignore"):
        assert np.array_equal(h2, oracle.rbf16(h * u))
