"""Block-scaled int8 / fp8 GEMM on the GPU vs the CPU oracle (hy_nomas/kernels.py:80-170).

int8: the int32 accumulators are exact and the fp32 epilogue runs the oracle's operation sequence, so the
outputs must match the oracle bit for bit.  gelu uses the hardware exp2 and reciprocal, so its bf16 outputs may differ
in rare last-bit cases (the reference test's tolerances apply).  fp8: fp32 accumulation inside the
matrix core has its own order; checked to 1e-2 max-abs-rel against the fp64 product of the dequantized
operands (and tightly against the oracle)."""
import numpy as np
import pytest
import torch

import oracle
from conftest import seeded
from test_quant_gpu import outlier_input

pytestmark = pytest.mark.gpu


def int8_weights(n, k, seed, per_channel=False):
    g = seeded(seed)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    if per_channel:
        sw = (torch.rand(n, 1, generator=g) * 4e-3 + 1e-3).float()
    else:
        sw = (torch.rand(n, k // 128, generator=g) * 4e-3 + 1e-3).float()
    bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    return w, sw, bias


def fp64_dequant_product(qa, sa, qw, sw, bias, kind="int8"):
    """(qa * sa)(qw * sw)^T + b in float64 (the dequantized-operand product)."""
    if kind == "fp8":
        table = oracle.e4m3_decode_table().astype(np.float64)
        a = table[np.asarray(qa).view(np.uint8)]
        w = table[np.asarray(qw).view(np.uint8)]
    else:
        a = np.asarray(qa, dtype=np.float64)
        w = np.asarray(qw, dtype=np.float64)
    k = a.shape[1]
    ra = np.repeat(np.asarray(sa, np.float64), k // sa.shape[1], axis=1)
    rw = np.repeat(np.asarray(sw, np.float64), k // sw.shape[1], axis=1)
    out = (a * ra) @ (w * rw).T
    if bias is not None:
        out += oracle.to_f32(bias).astype(np.float64)
    return out


def max_abs_rel(got, ref):
    return float(np.abs(got - ref).max() / np.abs(ref).max())


@pytest.mark.parametrize("m,n,k", [(100, 200, 256), (513, 768, 3072), (64, 256, 12288), (1, 3072, 128)])
def test_acc32_exact(dev, m, n, k):
    from hy_nomas import kernels

    print(f"acc32 m={m} n={n} k={k}", flush=True)
    g = seeded(m + n + k)
    qa = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8)
    qw = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    got = kernels.block_gemm_acc32(qa.to(dev), qw.to(dev)).cpu().numpy()
    ref = qa.numpy().astype(np.int64) @ qw.numpy().astype(np.int64).T
    assert np.array_equal(got.astype(np.int64), ref)


def test_acc32_extreme_codes(dev):
    """All +-127 codes over K = 12288: the largest accumulator magnitude (198 M) stays exact."""
    from hy_nomas import kernels

    k = 12288
    qa = torch.full((32, k), 127, dtype=torch.int8)
    qa[1::2] = -127
    qw = torch.full((256, k), -127, dtype=torch.int8)
    got = kernels.block_gemm_acc32(qa.to(dev), qw.to(dev)).cpu().numpy().astype(np.int64)
    ref = qa.numpy().astype(np.int64) @ qw.numpy().astype(np.int64).T
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("m,n,k,per_channel", [
    (300, 384, 1024, False), (257, 3072, 3072, False), (1, 256, 128, False), (1024, 640, 2048, False),
    (512, 1024, 3072, True), (100, 384, 12288, True), (1024, 3072, 3072, True)])
@pytest.mark.parametrize("with_bias", [True, False])
def test_int8_gemm_bit_exact(dev, m, n, k, per_channel, with_bias):
    from hy_nomas import kernels

    print(f"int8 gemm m={m} n={n} k={k} per_channel={per_channel} bias={with_bias}", flush=True)
    x = outlier_input(m, k, seed=m + n)
    w, sw, bias = int8_weights(n, k, seed=n + k, per_channel=per_channel)
    bias = bias if with_bias else None
    group = None if per_channel else 128
    qa, sa = oracle.quantize(x, group or k)
    out = kernels.block_gemm(torch.from_numpy(qa).to(dev), torch.from_numpy(sa).to(dev), w.to(dev), sw.to(dev),
                             bias.to(dev) if bias is not None else None)
    ref = oracle.block_gemm(qa, sa, w.numpy(), sw.numpy(), oracle.to_f32(bias) if bias is not None else None)
    ref_bf16 = torch.from_numpy(ref).to(torch.bfloat16)
    got = out.cpu()
    diff = (got != ref_bf16).nonzero()
    assert diff.numel() == 0, f"{len(diff)} outputs differ from the oracle, first {diff[:3].tolist()}"
    # and the 1e-2 max-abs-rel bar against the product of the dequantized operands
    assert max_abs_rel(got.float().numpy(), fp64_dequant_product(qa, sa, w.numpy(), sw.numpy(), bias)) < 1e-2


@pytest.mark.parametrize("with_bias", [True, False])
def test_int8_gemm_signed_zeros(dev, with_bias):
    """Exact-zero dot products (all-zero token rows and weight rows) under negative channel scales, with
    biases of -0 and +0: the output bits, the signs of zeros included, are the oracle's
    ((0 + (x sa) sw) + b in fp32, then bf16), for per-token scales and for the g128 layout."""
    from hy_nomas import kernels

    print(f"int8 gemm signed zeros bias={with_bias}", flush=True)
    m, n, k = 96, 256, 512
    x = outlier_input(m, k, seed=77)
    x[::7] = 0
    for per_channel in (True, False):
        w, sw, bias = int8_weights(n, k, seed=78, per_channel=per_channel)
        w[::5] = 0
        sw[::3] = -sw[::3]
        bias[::2] = -0.0
        bias[1::4] = 0.0
        bias = bias if with_bias else None
        qa, sa = oracle.quantize(x, k if per_channel else 128)
        out = kernels.block_gemm(torch.from_numpy(qa).to(dev), torch.from_numpy(sa).to(dev), w.to(dev), sw.to(dev),
                                 bias.to(dev) if bias is not None else None)
        ref = oracle.block_gemm(qa, sa, w.numpy(), sw.numpy(), oracle.to_f32(bias) if bias is not None else None)
        want = torch.from_numpy(ref).to(torch.bfloat16).view(torch.int16)
        got = out.cpu().view(torch.int16)
        # zero products in channels with sw < 0 and b = -0 (or no bias): a plain (x sa) sw + b gives -0 there
        assert (want == 0).any() and not (want == -32768).any()
        diff = (got != want).nonzero()
        assert diff.numel() == 0, f"per_channel={per_channel}: {len(diff)} output bit patterns differ, first {diff[:3].tolist()}"


@pytest.mark.parametrize("m,n,k,epilogue", [
    (64, 288, 256, None), (300, 1000, 384, None), (513, 520, 640, None), (40, 4096, 256, None),
    (130, 384, 384, None), (40, 4096, 256, "gelu_quant"), (130, 384, 384, "gelu_quant")])
def test_g128_stage_counts_and_ragged_tiles(dev, m, n, k, epilogue):
    """The g128 layout's block-major loop: two, three and five 128-deep stages (the last two stages of a tile
    take their own code paths, and a tile's first stage folds no previous block), tiles cut by M and N,
    N not a multiple of 8 (scalar stores), and the GELU + requantization epilogue; bit-exact vs the oracle."""
    from hy_nomas import kernels

    print(f"g128 int8 m={m} n={n} k={k} epilogue={epilogue}", flush=True)
    x = outlier_input(m, k, seed=m + 7 * n)
    w, sw, bias = int8_weights(n, k, seed=n + 3 * k)
    qa, sa = oracle.quantize(x, 128)
    args = (torch.from_numpy(qa).to(dev), torch.from_numpy(sa).to(dev), w.to(dev), sw.to(dev), bias.to(dev))
    if epilogue is None:
        out = kernels.block_gemm(*args)
        ref = oracle.block_gemm(qa, sa, w.numpy(), sw.numpy(), oracle.to_f32(bias))
        got, want = out.cpu(), torch.from_numpy(ref).to(torch.bfloat16)
        diff = (got != want).nonzero()
        assert diff.numel() == 0, f"{len(diff)} outputs differ from the oracle, first {diff[:3].tolist()}"
    else:
        # the codes of the GEMM's own bf16 GELU output: the quantization runs on what the GELU epilogue writes
        gelu = kernels.block_gemm(*args, epilogue="gelu")
        qh, sh = kernels.block_gemm(*args, epilogue="gelu_quant")
        q2, s2 = kernels.quantize_activations(gelu)
        assert torch.equal(qh.cpu(), q2.cpu()) and torch.equal(sh.cpu(), s2.cpu())


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
def test_int8_gemm_out_dtypes(dev, out_dtype):
    from hy_nomas import kernels

    m, n, k = 200, 512, 2048
    x = outlier_input(m, k, seed=11)
    w, sw, bias = int8_weights(n, k, seed=12)
    qa, sa = oracle.quantize(x)
    out = kernels.block_gemm(torch.from_numpy(qa).to(dev), torch.from_numpy(sa).to(dev), w.to(dev), sw.to(dev),
                             bias.to(dev), out_dtype=out_dtype)
    ref = oracle.block_gemm(qa, sa, w.numpy(), sw.numpy(), oracle.to_f32(bias))
    assert torch.equal(out.cpu(), torch.from_numpy(ref).to(out_dtype))


def test_int8_gemm_ragged_n(dev):
    """N not a multiple of 4 or of the tile: the scalar store path."""
    from hy_nomas import kernels

    m, n, k = 77, 301, 512
    x = outlier_input(m, k, seed=13)
    w, sw, bias = int8_weights(n, k, seed=14)
    qa, sa = oracle.quantize(x)
    out = kernels.block_gemm(torch.from_numpy(qa).to(dev), torch.from_numpy(sa).to(dev), w.to(dev), sw.to(dev),
                             bias.to(dev))
    ref = oracle.block_gemm(qa, sa, w.numpy(), sw.numpy(), oracle.to_f32(bias))
    assert torch.equal(out.cpu(), torch.from_numpy(ref).to(torch.bfloat16))


@pytest.mark.parametrize("per_channel", [False, True])
def test_gelu_epilogues(dev, per_channel):
    """hy_nomas tests/test_fused.py:63-78 tolerances, against the oracle's epilogue."""
    from hy_nomas import kernels

    m, k, n = 1000, 2048, 1024
    x = outlier_input(m, k, seed=21)
    w, sw, bias = int8_weights(n, k, seed=22, per_channel=per_channel)
    group = None if per_channel else 128
    qa, sa = oracle.quantize(x, group or k)
    args = (torch.from_numpy(qa).to(dev), torch.from_numpy(sa).to(dev), w.to(dev), sw.to(dev), bias.to(dev))
    gelu = kernels.block_gemm(*args, epilogue="gelu").cpu()
    ref = torch.from_numpy(oracle.block_gemm(qa, sa, w.numpy(), sw.numpy(), oracle.to_f32(bias), epilogue="gelu"))
    ref = ref.to(torch.bfloat16)
    assert (gelu != ref).float().mean().item() < 1e-3
    assert (gelu.float() - ref.float()).abs().max().item() <= 2 ** -6 * ref.float().abs().max().item()
    qh, sh = kernels.block_gemm(*args, epilogue="gelu_quant")
    q_ref, s_ref, _ = oracle.block_gemm(qa, sa, w.numpy(), sw.numpy(), oracle.to_f32(bias), epilogue="gelu_quant")
    assert (qh.cpu().numpy() != q_ref).mean() < 1e-3
    assert np.allclose(sh.cpu().numpy(), s_ref, rtol=1e-3)
    # gelu_quant codes are exactly the quantization of this same GEMM's gelu output
    q2, s2 = kernels.quantize_activations(gelu.to(dev))
    assert torch.equal(qh.cpu(), q2.cpu()) and torch.equal(sh.cpu(), s2.cpu())


@pytest.mark.parametrize("m,n,k,group", [(300, 512, 1024, 128), (1024, 1536, 3072, 128), (77, 384, 256, 128),
                                         (130, 640, 384, 128), (200, 384, 2048, None)])
def test_fp8_gemm(dev, m, n, k, group):
    from hy_nomas import kernels, pixelumm

    print(f"fp8 gemm m={m} n={n} k={k} group={group}", flush=True)
    g = seeded(m + n + k)
    x = outlier_input(m, k, seed=m)
    wf = torch.randn(n, k, generator=g) * 0.02
    bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    qw, sblk = pixelumm.quantize_fp8_block(wf)
    if group is None:
        sw = sblk.repeat_interleave(128, 0)[:, :1].contiguous()   # one scale per channel
        # only valid when a block row has one scale: use the first column's scale for the whole row
        wq_codes = qw
        sw_full = sw
    else:
        sw_full = sblk.repeat_interleave(128, 0)
        wq_codes = qw
    qa, sa = oracle.quantize(x, group or k, "fp8")
    out = kernels.block_gemm(torch.from_numpy(qa).view(torch.float8_e4m3fn).to(dev), torch.from_numpy(sa).to(dev),
                             wq_codes.to(dev), sw_full.to(dev), bias.to(dev), kind="fp8").cpu().float().numpy()
    w_codes = wq_codes.view(torch.uint8).numpy()
    ref = oracle.block_gemm(qa, sa, w_codes, sw_full.numpy(), oracle.to_f32(bias), kind="fp8")
    exact = fp64_dequant_product(qa, sa, w_codes, sw_full.numpy(), bias, kind="fp8")
    assert max_abs_rel(out, exact) < 1e-2
    assert max_abs_rel(out, ref) < 4e-3


@pytest.mark.parametrize("kind", ["fp8", "int8"])
@pytest.mark.parametrize("m,n,k", [(300, 384, 1024), (1024, 1536, 3072), (77, 200, 256), (64, 256, 128)])
def test_block_weight_scales(dev, kind, m, n, k):
    """Weight scales with one row per 128 output channels ([ceil(N/128), K/128], the fp8 128 x 128 block
    layout) against the same GEMM on the scales expanded to one row per channel: the fold multiplies by
    the product sa * sw instead of by sa, then sw, so the two agree to fp32 rounding, and both match the
    fp64 product of the dequantized operands."""
    from hy_nomas import kernels

    print(f"block weight scales {kind} m={m} n={n} k={k}", flush=True)
    g = seeded(m * 7 + n + k)
    x = outlier_input(m, k, seed=m + 1)
    nb = (n + 127) // 128
    sblk = (torch.rand(nb, k // 128, generator=g) * 4e-3 + 1e-3).float()
    if kind == "fp8":
        codes = (torch.randn(n, k, generator=g) * 100).clamp(-448, 448).to(torch.float8_e4m3fn)
        w_codes = codes.view(torch.uint8).numpy()
    else:
        codes = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
        w_codes = codes.numpy()
    bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    sw_full = sblk.repeat_interleave(128, 0)[:n].contiguous()
    qa, sa = oracle.quantize(x, 128, kind)
    qa_t = torch.from_numpy(qa)
    if kind == "fp8":
        qa_t = qa_t.view(torch.float8_e4m3fn)
    sa_t, sblk_t = torch.from_numpy(sa).to(dev), sblk.to(dev)
    assert kernels.validate_scales(sa_t, sblk_t)  # fp8: the block scales are read as stored
    args = (qa_t.to(dev), sa_t, codes.to(dev))
    # fp32 outputs, so that the fold's rounding is not hidden behind (or magnified by) a bf16 rounding
    got = kernels.block_gemm(*args, sblk_t, bias.to(dev), torch.float32, kind=kind).cpu().numpy()
    full = kernels.block_gemm(*args, sw_full.to(dev), bias.to(dev), torch.float32, kind=kind).cpu().numpy()
    exact = fp64_dequant_product(qa, sa, w_codes, sw_full.numpy(), bias, kind=kind)
    assert max_abs_rel(got, exact) < 1e-2
    assert max_abs_rel(got, full) < 4e-3
    if kind == "int8":   # exact int32 partials: only the fold's fp32 rounding differs
        assert max_abs_rel(got, full) < 1e-4


def test_fp8_block_scales_zero_and_inf(dev):
    """fp8 codes with 128 x 128 block weight scales that are not all positive and finite: one all-zero weight
    block at scale 0 and one all-zero activation group at scale 0 (the reference's fold multiplies them in
    as zeros), then one infinite activation scale.  The GEMM must not turn a zero scale into NaN for the
    whole block, as a running sum kept in units of the group's scale product would; the results follow the
    reference's per-group fold (the oracle), which reads the block scales repeated per channel."""
    from hy_nomas import kernels

    print("fp8 block scales with zeros", flush=True)
    m, n, k = 160, 384, 768
    g = seeded(777)
    x = outlier_input(m, k, seed=778)
    qa, sa = oracle.quantize(x, 128, "fp8")
    qa[5, 256:384] = 0
    sa[5, 2] = 0.0
    codes = (torch.randn(n, k, generator=g) * 100).clamp(-448, 448).to(torch.float8_e4m3fn)
    sblk = (torch.rand(n // 128, k // 128, generator=g) * 4e-3 + 1e-3).float()
    codes[128:256, 384:512] = 0
    sblk[1, 3] = 0.0
    w_codes = codes.view(torch.uint8).numpy()
    bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    sw_full = sblk.repeat_interleave(128, 0).contiguous()
    qa_t = torch.from_numpy(qa).view(torch.float8_e4m3fn).to(dev)
    got = kernels.block_gemm(qa_t, torch.from_numpy(sa).to(dev), codes.to(dev), sblk.to(dev), bias.to(dev),
                             torch.float32, kind="fp8").cpu().numpy()
    ref = oracle.block_gemm(qa, sa, w_codes, sw_full.numpy(), oracle.to_f32(bias), kind="fp8")
    assert np.isfinite(got).all()
    assert max_abs_rel(got, ref) < 4e-3
    # an infinite activation scale poisons its own token row only, as in the reference's fold
    sa_inf = sa.copy()
    sa_inf[9, 1] = np.inf
    got = kernels.block_gemm(qa_t, torch.from_numpy(sa_inf).to(dev), codes.to(dev), sblk.to(dev), bias.to(dev),
                             torch.float32, kind="fp8").cpu().numpy()
    rows = [r for r in range(m) if r != 9]
    assert np.isfinite(got[rows]).all()
    assert max_abs_rel(got[rows], ref[rows]) < 4e-3
    assert not np.isfinite(got[9]).all()


def test_fp8_block_linear(dev):
    """pixelumm.fp8_block_linear (block scales read directly) against F.linear on the dequantized fp8
    weights in fp32 (hy_nomas/pixelumm.py:147-155)."""
    from hy_nomas import pixelumm

    print("fp8 block linear", flush=True)
    g = seeded(4242)
    x = (torch.randn(3, 170, 1024, generator=g) * 0.5).to(torch.bfloat16)
    w = torch.randn(768, 1024, generator=g) * 0.02
    bias = (torch.randn(768, generator=g) * 0.02).to(torch.bfloat16)
    from hy_nomas import kernels

    qw, sblk = pixelumm.quantize_fp8_block(w)
    sblk_dev = sblk.to(dev)
    assert kernels.validate_scales(sblk_dev)
    got = pixelumm.fp8_block_linear(x.to(dev), qw.to(dev), sblk_dev, bias.to(dev)).cpu().float()
    ref = torch.nn.functional.linear(x.float(), pixelumm.dequantize_fp8_block(qw, sblk, torch.float32),
                                     bias.float())
    assert got.shape == (3, 170, 768)
    assert ((got - ref).abs().max() / ref.abs().max()).item() < 3e-2


@pytest.mark.parametrize("layout", ["g128", "per_token", "block"])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("n,k", [(18432, 3072), (200, 640), (3072, 12288)])
def test_skinny_m_equals_the_tile_kernel(dev, layout, m, n, k):
    """M <= 4 int8 runs the skinny v_dot4 kernel (the per-sample linears, e.g. the modulation linear
    3072 -> 18432 at batch 1-2).  Its rows must equal, bit for bit, the same rows of a large-M product
    (the MFMA tile kernel), for every scale layout, with a ragged N and a K that ends mid-step."""
    from hy_nomas import kernels

    print(f"skinny {layout} m={m} n={n} k={k}", flush=True)
    g = seeded(m * 7 + n + k)
    x = outlier_input(300, k, m * 7 + n + k)
    group = None if layout == "per_token" else 128
    qa, sa = kernels.quantize_activations(x.to(dev), "int8", group)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(dev)
    if layout == "per_token":
        sw = (torch.rand(n, 1, generator=g) * 4e-3 + 1e-3).to(dev)
    elif layout == "g128":
        sw = (torch.rand(n, k // 128, generator=g) * 4e-3 + 1e-3).to(dev)
    else:
        sw = (torch.rand((n + 127) // 128, k // 128, generator=g) * 4e-3 + 1e-3).to(dev)
    bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    for out_dtype, epi in ((torch.bfloat16, None), (torch.float32, None), (torch.bfloat16, "gelu"),
                           (torch.float16, None)):
        big = kernels.block_gemm(qa, sa, w, sw, bias, out_dtype, epilogue=epi)
        small = kernels.block_gemm(qa[:m].clone(), sa[:m].clone(), w, sw, bias, out_dtype, epilogue=epi)
        assert small.shape == (m, n)
        assert torch.equal(small.view(torch.int16) if out_dtype != torch.float32 else small,
                           big[:m].view(torch.int16) if out_dtype != torch.float32 else big[:m])
    nob = kernels.block_gemm(qa[:m].clone(), sa[:m].clone(), w, sw, None, torch.float32)
    assert torch.equal(nob, kernels.block_gemm(qa, sa, w, sw, None, torch.float32)[:m])
    if layout != "block" and n == 200:
        ref = oracle.block_gemm(qa[:m].cpu().numpy(), sa[:m].cpu().numpy(), w.cpu().numpy(), sw.cpu().numpy(),
                                oracle.to_f32(bias.cpu()))
        got = kernels.block_gemm(qa[:m].clone(), sa[:m].clone(), w, sw, bias, torch.float32).cpu().numpy()
        assert np.array_equal(got, ref)


def test_modulation_linear_from_silu_vec(dev):
    """The reference's Modulate (hy_nomas/model.py:306-314): linear(silu(vec)) with an int8 g128 weight at
    batch 1, through block_linear (quantize + skinny GEMM), vs the dequantized fp32 product."""
    from hy_nomas import kernels, ops

    print("modulation linear", flush=True)
    g = seeded(99)
    vec = torch.randn(1, 3072, generator=g).to(torch.bfloat16)
    w = torch.randn(6 * 3072, 3072, generator=g) * 0.02
    q, s = ops.quantize_g128(w)
    bias = (torch.randn(6 * 3072, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.nn.functional.silu(vec.to(dev))
    got = kernels.block_linear(x, q.to(dev), s.to(dev), bias.to(dev))
    ref = torch.nn.functional.linear(x.float().cpu(), ops.dequantize_g128(q, s, torch.float32), bias.float())
    assert got.shape == (1, 18432)
    assert ((got.float().cpu() - ref).norm() / ref.norm()).item() < 2e-2


def test_wrappers_reject_mismatched_operands(dev):
    """The C ABI sees pointers and strides only; the Python wrappers refuse operands whose shapes or dtypes
    would make a kernel read past a tensor (K mismatch, short scale or bias tensors, wrong code type)."""
    from hy_nomas import fused, kernels

    print("wrapper validation", flush=True)
    g = seeded(31)
    x = torch.randn(64, 256, generator=g).to(torch.bfloat16).to(dev)
    qa, sa = kernels.quantize_activations(x)
    w = torch.randint(-127, 128, (128, 256), generator=g, dtype=torch.int8).to(dev)
    sw = (torch.rand(128, 2, generator=g) * 1e-3 + 1e-3).to(dev)
    kernels.block_gemm(qa, sa, w, sw)                                  # the valid call
    bad = [
        lambda: kernels.block_gemm(qa, sa, w[:, :128].contiguous(), sw[:, :1].contiguous()),  # K mismatch
        lambda: kernels.block_gemm(qa, sa[:63], w, sw),                                       # short sa
        lambda: kernels.block_gemm(qa, sa, w, sw[:100]),                                      # short sw
        lambda: kernels.block_gemm(qa, sa, w, sw, torch.zeros(100, device=dev)),              # short bias
        lambda: kernels.block_gemm(qa, sa, w, sw, kind="fp8"),                                # int8 codes as fp8
        lambda: kernels.block_gemm_acc32(qa, w[:, :128].contiguous()),
        lambda: kernels.adaln_quant(x.view(1, 64, 256), torch.zeros(1, 128, device=dev), torch.zeros(1, 256, device=dev)),
        lambda: fused.adaln(x.view(1, 64, 256), torch.zeros(1, 256, device=dev), torch.zeros(1, 200, device=dev)),
        lambda: fused.gated_residual(x.view(1, 64, 256), x.view(1, 64, 256)[:, :32], torch.zeros(1, 256, device=dev)),
        lambda: fused.qk_norm_rope(x.view(1, 64, 2, 128), torch.ones(64, device=dev)),
    ]
    for i, fn in enumerate(bad):
        with pytest.raises(RuntimeError):
            fn()
        print(f"  rejected case {i}", flush=True)


def test_config0_half_even_chain(dev):
    """The single W8A8 linear of the CPU-baseline workload, chained on the GPU: x bf16 [1024, 3072] ~N(0, 1)
    with 1 % of the channels x20, per-token int8 quantization with round-half-even, per-channel int8
    weights [3072, 3072] with fp32 scales ~U(1e-3, 5e-3), bf16 bias, bf16 out.  Codes, scales and the bf16
    outputs equal the oracle's chain bit for bit; the outputs are within 1e-2 of the fp64 product of the
    dequantized operands."""
    from hy_nomas import kernels

    print("config 0 chain: half-even per-token quantization -> int8 GEMM, 1024 x 3072 -> 3072", flush=True)
    m, k, n = 1024, 3072, 3072
    g = seeded(0)
    x = torch.randn(m, k, generator=g)
    x[:, torch.randperm(k, generator=g)[: k // 100]] *= 20
    x = x.to(torch.bfloat16)
    w, sw, bias = int8_weights(n, k, seed=1, per_channel=True)
    qa, sa = kernels.quantize_activations(x.to(dev), "int8", None, rounding="half_even")
    out = kernels.block_gemm(qa, sa, w.to(dev), sw.to(dev), bias.to(dev))
    q_ref, s_ref = oracle.quantize(x, k, "int8", rounding="half_even")
    assert np.array_equal(qa.cpu().numpy(), q_ref) and np.array_equal(sa.cpu().numpy(), s_ref)
    # the half-even codes differ from half-away ones somewhere (ties occur at this size), so the
    # rounding mode really reached the kernel
    q_away, _ = oracle.quantize(x, k, "int8")
    assert (q_away != q_ref).any()
    ref = oracle.block_gemm(q_ref, s_ref, w.numpy(), sw.numpy(), oracle.to_f32(bias))
    assert torch.equal(out.cpu(), torch.from_numpy(ref).to(torch.bfloat16))
    exact = fp64_dequant_product(q_ref, s_ref, w.numpy(), sw.numpy(), bias)
    assert max_abs_rel(out.cpu().float().numpy(), exact) < 1e-2


@pytest.mark.parametrize("m,k,n,layout", [
    (1000, 3072, 1536, "g128"), (300, 1024, 640, "g128"), (77, 256, 384, "g128"),
    (1000, 3072, 1536, "per_token"), (513, 12288, 256, "per_token"), (5, 2048, 768, "per_token")])
def test_block_linear_equals_the_oracle_chain(dev, m, k, n, layout):
    """kernels.block_linear (one hn_block_linear call: activation quantization into a workspace, then the GEMM)
    against the oracle's quantize + block_gemm on the same bf16 input, bit for bit: g128 weights with
    per-token-and-group codes, per-channel weights with per-token codes (hy_nomas/kernels.py:210-222)."""
    from hy_nomas import kernels

    print(f"block_linear vs oracle chain {layout} m={m} k={k} n={n}", flush=True)
    x = outlier_input(m, k, seed=m + k + n)
    w, sw, bias = int8_weights(n, k, seed=n + 5 * k, per_channel=layout == "per_token")
    got = kernels.block_linear(x.view(1, m, k).to(dev), w.to(dev), sw.to(dev), bias.to(dev)).cpu()
    assert got.shape == (1, m, n) and got.dtype == torch.bfloat16
    qa, sa = oracle.quantize(x, 128 if layout == "g128" else k)
    ref = oracle.block_gemm(qa, sa, w.numpy(), sw.numpy(), oracle.to_f32(bias))
    want = torch.from_numpy(ref).to(torch.bfloat16)
    diff = (got[0].view(torch.int16) != want.view(torch.int16)).nonzero()
    assert diff.numel() == 0, f"{len(diff)} outputs differ from the oracle chain, first {diff[:3].tolist()}"


def test_block_linear_config0_half_even_equals_the_oracle_chain(dev):
    """Config 0 (x bf16 [1024, 3072] with 1 % outlier channels x20, per-channel int8 weights [3072, 3072], bf16
    bias) through the one-call linear with round-half-even per-token codes: bit-identical to the oracle's
    half-even quantization + GEMM, and within 1e-2 of the fp64 product of the dequantized operands."""
    from hy_nomas import kernels

    print("block_linear config 0 half-even", flush=True)
    m, k, n = 1024, 3072, 3072
    g = seeded(0)
    x = torch.randn(m, k, generator=g)
    x[:, torch.randperm(k, generator=g)[: k // 100]] *= 20
    x = x.to(torch.bfloat16)
    w, sw, bias = int8_weights(n, k, seed=1, per_channel=True)
    got = kernels.block_linear(x.to(dev), w.to(dev), sw.to(dev), bias.to(dev), rounding="half_even").cpu()
    q_ref, s_ref = oracle.quantize(x, k, "int8", rounding="half_even")
    ref = oracle.block_gemm(q_ref, s_ref, w.numpy(), sw.numpy(), oracle.to_f32(bias))
    assert torch.equal(got, torch.from_numpy(ref).to(torch.bfloat16))
    away = kernels.block_linear(x.to(dev), w.to(dev), sw.to(dev), bias.to(dev)).cpu()
    assert not torch.equal(away, got)  # ties occur at this size: the rounding mode reached the quantizer
    assert max_abs_rel(got.float().numpy(), fp64_dequant_product(q_ref, s_ref, w.numpy(), sw.numpy(), bias)) < 1e-2


@pytest.mark.parametrize("m,k,n", [(1000, 3072, 1536), (300, 1024, 640), (64, 12288, 384)])
def test_fp8_block_linear_equals_the_oracle_chain(dev, m, k, n):
    """pixelumm.fp8_block_linear (one hn_block_linear call, e4m3 codes per token and 128 channels, block weight
    scales read as stored) against the oracle's fp8 quantize + block_gemm on the scales repeated per channel:
    the codes and scales are the oracle's, so only the fp32 accumulation order differs (< 4e-3); and the same
    call on scales without a recorded verdict (the per-channel fold) agrees likewise."""
    from hy_nomas import kernels, pixelumm

    print(f"fp8 block_linear vs oracle chain m={m} k={k} n={n}", flush=True)
    g = seeded(m * 3 + k + n)
    x = outlier_input(m, k, seed=m + 17)
    qw, sblk = pixelumm.quantize_fp8_block(torch.randn(n, k, generator=g) * 0.02)
    bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    sblk_dev = sblk.to(dev)
    assert kernels.validate_scales(sblk_dev)
    # the bf16 values as fp32: the same codes and scales (exact division), and fp32 outputs, so the comparison
    # is not blurred by a bf16 rounding of the result
    xf = x.float().to(dev)
    got = pixelumm.fp8_block_linear(xf, qw.to(dev), sblk_dev, bias.to(dev)).cpu().numpy()
    assert got.dtype == np.float32
    qa, sa = oracle.quantize(x, 128, "fp8")
    sw_full = sblk.repeat_interleave(128, 0)[:n].contiguous().numpy()
    ref = oracle.block_gemm(qa, sa, qw.view(torch.uint8).numpy(), sw_full, oracle.to_f32(bias), kind="fp8")
    assert max_abs_rel(got, ref) < 4e-3
    exact = fp64_dequant_product(qa, sa, qw.view(torch.uint8).numpy(), sw_full, bias, kind="fp8")
    assert max_abs_rel(got, exact) < 1e-2
    unverified = pixelumm.fp8_block_linear(xf, qw.to(dev), sblk.to(dev), bias.to(dev)).cpu().numpy()
    assert max_abs_rel(unverified, ref) < 4e-3
    # and the bf16 input's own call: its output rounded once to bf16
    got16 = pixelumm.fp8_block_linear(x.to(dev), qw.to(dev), sblk_dev, bias.to(dev)).cpu()
    assert torch.equal(got16, torch.from_numpy(got).to(torch.bfloat16))


def test_fp8_block_dispatch_does_not_synchronize(dev):
    """With fp8 128 x 128 block weight scales, choosing the GEMM's scale layout never waits for the device:
    scales without a recorded verdict (a fresh device copy, an activation-scale copy) go to the per-channel
    fold, which is bit-identical to passing the scales repeated per channel; scales that passed
    `validate_scales` once are read as stored."""
    from hy_nomas import kernels, pixelumm

    print("fp8 block dispatch without synchronization", flush=True)
    g = seeded(515)
    m, k, n = 700, 1024, 640
    x = outlier_input(m, k, seed=516).to(dev)
    qa, sa = kernels.quantize_activations(x, "fp8")
    qw, sblk = pixelumm.quantize_fp8_block(torch.randn(n, k, generator=g) * 0.02)
    qw, sblk_dev, bias = qw.to(dev), sblk.to(dev), (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    sa_copy = sa.clone()
    sw_known = sblk_dev.clone()
    kernels.trust_scales(sw_known)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        fresh_sw = kernels.block_gemm(qa, sa, qw, sblk_dev, bias, torch.float32, kind="fp8")
        fresh_sa = kernels.block_gemm(qa, sa_copy, qw, sw_known, bias, torch.float32, kind="fp8")
        linear = kernels.block_linear(x, qw, sblk_dev, bias, kind="fp8")
    finally:
        torch.cuda.set_sync_debug_mode(0)
    expanded = sblk_dev.repeat_interleave(128, 0)[:n].contiguous()
    want = kernels.block_gemm(qa, sa, qw, expanded, bias, torch.float32, kind="fp8")
    assert torch.equal(fresh_sw, want) and torch.equal(fresh_sa, want)
    assert torch.equal(linear, kernels.block_linear(x, qw, expanded, bias, kind="fp8"))
    assert kernels.validate_scales(sblk_dev)
    stored = kernels.block_gemm(qa, sa, qw, sblk_dev, bias, torch.float32, kind="fp8")
    assert not torch.equal(stored, want)  # the rescaled running sum rounds differently...
    assert max_abs_rel(stored.cpu().numpy(), want.cpu().numpy()) < 4e-3  # ...within the fp8 tolerance


@pytest.mark.parametrize("layout", ["per_token", "g128", "fp8_block"])
def test_big_tiles_with_a_small_tile_tail(dev, layout):
    """A problem whose last round of 256 x 256 tiles would leave most compute units idle: M = 26400, N = 2048
    makes 832 such tiles (3 rounds and a quarter on 256 compute units), so the first 24576 rows run on big tiles
    and the rest on 128 x 128 tiles in a second launch.  Rows on both sides of the split, one in every 256-row
    tile, equal the oracle bit for bit (int8) or within the fp8 tolerance; the GELU epilogue takes the same
    split."""
    from hy_nomas import kernels, pixelumm

    m, k, n = 26400, 512, 2048
    print(f"tile split {layout} m={m} k={k} n={n}", flush=True)
    g = seeded(2640)
    x = outlier_input(m, k, seed=2641)
    split = 24576
    rows = sorted(set(list(range(0, m, 256)) + [255, 256, split - 257, split - 256, split - 1, split, split + 1,
                                                split + 127, split + 128, m - 129, m - 128, m - 2, m - 1]))
    if layout == "fp8_block":
        qw, sblk = pixelumm.quantize_fp8_block(torch.randn(n, k, generator=g) * 0.02)
        bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
        qa, sa = kernels.quantize_activations(x.to(dev), "fp8")
        sblk_dev = sblk.to(dev)
        assert kernels.validate_scales(sblk_dev)
        out = kernels.block_gemm(qa, sa, qw.to(dev), sblk_dev, bias.to(dev), torch.float32, kind="fp8")
        sw_full = sblk.repeat_interleave(128, 0).contiguous().numpy()
        ref = oracle.block_gemm(qa[rows].view(torch.uint8).cpu().numpy(), sa[rows].cpu().numpy(),
                                qw.view(torch.uint8).numpy(), sw_full, oracle.to_f32(bias), kind="fp8")
        assert max_abs_rel(out[rows].cpu().numpy(), ref) < 4e-3
        return
    w, sw, bias = int8_weights(n, k, seed=2642, per_channel=layout == "per_token")
    qa, sa = kernels.quantize_activations(x.to(dev), "int8", None if layout == "per_token" else 128)
    args = (qa, sa, w.to(dev), sw.to(dev), bias.to(dev))
    out = kernels.block_gemm(*args, torch.float32)
    ref = oracle.block_gemm(qa[rows].cpu().numpy(), sa[rows].cpu().numpy(), w.numpy(), sw.numpy(), oracle.to_f32(bias))
    got = out[rows].cpu().numpy()
    assert np.array_equal(got, ref), f"{int((got != ref).sum())} outputs differ in the sampled rows"
    out16 = kernels.block_gemm(*args)
    assert torch.equal(out16[rows].cpu(), torch.from_numpy(ref).to(torch.bfloat16))
    gelu = kernels.block_gemm(*args, epilogue="gelu")[rows].cpu()
    ref_gelu = torch.from_numpy(oracle.block_gemm(qa[rows].cpu().numpy(), sa[rows].cpu().numpy(), w.numpy(),
                                                  sw.numpy(), oracle.to_f32(bias), epilogue="gelu")).to(torch.bfloat16)
    assert (gelu != ref_gelu).float().mean().item() < 1e-3
