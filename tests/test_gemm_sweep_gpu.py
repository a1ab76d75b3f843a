"""A seeded sweep of GEMM shapes against the oracle (hy_nomas/kernels.py:80-170): token counts from one row
(the skinny kernel) through tile edges (127-129, 255-257, 511-513) to several rounds of tiles (the small-tile
tail of `choose_tiles` at many remainders), channel counts that are and are not multiples of 8 (the LDS-staged
and the direct 2-byte stores), K from one group to 32, per-token and g128 int8 and fp8 with 128 x 128 block
scales (with a partial last block of channels), with and without bias, the GELU epilogue, and bf16, fp16 and
fp32 outputs.  Rows are independent, so each case checks the rows around every 256-row tile boundary and 40
random rows against the oracle on those rows: bit for bit for int8 (GELU: the reference test's tolerance),
within 4e-3 of the oracle and 1e-2 of the fp64 product for fp8."""
import random

import numpy as np
import pytest
import torch

import oracle
from conftest import seeded
from test_gemm_gpu import fp64_dequant_product, int8_weights, max_abs_rel
from test_quant_gpu import outlier_input

pytestmark = pytest.mark.gpu

_M = [1, 2, 3, 4, 5, 31, 127, 128, 129, 255, 256, 257, 300, 511, 512, 513, 777, 1024, 1500, 2049, 4100, 9000]
_N = [8, 120, 128, 200, 256, 384, 1000, 1001, 1024, 1032, 2048, 3072, 4104]
_K = [128, 256, 384, 640, 1024, 2048, 3072, 4096]


def _cases(count=40, seed=2026):
    rnd = random.Random(seed)
    layouts = ["per_token", "g128", "fp8_block"]
    out = []
    for i in range(count):
        layout = layouts[i % 3]
        m, n, k = rnd.choice(_M), rnd.choice(_N), rnd.choice(_K)
        out_dt = rnd.choice(["bf16", "f16", "f32"])
        bias = rnd.random() < 0.75
        gelu = layout != "fp8_block" and rnd.random() < 0.25
        out.append(pytest.param(layout, m, n, k, out_dt, bias, gelu, i,
                                id=f"{i}-{layout}-m{m}-n{n}-k{k}-{out_dt}{'-bias' if bias else ''}{'-gelu' if gelu else ''}"))
    return out


def _rows(m, rnd):
    edges = [r for base in range(0, m + 256, 256) for r in (base - 1, base, base + 1, base + 127, base + 128)]
    picks = rnd.sample(range(m), min(m, 40))
    return sorted({r for r in edges + picks + [0, m - 1] if 0 <= r < m})


@pytest.mark.parametrize("layout,m,n,k,out_dt,with_bias,gelu,case", _cases())
def test_gemm_shape_sweep(dev, layout, m, n, k, out_dt, with_bias, gelu, case):
    from hy_nomas import kernels, pixelumm

    print(f"sweep case {case}: {layout} M={m} N={n} K={k} out={out_dt} bias={with_bias} gelu={gelu}", flush=True)
    rnd = random.Random(case)
    g = seeded(1000 + case)
    out_dtype = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[out_dt]
    x = outlier_input(m, k, seed=2000 + case)
    rows = _rows(m, rnd)
    if layout == "fp8_block":
        qa, sa = kernels.quantize_activations(x.to(dev), "fp8")
        # a weight of whole 128-row blocks (the layout's quantizer needs them), cut to n rows: the last block
        # row of scales then covers a partial block of channels
        npad = -(-n // 128) * 128
        qw, sblk = pixelumm.quantize_fp8_block(torch.randn(npad, k, generator=g) * 0.02)
        qw = qw[:n].contiguous()
        bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16) if with_bias else None
        sblk_dev = sblk.to(dev)
        assert kernels.validate_scales(sblk_dev)  # block scales read as stored
        got = kernels.block_gemm(qa, sa, qw.to(dev), sblk_dev, None if bias is None else bias.to(dev), out_dtype,
                                 kind="fp8")[rows].cpu().float().numpy().astype(np.float64)
        qa_r, sa_r = qa[rows].view(torch.uint8).cpu().numpy(), sa[rows].cpu().numpy()
        sw_full = sblk.repeat_interleave(128, 0)[:n].contiguous().numpy()
        b32 = None if bias is None else oracle.to_f32(bias)
        ref = oracle.block_gemm(qa_r, sa_r, qw.view(torch.uint8).numpy(), sw_full, b32, kind="fp8")
        exact = fp64_dequant_product(qa_r, sa_r, qw.view(torch.uint8).numpy(), sw_full, bias, kind="fp8")
        assert max_abs_rel(got, exact) < 1e-2
        assert max_abs_rel(got, ref.astype(np.float64)) < 4e-3
        return
    per_channel = layout == "per_token"
    w, sw, bias = int8_weights(n, k, seed=3000 + case, per_channel=per_channel)
    bias = bias if with_bias else None
    qa, sa = kernels.quantize_activations(x.to(dev), "int8", None if per_channel else 128)
    args = (qa, sa, w.to(dev), sw.to(dev), None if bias is None else bias.to(dev))
    got = kernels.block_gemm(*args, out_dtype, epilogue="gelu" if gelu else None)[rows].cpu()
    b32 = None if bias is None else oracle.to_f32(bias)
    ref = oracle.block_gemm(qa[rows].cpu().numpy(), sa[rows].cpu().numpy(), w.numpy(), sw.numpy(), b32,
                            epilogue="gelu" if gelu else None)
    ref = torch.from_numpy(ref).to(out_dtype)
    if not gelu:
        bits = (lambda t: t.view(torch.int32)) if out_dtype == torch.float32 else (lambda t: t.view(torch.int16))
        diff = (bits(got) != bits(ref)).nonzero()
        assert diff.numel() == 0, f"{len(diff)} outputs differ, first (row index, channel) {diff[:3].tolist()}"
    else:
        # the epilogue's sigmoid comes from the hardware exp2 / reciprocal (hy_nomas tests/test_fused.py:63-78)
        assert (got != ref).float().mean().item() < 1e-3
        assert (got.float() - ref.float()).abs().max().item() <= 2 ** -6 * ref.float().abs().max().item()
