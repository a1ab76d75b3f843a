"""The DiT-block GEMM stack at its full size (M = 32768 tokens, hidden 3072, FFN 12288), checked through
properties that do not need a full-size CPU product:
* rows are independent, so sampled rows of the full product must equal the oracle on those rows bit for bit
  (int8) or within the fp8 tolerance.  One random row of every 256-token tile is sampled (every output tile
  the persistent walk visits holds sampled rows), plus the rows at the tile edges 255 / 256 and the last row,
  for the fp32 epilogue and the LDS-staged bf16 epilogue;
* the int32 accumulators satisfy the exact checksum identity colsum(A B^T) = colsum(A) B^T in int64."""
import numpy as np
import pytest
import torch

import oracle
from conftest import seeded

pytestmark = pytest.mark.gpu

M = 32768
STACK = [("qkv", 3072, 9216), ("attn_out", 3072, 3072), ("ffn_up", 3072, 12288), ("ffn_down", 12288, 3072)]


TILE_M = 256  # token rows of a GEMM tile


def sample_rows(g, m, count=40):
    rows = torch.randperm(m, generator=g)[:count].tolist()
    return sorted(set(rows + [0, 1, m - 1]))


def tile_rows(g, m):
    """One random row of every TILE_M-row tile, plus rows 0, 1, TILE_M - 1, TILE_M and m - 1."""
    starts = torch.arange(0, m, TILE_M)
    span = torch.clamp(m - starts, max=TILE_M)
    picks = starts + (torch.rand(len(starts), generator=g) * span).long()
    return sorted(set(picks.tolist() + [0, 1, TILE_M - 1, TILE_M, m - 1]))


@pytest.mark.parametrize("layout", ["per_token", "g128"])
@pytest.mark.parametrize("name,k,n", STACK)
def test_full_size_int8_rows_equal_the_oracle(dev, layout, name, k, n):
    from hy_nomas import kernels

    print(f"full size int8 {layout} {name} M={M} K={k} N={n}", flush=True)
    g = seeded(k + n + (layout == "g128"))
    x = torch.randn(M, k, generator=g)
    ch = torch.randperm(k, generator=g)[: k // 100]
    x[:, ch] *= 20
    group = None if layout == "per_token" else 128
    qa, sa = kernels.quantize_activations(x.to(torch.bfloat16).to(dev), "int8", group)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    sw = torch.rand(n, 1 if group is None else k // 128, generator=g) * 4e-3 + 1e-3
    bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    args = (qa, sa, w.to(dev), sw.to(dev), bias.to(dev))
    out = kernels.block_gemm(*args, torch.float32)
    rows = tile_rows(g, M)
    assert len(rows) >= M // TILE_M
    ref = oracle.block_gemm(qa[rows].cpu().numpy(), sa[rows].cpu().numpy(), w.numpy(), sw.numpy(),
                            oracle.to_f32(bias))
    got = out[rows].cpu().numpy()
    assert np.array_equal(got, ref), f"{int((got != ref).sum())} outputs differ in the sampled rows"
    del out
    # the bf16 output (the staged 16-byte store path) on the same rows
    out16 = kernels.block_gemm(*args, torch.bfloat16)
    got16 = out16[rows].cpu().view(torch.int16)
    want16 = torch.from_numpy(ref).to(torch.bfloat16).view(torch.int16)
    diff = (got16 != want16).nonzero()
    assert diff.numel() == 0, f"{len(diff)} bf16 outputs differ in the sampled rows, first {diff[:3].tolist()}"


def test_full_size_acc32_checksums(dev):
    """FFN-down (K = 12288, the largest accumulators): exact int64 column and row checksums of the
    full 32768 x 3072 int32 product."""
    from hy_nomas import kernels

    print("full size acc32 checksums", flush=True)
    g = seeded(5)
    k, n = 12288, 3072
    qa = torch.randint(-127, 128, (M, k), generator=g, dtype=torch.int8)
    qw = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    acc = kernels.block_gemm_acc32(qa.to(dev), qw.to(dev))
    col = acc.to(torch.int64).sum(dim=0).cpu()
    row = acc.to(torch.int64).sum(dim=1).cpu()
    a64, w64 = qa.to(torch.int64), qw.to(torch.int64)
    assert torch.equal(col, a64.sum(dim=0) @ w64.t())
    assert torch.equal(row, a64 @ w64.sum(dim=0))
    rows = sample_rows(g, M, 8)
    assert torch.equal(acc[rows].cpu().to(torch.int64), a64[rows] @ w64.t())


@pytest.mark.parametrize("name,k,n", STACK)
def test_full_size_fp8_block_rows(dev, name, k, n):
    """fp8 with 128 x 128 block weight scales at full size: sampled rows within 1e-2 max-abs-rel of the
    fp64 product of the dequantized operands, and within 4e-3 of the oracle."""
    from hy_nomas import kernels, pixelumm

    print(f"full size fp8 {name} M={M} K={k} N={n}", flush=True)
    g = seeded(k * 3 + n)
    x = torch.randn(M, k, generator=g).to(torch.bfloat16)
    qa, sa = kernels.quantize_activations(x.to(dev), "fp8")
    qw, sblk = pixelumm.quantize_fp8_block(torch.randn(n, k, generator=g) * 0.02)
    sblk_dev = sblk.to(dev)
    assert kernels.validate_scales(sblk_dev)  # the block scales are read as stored
    out = kernels.block_gemm(qa, sa, qw.to(dev), sblk_dev, None, torch.float32, kind="fp8")
    rows = tile_rows(g, M)
    table = oracle.e4m3_decode_table().astype(np.float64)
    a = table[qa[rows].view(torch.uint8).cpu().numpy()] * np.repeat(sa[rows].cpu().numpy().astype(np.float64), 128, 1)
    wd = pixelumm.dequantize_fp8_block(qw, sblk, torch.float32).double().numpy()
    exact = a @ wd.T
    got = out[rows].cpu().numpy().astype(np.float64)
    assert np.abs(got - exact).max() / np.abs(exact).max() < 1e-2
    sw_full = sblk.repeat_interleave(128, 0)[:n].contiguous().numpy()
    ref = oracle.block_gemm(qa[rows].view(torch.uint8).cpu().numpy(), sa[rows].cpu().numpy(),
                            qw.view(torch.uint8).numpy(), sw_full, None, kind="fp8")
    assert np.abs(got - ref).max() / np.abs(ref).max() < 4e-3
