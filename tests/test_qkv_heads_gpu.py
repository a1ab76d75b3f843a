"""QKV projection with QK-norm + RoPE in the GEMM epilogue, written head-major (model.py:253-267 with
fused.py:65-105), against the unfused sequence: block_gemm to [B * L, 3 * hidden] bf16, then
fused.qk_norm_rope on the q and k views.  v is the same GEMM output, so it must match bit for bit; q and k
sum their squares in another order (the reference's tolerance for the norm applies)."""
import pytest
import torch

import oracle
from conftest import seeded

pytestmark = pytest.mark.gpu


def make_qkv(g, hidden, k, layout, dev):
    n = 3 * hidden
    qw = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    cols = 1 if layout == "per_token" else k // 128
    sw = torch.rand(n, cols, generator=g) * 2e-3 + 5e-4
    bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    return qw.to(dev), sw.to(dev), bias.to(dev)


def rope_tables(g, length):
    ang = torch.rand(length, 64, generator=g) * 6.283
    cos = torch.cos(ang).repeat_interleave(2, dim=1)
    sin = torch.sin(ang).repeat_interleave(2, dim=1)
    return cos.float(), sin.float()


@pytest.mark.parametrize("layout", ["g128", "per_token"])
@pytest.mark.parametrize("b,l,hidden,k,with_rope", [(1, 300, 512, 512, True), (2, 129, 384, 256, False),
                                                    (1, 1024, 3072, 3072, True)])
def test_qkv_heads_matches_gemm_then_qk_norm_rope(dev, layout, b, l, hidden, k, with_rope):
    from hy_nomas import fused, kernels

    print(f"qkv_heads {layout} b={b} l={l} hidden={hidden} k={k} rope={with_rope}", flush=True)
    g = seeded(b * 1000 + l + hidden + k)
    x = (torch.randn(b * l, k, generator=g) * 2).to(torch.bfloat16).to(dev)
    qa, sa = kernels.quantize_activations(x, "int8", None if layout == "per_token" else 128)
    qw, sw, bias = make_qkv(g, hidden, k, layout, dev)
    wq = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16).to(dev)
    wk = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16).to(dev)
    rope = tuple(t.to(dev) for t in rope_tables(g, l)) if with_rope else None
    hm = kernels.qkv_heads(qa, sa, qw, sw, bias, wq, wk, b, rope)
    h = hidden // 128
    assert hm.shape == (3, b, h, l, 128)
    flat = kernels.block_gemm(qa, sa, qw, sw, bias).view(b, l, 3, h, 128)
    v_ref = flat[:, :, 2].transpose(1, 2)
    assert torch.equal(hm[2], v_ref)
    for part, w in ((0, wq), (1, wk)):
        ref = fused.qk_norm_rope(flat[:, :, part], w, rope).transpose(1, 2)
        got = hm[part]
        assert (got != ref).float().mean().item() < 1e-2
        assert ((got.float() - ref.float()).norm() / ref.float().norm()).item() < 1e-3
        rope_cpu = tuple(t.cpu() for t in rope) if rope is not None else None
        ora = torch.from_numpy(oracle.qk_norm_rope(flat[:, :, part].contiguous().cpu(), w.cpu(), rope_cpu))
        ora = ora.to(torch.bfloat16).transpose(1, 2)
        assert (got.cpu() != ora).float().mean().item() < 1e-2


def test_qkv_heads_two_streams_share_one_buffer(dev):
    """Image and text projections written into one head-major buffer at their token offsets (the joint
    attention's torch.cat order), fp8 block scales for the text stream."""
    from hy_nomas import kernels, pixelumm

    print("qkv_heads two streams", flush=True)
    g = seeded(21)
    hidden, k, li, lt = 256, 256, 200, 37
    xi = torch.randn(li, k, generator=g).to(torch.bfloat16).to(dev)
    xt = torch.randn(lt, k, generator=g).to(torch.bfloat16).to(dev)
    qi, si = kernels.quantize_activations(xi)
    wi, swi, bi = make_qkv(g, hidden, k, "g128", dev)
    qt, st = kernels.quantize_activations(xt, "fp8")
    wt, sblk = pixelumm.quantize_fp8_block(torch.randn(3 * hidden, k, generator=g) * 0.02)
    wt, sblk = wt.to(dev), sblk.to(dev)
    assert kernels.validate_scales(sblk)  # read as stored by the GEMM
    wq = torch.ones(128, device=dev)
    wk = (torch.rand(128, generator=g) + 0.5).to(dev)
    rope = tuple(t.to(dev) for t in rope_tables(g, li))
    hm = torch.full((3, 1, 2, li + lt, 128), float("nan"), device=dev, dtype=torch.bfloat16)
    kernels.qkv_heads(qi, si, wi, swi, bi, wq, wk, 1, rope, out=hm, l_offset=0)
    kernels.qkv_heads(qt, st, wt, sblk, None, wq, wk, 1, None, kind="fp8", out=hm, l_offset=li)
    assert not torch.isnan(hm.float()).any()
    alone_i = kernels.qkv_heads(qi, si, wi, swi, bi, wq, wk, 1, rope)
    alone_t = kernels.qkv_heads(qt, st, wt, sblk, None, wq, wk, 1, None, kind="fp8")
    assert torch.equal(hm[:, :, :, :li], alone_i)
    assert torch.equal(hm[:, :, :, li:], alone_t)
    v_t = kernels.block_gemm(qt, st, wt, sblk, kind="fp8").view(lt, 3, 2, 128)[:, 2].transpose(0, 1)
    assert torch.equal(alone_t[2, 0], v_t)
    with pytest.raises(RuntimeError):
        kernels.qkv_heads(qt, st, wt, sblk, None, wq, wk, 1, None, kind="fp8", out=hm, l_offset=li + 1)


@pytest.mark.parametrize("layout", ["g128", "per_token"])
def test_qkv_heads_vt_matches_head_major(dev, layout):
    """v written straight into the HIP attention's V^T layout (hn_qkv_heads_vt): equal bit for bit to the V^T
    copy of the head-major v (attention.transpose_values), q and k to the head-major call's; two streams at
    their key offsets (an image stream of 2 x 320 tokens, then 32 text tokens with fp8 block scales), hidden
    384 (a tile holding a k head and a v head), the padding keys up to 384 left as they were."""
    from hy_nomas import attention, kernels, pixelumm

    print(f"qkv_heads V^T {layout}", flush=True)
    g = seeded(31)
    hidden, k, b, li, lt = 384, 256, 2, 320, 32
    ltot = li + lt
    xi = torch.randn(b * li, k, generator=g).to(torch.bfloat16).to(dev)
    xt = torch.randn(b * lt, k, generator=g).to(torch.bfloat16).to(dev)
    qi, si = kernels.quantize_activations(xi, "int8", None if layout == "per_token" else 128)
    wi, swi, bi = make_qkv(g, hidden, k, layout, dev)
    qt, st = kernels.quantize_activations(xt, "fp8")
    wt, sblk = pixelumm.quantize_fp8_block(torch.randn(3 * hidden, k, generator=g) * 0.02)
    wt, sblk = wt.to(dev), sblk.to(dev)
    assert kernels.validate_scales(sblk)  # read as stored by the GEMM
    wq = (torch.rand(128, generator=g) + 0.5).to(dev)
    wk = (torch.rand(128, generator=g) + 0.5).to(dev)
    rope = tuple(t.to(dev) for t in rope_tables(g, li))
    hm = torch.empty((3, b, hidden // 128, ltot, 128), device=dev, dtype=torch.bfloat16)
    kernels.qkv_heads(qi, si, wi, swi, bi, wq, wk, b, rope, out=hm, l_offset=0)
    kernels.qkv_heads(qt, st, wt, sblk, None, wq, wk, b, None, kind="fp8", out=hm, l_offset=li)
    vt_ref = attention.transpose_values(hm[2])
    qk = torch.full((2, b, hidden // 128, ltot, 128), float("nan"), device=dev, dtype=torch.bfloat16)
    vt = torch.full(tuple(vt_ref.shape), float("nan"), device=dev, dtype=torch.bfloat16)
    kernels.qkv_heads(qi, si, wi, swi, bi, wq, wk, b, rope, out=qk, l_offset=0, vt=vt)
    assert torch.isnan(vt[..., li:].float()).all()          # the text keys are not this call's
    kernels.qkv_heads(qt, st, wt, sblk, None, wq, wk, b, None, kind="fp8", out=qk, l_offset=li, vt=vt)
    assert torch.equal(qk, hm[:2])
    assert torch.equal(vt[..., :ltot], vt_ref[..., :ltot])
    assert vt.shape[3] == 384 and torch.isnan(vt[..., ltot:].float()).all()   # padding keys untouched
    pad = attention.values_buffer(b, hidden // 128, ltot, dev)
    assert pad.shape == vt_ref.shape and not pad[..., ltot:].any()
    with pytest.raises(RuntimeError):                       # 36 tokens: not whole 32-token blocks
        kernels.qkv_heads(qt[:36], st[:36], wt, sblk, None, wq, wk, 1, None, kind="fp8", l_offset=li, vt=vt)
