"""The double-stream DiT block on the int8 path (hy_nomas/model.py:230-286) against the same block in float32
torch arithmetic with dequantized weights and unquantized activations (the reference's exact-matmul path).
The int8 path quantizes every activation, so the bar is a relative error, for both activation layouts."""
import pytest
import torch

from conftest import seeded

pytestmark = pytest.mark.gpu


def make_linear(n, k, g, per_channel, dev):
    from hy_nomas import block

    qw = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    cols = 1 if per_channel else k // 128
    sw = (torch.rand(n, cols, generator=g) * 2e-3 + 5e-4).float()
    bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    return block.Int8Linear(qw.to(dev), sw.to(dev), bias.to(dev))


def make_stream(d, heads, mlp, g, per_token, dev):
    from hy_nomas import block

    lins = [make_linear(n, k, g, per_token, dev) for n, k in ((3 * d, d), (d, d), (mlp, d), (d, mlp))]
    hd = d // heads
    qn = (torch.rand(hd, generator=g) + 0.5).to(torch.bfloat16).to(dev)
    kn = (torch.rand(hd, generator=g) + 0.5).to(torch.bfloat16).to(dev)
    return block.DiTBlockInt8(*lins, qn, kn, heads, per_token=per_token)


@pytest.mark.parametrize("per_token", [False, True])
def test_double_stream_block(dev, per_token):
    from hy_nomas import block
    from oracle import torch_forms

    print(f"double-stream block per_token={per_token}", flush=True)
    d, heads, mlp, lv, lt = 256, 2, 1024, 200, 40
    g = seeded(91 + per_token)
    img_blk = make_stream(d, heads, mlp, g, per_token, dev)
    txt_blk = make_stream(d, heads, mlp, g, per_token, dev)
    img = torch.randn(1, lv, d, generator=g).to(torch.bfloat16)
    txt = torch.randn(1, lt, d, generator=g).to(torch.bfloat16)
    img_mods = [(torch.randn(1, d, generator=g) * 0.1).to(torch.bfloat16) for _ in range(6)]
    txt_mods = [(torch.randn(1, d, generator=g) * 0.1).to(torch.bfloat16) for _ in range(6)]
    rope = torch_forms.rope_freqs([32, 48, 48], 256, 2, 10, 10)
    blk = block.DoubleStreamBlockInt8(img_blk, txt_blk)
    with torch.no_grad():
        gi, gt = blk.forward(img.to(dev), txt.to(dev), [m.to(dev) for m in img_mods], [m.to(dev) for m in txt_mods],
                             (rope[0].to(dev), rope[1].to(dev)))
        ri, rt = torch_forms.reference_double_stream(img_blk, txt_blk, img.to(dev), txt.to(dev),
                                               [m.to(dev) for m in img_mods], [m.to(dev) for m in txt_mods],
                                               (rope[0].to(dev), rope[1].to(dev)))
    for got, ref in ((gi, ri), (gt, rt)):
        assert got.dtype == torch.bfloat16 and got.shape == ref.shape
        err = ((got.float() - ref).norm() / ref.norm()).item()
        assert err < 2e-2, err
        # and the block really changed the stream (a wiring mistake that drops a branch fails here)
        assert ((got.float() - (img if got is gi else txt).to(dev).float()).norm() / ref.norm()).item() > 1e-2


def make_linear_on(dev, gen, n, k, per_channel):
    """Random int8 codes, fp32 scales ([N, 1] per channel or [N, K/128]) and bf16 bias, drawn on `dev`."""
    from hy_nomas import block

    qw = torch.randint(-127, 128, (n, k), generator=gen, device=dev, dtype=torch.int8)
    sw = torch.rand(n, 1 if per_channel else k // 128, generator=gen, device=dev) * 2e-3 + 5e-4
    bias = (torch.randn(n, generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    return block.Int8Linear(qw, sw.float(), bias)


@pytest.mark.parametrize("per_token,backend", [(True, "sdpa"), (False, "sdpa"), (True, "hip"), (False, "hip")])
def test_double_stream_block_full_size(dev, per_token, backend):
    """The config-4 block at its real size: hidden 3072, 24 heads x 128, FFN 12288, 57344 image tokens on a
    14 x 64 x 64 RoPE grid plus 256 text tokens, both activation layouts, both attention backends (the HIP one
    with v written straight into its V^T layout by the QKV epilogues).  The float32 reference (dequantized
    weights, unquantized activations, hy_nomas/model.py:230-303) computes q/k/v for every token and the
    attention and row-local rest of the block for sampled rows of each stream; the int8 block's rows must
    match within 2e-2 relative (as the small-block test), and so must the block's change to the stream."""
    from hy_nomas import block
    from oracle import torch_forms

    d, heads, mlp, lv, lt = 3072, 24, 12288, 57344, 256
    print(f"double-stream block full size per_token={per_token} backend={backend} ({lv}+{lt} tokens)", flush=True)
    gen = torch.Generator(device=dev).manual_seed(2024 + per_token)

    def stream():
        lins = [make_linear_on(dev, gen, n, k, per_token) for n, k in ((3 * d, d), (d, d), (mlp, d), (d, mlp))]
        qn = (torch.rand(d // heads, generator=gen, device=dev) + 0.5).to(torch.bfloat16)
        kn = (torch.rand(d // heads, generator=gen, device=dev) + 0.5).to(torch.bfloat16)
        return block.DiTBlockInt8(*lins, qn, kn, heads, per_token=per_token)

    img_blk, txt_blk = stream(), stream()
    img = torch.randn(1, lv, d, generator=gen, device=dev).to(torch.bfloat16)
    txt = torch.randn(1, lt, d, generator=gen, device=dev).to(torch.bfloat16)
    img_mods = [(torch.randn(1, d, generator=gen, device=dev) * 0.1).to(torch.bfloat16) for _ in range(6)]
    txt_mods = [(torch.randn(1, d, generator=gen, device=dev) * 0.1).to(torch.bfloat16) for _ in range(6)]
    rope = torch_forms.rope_freqs([16, 56, 56], 256, 14, 64, 64, device=dev)
    blk = block.DoubleStreamBlockInt8(img_blk, txt_blk)
    with torch.no_grad():
        gi, gt = blk.forward(img, txt, img_mods, txt_mods, rope, backend)
        torch.cuda.synchronize()
        g = seeded(55 + per_token)
        img_rows = sorted(set(torch.randperm(lv, generator=g)[:30].tolist() + [0, lv - 1]))
        txt_rows = sorted(set(torch.randperm(lt, generator=g)[:30].tolist() + [0, lt - 1]))
        ri, rt = torch_forms.double_stream_rows(img_blk, txt_blk, img, txt, img_mods, txt_mods, rope, img_rows,
                                                txt_rows)
    assert gi.shape == (1, lv, d) and gt.shape == (1, lt, d) and gi.dtype == torch.bfloat16
    for name, got, x, rows, ref in (("img", gi, img, img_rows, ri), ("txt", gt, txt, txt_rows, rt)):
        got_r, x_r = got[0, rows].float(), x[0, rows].float()
        err = ((got_r - ref).norm() / ref.norm()).item()
        delta_err = ((got_r - ref).norm() / (ref - x_r).norm()).item()
        print(f"  {name}: relative error {err:.3e}, of the block's change {delta_err:.3e}", flush=True)
        assert torch.isfinite(got_r).all()
        assert err < 2e-2, err
        assert delta_err < 2e-2, delta_err
