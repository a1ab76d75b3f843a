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

    print(f"double-stream block per_token={per_token}", flush=True)
    d, heads, mlp, lv, lt = 256, 2, 1024, 200, 40
    g = seeded(91 + per_token)
    img_blk = make_stream(d, heads, mlp, g, per_token, dev)
    txt_blk = make_stream(d, heads, mlp, g, per_token, dev)
    img = torch.randn(1, lv, d, generator=g).to(torch.bfloat16)
    txt = torch.randn(1, lt, d, generator=g).to(torch.bfloat16)
    img_mods = [(torch.randn(1, d, generator=g) * 0.1).to(torch.bfloat16) for _ in range(6)]
    txt_mods = [(torch.randn(1, d, generator=g) * 0.1).to(torch.bfloat16) for _ in range(6)]
    rope = block.rope_freqs([32, 48, 48], 256, 2, 10, 10)
    blk = block.DoubleStreamBlockInt8(img_blk, txt_blk)
    with torch.no_grad():
        gi, gt = blk.forward(img.to(dev), txt.to(dev), [m.to(dev) for m in img_mods], [m.to(dev) for m in txt_mods],
                             (rope[0].to(dev), rope[1].to(dev)))
        ri, rt = block.reference_double_stream(img_blk, txt_blk, img.to(dev), txt.to(dev),
                                               [m.to(dev) for m in img_mods], [m.to(dev) for m in txt_mods],
                                               (rope[0].to(dev), rope[1].to(dev)))
    for got, ref in ((gi, ri), (gt, rt)):
        assert got.dtype == torch.bfloat16 and got.shape == ref.shape
        err = ((got.float() - ref).norm() / ref.norm()).item()
        assert err < 2e-2, err
        # and the block really changed the stream (a wiring mistake that drops a branch fails here)
        assert ((got.float() - (img if got is gi else txt).to(dev).float()).norm() / ref.norm()).item() > 1e-2
