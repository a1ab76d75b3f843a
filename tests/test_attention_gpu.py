"""The HIP attention kernel (hn_attention) against float32 softmax attention and against torch SDPA
(hy_nomas/model.py:145-223): ragged lengths, strided head-major operands as the QKV epilogue writes them,
large score magnitudes, the full config-4 length, segment attention with history keys and query groups,
and the double-stream block on the HIP backend.  bf16 operands and probabilities: the bar is relative."""
import pytest
import torch

from conftest import seeded

pytestmark = pytest.mark.gpu


def ref_attention(q, k, v):
    """float32 softmax(q k^T / sqrt(d)) v; q [B, Lq, H, D], k / v [B, Lk, H, D] -> [B, Lq, H, D] float32."""
    qf, kf, vf = (t.float().transpose(1, 2).contiguous() for t in (q, k, v))
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * q.shape[-1] ** -0.5
    return torch.matmul(torch.softmax(s, dim=-1), vf).transpose(1, 2)


def rel(got, ref):
    got, ref = got.float(), ref.float()
    return ((got - ref).norm() / ref.norm()).item(), ((got - ref).abs().max() / ref.abs().max()).item()


@pytest.mark.parametrize("b,h,lq,lk,mag", [(2, 3, 200, 130, 1.0), (1, 2, 128, 64, 1.0), (1, 1, 1, 1, 1.0),
                                           (1, 2, 77, 65, 4.0), (2, 1, 300, 1000, 2.0), (1, 4, 256, 513, 8.0)])
def test_attention_matches_float32(dev, b, h, lq, lk, mag):
    from hy_nomas import attention

    print(f"attention b={b} h={h} lq={lq} lk={lk} magnitude x{mag}", flush=True)
    g = seeded(lq * 7 + lk)
    q = (torch.randn(b, lq, h, 128, generator=g) * mag).to(torch.bfloat16).to(dev)
    k = (torch.randn(b, lk, h, 128, generator=g) * mag).to(torch.bfloat16).to(dev)
    v = torch.randn(b, lk, h, 128, generator=g).to(torch.bfloat16).to(dev)
    got = attention.attention(q, k, v, backend="hip")
    assert got.shape == (b, lq, h, 128) and got.dtype == torch.bfloat16 and torch.isfinite(got.float()).all()
    fro, mx = rel(got, ref_attention(q, k, v))
    assert fro < 1e-2 and mx < 3e-2, (fro, mx)
    fro_s, _ = rel(got, attention.attention(q, k, v, backend="sdpa"))
    assert fro_s < 1e-2, fro_s


@pytest.mark.parametrize("lk", [1000, 4096])
def test_attention_growing_scores(dev, lk):
    """Keys whose scale grows along the sequence, so the tile max rises tile after tile and the lazy
    reference moves many times (each move rescales the running sums after the previous tile's probabilities
    have joined them), and a last block of keys far above the rest (a late jump of the reference): against
    float32 softmax attention at the usual tolerances."""
    from hy_nomas import attention

    print(f"attention growing scores lk={lk}", flush=True)
    g = seeded(lk + 3)
    b, h, lq = 1, 2, 160
    q = torch.randn(b, lq, h, 128, generator=g)
    k = torch.randn(b, lk, h, 128, generator=g) * torch.linspace(0.2, 3.0, lk).view(1, lk, 1, 1)
    k[:, -40:] *= 2.5
    v = torch.randn(b, lk, h, 128, generator=g)
    q, k, v = (t.to(torch.bfloat16).to(dev) for t in (q, k, v))
    got = attention.attention(q, k, v, backend="hip")
    assert torch.isfinite(got.float()).all()
    fro, mx = rel(got, ref_attention(q, k, v))
    assert fro < 1e-2 and mx < 3e-2, (fro, mx)


def test_attention_heads_on_strided_qkv(dev):
    """Head-major q, k, v as views of one [3, B, H, L, 128] buffer (the QKV epilogue's output)."""
    from hy_nomas import attention

    g = seeded(12)
    hm = torch.randn(3, 2, 4, 333, 128, generator=g).to(torch.bfloat16).to(dev)
    got = attention.attention_heads(hm[0], hm[1], hm[2], backend="hip")
    ref = ref_attention(*(t.transpose(1, 2) for t in hm))
    assert got.shape == (2, 333, 4, 128)
    fro, mx = rel(got, ref)
    assert fro < 1e-2 and mx < 3e-2, (fro, mx)


def test_attention_full_config4_length(dev):
    """57344 image + 256 text tokens, 24 heads x 128 (the config-4 block): sampled query rows of every head
    against float32 attention over all 57600 keys."""
    from hy_nomas import attention

    print("attention at 57600 tokens x 24 heads", flush=True)
    gen = torch.Generator(device=dev).manual_seed(5)
    L, H = 57600, 24
    hm = torch.randn(3, 1, H, L, 128, generator=gen, device=dev).to(torch.bfloat16)
    got = attention.attention_heads(hm[0], hm[1], hm[2], backend="hip")
    rows = torch.tensor(sorted(set(torch.randperm(L, generator=seeded(6))[:48].tolist() + [0, L - 1])), device=dev)
    qh, kh, vh = (t[0].float() for t in hm)                       # [H, L, 128]
    s = torch.matmul(qh[:, rows], kh.transpose(-1, -2).contiguous()) * 128 ** -0.5
    ref = torch.matmul(torch.softmax(s, dim=-1), vh).transpose(0, 1)  # [rows, H, 128]
    fro, mx = rel(got[0, rows], ref)
    print(f"  relative error {fro:.3e}, max {mx:.3e}", flush=True)
    assert fro < 1e-2 and mx < 3e-2, (fro, mx)


class Plan:
    def __init__(self, video_tokens, groups):
        self.video_tokens, self.groups = video_tokens, groups


def test_segment_attention_history_and_groups(dev):
    """segment_attention (hy_nomas/model.py:199-223) with history keys and query groups: the HIP backend against
    float32 attention over each group's keys [history | current video | the group's text keys]."""
    from hy_nomas import attention

    g = seeded(21)
    b, h, lv, lt, lh = 1, 2, 150, 40, 96
    q, k, v = (torch.randn(b, lv + lt, h, 128, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
    hk, hv = (torch.randn(1, lh, h, 128, generator=g).to(torch.bfloat16).to(dev) for _ in range(2))
    groups = [(torch.cat([torch.arange(0, 90), torch.arange(lv, lv + 10)]).to(dev), torch.arange(0, 10).to(dev)),
              (torch.cat([torch.arange(90, lv), torch.arange(lv + 10, lv + lt)]).to(dev), torch.arange(10, 40).to(dev))]
    for plan in (Plan(lv, None), Plan(lv, groups)):
        got = attention.segment_attention(q, k, v, (hk, hv), plan, None, backend="hip")
        ref = torch.empty(b, lv + lt, h, 128, device=dev)
        for q_idx, t_idx in (plan.groups or [(torch.arange(lv + lt, device=dev), torch.arange(lt, device=dev))]):
            keys = torch.cat([hk, k[:, :lv], k[:, lv + t_idx]], dim=1)
            vals = torch.cat([hv, v[:, :lv], v[:, lv + t_idx]], dim=1)
            ref[:, q_idx] = ref_attention(q[:, q_idx], keys, vals)
        fro, mx = rel(got, ref)
        assert fro < 1e-2 and mx < 3e-2, (plan.groups is None, fro, mx)
        fro_s, _ = rel(got, attention.segment_attention(q, k, v, (hk, hv), plan, {}, backend="sdpa"))
        assert fro_s < 1e-2


@pytest.mark.parametrize("per_token,lv,lt", [(False, 200, 40), (True, 200, 40), (False, 224, 64), (True, 224, 64)])
def test_double_stream_block_on_the_hip_backend(dev, per_token, lv, lt, monkeypatch):
    """The double-stream block with the HIP attention kernel against the float32 block (as the SDPA run).  With
    whole 32-token blocks in both streams (224 + 64) the QKV epilogues write v straight into V^T; the block's
    output then equals, bit for bit, the run that writes v head-major and copies it to V^T."""
    from hy_nomas import block, kernels
    from oracle import torch_forms
    from test_block_gpu import make_stream

    d, heads, mlp = 256, 2, 1024
    print(f"double-stream block on hip per_token={per_token} {lv}+{lt}", flush=True)
    g = seeded(191 + per_token)
    img_blk = make_stream(d, heads, mlp, g, per_token, dev)
    txt_blk = make_stream(d, heads, mlp, g, per_token, dev)
    img = torch.randn(1, lv, d, generator=g).to(torch.bfloat16).to(dev)
    txt = torch.randn(1, lt, d, generator=g).to(torch.bfloat16).to(dev)
    img_mods = [(torch.randn(1, d, generator=g) * 0.1).to(torch.bfloat16).to(dev) for _ in range(6)]
    txt_mods = [(torch.randn(1, d, generator=g) * 0.1).to(torch.bfloat16).to(dev) for _ in range(6)]
    grid = (2, 10, 10) if lv == 200 else (2, 8, 14)
    rope = [t.to(dev) for t in torch_forms.rope_freqs([32, 48, 48], 256, *grid)]
    blk = block.DoubleStreamBlockInt8(img_blk, txt_blk)
    with torch.no_grad():
        gi, gt = blk.forward(img, txt, img_mods, txt_mods, rope, "hip")
        si, st = blk.forward(img, txt, img_mods, txt_mods, rope, "sdpa")
        ri, rt = torch_forms.reference_double_stream(img_blk, txt_blk, img, txt, img_mods, txt_mods, rope)
    for got, sd, ref in ((gi, si, ri), (gt, st, rt)):
        assert rel(got, ref)[0] < 2e-2
        assert rel(got, sd)[0] < 1e-2
    if kernels.vt_direct_ok(lv, 0) and kernels.vt_direct_ok(lt, lv):
        monkeypatch.setattr(kernels, "vt_direct_ok", lambda *a: False)
        with torch.no_grad():
            ci, ct = blk.forward(img, txt, img_mods, txt_mods, rope, "hip")
        assert torch.equal(ci, gi) and torch.equal(ct, gt)


@pytest.mark.parametrize("backend", ["hip", "sdpa"])
def test_double_stream_block_with_history_plan_and_capture(dev, backend):
    """The block's attention with the reference's segment inputs (hy_nomas/model.py:288-297): cached history keys
    and values, an action plan's query groups, and the capture hook, against the float32 block with the same
    segment attention; the captured keys / values are the QKV epilogue's own."""
    from hy_nomas import block
    from oracle import torch_forms
    from test_block_gpu import make_stream

    d, heads, mlp, lv, lt, lh = 256, 2, 1024, 200, 40, 64
    g = seeded(217)
    img_blk = make_stream(d, heads, mlp, g, False, dev)
    txt_blk = make_stream(d, heads, mlp, g, False, dev)
    img = torch.randn(1, lv, d, generator=g).to(torch.bfloat16).to(dev)
    txt = torch.randn(1, lt, d, generator=g).to(torch.bfloat16).to(dev)
    img_mods = [(torch.randn(1, d, generator=g) * 0.1).to(torch.bfloat16).to(dev) for _ in range(6)]
    txt_mods = [(torch.randn(1, d, generator=g) * 0.1).to(torch.bfloat16).to(dev) for _ in range(6)]
    rope = [t.to(dev) for t in torch_forms.rope_freqs([32, 48, 48], 256, 2, 10, 10)]
    history = tuple(torch.randn(1, lh, heads, d // heads, generator=g).to(torch.bfloat16).to(dev) for _ in range(2))
    groups = [(torch.cat([torch.arange(0, 120), torch.arange(lv, lv + 15)]).to(dev), torch.arange(0, 15).to(dev)),
              (torch.cat([torch.arange(120, lv), torch.arange(lv + 15, lv + lt)]).to(dev),
               torch.cat([torch.arange(0, 5), torch.arange(15, lt)]).to(dev))]

    class Plan:
        video_tokens = lv

    plan = Plan()
    plan.groups = groups
    captured = []
    blk = block.DoubleStreamBlockInt8(img_blk, txt_blk)
    with torch.no_grad():
        for hist, pl in ((history, None), (None, plan), (history, plan)):
            captured.clear()
            gi, gt = blk.forward(img, txt, img_mods, txt_mods, rope, backend, history=hist, plan=pl,
                                 capture=lambda k, v: captured.append((k.clone(), v.clone())))
            ri, rt = torch_forms.reference_double_stream(img_blk, txt_blk, img, txt, img_mods, txt_mods, rope,
                                                         history=hist, groups=pl.groups if pl else None)
            for got, ref in ((gi, ri), (gt, rt)):
                assert rel(got, ref)[0] < 2e-2, (hist is None, pl is None, rel(got, ref))
            (ck, cv), = captured
            assert ck.shape == (1, lv + lt, heads, d // heads) and cv.shape == ck.shape
    # the captured keys / values (image tokens first) against the float32 block's own q / k / v of each stream
    _, rki, rvi = torch_forms._qkv(img_blk, img.float(), img_mods, rope, 1e-6)
    _, rkt, rvt = torch_forms._qkv(txt_blk, txt.float(), txt_mods, None, 1e-6)
    assert rel(ck, torch.cat([rki, rkt], dim=1))[0] < 1e-2
    assert rel(cv, torch.cat([rvi, rvt], dim=1))[0] < 1e-2
