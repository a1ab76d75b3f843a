"""The Linear op family that loads Tencent's int8 g128 weights and picks the matmul (hy_nomas/ops.py:104-191):
state-dict loading and its errors, the exact path against the dequantized weight, the matmul-mode switches
(`with_matmul`, HY_NOMAS_MATMUL), re-quantization on `set_weight`, `fast_int8` / `int8_weights`, and on the
GPU the int8 matrix-core path against block_linear and against the exact path."""
import numpy as np
import pytest
import torch

import oracle
from conftest import seeded


def tencent_pair(n, k, seed):
    """A `weight_q` / `weight_scale` pair as the reference's checkpoints hold it (ops.py:41-52 on a bf16 weight)."""
    w = (torch.randn(n, k, generator=seeded(seed)) * 0.02).to(torch.bfloat16)
    q, s = oracle.quantize_g128(w)
    return torch.from_numpy(q), torch.from_numpy(s)


def make_linear(ops_cls, n, k, seed, bias=True, dtype=torch.bfloat16):
    from hy_nomas import ops

    lin = ops_cls.Linear(k, n, bias=bias, dtype=dtype)
    q, s = tencent_pair(n, k, seed)
    sd = {"weight_q": q, "weight_scale": s}
    b = (torch.randn(n, generator=seeded(seed + 1)) * 0.02).to(torch.bfloat16)
    if bias:
        sd["bias"] = b
    missing, errors = [], []
    lin._load_from_state_dict(sd, "", {}, True, missing, [], errors)
    assert not missing and not errors
    assert ops.is_quantized(lin.weight)
    return lin, q, s, b


def test_load_and_exact_forward_is_dequantize_then_linear():
    from hy_nomas import ops

    n, k = 96, 300  # K not a multiple of 128: the last group is partial
    lin, q, s, b = make_linear(ops.NomasOps, n, k, seed=3)
    assert torch.equal(lin.weight._qdata, q) and torch.equal(lin.weight._params.scale, s)
    x = torch.randn(2, 5, k, generator=seeded(4)).to(torch.bfloat16)
    got = lin(x)
    w = torch.from_numpy(oracle.dequantize_g128(q.numpy(), s.numpy())).to(torch.bfloat16)
    assert torch.equal(got, torch.nn.functional.linear(x, w, b))
    assert got.shape == (2, 5, n) and got.dtype == torch.bfloat16


def test_load_errors_and_plain_weights():
    from hy_nomas import ops

    q, s = tencent_pair(64, 128, seed=5)
    lin = ops.NomasOps.Linear(128, 64, bias=True)
    missing, errors = [], []
    lin._load_from_state_dict({"blk.weight_q": q}, "blk.", {}, True, missing, [], errors)
    assert errors == ["blk.weight_q without blk.weight_scale"] and lin.weight is None
    errors.clear()
    lin._load_from_state_dict({"blk.weight_q": q[:, :64], "blk.weight_scale": s}, "blk.", {}, True, missing, [],
                             errors)
    assert len(errors) == 1 and "expected (64, 128)" in errors[0]
    errors.clear()
    lin._load_from_state_dict({}, "blk.", {}, True, missing, [], errors)
    assert missing == ["blk.weight"]
    missing.clear()
    # a plain weight stays a plain parameter, cast to the layer dtype; a missing bias is reported
    lin = ops.NomasOps.Linear(128, 64, bias=True, dtype=torch.bfloat16)
    plain = torch.randn(64, 128, generator=seeded(6))
    lin._load_from_state_dict({"blk.weight": plain}, "blk.", {}, True, missing, [], errors)
    assert missing == ["blk.bias"] and not errors
    assert not ops.is_quantized(lin.weight) and lin.weight.dtype == torch.bfloat16
    assert ops.quantized_linears(torch.nn.Sequential(lin)) == []


def test_matmul_mode_switches(monkeypatch):
    from hy_nomas import ops

    int8_ops = ops.NomasOps.with_matmul("int8")
    assert int8_ops.Linear.default_matmul == "int8" and ops.NomasOps.Linear.default_matmul == "exact"
    assert issubclass(int8_ops.Linear, ops.NomasOps.Linear)
    lin, _, _, _ = make_linear(int8_ops, 64, 256, seed=7)
    x = torch.randn(3, 256, generator=seeded(8)).to(torch.bfloat16)
    # CPU input: never the int8 path, whatever the mode
    assert not lin.fast_int8(x)
    exact, _, _, _ = make_linear(ops.NomasOps, 64, 256, seed=7)
    assert torch.equal(lin(x), exact(x))
    monkeypatch.setenv(ops.MATMUL_ENV, "int8")
    assert ops.matmul_mode() == "int8"
    monkeypatch.delenv(ops.MATMUL_ENV)
    assert ops.matmul_mode() == "exact" and ops.matmul_mode("int8") == "int8"


def test_set_weight_requantizes_and_int8_weights_yields_the_codes():
    from hy_nomas import ops

    lin, q, s, b = make_linear(ops.NomasOps, 64, 256, seed=9)
    new = (torch.randn(64, 256, generator=seeded(10)) * 0.05).to(torch.bfloat16)
    lin.set_weight(new)
    q2, s2 = oracle.quantize_g128(new)
    assert torch.equal(lin.weight._qdata, torch.from_numpy(q2))
    assert np.array_equal(lin.weight._params.scale.numpy(), s2)
    with lin.int8_weights(torch.zeros(1, 256, dtype=torch.bfloat16)) as (qd, sc, bias):
        assert torch.equal(qd, torch.from_numpy(q2)) and torch.equal(bias, b)


@pytest.mark.gpu
def test_int8_mode_runs_the_matrix_core_path(dev):
    """int8 mode on a device input: bit-identical to block_linear (per-token-and-group quantization + the
    g128 GEMM), within 1e-2 max-abs-rel of the exact path, and `fast_int8` holds."""
    from hy_nomas import kernels, ops

    print("ops.Linear int8 mode", flush=True)
    lin, q, s, b = make_linear(ops.NomasOps.with_matmul("int8"), 384, 1024, seed=11)
    lin = lin.to(dev)
    x = (torch.randn(2, 77, 1024, generator=seeded(12)) * 2).to(torch.bfloat16).to(dev)
    assert lin.fast_int8(x)
    got = lin(x)
    ref = kernels.block_linear(x, q.to(dev), s.to(dev), b.to(dev))
    assert torch.equal(got, ref)
    exact = ops.NomasOps.Linear(1024, 384, bias=True, dtype=torch.bfloat16)
    exact._load_from_state_dict({"weight_q": q, "weight_scale": s, "bias": b}, "", {}, True, [], [], [])
    want = exact.to(dev)(x).float()
    assert ((got.float() - want).abs().max() / want.abs().max()).item() < 1e-2
    with lin.int8_weights(x) as (qd, sc, bias):
        assert qd.device == x.device and torch.equal(qd.cpu(), q)


@pytest.mark.gpu
def test_block_linear_takes_the_reference_fallback_for_empty_and_ragged_k(dev):
    """M = 0 and K % 128 != 0 take the reference's dequantize + F.linear branch (kernels.py:216-218)."""
    from hy_nomas import kernels

    print("block_linear fallback shapes", flush=True)
    q, s = tencent_pair(64, 256, seed=13)
    out = kernels.block_linear(torch.empty(0, 256, dtype=torch.bfloat16, device=dev), q.to(dev), s.to(dev))
    assert out.shape == (0, 64) and out.dtype == torch.bfloat16
    q, s = tencent_pair(64, 200, seed=14)
    x = torch.randn(2, 3, 200, generator=seeded(15)).to(torch.bfloat16)
    b = (torch.randn(64, generator=seeded(16)) * 0.02).to(torch.bfloat16)
    got = kernels.block_linear(x.to(dev), q.to(dev), s.to(dev), b.to(dev)).cpu()
    w = torch.from_numpy(oracle.dequantize_g128(q.numpy(), s.numpy())).to(torch.bfloat16)
    want = torch.nn.functional.linear(x.float(), w.float(), b.float())
    assert got.shape == (2, 3, 64)
    assert ((got.float() - want).abs().max() / want.abs().max()).item() < 1e-2


def test_fused_gate(monkeypatch):
    """fused.available: HY_NOMAS_FUSED != "0" at import, a device tensor, bf16 (fused.py:22-26)."""
    import importlib

    from hy_nomas import fused

    assert fused.ENABLED
    assert not fused.available(torch.zeros(2, dtype=torch.bfloat16))
    monkeypatch.setenv("HY_NOMAS_FUSED", "0")
    try:
        assert not importlib.reload(fused).ENABLED
    finally:
        monkeypatch.delenv("HY_NOMAS_FUSED")
        importlib.reload(fused)
    assert fused.ENABLED
    if torch.cuda.is_available():
        assert fused.available(torch.zeros(2, dtype=torch.bfloat16, device="cuda"))
        assert not fused.available(torch.zeros(2, dtype=torch.float16, device="cuda"))


def test_kv_host_path_and_odd_head_dims():
    """quantize_kv / dequantize_kv on host tensors and on head dims that are not multiples of 128 take the
    reference's torch steps (hy_nomas/world.py:83-94): codes and scales equal the oracle's."""
    from hy_nomas import kv

    g = seeded(31)
    for shape in ((50, 3, 128), (7, 2, 96), (5, 1, 200)):
        x = torch.randn(*shape, generator=g).to(torch.bfloat16)
        x[0, 0] = 0  # an all-zero (token, head) row: scale 1, codes 0
        x[1, 0, 3] = 0.5 * x[1, 0].abs().max()   # half of the peak: an exact .5 tie of x / scale
        q, s = kv.quantize_kv(x)
        q_ref, s_ref = oracle.quantize_kv(x)
        assert q.dtype == torch.int8 and s.shape == shape[:2] + (1,)
        assert np.array_equal(q.numpy(), q_ref) and np.array_equal(s.numpy(), s_ref)
        back = kv.dequantize_kv(q, s)
        assert torch.equal(back, torch.from_numpy(oracle.dequantize_kv(q_ref, s_ref)))


def test_qk_kernels_reject_other_dtypes():
    """The QK kernels read bf16 bits: fp16 / fp32 inputs raise instead of being read as bf16."""
    from hy_nomas import fused

    x = torch.randn(1, 4, 2, 128)
    w = torch.ones(128)
    for dtype in (torch.float32, torch.float16):
        with pytest.raises(RuntimeError, match="bfloat16"):
            fused.qk_norm_rope(x.to(dtype), w)
        with pytest.raises(RuntimeError, match="bfloat16"):
            fused.pixelumm_qk(x.to(dtype), w[:64], w[:64], torch.ones(4, 128), torch.zeros(4, 128))


def test_whole_k_int8_routes_long_k_to_the_group_fold(monkeypatch):
    """A per-token x per-channel int8 GEMM with K >= 2^17 would overflow a whole-K int32 sum: the wrapper
    hands it to the per-group fold instead (scales repeated per group); shorter K keeps whole-K mode."""
    from hy_nomas import kernels

    sw = torch.ones(8, 1)
    assert kernels._layout(sw, 8, 3072, "int8", 1)[2:] == (3072, 1)
    assert kernels._layout(sw, 8, 131072, "int8", 1)[2:] == (128, 1024)
    assert kernels._layout(sw, 8, 131072, "fp8", 1)[2:] == (131072, 1)


def test_attention_backend_selection_and_value_layout(monkeypatch):
    """The attention backend switch (HY_NOMAS_ATTENTION) and the kernel's V^T layout: keys along the last dim in
    the grouped order, padded with zeros up to the 64-key tile."""
    from hy_nomas import attention

    monkeypatch.delenv(attention.BACKEND_ENV, raising=False)
    assert attention.choose_backend() == "sdpa" and attention.choose_backend("hip") == "hip"
    monkeypatch.setenv(attention.BACKEND_ENV, "hip")
    assert attention.choose_backend() == "hip" and attention.choose_backend("sdpa") == "sdpa"
    monkeypatch.setenv(attention.BACKEND_ENV, "flash")
    with pytest.raises(ValueError):
        attention.choose_backend()
    for lk in (70, 64, 5, 130):
        vh = torch.randn(2, 3, lk, 128).to(torch.bfloat16)
        vt = attention.transpose_values(vh)
        pad = -(-lk // 64) * 64
        assert vt.shape == (2, 3, 128, pad)
        # key j at position 16 (j // 16) + 8 ((j // 4) % 2) + 4 ((j // 8) % 2) + j % 4; the other positions are 0
        pos = [16 * (j // 16) + 8 * ((j // 4) % 2) + 4 * ((j // 8) % 2) + j % 4 for j in range(lk)]
        assert len(set(pos)) == lk and max(pos) < pad
        assert torch.equal(vt[..., pos], vh.transpose(-1, -2))
        rest = sorted(set(range(pad)) - set(pos))
        assert not vt[..., rest].any()
    # values_buffer for writers that fill only the real keys: every padding key is zero, including those of a
    # partial last 16-key group that the grouped order places below Lk.  torch.empty is made to return NaN
    # bits, so that memory which happens to be zero cannot hide a position the buffer leaves uninitialised.
    real_empty = torch.empty
    for lk in (70, 64, 37, 5, 130, 16):
        with monkeypatch.context() as mp:
            mp.setattr(torch, "empty", lambda *a, **kw: real_empty(*a, **kw).fill_(float("nan")))
            buf = attention.values_buffer(2, 3, lk, "cpu")
        pad = -(-lk // 64) * 64
        assert buf.shape == (2, 3, 128, pad)
        pos = [16 * (j // 16) + 8 * ((j // 4) % 2) + 4 * ((j // 8) % 2) + j % 4 for j in range(lk)]
        rest = sorted(set(range(pad)) - set(pos))
        assert not buf[..., rest].any(), f"lk={lk}: padding keys left uninitialised"
        if lk % 16 > 4:
            assert min(rest) < lk  # the case the grouped order creates
    # a token-major value tensor viewed head-major (the layout attention() passes)
    v = torch.randn(1, 40, 2, 128).to(torch.bfloat16)
    assert torch.equal(attention.transpose_values(v.transpose(1, 2)), attention.transpose_values(v.transpose(1, 2).contiguous()))
    k = torch.randn(1, 5, 2, 128)
    hk = torch.randn(1, 3, 2, 128)
    keys, vals = attention._keys([(hk, hk + 1), None, (k, k + 1), (k[:, :0], k[:, :0])])
    assert torch.equal(keys, torch.cat([hk, k], dim=1)) and torch.equal(vals, torch.cat([hk + 1, k + 1], dim=1))


def test_attention_reference_signature_and_segments_cpu():
    """attention / segment_attention called as the reference's model.py calls them (transformer_options in the
    4th / 6th position), on float32 CPU tensors (the SDPA backend), against explicit softmax attention: every
    query group attends to [history | all current video keys | its own text keys] (model.py:199-223)."""
    from hy_nomas import attention

    g = torch.Generator().manual_seed(31)
    b, h, lv, lt, lh, d = 2, 2, 30, 12, 9, 128
    q, k, v = (torch.randn(b, lv + lt, h, d, generator=g) for _ in range(3))
    hk, hv = (torch.randn(1, lh, h, d, generator=g) for _ in range(2))

    def softmax_attn(qq, kk, vv):
        s = torch.einsum("bqhd,bkhd->bhqk", qq, kk) / d ** 0.5
        return torch.einsum("bhqk,bkhd->bqhd", torch.softmax(s, dim=-1), vv)

    out = attention.attention(q, k, v, {"patches": {}})
    assert torch.allclose(out, softmax_attn(q, k, v), atol=1e-5)

    class Plan:
        video_tokens = lv
        groups = [(torch.cat([torch.arange(0, 20), torch.arange(lv, lv + 5)]), torch.arange(0, 5)),
                  (torch.cat([torch.arange(20, lv), torch.arange(lv + 5, lv + lt)]), torch.tensor([0, 5, 6, 7, 8, 9, 10, 11])),
                  ]

    got = attention.segment_attention(q, k, v, (hk, hv), Plan(), {})
    want = torch.empty_like(q)
    for q_idx, t_idx in Plan.groups:
        keys = torch.cat([hk.expand(b, -1, -1, -1), k[:, :lv], k[:, lv + t_idx]], dim=1)
        vals = torch.cat([hv.expand(b, -1, -1, -1), v[:, :lv], v[:, lv + t_idx]], dim=1)
        want[:, q_idx] = softmax_attn(q[:, q_idx], keys, vals)
    assert torch.allclose(got, want, atol=1e-5)

    class NoGroups:
        video_tokens = lv
        groups = None

    got = attention.segment_attention(q, k, v, None, NoGroups(), None)
    assert torch.allclose(got, softmax_attn(q, k, v), atol=1e-5)
    # the float32 form the block tests compare with agrees (with and without history, with and without groups)
    from oracle import torch_forms
    for hist in (None, (hk, hv)):
        for plan in (NoGroups(), Plan()):
            assert torch.allclose(torch_forms.segment_attention(q, k, v, hist, plan.groups, lv),
                                  attention.segment_attention(q, k, v, hist, plan, {}), atol=1e-5)


def test_fp8_block_scale_dispatch_reads_only_recorded_verdicts():
    """fp8 with 128 x 128 block weight scales: the GEMM reads them as stored only when the activation and weight
    scales are recorded as positive and finite (this package's quantizers, or `validate_scales`); otherwise the
    block rows are repeated per channel, the layout whose fold takes any values.  Deciding never reads a scale
    tensor, and an in-place change drops the verdict."""
    from hy_nomas import kernels

    n, k = 300, 512
    g = torch.Generator().manual_seed(40)
    s = torch.rand(3, 4, generator=g) + 0.1
    sw, rows, group, groups = kernels._layout(s, n, k, "fp8", 4)
    assert rows == 1 and group == 128 and groups == 4 and sw.shape == (n, 4)
    assert torch.equal(sw, s.repeat_interleave(128, 0)[:n])
    assert kernels.validate_scales(s)
    sw, rows, _, _ = kernels._layout(s, n, k, "fp8", 4)
    assert rows == 128 and sw is s
    s[0, 0] = 0.0                      # in place: the verdict no longer applies
    assert kernels._layout(s, n, k, "fp8", 4)[1] == 1
    assert not kernels.validate_scales(s)
    assert kernels._layout(s, n, k, "fp8", 4)[1] == 1
    for bad in (float("inf"), float("nan"), -1e-3):
        t = torch.rand(3, 4, generator=g) + 0.1
        t[2, 3] = bad
        assert not kernels.validate_scales(t) and kernels._layout(t, n, k, "fp8", 4)[1] == 1
    # activation scales from elsewhere need a verdict too
    sw_ok = torch.rand(3, 4, generator=g) + 0.1
    kernels.trust_scales(sw_ok)
    sa = torch.rand(8, 4, generator=g) + 0.1
    assert kernels._layout(sw_ok, n, k, "fp8", 4, sa)[1] == 1
    assert kernels.validate_scales(sa) and kernels._layout(sw_ok, n, k, "fp8", 4, sa)[1] == 128
    # int8 block scales fold without a ratio: no verdict needed
    assert kernels._layout(torch.rand(3, 4, generator=g), n, k, "int8", 4)[1] == 128
