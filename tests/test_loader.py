"""Checkpoint detection, load-time quantization and block construction (hy_nomas/loader.py:25-115), on synthetic
safetensors files written here (CPU); the GPU test runs a block built from such a file."""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from conftest import seeded

D, HEADS, MLP = 256, 2, 1024


def float_state_dict(g, blocks=1):
    sd = {}
    for i in range(blocks):
        for side in ("img", "txt"):
            p = f"double_blocks.{i}.{side}"
            for n, (o, k) in {"attn_q": (D, D), "attn_k": (D, D), "attn_v": (D, D), "attn_proj": (D, D),
                              "mlp.fc1": (MLP, D), "mlp.fc2": (D, MLP), "mod.linear": (6 * D, D)}.items():
                sd[f"{p}_{n}.weight"] = (torch.randn(o, k, generator=g) * 0.05).to(torch.bfloat16)
                sd[f"{p}_{n}.bias"] = (torch.randn(o, generator=g) * 0.02).to(torch.bfloat16)
            sd[f"{p}_attn_q_norm.weight"] = (torch.rand(D // HEADS, generator=g) + 0.5).to(torch.bfloat16)
            sd[f"{p}_attn_k_norm.weight"] = (torch.rand(D // HEADS, generator=g) + 0.5).to(torch.bfloat16)
    sd["img_in.proj.weight"] = torch.randn(D, 128, generator=g).to(torch.bfloat16)        # kept float (KEEP_FLOAT)
    sd["txt_in.odd.weight"] = torch.randn(D, 100, generator=g).to(torch.bfloat16)         # K % 128 != 0: kept
    sd["action_modules.0.weight"] = torch.randn(D, 256, generator=g).float()              # camera module
    return sd


def test_detect_and_config(tmp_path):
    from hy_nomas import loader

    g = seeded(1)
    sd = float_state_dict(g, blocks=3)
    assert loader.detect(sd, {}) == "float"
    assert loader.detect({"double_blocks.0.img_attn_q.weight_q": torch.zeros(1)}, None) == "int8"
    assert loader.detect({}, {"format": "nomas-int8-bf16-single-v1"}) == "int8"
    with pytest.raises(ValueError):
        loader.detect({"x.weight": torch.zeros(1)}, {})
    cfg = loader.config_from_state_dict(sd)
    assert cfg["mm_double_blocks_depth"] == 3 and cfg["camera"] is True and cfg["hidden_size"] == 2048


def test_quantize_state_dict_matches_oracle_and_keeps_float_modules():
    from hy_nomas import loader

    g = seeded(2)
    sd = float_state_dict(g)
    q = loader.quantize_state_dict(sd)
    w = sd["double_blocks.0.img_attn_q.weight"]
    qo, so = oracle.quantize(w.float().numpy())
    assert np.array_equal(q["double_blocks.0.img_attn_q.weight_q"].numpy(), qo)
    assert np.array_equal(q["double_blocks.0.img_attn_q.weight_scale"].numpy(), so)
    assert "double_blocks.0.img_attn_q.weight" not in q
    assert torch.equal(q["double_blocks.0.img_attn_q.bias"], sd["double_blocks.0.img_attn_q.bias"])
    for kept in ("img_in.proj.weight", "txt_in.odd.weight", "action_modules.0.weight"):
        assert torch.equal(q[kept], sd[kept])
    assert q["double_blocks.0.txt_mlp.fc2.weight_scale"].shape == (D, MLP // 128)


def test_load_state_dict_float_int8_and_metadata(tmp_path):
    from safetensors.torch import save_file

    from hy_nomas import loader

    g = seeded(3)
    sd = float_state_dict(g)
    sd["action_modules.0.weight"] = sd["action_modules.0.weight"].float()
    path = os.path.join(tmp_path, "float.safetensors")
    save_file(sd, path, metadata={"model_type": "hy-nomas", "format": "plain"})
    f_sd, meta, kind = loader.load_state_dict(path)
    assert kind == "float" and f_sd["action_modules.0.weight"].dtype == torch.bfloat16
    q_sd, _, kind_q = loader.load_state_dict(path, quantize=True)
    assert kind_q == "int8" and q_sd["double_blocks.0.img_mlp.fc1.weight_q"].dtype == torch.int8
    assert json.loads(loader.describe_file(path)) == {"format": "plain", "model_type": "hy-nomas"}
    ipath = os.path.join(tmp_path, "int8.safetensors")
    save_file(loader.quantize_state_dict(sd), ipath, metadata={"format": "nomas-int8-bf16-single-v1"})
    i_sd, imeta, ikind = loader.load_state_dict(ipath)
    assert ikind == "int8" and loader.info(imeta) == {"format": "nomas-int8-bf16-single-v1"}
    assert torch.equal(i_sd["double_blocks.0.img_attn_q.weight_q"], q_sd["double_blocks.0.img_attn_q.weight_q"])
    assert loader.describe_file(os.path.join(tmp_path, "missing.safetensors")) == "{}"


def test_double_block_needs_int8_weights():
    from hy_nomas import loader

    with pytest.raises(ValueError, match="no int8 weight"):
        loader.double_block(float_state_dict(seeded(4)), 0, HEADS, device="cpu")


@pytest.mark.gpu
def test_block_from_checkpoint_runs_on_the_int8_path(dev, tmp_path):
    """A double-stream block built from a (quantized) checkpoint file against the float32 block on the same
    dequantized weights; the QKV GEMM's weight is the concatenation of the file's q, k, v."""
    from safetensors.torch import save_file

    from hy_nomas import loader
    from oracle import torch_forms

    print("block from checkpoint", flush=True)
    g = seeded(5)
    sd = float_state_dict(g)
    path = os.path.join(tmp_path, "int8.safetensors")
    save_file(loader.quantize_state_dict(sd), path, metadata={"format": "nomas-int8-bf16-single-v1"})
    state, _, kind = loader.load_state_dict(path)
    assert kind == "int8"
    blk = loader.double_block(state, 0, HEADS, device=dev)
    assert torch.equal(blk.img.qkv.qw[:D].cpu(), state["double_blocks.0.img_attn_q.weight_q"])
    assert torch.equal(blk.img.qkv.qw[2 * D:].cpu(), state["double_blocks.0.img_attn_v.weight_q"])
    lv, lt = 96, 32
    img = torch.randn(1, lv, D, generator=g).to(torch.bfloat16).to(dev)
    txt = torch.randn(1, lt, D, generator=g).to(torch.bfloat16).to(dev)
    img_mods = [(torch.randn(1, D, generator=g) * 0.1).to(torch.bfloat16).to(dev) for _ in range(6)]
    txt_mods = [(torch.randn(1, D, generator=g) * 0.1).to(torch.bfloat16).to(dev) for _ in range(6)]
    rope = [t.to(dev) for t in torch_forms.rope_freqs([32, 48, 48], 256, 2, 8, 6)]
    with torch.no_grad():
        gi, gt = blk.forward(img, txt, img_mods, txt_mods, rope)
        ri, rt = torch_forms.reference_double_stream(blk.img, blk.txt, img, txt, img_mods, txt_mods, rope)
    for got, ref in ((gi, ri), (gt, rt)):
        assert ((got.float() - ref).norm() / ref.norm()).item() < 2e-2


def test_pixelumm_fp8_checkpoint_round_trip_and_gate_up_interleave(tmp_path):
    """The decoder's single-file FP8 format (hy_nomas/pixelumm.py:35, 470-485): fp8_weight / fp8_scale pairs
    under decoder.*, detected by metadata or keys; the fused gate/up weight alternates 128-row blocks."""
    from safetensors.torch import save_file

    from hy_nomas import pixelumm

    g = seeded(11)
    sd = {"layers.0.mlp.gate_proj.weight": torch.randn(384, 256, generator=g) * 0.02,
          "layers.0.mlp.up_proj.weight": torch.randn(384, 256, generator=g) * 0.02,
          "layers.0.mlp.down_proj.weight": torch.randn(256, 384, generator=g) * 0.02,
          "layers.0.input_norm.weight": torch.rand(256, generator=g) + 0.5,
          "head.linear.bias": torch.randn(100, generator=g)}
    fp8 = pixelumm.fp8_state_dict(sd)
    assert fp8["layers.0.mlp.gate_proj.fp8_weight"].dtype == torch.float8_e4m3fn
    assert fp8["layers.0.mlp.gate_proj.fp8_scale"].shape == (3, 2)
    assert fp8["layers.0.input_norm.weight"].dtype == torch.bfloat16
    path = os.path.join(tmp_path, "decoder_fp8.safetensors")
    save_file({"decoder." + k: v for k, v in fp8.items()} | {"dcae.enc.weight": torch.zeros(2)}, path,
              metadata={"format": pixelumm.FP8_FORMAT})
    state, is_fp8 = pixelumm.load_state_dict(path)
    assert is_fp8 and set(state) == set(fp8)
    assert torch.equal(state["layers.0.mlp.up_proj.fp8_weight"].view(torch.uint8),
                       fp8["layers.0.mlp.up_proj.fp8_weight"].view(torch.uint8))
    bf_path = os.path.join(tmp_path, "decoder_bf16.safetensors")
    save_file({"decoder." + k: v.to(torch.bfloat16) for k, v in sd.items()}, bf_path)
    assert pixelumm.load_state_dict(bf_path)[1] is False
    with pytest.raises(ValueError):
        save_file({"other.weight": torch.zeros(2)}, os.path.join(tmp_path, "x.safetensors"))
        pixelumm.load_state_dict(os.path.join(tmp_path, "x.safetensors"))
    # dequantized fp8 blocks stay within the e4m3 step of the weights
    w = sd["layers.0.mlp.gate_proj.weight"]
    wd = pixelumm.dequantize_fp8_block(fp8["layers.0.mlp.gate_proj.fp8_weight"],
                                       fp8["layers.0.mlp.gate_proj.fp8_scale"], torch.float32)
    assert ((wd - w).abs().max() / w.abs().max()).item() < 2 ** -3
    gate = (fp8["layers.0.mlp.gate_proj.fp8_weight"], fp8["layers.0.mlp.gate_proj.fp8_scale"])
    up = (fp8["layers.0.mlp.up_proj.fp8_weight"], fp8["layers.0.mlp.up_proj.fp8_scale"])
    q, s = pixelumm.interleave_gate_up(gate, up)
    assert q.shape == (768, 256) and s.shape == (6, 2) and q.dtype == torch.float8_e4m3fn
    for b in range(3):
        assert torch.equal(q[256 * b:256 * b + 128].view(torch.uint8), gate[0][128 * b:128 * (b + 1)].view(torch.uint8))
        assert torch.equal(q[256 * b + 128:256 * (b + 1)].view(torch.uint8), up[0][128 * b:128 * (b + 1)].view(torch.uint8))
        assert torch.equal(s[2 * b], gate[1][b]) and torch.equal(s[2 * b + 1], up[1][b])


def test_decoder_mlp_dequant_path_is_the_reference_expression():
    """pixelumm.MLP with matmul="dequant" (CPU): down_proj(F.silu(gate_proj(x)) * up_proj(x)) on the
    dequantized bf16 weights (hy_nomas/pixelumm.py:314-323, 150-155)."""
    from hy_nomas import pixelumm

    g = seeded(12)
    arch = pixelumm.Arch(hidden_size=256, intermediate_size=384)
    mlp = pixelumm.MLP(arch, pixelumm.DecoderOps.with_matmul("dequant"))
    sd = {}
    for name, (o, k) in {"gate_proj": (384, 256), "up_proj": (384, 256), "down_proj": (256, 384)}.items():
        q, s = pixelumm.quantize_fp8_block(torch.randn(o, k, generator=g) * 0.03)
        sd[f"{name}.fp8_weight"], sd[f"{name}.fp8_scale"] = q, s
    mlp.load_state_dict(sd, strict=False)
    x = torch.randn(5, 256, generator=g).to(torch.bfloat16)
    wd = {n: pixelumm.dequantize_fp8_block(sd[f"{n}.fp8_weight"], sd[f"{n}.fp8_scale"], torch.bfloat16)
          for n in ("gate_proj", "up_proj", "down_proj")}
    ref = torch.nn.functional.linear(
        torch.nn.functional.silu(torch.nn.functional.linear(x, wd["gate_proj"])) *
        torch.nn.functional.linear(x, wd["up_proj"]), wd["down_proj"])
    assert torch.equal(mlp(x), ref)
    # codes without their block scales are reported as missing
    missing = []
    lin = pixelumm.DecoderOps.Linear(256, 384, bias=False)
    lin._load_from_state_dict({"g.fp8_weight": sd["gate_proj.fp8_weight"]}, "g.", {}, True, missing, [], [])
    assert missing == ["g.fp8_scale"] and lin.weight is None
