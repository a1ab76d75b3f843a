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

    from hy_nomas import block, loader

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
    rope = [t.to(dev) for t in block.rope_freqs([32, 48, 48], 256, 2, 8, 6)]
    with torch.no_grad():
        gi, gt = blk.forward(img, txt, img_mods, txt_mods, rope)
        ri, rt = block.reference_double_stream(blk.img, blk.txt, img, txt, img_mods, txt_mods, rope)
    for got, ref in ((gi, ri), (gt, rt)):
        assert ((got.float() - ref).norm() / ref.norm()).item() < 2e-2
