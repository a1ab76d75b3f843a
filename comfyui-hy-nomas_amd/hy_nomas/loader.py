"""Hy-Nomas DiT checkpoints -> the int8 linear path (hy_nomas/loader.py:25-115).

Files are detected from their tensors, as the reference does:
* Tencent's INT8 file (`nomas-int8-bf16-single-v1`): `weight_q` int8 [N, K] + `weight_scale` fp32 [N, K/128] per
  Linear, everything else bf16.  Used as stored.
* a float file with plain `weight` tensors: cast to bf16, or quantized at load to the same int8 layout.

Files are read with safetensors (no code runs from a file).  The reference builds a ComfyUI MODEL from the state
dict; without ComfyUI this module builds the double-stream blocks of `block.py` instead, so a checkpoint's
weights run on the HIP GEMMs directly.
"""
import json

import torch

from . import ops as nomas_ops

UNET_CONFIG = {
    "in_channels": 32, "out_channels": 32, "hidden_size": 2048, "heads_num": 16, "mlp_width_ratio": 4,
    "mm_double_blocks_depth": 54, "rope_dim_list": [16, 56, 56], "rope_theta": 256, "text_states_dim": 3584,
}
# small modules the int8 path keeps unquantized when quantizing a float checkpoint, as Tencent's file does
KEEP_FLOAT = ("action_modules.", "extrinsics_embedding_camctrl", "c2ws_hidden_states_layer", "img_in.")
INT8_FORMAT = "nomas-int8-bf16-single-v1"


def detect(state_dict, metadata):
    """"int8" or "float" (hy_nomas/loader.py:34-40); anything else raises ValueError."""
    fmt = (metadata or {}).get("format")
    if fmt == INT8_FORMAT or any(k.endswith(".weight_q") for k in state_dict):
        return "int8"
    if "double_blocks.0.img_attn_q.weight" in state_dict:
        return "float"
    raise ValueError("not a Hy-Nomas DiT checkpoint (no double_blocks.0.img_attn_q weights)")


def config_from_state_dict(state_dict):
    """The reference's UNET_CONFIG with the block depth and camera flag read from the keys (loader.py:43-48)."""
    cfg = dict(UNET_CONFIG)
    depth = 1 + max(int(k.split(".")[1]) for k in state_dict if k.startswith("double_blocks."))
    cfg["mm_double_blocks_depth"] = depth
    cfg["camera"] = any(k.startswith("action_modules.") for k in state_dict)
    return cfg


def quantize_state_dict(state_dict):
    """A float checkpoint's Linear weights -> Tencent's int8 g128 pairs (hy_nomas/loader.py:51-62).  Weights on a
    GPU are quantized by the device kernel; CPU tensors by the reference's torch steps (`ops.quantize_g128`)."""
    out = {}
    for key, value in state_dict.items():
        if (key.endswith(".weight") and value.ndim == 2 and not key.startswith(KEEP_FLOAT)
                and value.shape[1] % 128 == 0):
            q, s = nomas_ops.quantize_g128(value)
            out[key[:-len("weight")] + "weight_q"] = q
            out[key[:-len("weight")] + "weight_scale"] = s
        else:
            out[key] = value
    return out


def load_state_dict(path, quantize=False):
    """(state_dict, metadata, kind) of a safetensors checkpoint (the reference's `load_dit` minus the ComfyUI
    model): float files are cast to bf16 and, with `quantize`, turned into int8 pairs."""
    from safetensors import safe_open
    from safetensors.torch import load_file

    with safe_open(path, framework="pt", device="cpu") as handle:
        metadata = handle.metadata() or {}
    state_dict = load_file(path, device="cpu")
    kind = detect(state_dict, metadata)
    if kind == "float":
        state_dict = {k: (v.to(torch.bfloat16) if v.is_floating_point() else v) for k, v in state_dict.items()}
        if quantize:
            state_dict = quantize_state_dict(state_dict)
            kind = "int8"
    return state_dict, metadata, kind


def _linear(state_dict, prefix, device):
    from .block import Int8Linear

    try:
        q, s = state_dict[prefix + ".weight_q"], state_dict[prefix + ".weight_scale"]
    except KeyError:
        raise ValueError(f"checkpoint has no int8 weight for {prefix} (quantize a float file first)") from None
    bias = state_dict.get(prefix + ".bias")
    return Int8Linear(q.to(device).contiguous(), s.to(device).float().contiguous(),
                      None if bias is None else bias.to(device, torch.bfloat16).contiguous())


def double_block(state_dict, index, heads, device="cuda"):
    """The int8 double-stream block `double_blocks.<index>` (hy_nomas/model.py:230-244 names) as a
    `block.DoubleStreamBlockInt8` on `device`: per stream, q/k/v concatenated into one QKV GEMM, the out
    projection, the MLP and the QK-norm weights.  The modulation linears (`<side>_mod`) stay with the caller,
    whose per-sample adaLN vectors the block takes as inputs."""
    from .block import DiTBlockInt8, DoubleStreamBlockInt8, Int8Linear

    sides = {}
    for side in ("img", "txt"):
        p = f"double_blocks.{index}.{side}"
        qkv = Int8Linear.cat([_linear(state_dict, f"{p}_attn_{n}", device) for n in ("q", "k", "v")])
        sides[side] = DiTBlockInt8(
            qkv, _linear(state_dict, f"{p}_attn_proj", device), _linear(state_dict, f"{p}_mlp.fc1", device),
            _linear(state_dict, f"{p}_mlp.fc2", device),
            state_dict[f"{p}_attn_q_norm.weight"].to(device, torch.bfloat16),
            state_dict[f"{p}_attn_k_norm.weight"].to(device, torch.bfloat16), heads)
    return DoubleStreamBlockInt8(sides["img"], sides["txt"])


def info(metadata):
    """The descriptive metadata keys of a checkpoint (hy_nomas/loader.py:102-106)."""
    if not metadata:
        return {}
    keep = ("format", "model_type", "quantization", "group_size", "source_sha256")
    return {k: metadata[k] for k in keep if k in metadata}


def describe_file(path):
    """`info` of a file as JSON, "{}" when it cannot be read (hy_nomas/loader.py:109-115)."""
    try:
        from safetensors import safe_open
        with safe_open(path, framework="pt", device="cpu") as handle:
            return json.dumps(info(handle.metadata()))
    except Exception:
        return "{}"
