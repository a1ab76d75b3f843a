"""Hy-Nomas DiT checkpoints -> the int8 linear path (the reference's hy_nomas/loader.py:25-115).

The on-disk formats, as the reference's loader accepts them:

* Tencent's int8 release, metadata ``format = nomas-int8-bf16-single-v1``: every quantized Linear stores
  ``<name>.weight_q`` (int8 [N, K]) and ``<name>.weight_scale`` (fp32 [N, ceil(K / 128)], one scale per
  output channel and 128 input channels); all other tensors are bf16.  It is used as stored.
* float releases (fp32 or bf16 ``<name>.weight``), recognised by the first block's image q projection.  They
  are cast to bf16 and may be quantized at load to the int8 layout above: every 2-D ``.weight`` whose K is a
  multiple of 128, except the small modules the int8 release also keeps in bf16.

Files are read with safetensors (tensors) and by parsing the safetensors JSON header (names and metadata); no
code runs from a file.  Without ComfyUI this module builds the double-stream blocks of `block.py` from the
state dict, so a checkpoint's weights run on the HIP GEMMs directly.
"""
import json
import struct

import torch

from . import ops as nomas_ops

INT8_FORMAT = "nomas-int8-bf16-single-v1"
CODES_SUFFIX, SCALES_SUFFIX = "weight_q", "weight_scale"
# a float file holds this tensor; an int8 file holds its codes / scales instead
FLOAT_MARKER = "double_blocks.0.img_attn_q.weight"
# the released model's shape; the block depth and the camera flag are read from the keys
UNET_CONFIG = {
    "in_channels": 32, "out_channels": 32, "hidden_size": 2048, "heads_num": 16, "mlp_width_ratio": 4,
    "mm_double_blocks_depth": 54, "rope_dim_list": [16, 56, 56], "rope_theta": 256, "text_states_dim": 3584,
}
# key prefixes whose weights the int8 release stores in bf16 (patch embedding, camera and action modules)
KEEP_FLOAT = ("action_modules.", "extrinsics_embedding_camctrl", "c2ws_hidden_states_layer", "img_in.")
# metadata entries a checkpoint description reports
DESCRIPTIVE_KEYS = ("format", "model_type", "quantization", "group_size", "source_sha256")
_HEADER_LIMIT = 1 << 28   # bytes of JSON header accepted before the file is taken as something else


def read_header(path):
    """(tensor table, metadata) of a safetensors file, from its header alone: an 8-byte little-endian length,
    then that many bytes of JSON mapping tensor names to {dtype, shape, data_offsets}, with the optional
    string map ``__metadata__``.  Raises OSError / ValueError for a file that is not one."""
    with open(path, "rb") as handle:
        raw = handle.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: too short for a safetensors header")
        (size,) = struct.unpack("<Q", raw)
        if size == 0 or size > _HEADER_LIMIT:
            raise ValueError(f"{path}: implausible safetensors header size {size}")
        body = handle.read(size)
    if len(body) != size:
        raise ValueError(f"{path}: truncated safetensors header")
    table = json.loads(body.decode("utf-8"))
    if not isinstance(table, dict):
        raise ValueError(f"{path}: the safetensors header is not a JSON object")
    metadata = table.pop("__metadata__", None) or {}
    return table, metadata


def _block_layout(keys):
    """(number of double blocks, has a camera module) from the state-dict keys."""
    top = -1
    camera = False
    for key in keys:
        parts = key.split(".", 2)
        if parts[0] == "double_blocks" and len(parts) > 1 and parts[1].isdigit():
            top = max(top, int(parts[1]))
        elif parts[0] == "action_modules":
            camera = True
    return top + 1, camera


def detect(state_dict, metadata):
    """The checkpoint kind, "int8" or "float" (the reference's loader.py:34-40); ValueError for anything that
    is not a Hy-Nomas DiT file.  The metadata's format tag decides first, then the tensor names."""
    if (metadata or {}).get("format") == INT8_FORMAT:
        return "int8"
    codes = "." + CODES_SUFFIX
    for key in state_dict:
        if key.endswith(codes):
            return "int8"
    if FLOAT_MARKER in state_dict:
        return "float"
    raise ValueError(f"not a Hy-Nomas DiT checkpoint: no {INT8_FORMAT} code tensors and no {FLOAT_MARKER}")


def config_from_state_dict(state_dict):
    """The model config for a state dict: the released shape with the block depth and the camera flag taken
    from the keys (loader.py:43-48)."""
    depth, camera = _block_layout(state_dict)
    if depth == 0:
        raise ValueError("state dict has no double_blocks.<i> tensors")
    return {**UNET_CONFIG, "mm_double_blocks_depth": depth, "camera": camera}


def quantizable(key, tensor):
    """True for the weights the int8 release stores as code / scale pairs: 2-D Linear weights whose input
    width is a multiple of 128, outside the modules kept in bf16."""
    return (key.endswith(".weight") and tensor.ndim == 2 and tensor.shape[1] % 128 == 0
            and not key.startswith(KEEP_FLOAT))


def quantize_state_dict(state_dict):
    """A float state dict with every quantizable weight replaced by its int8 g128 pair (loader.py:51-62, with
    ops.quantize_g128: the device kernel for GPU tensors, the reference's torch steps for host tensors).
    Other tensors are passed through unchanged."""
    out = {}
    for key, tensor in state_dict.items():
        if quantizable(key, tensor):
            stem = key[: -len("weight")]
            out[stem + CODES_SUFFIX], out[stem + SCALES_SUFFIX] = nomas_ops.quantize_g128(tensor)
        else:
            out[key] = tensor
    return out


def load_state_dict(path, quantize=False):
    """(state_dict, metadata, kind) of a checkpoint file (the reference's load_dit up to the model build):
    a float file is cast to bf16 and, with `quantize`, turned into int8 pairs (kind "int8" then)."""
    from safetensors.torch import load_file

    _, metadata = read_header(path)
    state_dict = load_file(path, device="cpu")
    kind = detect(state_dict, metadata)
    if kind == "float":
        state_dict = {k: v.to(torch.bfloat16) if v.is_floating_point() else v for k, v in state_dict.items()}
        if quantize:
            state_dict, kind = quantize_state_dict(state_dict), "int8"
    return state_dict, metadata, kind


def _linear(state_dict, prefix, device):
    from .block import Int8Linear

    codes, scales = state_dict.get(f"{prefix}.{CODES_SUFFIX}"), state_dict.get(f"{prefix}.{SCALES_SUFFIX}")
    if codes is None or scales is None:
        raise ValueError(f"checkpoint has no int8 weight for {prefix} (quantize a float file first)")
    bias = state_dict.get(prefix + ".bias")
    return Int8Linear(codes.to(device).contiguous(), scales.to(device).float().contiguous(),
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
    """The descriptive entries of a checkpoint's metadata (loader.py:102-106)."""
    metadata = metadata or {}
    return {key: metadata[key] for key in DESCRIPTIVE_KEYS if key in metadata}


def describe_file(path):
    """`info` of a file's metadata as JSON, or "{}" when the file cannot be read as safetensors
    (loader.py:109-115)."""
    try:
        _, metadata = read_header(path)
    except (OSError, ValueError):
        return "{}"
    return json.dumps(info(metadata))
