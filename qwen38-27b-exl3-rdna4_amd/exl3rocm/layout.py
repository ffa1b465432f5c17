"""Checkpoint layout discovery from safetensors headers (no tensor data is read).

Restates the reference's `_norm_key` and `_read_checkpoint_layout`
(vllm_plugin/exl3rocm/plugin.py:48-79): for every `<module>.trellis` tensor the EXL3 bitrate
K = shape[-1] // 16 and the layer shape k = shape[0] * 16, n = shape[1] * 16 are recorded
under a normalized module name shared by checkpoint keys and vLLM prefixes.
"""
from __future__ import annotations

import glob
import json
import os
import re
import struct

# vLLM fused module -> checkpoint constituents, in output order (reference plugin.py:38-44)
FUSED = {
    "gate_up_proj": ["gate_proj", "up_proj"],
    "qkv_proj": ["q_proj", "k_proj", "v_proj"],
    "in_proj_qkvz": ["in_proj_qkv", "in_proj_z"],
    "in_proj_ba": ["in_proj_b", "in_proj_a"],
    "qkv": ["q_proj", "k_proj", "v_proj"],
}
QKV_IDS = {"q": 0, "k": 1, "v": 2}


def norm_key(k: str) -> str:
    """'model.language_model.layers.3.mlp.gate_proj' -> 'layers.3.mlp.gate_proj';
    '...mtp.layers.0.x' -> 'mtp.layers.0.x'; '...visual.blocks.0.y' -> 'visual.blocks.0.y';
    anything else -> its last component (e.g. 'lm_head')."""
    parts = k.split(".")
    if "visual" in parts:
        return "visual." + ".".join(parts[parts.index("visual") + 1:])
    if "mtp" in parts:
        return "mtp." + ".".join(parts[parts.index("mtp") + 1:])
    m = re.search(r"(layers\.\d+\..*)$", k)
    if m:
        return m.group(1)
    return parts[-1]


def read_header(path: str) -> dict:
    """JSON header of one safetensors file (8-byte little-endian length, then JSON)."""
    with open(path, "rb") as fh:
        raw = fh.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: truncated safetensors header")
        n = struct.unpack("<Q", raw)[0]
        return json.loads(fh.read(n))


def read_checkpoint_layout(model_dir: str):
    """({normalized module: (K, k, n)} for every '<module>.trellis' tensor,
        {tensor name: dtype string}, {tensor name: shape}) over every *.safetensors file."""
    out, dtypes, shapes = {}, {}, {}
    for f in sorted(glob.glob(os.path.join(model_dir, "*.safetensors"))):
        for name, v in read_header(f).items():
            if name == "__metadata__":
                continue
            dtypes[name] = v["dtype"]
            shapes[name] = tuple(v["shape"])
            if name.endswith(".trellis"):
                s = v["shape"]
                out[norm_key(name[: -len(".trellis")])] = (s[-1] // 16, s[0] * 16, s[1] * 16)
    return out, dtypes, shapes


def groups_for(modules: dict, prefix: str, vision_qkv_bf16: bool = False):
    """Checkpoint members of the (possibly fused) module at `prefix` as [(member, K, k, n)], or
    None when the module is not EXL3 (reference plugin.py:133-147)."""
    key = norm_key(prefix)
    if key.endswith(".attn.qkv") and key.startswith("visual.") and vision_qkv_bf16:
        return None
    base, _, leaf = key.rpartition(".")
    members = [f"{base}.{p}" if base else p for p in FUSED.get(leaf, [leaf])]
    found = [modules.get(m) for m in members]
    if all(f is None for f in found):
        return None
    if not all(f is not None for f in found):
        raise AssertionError(f"exl3rocm: partially quantized fused module {prefix}")
    return [(m, *f) for m, f in zip(members, found)]
