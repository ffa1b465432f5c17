"""Where the EXL3 modules of a checkpoint are and what shape they have, from the safetensors
headers alone (tensor data is never read here).

A trellis tensor is (k / 16, n / 16, 16 K) 16-bit words, so its header shape gives the module's
input width k, output width n and bitrate K.  Checkpoint tensor names and vLLM module prefixes
spell the same module differently ("model.language_model.layers.3..." against
"model.layers.3..."); both are reduced to one key.  Same behaviour as the reference's
`_norm_key` / `_read_checkpoint_layout` (vllm_plugin/exl3rocm/plugin.py:48-79).
"""
from __future__ import annotations

import glob
import json
import os
import re
import struct

# modules vLLM fuses, and the checkpoint modules they hold, in output-column order (the
# reference plugin's table, plugin.py:38-44: the checkpoint's naming)
FUSED = {
    "gate_up_proj": ["gate_proj", "up_proj"],
    "qkv_proj": ["q_proj", "k_proj", "v_proj"],
    "in_proj_qkvz": ["in_proj_qkv", "in_proj_z"],
    "in_proj_ba": ["in_proj_b", "in_proj_a"],
    "qkv": ["q_proj", "k_proj", "v_proj"],
}
QKV_IDS = {"q": 0, "k": 1, "v": 2}


def norm_key(k: str) -> str:
    """The key of a module name: decoder layers from "layers.<i>" on, the MTP head and the vision
    tower under "mtp." / "visual.", and any other module by its last name component."""
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
    """Three maps over all *.safetensors files of the directory: module key -> (K, k, n) of each
    module that has a trellis, and tensor name -> dtype string / shape for every tensor."""
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
    """The checkpoint modules behind vLLM module `prefix` (its FUSED members in output order, or
    itself) as [(key, K, k, n)]; None when none of them is EXL3, an error when only some are
    (the reference's Exl3Config._groups_for, plugin.py:133-147)."""
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
