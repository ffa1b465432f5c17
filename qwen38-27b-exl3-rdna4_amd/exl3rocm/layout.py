"""Where the EXL3 modules of a checkpoint are and what shape they have, from the safetensors
headers alone (tensor data is never read here).

A trellis tensor is (k / 16, n / 16, 16 K) 16-bit words, so its header shape gives the module's
input width k, output width n and bitrate K.  Checkpoint tensor names and vLLM module prefixes
spell the same module differently ("model.language_model.layers.3..." against
"model.layers.3..."); both reduce to one key.  The keys and maps are the reference's
(`_norm_key` / `_read_checkpoint_layout`, vllm_plugin/exl3rocm/plugin.py:48-79): the checkpoint
format and vLLM's module naming fix them.
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


# sub-trees whose modules are keyed from their own root ("<anchor>.<rest>"), checked in this order
SUBTREE_ROOTS = ("visual", "mtp")


def norm_key(name: str) -> str:
    """The key of a module name: inside the vision tower or the MTP head, the path below that
    root prefixed with the root's name; inside the decoder stack, the path from "layers.<i>" on;
    anything else (lm_head, embeddings) by its last component."""
    parts = name.split(".")
    for root in SUBTREE_ROOTS:
        if root in parts:
            return ".".join([root] + parts[parts.index(root) + 1:])
    for i in range(len(parts) - 2):
        if parts[i] == "layers" and parts[i + 1].isdigit():
            return ".".join(parts[i:])
    return parts[-1]


def read_header(path: str) -> dict:
    """JSON header of one safetensors file (8-byte little-endian length, then JSON)."""
    with open(path, "rb") as fh:
        raw = fh.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: truncated safetensors header")
        n = struct.unpack("<Q", raw)[0]
        return json.loads(fh.read(n))


def _tensor_entries(model_dir: str):
    """(name, header entry) of every tensor in the directory's *.safetensors files, files in name order."""
    for path in sorted(glob.glob(os.path.join(model_dir, "*.safetensors"))):
        yield from ((name, v) for name, v in read_header(path).items() if name != "__metadata__")


def trellis_dims(shape) -> tuple:
    """(K, k, n) of a trellis tensor of shape (k / 16, n / 16, 16 K)."""
    kt, nt, words = shape[0], shape[1], shape[-1]
    return words // 16, kt * 16, nt * 16


def read_checkpoint_layout(model_dir: str):
    """Three maps over all *.safetensors files of the directory: module key -> (K, k, n) of each
    module that has a trellis, and tensor name -> dtype string / shape for every tensor."""
    modules, dtypes, shapes = {}, {}, {}
    suffix = ".trellis"
    for name, entry in _tensor_entries(model_dir):
        dtypes[name], shapes[name] = entry["dtype"], tuple(entry["shape"])
        if name.endswith(suffix):
            modules[norm_key(name[:-len(suffix)])] = trellis_dims(entry["shape"])
    return modules, dtypes, shapes


def groups_for(modules: dict, prefix: str, vision_qkv_bf16: bool = False):
    """The checkpoint modules behind vLLM module `prefix` (its FUSED members in output order, or
    the module itself) as [(key, K, k, n)]; None when none of them is EXL3, an error when only
    some are (the reference's Exl3Config._groups_for, plugin.py:133-147).  vision_qkv_bf16: the
    vision tower's attention q/k/v stays unquantized."""
    key = norm_key(prefix)
    if vision_qkv_bf16 and key.startswith("visual.") and key.endswith(".attn.qkv"):
        return None
    parent, _, leaf = key.rpartition(".")
    names = [".".join(filter(None, (parent, member))) for member in FUSED.get(leaf, [leaf])]
    dims = {nm: modules[nm] for nm in names if nm in modules}
    if not dims:
        return None
    if len(dims) != len(names):
        absent = [nm for nm in names if nm not in dims]
        raise AssertionError(f"exl3rocm: fused module {prefix}: {absent} have no trellis, the rest do")
    return [(nm, *dims[nm]) for nm in names]
