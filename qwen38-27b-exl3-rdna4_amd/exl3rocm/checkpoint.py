"""Load EXL3 linear modules straight from a local checkpoint directory, without vLLM.

vLLM drives Exl3LinearMethod through its own weight iterator; this module does the same for one
(possibly fused) module: it finds the module's checkpoint tensors from the safetensors headers,
reads their data with the safetensors loader (no pickle), routes every tensor through the
registered load targets with the shard ids vLLM would pass, and finishes with
process_weights_after_loading.  Used by tests and benchmarks that start from files, and by any
caller that wants one EXL3 layer outside a vLLM model.
"""
from __future__ import annotations

import glob
import os

import torch

from . import layout, plugin


def tensor_index(model_dir: str) -> dict:
    """{normalized module: {tensor kind: (file, full tensor name)}} over every *.safetensors file;
    kinds are the suffixes after the module name (trellis, suh, svh, mul1, mcg, bias, ...)."""
    out: dict = {}
    for f in sorted(glob.glob(os.path.join(model_dir, "*.safetensors"))):
        for name in layout.read_header(f):
            if name == "__metadata__" or "." not in name:
                continue
            module, kind = name.rsplit(".", 1)
            out.setdefault(layout.norm_key(module), {})[kind] = (f, name)
    return out


def _read(path: str, name: str) -> torch.Tensor:
    from safetensors import safe_open
    with safe_open(path, framework="pt") as fh:
        return fh.get_tensor(name)


def load_linear(model_dir: str, prefix: str, device="cuda", codebook: str = "mul1", config=None):
    """(Exl3LinearMethod, layer) for the EXL3 module at vLLM prefix `prefix` (e.g.
    "model.layers.0.self_attn.qkv_proj"), its buffers filled from the checkpoint on `device`.
    Raises KeyError when the prefix is not an EXL3 module, plugin.Exl3FormatError for a
    checkpoint the kernels cannot decode."""
    cfg = config
    if cfg is None:
        cfg = plugin.Exl3Config(codebook)
        cfg.maybe_update_config(model_dir)
    groups = cfg._groups_for(prefix)
    if groups is None:
        raise KeyError(f"exl3rocm: {prefix} is not an EXL3 module of {model_dir}")
    method = plugin.Exl3LinearMethod(cfg, groups)
    layer = torch.nn.Module()
    k = groups[0][2]
    widths = [g[3] for g in groups]
    method.create_weights(layer, k, widths, k, sum(widths), torch.float16)
    layer.to(device)
    index = tensor_index(model_dir)
    kinds = plugin.TENSOR_KINDS + ((cfg.codebook,) if cfg.codebook in plugin.SCALAR_KINDS else ())
    for gi, (key, *_rest) in enumerate(groups):
        tensors = index.get(key, {})
        # vLLM's shard id for this group: the output partitions it covers (one partition per group here)
        shard = None if len(groups) == 1 else gi
        for kind in kinds:
            if kind not in tensors:
                continue              # a missing trellis / suh / svh is reported by process_weights_after_loading
            path, name = tensors[kind]
            target = getattr(layer, kind)
            target.weight_loader(target, _read(path, name), shard)
    method.process_weights_after_loading(layer)
    return method, layer
