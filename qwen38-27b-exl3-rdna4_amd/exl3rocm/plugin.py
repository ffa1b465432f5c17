"""
vLLM quantization plugin surface for EXL3 weights on MI355X: `Exl3Config` and
`Exl3LinearMethod` with the reference's create_weights / weight loading /
process_weights_after_loading / apply contract (vllm_plugin/exl3rocm/plugin.py:82-372).

Weights are kept per checkpoint tensor ("group") with that group's own K, trellis, suh and svh,
because vLLM fuses sibling projections (qkv, gate/up) whose checkpoint tensors may differ in
bitrate; the fused output is the concatenation of per-group results, computed inside the
opaque `exl3rocm::linear_groups` op.

vLLM is optional: when it is importable the config registers itself as quantization "exl3";
without it the same classes work on any torch.nn.Module (what the tests drive).
"""
from __future__ import annotations

import logging
import os
from typing import Any

import torch
from torch.nn import Parameter

from . import layout
from .layout import FUSED, QKV_IDS  # noqa: F401  (re-exported names of the reference module)

try:  # pragma: no cover - exercised only where vLLM is installed
    from vllm.logger import init_logger
    from vllm.model_executor.layers.linear import LinearBase, LinearMethodBase, UnquantizedLinearMethod
    from vllm.model_executor.layers.quantization import register_quantization_config
    from vllm.model_executor.layers.quantization.base_config import QuantizationConfig
    from vllm.model_executor.layers.vocab_parallel_embedding import ParallelLMHead
    HAVE_VLLM = True
    logger = init_logger("vllm.exl3rocm")
except Exception:  # vLLM absent: plain stand-ins with the same roles
    HAVE_VLLM = False
    logger = logging.getLogger("vllm.exl3rocm")

    class LinearBase(torch.nn.Module):
        pass

    class ParallelLMHead(torch.nn.Module):
        pass

    class LinearMethodBase:
        pass

    class UnquantizedLinearMethod(LinearMethodBase):
        pass

    class QuantizationConfig:
        def __init__(self):
            pass

    def register_quantization_config(name):
        def deco(cls):
            return cls
        return deco

# mul1 / mcg multipliers the kernels implement (codebook hash constants)
CODEBOOK_MULTIPLIERS = {"mul1": 0x83DCD12D, "mcg": 0xCBAC1FED}


def check_codebook_scalar(kind: str, value: int) -> bool:
    """True when a checkpoint's `mul1` / `mcg` scalar names the multiplier the kernels use (as an
    unsigned or signed 32-bit integer).  The reference only checks presence (plugin.py:334-335);
    a mismatch is logged, and the scalar's presence still selects the codebook."""
    want = CODEBOOK_MULTIPLIERS[kind]
    ok = (int(value) & 0xFFFFFFFF) == want
    if not ok:
        logger.warning("exl3rocm: checkpoint %s scalar %#x differs from the kernel multiplier %#x",
                       kind, int(value) & 0xFFFFFFFF, want)
    return ok


@register_quantization_config("exl3")
class Exl3Config(QuantizationConfig):

    def __init__(self, codebook: str = "mul1"):
        super().__init__()
        self.codebook = codebook
        self.modules: dict[str, tuple[int, int, int]] = {}

    def __repr__(self):
        return f"Exl3Config(codebook={self.codebook}, modules={len(self.modules)})"

    def get_name(self):
        return "exl3"

    def get_supported_act_dtypes(self):
        return [torch.float16]

    @classmethod
    def get_min_capability(cls) -> int:
        return 0

    @staticmethod
    def get_config_filenames() -> list[str]:
        return []

    @classmethod
    def from_config(cls, config: dict[str, Any]) -> "Exl3Config":
        return cls(codebook=config.get("codebook", "mul1"))

    def maybe_update_config(self, model_name: str, hf_config=None, revision=None):
        if not os.path.isdir(model_name):
            raise NotImplementedError("exl3rocm: pass a local checkpoint directory")
        self.modules, _, _ = layout.read_checkpoint_layout(model_name)
        logger.info("exl3rocm: %d EXL3 modules", len(self.modules))

    def _groups_for(self, prefix: str):
        return layout.groups_for(self.modules, prefix, os.environ.get("EXL3_VISION_QKV_BF16") == "1")

    def get_quant_method(self, layer: torch.nn.Module, prefix: str):
        if isinstance(layer, (LinearBase, ParallelLMHead)):
            groups = self._groups_for(prefix)
            if groups is None:
                return UnquantizedLinearMethod() if isinstance(layer, LinearBase) else None
            return Exl3LinearMethod(self, groups)
        return None


class Exl3LinearMethod(LinearMethodBase):
    """Per-group EXL3 storage.  The registered Parameters `trellis`, `suh`, `svh`, `mul1`|`mcg`
    are 0-size load targets; their weight_loader routes each checkpoint tensor into that group's
    non-persistent buffers."""

    def __init__(self, config: Exl3Config, groups):
        self.config = config
        self.groups = groups  # [(member_key, K, k, n)]

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size,
                       output_size, params_dtype, **extra_weight_attrs):
        k = input_size_per_partition
        if k != input_size:
            raise NotImplementedError("exl3rocm: tensor parallelism is not supported")
        parts = list(output_partition_sizes)
        # map output partitions onto checkpoint groups (a group may span partitions)
        group_n = [g[3] for g in self.groups]
        part_to_group, gi, acc = [], 0, 0
        for p in parts:
            assert gi < len(group_n), f"exl3rocm: partitions {parts} do not tile groups {group_n}"
            part_to_group.append(gi)
            acc += p
            assert acc <= group_n[gi], f"exl3rocm: partitions {parts} do not tile groups {group_n}"
            if acc == group_n[gi]:
                gi, acc = gi + 1, 0
        assert gi == len(group_n), f"exl3rocm: partitions {parts} do not tile groups {group_n}"
        layer.exl3_part_to_group = part_to_group
        layer.exl3_K = [g[1] for g in self.groups]
        layer.exl3_n = [g[3] for g in self.groups]
        for i, (_, K, gk, n) in enumerate(self.groups):
            assert gk == k, f"exl3rocm: {self.groups[i][0]} k={gk} vs layer k={k}"
            layer.register_buffer(f"exl3_trellis_{i}", torch.empty((k // 16, n // 16, 16 * K), dtype=torch.int16),
                                  persistent=False)
            layer.register_buffer(f"exl3_suh_{i}", torch.empty((k,), dtype=torch.float16), persistent=False)
            layer.register_buffer(f"exl3_svh_{i}", torch.empty((n,), dtype=torch.float16), persistent=False)
        layer.exl3_loaded = set()
        layer.exl3_mul1 = None
        layer.exl3_mcg = None

        def reg(name, loader):
            p = Parameter(torch.empty(0, dtype=torch.int8), requires_grad=False)
            p.weight_loader = loader
            layer.register_parameter(name, p)

        reg("trellis", self._loader(layer, "trellis"))
        reg("suh", self._loader(layer, "suh"))
        reg("svh", self._loader(layer, "svh"))
        if self.config.codebook in ("mul1", "mcg"):
            reg(self.config.codebook, self._loader(layer, self.config.codebook))

    @staticmethod
    def _group_of(layer, shard_id) -> int:
        if shard_id is None:
            assert len(layer.exl3_n) == 1, "exl3rocm: unsharded load into fused module"
            return 0
        if isinstance(shard_id, str):
            parts = [QKV_IDS[shard_id]]
        elif isinstance(shard_id, int):
            parts = [shard_id]
        else:
            parts = list(shard_id)
        gs = {layer.exl3_part_to_group[p] for p in parts}
        assert len(gs) == 1, f"exl3rocm: shard {shard_id} spans groups {gs}"
        return gs.pop()

    def _loader(self, layer, kind):
        def load(param, w, shard_id=None, *args, **kwargs):
            if shard_id is None:
                shard_id = getattr(w, "exl3_shard", None)
            g = self._group_of(layer, shard_id)
            if kind in ("mul1", "mcg"):
                val = int(w.item())
                prev = getattr(layer, f"exl3_{kind}")
                assert prev is None or prev == val, f"exl3rocm: {kind} differs across groups"
                setattr(layer, f"exl3_{kind}", val)
            else:
                buf = getattr(layer, f"exl3_{kind}_{g}")
                assert tuple(w.shape) == tuple(buf.shape), \
                    f"exl3rocm: {kind} shape {tuple(w.shape)} vs {tuple(buf.shape)} (group {g})"
                buf.copy_(w)
            layer.exl3_loaded.add((kind, g))
        return load

    def process_weights_after_loading(self, layer):
        ng = len(layer.exl3_n)
        missing = [(k, g) for k in ("trellis", "suh", "svh") for g in range(ng) if (k, g) not in layer.exl3_loaded]
        assert not missing, f"exl3rocm: missing tensors {missing}"
        layer.exl3_is_mul1 = layer.exl3_mul1 is not None
        layer.exl3_is_mcg = layer.exl3_mcg is not None
        for kind in ("mul1", "mcg"):
            if getattr(layer, f"exl3_{kind}") is not None:
                check_codebook_scalar(kind, getattr(layer, f"exl3_{kind}"))
        k = layer.exl3_trellis_0.shape[0] * 16
        dev = layer.exl3_trellis_0.device
        if dev.type == "cuda":
            # reserve everything the forward needs now, so graph capture never allocates
            from . import ops
            for K, n in zip(layer.exl3_K, layer.exl3_n):
                ops.reserve_workspace(dev, k, n, K, groups=min(ng, 4))
            if ops.PREFILL_ROUTE == "recon":
                ops.reserve_weight_buffer(dev, max(k * min(n, ops.RECON_SLICE_N) for n in layer.exl3_n))
        # grouped M == 1 path over pointer tables for modules whose groups share K and width
        layer.exl3_mgemm_ptrs = None
        if 1 < ng <= 4 and len(set(layer.exl3_K)) == 1 and len(set(layer.exl3_n)) == 1 \
                and os.environ.get("EXL3_MGEMM", "1") != "0":
            def ptrs(kind):
                t = torch.tensor([getattr(layer, f"exl3_{kind}_{i}").data_ptr() for i in range(ng)],
                                 dtype=torch.long, device=dev)
                layer.register_buffer(f"exl3_ptrs_{kind}", t, persistent=False)
                return t
            layer.exl3_mgemm_ptrs = [ptrs("trellis"), ptrs("suh"), ptrs("svh")]
        # drop the 0-size load targets so nothing downstream mistakes them for weights
        for name in ("trellis", "suh", "svh", "mul1", "mcg"):
            if name in layer._parameters:
                del layer._parameters[name]

    def apply(self, layer, x, bias=None):
        from . import ops  # noqa: F401  (registers the custom ops)
        ng = len(layer.exl3_n)
        # one opaque op per module: never concatenate per-group outputs in traced code
        y = torch.ops.exl3rocm.linear_groups(
            x,
            [getattr(layer, f"exl3_trellis_{i}") for i in range(ng)],
            [getattr(layer, f"exl3_suh_{i}") for i in range(ng)],
            [getattr(layer, f"exl3_svh_{i}") for i in range(ng)],
            list(layer.exl3_K), layer.exl3_is_mcg, layer.exl3_is_mul1,
            *(layer.exl3_mgemm_ptrs or (None, None, None)))
        if y.dtype != x.dtype:
            y = y.to(x.dtype)
        if bias is not None:
            y = y + bias
        return y

    def embedding(self, layer, input_):
        raise NotImplementedError("exl3rocm: quantized input embeddings are not supported")


def register():
    """vLLM general-plugin entry point: importing registers the config and the custom ops."""
    from . import ops  # noqa: F401
    return None
