"""
vLLM quantization surface for EXL3 weights on MI355X: `Exl3Config` and `Exl3LinearMethod`.

The contract is the reference plugin's (vllm_plugin/exl3rocm/plugin.py:82-372): vLLM calls
`create_weights`, streams checkpoint tensors through the registered parameters' `weight_loader`
(with vLLM's shard ids), then `process_weights_after_loading`, then `apply` per forward.

Storage is per checkpoint tensor ("group"): vLLM fuses sibling projections (qkv_proj, gate_up_proj,
in_proj_qkvz) whose checkpoint tensors may differ in bitrate (the reference checkpoint pairs a 2-bit
q with 5-bit k / v), so each group keeps its own K, trellis, suh and svh, and the fused output is the
concatenation of the groups' outputs, computed inside one opaque `exl3rocm::linear_groups` op.

Design here:
  * a layer's groups are described by their cumulative column offsets; vLLM's output partitions
    are mapped onto groups by bisection over those offsets (a group may span partitions, never the
    reverse);
  * each registered load target carries a `_Router` for one tensor kind, which resolves vLLM's
    shard id to a group and validates shape and dtype before copying;
  * the codebook scalar (`mul1` / `mcg`) is a hard contract: the kernels implement exactly one
    multiplier per codebook, so a checkpoint scalar (or a `quantization_config.json`
    `mul1_multiplier`) naming another one raises instead of decoding wrong weights.

vLLM is optional: when it is importable the config registers itself as quantization "exl3";
without it the same classes work on any torch.nn.Module (what the tests and
`exl3rocm.checkpoint` drive).
"""
from __future__ import annotations

import bisect
import json
import logging
import os
from typing import Any, Optional

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

# The hash multipliers the kernels implement, per codebook (csrc/exl3_device.h Codebook<>): a
# checkpoint scalar selects its codebook and must name exactly this multiplier.
CODEBOOK_MULTIPLIERS = {"mul1": 0x83DCD12D, "mcg": 0xCBAC1FED}
SCALAR_KINDS = tuple(CODEBOOK_MULTIPLIERS)
TENSOR_KINDS = ("trellis", "suh", "svh")


class Exl3FormatError(ValueError):
    """A checkpoint that the kernels cannot decode as stored (wrong codebook multiplier,
    inconsistent bitrate)."""


class Exl3LoadError(AssertionError):
    """A checkpoint tensor that does not fit the layer it is loaded into (shape, shard id, a
    missing tensor, partitions that do not tile the groups).  An AssertionError, the kind vLLM's
    loaders and the reference plugin raise for these, but raised explicitly: it survives
    `python -O`."""


def _as_u32(value) -> int:
    """A multiplier as stored: an integer (signed or unsigned 32-bit, e.g. an int32 tensor's
    item()) or a string in any base int() reads with base 0 ("0x83DCD12D", "2212286765").  How
    a real checkpoint stores it is not fixed by any reference fixture, so every such form is read."""
    if isinstance(value, str):
        try:
            value = int(value.strip(), 0)
        except ValueError as e:
            raise Exl3FormatError(f"exl3rocm: codebook multiplier {value!r} is not an integer") from e
    return int(value) & 0xFFFFFFFF


def check_codebook_scalar(kind: str, value) -> bool:
    """True when `value` (a signed or unsigned 32-bit integer, or its text) is the multiplier the
    kernels implement for codebook `kind`."""
    return _as_u32(value) == CODEBOOK_MULTIPLIERS[kind]


def require_codebook_scalar(kind: str, value, where: str = "") -> int:
    """The scalar as an unsigned 32-bit multiplier; raises Exl3FormatError when it is not the
    kernels' (the reference only checks that the scalar is present, plugin.py:334-335)."""
    v = _as_u32(value)
    if v != CODEBOOK_MULTIPLIERS[kind]:
        raise Exl3FormatError(f"exl3rocm: {where or kind} multiplier {v:#010x} is not the {kind} codebook's "
                              f"{CODEBOOK_MULTIPLIERS[kind]:#010x}; the kernels cannot decode these weights")
    return v


def read_quantization_config(model_dir: str) -> dict:
    """{normalized module: {"bits": int | None, "mul1_multiplier": int | None}} from the
    checkpoint's quantization_config.json `tensor_storage` (the fields the reference's
    tools/build_shape_manifest.py:69-105 reads); {} when the file is absent."""
    path = os.path.join(model_dir, "quantization_config.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        q = json.load(f)
    out = {}
    for name, entry in (q.get("tensor_storage") or {}).items():
        if entry.get("bits_per_weight") is None:
            continue                                   # not an EXL3 module (norms, embeddings)
        out[layout.norm_key(name)] = {"bits": int(entry["bits_per_weight"]),
                                      "mul1_multiplier": entry.get("mul1_multiplier")}
    return out


@register_quantization_config("exl3")
class Exl3Config(QuantizationConfig):
    """Checkpoint-wide EXL3 settings: the codebook and, after maybe_update_config, every EXL3
    module's (K, k, n) from the safetensors headers (validated against quantization_config.json
    where the checkpoint has one)."""

    def __init__(self, codebook: str = "mul1"):
        super().__init__()
        self.codebook = codebook
        self.modules: dict[str, tuple[int, int, int]] = {}
        self.multipliers: dict[str, int] = {}

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
        for key, meta in read_quantization_config(model_name).items():
            K = self.modules.get(key, (None,))[0]
            if K is not None and meta["bits"] is not None and meta["bits"] != K:
                raise Exl3FormatError(f"exl3rocm: {key}: quantization_config.json says {meta['bits']} bits, "
                                      f"its trellis holds {K}")
            if meta["mul1_multiplier"] is not None:
                self.multipliers[key] = require_codebook_scalar("mul1", meta["mul1_multiplier"], key)
        logger.info("exl3rocm: %d EXL3 modules", len(self.modules))

    def _groups_for(self, prefix: str):
        return layout.groups_for(self.modules, prefix, os.environ.get("EXL3_VISION_QKV_BF16") == "1")

    def get_quant_method(self, layer: torch.nn.Module, prefix: str):
        if not isinstance(layer, (LinearBase, ParallelLMHead)):
            return None
        groups = self._groups_for(prefix)
        if groups is not None:
            return Exl3LinearMethod(self, groups)
        return UnquantizedLinearMethod() if isinstance(layer, LinearBase) else None


def _partition_groups(parts: list, widths: list) -> list:
    """Group index of every output partition.  Group boundaries are the cumulative widths; every
    group boundary must also end a partition, and each partition must lie inside one group."""
    ends = [0]
    for w in widths:
        ends.append(ends[-1] + w)
    starts, off = [], 0
    for p in parts:
        starts.append(off)
        off += p
    tiled = off == ends[-1] and all(e in set(starts) | {off} for e in ends)
    if not tiled:
        raise Exl3LoadError(f"exl3rocm: output partitions {parts} do not tile the checkpoint groups {widths}")
    return [bisect.bisect_right(ends, s) - 1 for s in starts]


def _shard_partitions(shard_id) -> tuple:
    """vLLM's shard id as the output partitions it names: "q" / "k" / "v", one partition index,
    or a tuple of them (a checkpoint tensor covering several partitions)."""
    if isinstance(shard_id, str):
        return (QKV_IDS[shard_id],)
    if isinstance(shard_id, int):
        return (shard_id,)
    return tuple(shard_id)


def _shard_group(layer, shard_id) -> int:
    """The group a checkpoint tensor fills.  Without a shard id the module must have a single
    group; otherwise every partition the id names must map to the same group."""
    if shard_id is None:
        if len(layer.exl3_n) != 1:
            raise Exl3LoadError(f"exl3rocm: a tensor with no shard id cannot choose among "
                                f"{len(layer.exl3_n)} groups of a fused module")
        return 0
    parts = _shard_partitions(shard_id)
    targets = sorted({layer.exl3_part_to_group[p] for p in parts})
    if len(targets) != 1:
        raise Exl3LoadError(f"exl3rocm: shard id {shard_id!r} names partitions {list(parts)} of groups "
                            f"{targets}; a checkpoint tensor fills exactly one group")
    return targets[0]


class _Router:
    """weight_loader of one load target: routes a checkpoint tensor of kind `kind` into its
    group's buffer (or records the codebook scalar)."""

    def __init__(self, layer, kind: str, expected_multiplier: Optional[int]):
        self.layer = layer
        self.kind = kind
        self.expected = expected_multiplier

    def __call__(self, param, w, shard_id=None, *args, **kwargs):
        layer = self.layer
        g = _shard_group(layer, getattr(w, "exl3_shard", None) if shard_id is None else shard_id)
        if self.kind in SCALAR_KINDS:
            v = require_codebook_scalar(self.kind, int(w.item()), f"{self.kind} of group {g}")
            if self.expected is not None and v != self.expected:
                raise Exl3FormatError(f"exl3rocm: {self.kind} scalar {v:#010x} differs from the checkpoint's "
                                      f"quantization_config {self.expected:#010x}")
            seen = getattr(layer, f"exl3_{self.kind}")
            if seen is not None and seen != v:
                raise Exl3LoadError(f"exl3rocm: group {g} names {self.kind} {v:#010x}, an earlier group "
                                    f"{seen:#010x}")
            setattr(layer, f"exl3_{self.kind}", v)
        else:
            dst = getattr(layer, f"exl3_{self.kind}_{g}")
            if tuple(w.shape) != tuple(dst.shape):
                raise Exl3LoadError(f"exl3rocm: group {g} holds a {self.kind} of shape {tuple(dst.shape)}; "
                                    f"the checkpoint tensor is {tuple(w.shape)}")
            dst.copy_(w)
        layer.exl3_loaded.add((self.kind, g))


class Exl3LinearMethod(LinearMethodBase):
    """EXL3 linear over per-group buffers `exl3_{trellis,suh,svh}_{i}` (non-persistent).  The
    registered Parameters `trellis`, `suh`, `svh` and the codebook scalar are 0-size load targets
    whose weight_loader fills those buffers."""

    def __init__(self, config: Exl3Config, groups):
        self.config = config
        self.groups = groups  # [(member_key, K, k, n)]

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size,
                       output_size, params_dtype, **extra_weight_attrs):
        k = input_size_per_partition
        if k != input_size:
            raise NotImplementedError("exl3rocm: tensor parallelism is not supported")
        keys = [g[0] for g in self.groups]
        Ks = [g[1] for g in self.groups]
        widths = [g[3] for g in self.groups]
        for key, gk in zip(keys, (g[2] for g in self.groups)):
            if gk != k:
                raise Exl3LoadError(f"exl3rocm: checkpoint tensor {key} has {gk} inputs, the layer {k}")
        layer.exl3_part_to_group = _partition_groups(list(output_partition_sizes), widths)
        layer.exl3_K, layer.exl3_n = Ks, widths
        for i, (K, n) in enumerate(zip(Ks, widths)):
            shapes = {"trellis": ((k // 16, n // 16, 16 * K), torch.int16), "suh": ((k,), torch.float16),
                      "svh": ((n,), torch.float16)}
            for kind, (shape, dt) in shapes.items():
                layer.register_buffer(f"exl3_{kind}_{i}", torch.empty(shape, dtype=dt), persistent=False)
        layer.exl3_loaded = set()
        layer.exl3_mul1 = layer.exl3_mcg = None
        # the checkpoint's quantization_config multiplier, when every group names the same one
        known = {self.config.multipliers.get(key) for key in keys}
        expected = known.pop() if len(known) == 1 else None
        # load targets: the tensor kinds, and only the codebook scalar the checkpoint stores
        # (vLLM rejects registered parameters that are never loaded)
        kinds = TENSOR_KINDS + ((self.config.codebook,) if self.config.codebook in SCALAR_KINDS else ())
        for kind in kinds:
            target = Parameter(torch.empty(0, dtype=torch.int8), requires_grad=False)
            target.weight_loader = _Router(layer, kind, expected if kind == "mul1" else None)
            layer.register_parameter(kind, target)

    @staticmethod
    def _group_of(layer, shard_id) -> int:
        return _shard_group(layer, shard_id)

    def process_weights_after_loading(self, layer):
        ng = len(layer.exl3_n)
        missing = sorted({(kind, g) for kind in TENSOR_KINDS for g in range(ng)} - layer.exl3_loaded)
        if missing:
            raise Exl3LoadError(f"exl3rocm: never loaded, as (kind, group): {missing} (missing tensors)")
        layer.exl3_is_mul1 = layer.exl3_mul1 is not None
        layer.exl3_is_mcg = layer.exl3_mcg is not None
        dev = layer.exl3_trellis_0.device
        if dev.type == "cuda":
            # every buffer the forward uses is reserved now, so graph capture never allocates
            from . import ops
            k = layer.exl3_trellis_0.shape[0] * 16
            for K, n in zip(layer.exl3_K, layer.exl3_n):
                ops.reserve_workspace(dev, k, n, K, groups=min(ng, 4))
            # the prefill's split workspace: one size serves every shape (each further stream
            # allocates it on its first eager prefill call)
            ops.E.reserve_prefill_workspace(dev)
            if ops.PREFILL_ROUTE == "recon":
                ops.reserve_weight_buffer(dev, k * min(max(layer.exl3_n), ops.RECON_SLICE_N))
        # equal-K, equal-width groups (gate/up) take the pointer-table launch at M == 1
        layer.exl3_mgemm_ptrs = None
        same_shape = len(set(layer.exl3_K)) == 1 and len(set(layer.exl3_n)) == 1
        if 1 < ng <= 4 and same_shape and os.environ.get("EXL3_MGEMM", "1") != "0":
            tables = []
            for kind in TENSOR_KINDS:
                t = torch.tensor([getattr(layer, f"exl3_{kind}_{i}").data_ptr() for i in range(ng)],
                                 dtype=torch.long, device=dev)
                layer.register_buffer(f"exl3_ptrs_{kind}", t, persistent=False)
                tables.append(t)
            layer.exl3_mgemm_ptrs = tables
        # the 0-size load targets are done: nothing downstream should take them for weights
        for name in TENSOR_KINDS + SCALAR_KINDS:
            layer._parameters.pop(name, None)

    def apply(self, layer, x, bias=None):
        from . import ops  # noqa: F401  (registers the custom ops)
        ng = len(layer.exl3_n)
        per = [[getattr(layer, f"exl3_{kind}_{i}") for i in range(ng)] for kind in TENSOR_KINDS]
        # one opaque op per module: the groups' outputs are concatenated inside it
        y = torch.ops.exl3rocm.linear_groups(x, *per, list(layer.exl3_K), layer.exl3_is_mcg, layer.exl3_is_mul1,
                                             *(layer.exl3_mgemm_ptrs or (None, None, None)))
        y = y if y.dtype == x.dtype else y.to(x.dtype)
        return y if bias is None else y + bias

    def apply_silu_mul(self, layer, gate_up, bias=None):
        """The layer's linear of act = fp16(fp16(silu(gate)) * up), gate_up = [gate | up] (the
        [*, 2k] output of the MLP's gate/up module): what `apply(layer, act_fn(gate_up))` gives with
        vLLM's SiluAndMul, bitwise, as one op (exl3rocm::silu_mul_linear: the GEMV or the
        prefill's input transform forms act as it loads, so act is never written).  No counterpart
        in the reference plugin, whose MLP runs SiluAndMul and then the down linear.  For MLP code
        that owns both steps; the layer holds one group (a down projection).  Like `apply`, this
        is the local product only: a row-parallel caller still reduces across ranks."""
        from . import ops  # noqa: F401  (registers the custom ops)
        if len(layer.exl3_n) != 1:
            raise ValueError(f"exl3rocm: apply_silu_mul takes a layer of one group, got {len(layer.exl3_n)}")
        k = layer.exl3_suh_0.shape[0]
        if gate_up.shape[-1] != 2 * k:
            raise ValueError(f"exl3rocm: apply_silu_mul takes [gate | up] of 2 x {k} columns, got {gate_up.shape[-1]}")
        gu = gate_up if gate_up.dtype == torch.float16 else gate_up.to(torch.float16)
        y = torch.ops.exl3rocm.silu_mul_linear(gu, layer.exl3_trellis_0, layer.exl3_suh_0, layer.exl3_svh_0,
                                                layer.exl3_K[0], layer.exl3_is_mcg, layer.exl3_is_mul1)
        y = y if y.dtype == gate_up.dtype else y.to(gate_up.dtype)
        return y if bias is None else y + bias

    def embedding(self, layer, input_):
        raise NotImplementedError("exl3rocm: quantized input embeddings are not supported")


def register():
    """vLLM general-plugin entry point: importing registers the config and the custom ops."""
    from . import ops  # noqa: F401
    return None
