"""CPU tests of the host-side surface: checkpoint layout discovery, the linear-method weight
loading contract, and the custom ops' fake (meta) implementations."""
import json
import os
import struct

import numpy as np
import pytest
import torch

from exl3rocm import layout, plugin
from exl3rocm import ops  # noqa: F401  (registers torch.ops.exl3rocm.*)


def write_safetensors_header(path, tensors: dict):
    """A header-only safetensors file (the layout reader never touches tensor data)."""
    header, off = {}, 0
    for name, (dtype, shape) in tensors.items():
        nbytes = int(np.prod(shape)) * {"I16": 2, "F16": 2, "I32": 4, "F8_E4M3": 1}[dtype]
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + nbytes]}
        off += nbytes
    blob = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(blob)))
        f.write(blob)


@pytest.fixture
def checkpoint(tmp_path):
    pre = "model.language_model.layers.0"
    t = {
        f"{pre}.mlp.gate_proj.trellis": ("I16", (320, 1088, 64)),
        f"{pre}.mlp.up_proj.trellis": ("I16", (320, 1088, 64)),
        f"{pre}.mlp.down_proj.trellis": ("I16", (1088, 320, 48)),
        f"{pre}.self_attn.q_proj.trellis": ("I16", (320, 320, 32)),
        f"{pre}.self_attn.k_proj.trellis": ("I16", (320, 64, 80)),
        f"{pre}.self_attn.v_proj.trellis": ("I16", (320, 64, 80)),
        f"{pre}.mlp.gate_proj.suh": ("F16", (5120,)),
        "model.language_model.embed_tokens.weight": ("F8_E4M3", (1000, 5120)),
        "lm_head.trellis": ("I16", (320, 100, 64)),
    }
    write_safetensors_header(str(tmp_path / "model-00001.safetensors"), t)
    return str(tmp_path)


def test_norm_key():
    assert layout.norm_key("model.language_model.layers.3.mlp.gate_proj") == "layers.3.mlp.gate_proj"
    assert layout.norm_key("language_model.model.layers.3.mlp.gate_proj") == "layers.3.mlp.gate_proj"
    assert layout.norm_key("model.mtp.layers.0.x") == "mtp.layers.0.x"
    assert layout.norm_key("model.visual.blocks.0.mlp.linear_fc1") == "visual.blocks.0.mlp.linear_fc1"
    assert layout.norm_key("lm_head") == "lm_head"


def test_checkpoint_layout(checkpoint):
    mods, dtypes, shapes = layout.read_checkpoint_layout(checkpoint)
    assert mods["layers.0.mlp.gate_proj"] == (4, 5120, 17408)
    assert mods["layers.0.mlp.down_proj"] == (3, 17408, 5120)
    assert mods["layers.0.self_attn.k_proj"] == (5, 5120, 1024)
    assert mods["lm_head"] == (4, 5120, 1600)
    assert dtypes["model.language_model.embed_tokens.weight"] == "F8_E4M3"
    assert shapes["model.language_model.layers.0.mlp.gate_proj.suh"] == (5120,)


def test_groups_for_fused_modules(checkpoint):
    mods, _, _ = layout.read_checkpoint_layout(checkpoint)
    g = layout.groups_for(mods, "model.layers.0.mlp.gate_up_proj")
    assert [m for m, *_ in g] == ["layers.0.mlp.gate_proj", "layers.0.mlp.up_proj"]
    qkv = layout.groups_for(mods, "model.layers.0.self_attn.qkv_proj")
    assert [x[1] for x in qkv] == [2, 5, 5]
    assert layout.groups_for(mods, "model.layers.0.self_attn.o_proj") is None
    with pytest.raises(AssertionError):
        layout.groups_for({"layers.0.mlp.gate_proj": (4, 128, 128)}, "model.layers.0.mlp.gate_up_proj")


def test_config_surface(checkpoint):
    cfg = plugin.Exl3Config.from_config({"codebook": "mcg"})
    assert cfg.get_name() == "exl3" and cfg.codebook == "mcg"
    assert cfg.get_supported_act_dtypes() == [torch.float16]
    cfg.maybe_update_config(checkpoint)
    assert len(cfg.modules) == 7
    with pytest.raises(NotImplementedError):
        cfg.maybe_update_config(os.path.join(checkpoint, "missing"))
    layer = plugin.LinearBase()
    m = cfg.get_quant_method(layer, "model.layers.0.mlp.gate_up_proj")
    assert isinstance(m, plugin.Exl3LinearMethod) and len(m.groups) == 2
    assert isinstance(cfg.get_quant_method(layer, "model.layers.0.self_attn.o_proj"), plugin.UnquantizedLinearMethod)


def make_layer(groups, codebook="mul1"):
    cfg = plugin.Exl3Config(codebook)
    method = plugin.Exl3LinearMethod(cfg, groups)
    layer = torch.nn.Module()
    k = groups[0][2]
    method.create_weights(layer, k, [g[3] for g in groups], k, sum(g[3] for g in groups), torch.float16)
    return method, layer


def test_create_weights_and_loading():
    groups = [("q", 2, 256, 256), ("k", 5, 256, 128), ("v", 5, 256, 128)]
    method, layer = make_layer(groups)
    assert layer.exl3_K == [2, 5, 5] and layer.exl3_n == [256, 128, 128]
    assert tuple(layer.exl3_trellis_1.shape) == (16, 8, 80) and layer.exl3_trellis_1.dtype == torch.int16
    assert "exl3_trellis_0" not in layer.state_dict()            # non-persistent buffers
    for name in ("trellis", "suh", "svh", "mul1"):
        assert layer._parameters[name].numel() == 0
    rng = np.random.default_rng(0)
    for sid, (_, K, k, n) in zip("qkv", groups):
        tr = torch.from_numpy(rng.integers(-32768, 32767, (k // 16, n // 16, 16 * K), dtype=np.int16))
        layer.trellis.weight_loader(layer.trellis, tr, sid)
        layer.suh.weight_loader(layer.suh, torch.ones(k, dtype=torch.float16), sid)
        layer.svh.weight_loader(layer.svh, torch.ones(n, dtype=torch.float16), sid)
        layer.mul1.weight_loader(layer.mul1, torch.tensor(0x83DCD12D - (1 << 32), dtype=torch.int64), sid)
    assert torch.equal(layer.exl3_trellis_2, tr)
    with pytest.raises(AssertionError):
        layer.trellis.weight_loader(layer.trellis, torch.zeros(1, dtype=torch.int16), "q")
    with pytest.raises(plugin.Exl3FormatError):
        layer.mul1.weight_loader(layer.mul1, torch.tensor(7), "k")             # not the kernels' multiplier
    method.process_weights_after_loading(layer)
    assert layer.exl3_is_mul1 and not layer.exl3_is_mcg
    assert "trellis" not in layer._parameters and "mul1" not in layer._parameters
    assert layer.exl3_mgemm_ptrs is None                                   # groups differ in K / width


def test_partition_mapping_and_errors():
    # one group spanning two output partitions (in_proj_qkv covers q, k, v of in_proj_qkvz)
    method, layer = make_layer([("qkv", 4, 128, 384), ("z", 4, 128, 128)])
    assert layer.exl3_part_to_group == [0, 1]
    cfg = plugin.Exl3Config()
    m = plugin.Exl3LinearMethod(cfg, [("a", 4, 128, 256)])
    l2 = torch.nn.Module()
    m.create_weights(l2, 128, [128, 128], 128, 256, torch.float16)
    assert l2.exl3_part_to_group == [0, 0]
    with pytest.raises(NotImplementedError):
        m.create_weights(torch.nn.Module(), 64, [256], 128, 256, torch.float16)   # tensor parallel
    with pytest.raises(AssertionError):
        m.create_weights(torch.nn.Module(), 128, [200], 128, 200, torch.float16)  # does not tile
    with pytest.raises(AssertionError):
        plugin.Exl3LinearMethod._group_of(l2, (0, 1)) if len(set(l2.exl3_part_to_group)) > 1 else \
            plugin.Exl3LinearMethod._group_of(layer, (0, 1))


def test_apply_silu_mul_rejects_fused_modules():
    """The MLP hook takes a down projection (one group): a gate/up module is rejected before any
    launch."""
    method, layer = make_layer([("gate", 4, 128, 128), ("up", 4, 128, 128)])
    with pytest.raises(ValueError, match="one group"):
        method.apply_silu_mul(layer, torch.zeros(1, 256, dtype=torch.float16))


def test_missing_tensor_is_reported():
    method, layer = make_layer([("a", 4, 128, 128)])
    layer.trellis.weight_loader(layer.trellis, torch.zeros(8, 8, 64, dtype=torch.int16))
    with pytest.raises(AssertionError, match="missing"):
        method.process_weights_after_loading(layer)


def test_codebook_scalar_check():
    assert plugin.check_codebook_scalar("mul1", 0x83DCD12D)
    assert plugin.check_codebook_scalar("mul1", 0x83DCD12D - (1 << 32))
    assert not plugin.check_codebook_scalar("mcg", 0x83DCD12D)
    assert plugin.require_codebook_scalar("mcg", 0xCBAC1FED - (1 << 32)) == 0xCBAC1FED
    with pytest.raises(plugin.Exl3FormatError, match="0x83dcd12d"):
        plugin.require_codebook_scalar("mul1", 0x83DCD12C)


def test_partition_mapping_by_offsets():
    assert plugin._partition_groups([128, 128], [256]) == [0, 0]
    assert plugin._partition_groups([5120, 1024, 1024], [5120, 1024, 1024]) == [0, 1, 2]
    assert plugin._partition_groups([128, 256, 128, 128], [384, 256]) == [0, 0, 1, 1]
    for parts, widths in (([512], [384, 128]), ([256, 256], [384, 128]), ([200], [256]), ([128], [128, 128])):
        with pytest.raises(AssertionError):
            plugin._partition_groups(parts, widths)


# ---------------------------------------------------------------------------------------------
# real checkpoint files: safetensors with tensor data, and quantization_config.json
# ---------------------------------------------------------------------------------------------
def write_exl3_checkpoint(path, modules: dict, mul1=0x83DCD12D, qconfig=None):
    """modules: {checkpoint module name: (K, k, n)} -> one safetensors file with seeded trellis /
    suh / svh data and a mul1 scalar per module; returns {module: (trellis, suh, svh)}."""
    from safetensors.torch import save_file
    rng = np.random.default_rng(11)
    tensors, data = {}, {}
    for name, (K, k, n) in modules.items():
        tr = rng.integers(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=np.int16)
        su = rng.standard_normal(k).astype(np.float16)
        sv = rng.standard_normal(n).astype(np.float16)
        tensors[f"{name}.trellis"] = torch.from_numpy(tr)
        tensors[f"{name}.suh"] = torch.from_numpy(su)
        tensors[f"{name}.svh"] = torch.from_numpy(sv)
        tensors[f"{name}.mul1"] = torch.tensor(mul1 - (1 << 32) if mul1 >= (1 << 31) else mul1, dtype=torch.int32)
        data[name] = (tr, su, sv)
    save_file(tensors, str(path / "model-00001-of-00001.safetensors"))
    if qconfig is not None:
        with open(path / "quantization_config.json", "w") as f:
            json.dump(qconfig, f)
    return data


QKV = {"model.language_model.layers.0.self_attn.q_proj": (2, 256, 256),
       "model.language_model.layers.0.self_attn.k_proj": (5, 256, 128),
       "model.language_model.layers.0.self_attn.v_proj": (5, 256, 128)}


def _qconfig(modules, mul1=0x83DCD12D, bits=None):
    return {"codebook": "mul1", "tensor_storage": {
        name: {"bits_per_weight": bits or K, "quant_format": "exl3", "mul1_multiplier": mul1,
               "stored_tensors": {f"{name}.trellis": {"shape": [k // 16, n // 16, 16 * K], "dtype": "int16"}}}
        for name, (K, k, n) in modules.items()} | {"model.norm": {"stored_tensors": {}}}}


def test_load_linear_from_real_safetensors(tmp_path):
    from exl3rocm import checkpoint
    data = write_exl3_checkpoint(tmp_path, QKV, qconfig=_qconfig(QKV))
    method, layer = checkpoint.load_linear(str(tmp_path), "model.layers.0.self_attn.qkv_proj", device="cpu")
    assert layer.exl3_K == [2, 5, 5] and layer.exl3_n == [256, 128, 128]
    assert layer.exl3_is_mul1 and layer.exl3_mul1 == 0x83DCD12D
    for i, name in enumerate(QKV):
        tr, su, sv = data[name]
        assert np.array_equal(getattr(layer, f"exl3_trellis_{i}").numpy(), tr)
        assert np.array_equal(getattr(layer, f"exl3_suh_{i}").numpy().view(np.uint16), su.view(np.uint16))
        assert np.array_equal(getattr(layer, f"exl3_svh_{i}").numpy().view(np.uint16), sv.view(np.uint16))
    assert "trellis" not in layer._parameters
    with pytest.raises(KeyError):
        checkpoint.load_linear(str(tmp_path), "model.layers.0.mlp.gate_up_proj", device="cpu")


def test_wrong_multiplier_in_the_file_is_refused(tmp_path):
    from exl3rocm import checkpoint
    write_exl3_checkpoint(tmp_path, QKV, mul1=0x83DCD12D ^ 0x100)
    with pytest.raises(plugin.Exl3FormatError):
        checkpoint.load_linear(str(tmp_path), "model.layers.0.self_attn.qkv_proj", device="cpu")


def test_quantization_config_is_a_contract(tmp_path):
    write_exl3_checkpoint(tmp_path, QKV, qconfig=_qconfig(QKV))
    cfg = plugin.Exl3Config()
    cfg.maybe_update_config(str(tmp_path))
    assert set(cfg.multipliers.values()) == {0x83DCD12D} and len(cfg.multipliers) == 3
    for bad in (_qconfig(QKV, mul1=0x12345678), _qconfig(QKV, bits=3)):
        with open(tmp_path / "quantization_config.json", "w") as f:
            json.dump(bad, f)
        with pytest.raises(plugin.Exl3FormatError):
            plugin.Exl3Config().maybe_update_config(str(tmp_path))
    # a scalar in the weights that disagrees with the config's multiplier is refused at load time
    cfg.multipliers = {k: 0x83DCD12D for k in cfg.multipliers}
    method = plugin.Exl3LinearMethod(cfg, cfg._groups_for("model.layers.0.self_attn.qkv_proj"))
    layer = torch.nn.Module()
    method.create_weights(layer, 256, [256, 128, 128], 256, 512, torch.float16)
    assert layer.mul1.weight_loader.expected == 0x83DCD12D


def test_fake_impls_shapes():
    x = torch.empty(2, 3, 256, device="meta", dtype=torch.float16)
    tr = torch.empty(16, 8, 64, device="meta", dtype=torch.int16)
    su = torch.empty(256, device="meta", dtype=torch.float16)
    sv = torch.empty(128, device="meta", dtype=torch.float16)
    y = torch.ops.exl3rocm.linear(x, tr, su, sv, 4, False, True)
    assert y.shape == (2, 3, 128) and y.dtype == torch.float16
    yg = torch.ops.exl3rocm.linear_groups(x, [tr, tr], [su, su], [sv, sv], [4, 4], False, True)
    assert yg.shape == (2, 3, 256)


def test_cpu_tensors_fail_loudly():
    x = torch.zeros(1, 128, dtype=torch.float16)
    tr = torch.zeros(8, 8, 64, dtype=torch.int16)
    s = torch.ones(128, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU"):
        torch.ops.exl3rocm.linear(x, tr, s, s, 4, False, True)


def test_vllm_entry_point_is_declared():
    """The package declares the vLLM general-plugin entry point, and it names a callable that
    registers the custom ops (the reference's vllm_plugin/pyproject.toml:12-13)."""
    import importlib
    import tomli
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "qwen38-27b-exl3-rdna4_amd")
    with open(os.path.join(pkg, "pyproject.toml"), "rb") as f:
        meta = tomli.load(f)
    target = meta["project"]["entry-points"]["vllm.general_plugins"]["exl3rocm"]
    mod, fn = target.split(":")
    assert callable(getattr(importlib.import_module(mod), fn))
    assert "libexl3_mi355x.so" in meta["tool"]["setuptools"]["package-data"]["exl3rocm"]


def test_approx_route_setting():
    """EXL3_GEMV_APPROX: off values select the faithful GEMV, the two routes by name (any case),
    anything else is refused rather than silently ignored."""
    for off in (None, "", "0", "off", "OFF", " none ", "faithful"):
        assert ops.approx_mode(off) == ""
    assert ops.approx_mode("affine") == "affine"
    assert ops.approx_mode(" INT8") == "int8"
    for bad in ("1", "7", "int4", "affin"):
        with pytest.raises(ValueError):
            ops.approx_mode(bad)


@pytest.mark.parametrize("mode", ["", "affine", "int8"])
def test_empty_batch_launches_nothing_on_every_route(monkeypatch, mode):
    """A zero-row input returns an empty [0, sum(widths)] output before any route is chosen: the
    approximate GEMV (which declines m = 0) is never reached.  No launch happens, so CPU tensors
    show it without a GPU."""
    monkeypatch.setattr(ops, "GEMV_APPROX", mode)
    x = torch.zeros(0, 256, dtype=torch.float16)
    tr = [torch.zeros(16, 8, 64, dtype=torch.int16) for _ in range(2)]
    s = [torch.ones(256, dtype=torch.float16)] * 2
    v = [torch.ones(128, dtype=torch.float16)] * 2
    y = torch.ops.exl3rocm.linear_groups(x, tr, s, v, [4, 4], False, True)
    assert tuple(y.shape) == (0, 256) and y.dtype == torch.float16
    y3 = torch.ops.exl3rocm.linear_groups(x.view(1, 0, 256), tr, s, v, [4, 4], False, True)
    assert tuple(y3.shape) == (1, 0, 256)


# ---------------------------------------------------------------------------------- GEMV / GEMM route
def test_route_boundary_table_and_override(monkeypatch):
    """Each launch shape in the measured table routes its own boundary b to the GEMV and b + 1 to
    the prefill GEMM; the fused-epilogue forms stop at 32 rows; shapes outside the table take
    DEFAULT_MR; EXL3_MR_MAX fixes one boundary for every shape, capped at the GEMV's 64 rows."""
    from exl3rocm import _lib
    monkeypatch.setattr(ops, "MR_MAX", None)
    for (k, w), b in ops.GEMV_CROSSOVER.items():
        assert 1 <= b <= _lib.GEMV_MAX_ROWS
        assert ops.gemv_rows(b, k, w) and not ops.gemv_rows(b + 1, k, w)
        assert ops.fused_rows(min(b, 32), k, w) and not ops.fused_rows(33, k, w)
    assert ops.gemv_max_rows(512, 512) == ops.DEFAULT_MR
    monkeypatch.setattr(ops, "MR_MAX", 16)
    assert ops.gemv_max_rows(5120, 34816) == 16 and ops.gemv_max_rows(512, 512) == 16
    monkeypatch.setenv("EXL3_MR_MAX", "64")
    assert ops._env_rows("EXL3_MR_MAX") == _lib.GEMV_MAX_ROWS
    monkeypatch.setenv("EXL3_MR_MAX", " ")
    assert ops._env_rows("EXL3_MR_MAX") is None


class _Launches:
    """Stands in for the kernels module: records each launch linear_groups makes (no GPU)."""

    def __init__(self):
        self.calls = []

    def __getattr__(self, name):
        def launch(*args, **kw):
            svh = args[5] if name.startswith("exl3_gemm_trellis") else \
                args[4] if name == "exl3_gemv_mr_grouped_widths" else args[5]
            self.calls.append((name, [int(s.shape[0]) for s in svh] if isinstance(svh, list) else [int(svh.shape[0])]))
            return 0
        return launch


@pytest.mark.parametrize("m,expect", [
    (20, [("exl3_gemv_mr", [12288]), ("exl3_gemv_mr_grouped", [1024, 1024])]),
    (25, [("exl3_gemv_mr", [12288]), ("exl3_gemm_trellis_grouped", [1024, 1024])]),
    (31, [("exl3_gemm_trellis_grouped", [12288]), ("exl3_gemm_trellis_grouped", [1024, 1024])]),
])
def test_linear_groups_routes_each_run_by_its_shape(monkeypatch, m, expect):
    """A checkpoint's q (2 bpw, 5120 -> 12288) and k / v (5 bpw, 1024 each): two runs of equal K,
    each routed by its own launch shape (crossovers set here to 30 and 21 rows)."""
    rec = _Launches()
    monkeypatch.setattr(ops, "E", rec)
    monkeypatch.setattr(ops, "MR_MAX", None)
    monkeypatch.setattr(ops, "GEMV_CROSSOVER", {(5120, 12288): 30, (5120, 2048): 21})
    monkeypatch.setattr(ops, "GEMV_APPROX", "")
    x = torch.zeros(m, 5120, dtype=torch.float16)
    tr = [torch.zeros(320, n // 16, 16 * K, dtype=torch.int16) for n, K in ((12288, 2), (1024, 5), (1024, 5))]
    su = [torch.ones(5120, dtype=torch.float16)] * 3
    sv = [torch.ones(n, dtype=torch.float16) for n in (12288, 1024, 1024)]
    y = torch.ops.exl3rocm.linear_groups(x, tr, su, sv, [2, 5, 5], False, True)
    assert tuple(y.shape) == (m, 14336)
    assert rec.calls == expect
