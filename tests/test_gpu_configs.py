"""GPU parity at the benchmark configurations' full shapes (run with -m gpu on an MI355X).

* config 4 (prefill, M = 2048, Qwen-27B layer shapes): o and down with their 4-piece K-split
  tail, the grouped q/k/v launch (448 tiles) and the grouped gate/up launch (2176 tiles, 2-piece
  split).  Oracle on row subsets taken from whole tiles and from split tiles; whole tiles bitwise
  equal to the never-splitting reference entry point exl3_gemm_trellis.
* config 3 (M = 16 / 32, heavy-tail x, 4 bpw) on gate/up (5120 -> 17408) and down
  (17408 -> 5120): oracle, and every row bitwise equal to its M = 1 call.
* a mixed-bitrate fused module (q = 2 bpw, k / v = 5 bpw, as in the reference checkpoint's
  qkv_proj) through the plugin at M = 1, 4 and 64 against the oracle.
* the boundary: the exl3_gemm row dispatcher through the C ABI, the reference's reconstruct +
  hgemm prefill route through the op, and the serving sequence (load, eager warm-up on a side
  stream, graph capture on it) with no manual workspace reservation.
Expected values come from oracle/libexl3cpu.so (pinned in test_oracle.py).
"""
import ctypes

import numpy as np
import pytest
import torch

import cpu
from exl3rocm import _lib, kernels as E, ops, synth
from test_gpu_parity import DEV, assert_close, to_dev

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

M4 = 2048


def plan(m, k, widths):
    wa = (ctypes.c_int * len(widths))(*widths)
    return int(_lib.lib().exl3_gemm_trellis_workspace_size(m, k, wa, len(widths)))


# ---------------------------------------------------------------------------------- config 4
@pytest.mark.parametrize("name,k,n", [("o", 5120, 5120), ("down", 17408, 5120)])
def test_config4_prefill_split4(name, k, n):
    """320 tiles of 256 x 128: 256 whole tiles, then 64 tiles split along K into 4 pieces."""
    bits = 4
    tr, su, sv = synth.layer("cfg4", name, k, n, bits)
    x = synth.activations(synth.key_of("cfg4", name, "x"), M4, k)
    X, T, SU, SV = to_dev(x, tr.view(np.int16), su, sv)
    tiles_n = n // 128
    assert plan(M4, k, [n]) > 0                         # the tail is split
    print(f"config4 {name}: m={M4} k={k} n={n}", flush=True)
    y = torch.ops.exl3rocm.linear(X, T, SU, SV, bits, False, True)
    y0 = torch.empty_like(y)
    E.exl3_gemm_trellis(X, T, y0, SU, torch.empty_like(X), SV, bits, False, True)
    torch.cuda.synchronize()
    # whole tiles: u < 256 -> row tile u // tiles_n, column tile u % tiles_n
    full_rows = 256 // tiles_n                          # row tiles made only of whole tiles (6)
    whole_cols = (256 - full_rows * tiles_n) * 128      # whole columns of row tile 6
    r6 = full_rows * 256
    assert torch.equal(y[:r6].view(torch.int16), y0[:r6].view(torch.int16))
    assert torch.equal(y[r6:r6 + 256, :whole_cols].view(torch.int16), y0[r6:r6 + 256, :whole_cols].view(torch.int16))
    # split tiles: the rest of row tile 6 and all of row tile 7
    assert_close(y[r6:].cpu().numpy(), y0[r6:].cpu().numpy(), "split vs unsplit")
    rows = [0, 1, 255, 1024, r6, r6 + 77, 2046, 2047]
    ref = cpu.linear(x[rows], tr, bits, su, sv, 2)
    assert_close(y[rows].cpu().numpy(), ref, f"{name} vs oracle")
    y2 = torch.ops.exl3rocm.linear(X, T, SU, SV, bits, False, True)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))     # counters left zero: repeatable


def _grouped(tag, k, widths, bits):
    mats = [synth.layer("cfg4", f"{tag}{i}", k, n, bits) for i, n in enumerate(widths)]
    x = synth.activations(synth.key_of("cfg4", tag, "x"), M4, k)
    X = to_dev(x)[0]
    Ts = [to_dev(t.view(np.int16))[0] for t, _, _ in mats]
    SUs = [to_dev(s)[0] for _, s, _ in mats]
    SVs = [to_dev(s)[0] for _, _, s in mats]
    return x, mats, X, Ts, SUs, SVs


def test_config4_grouped_qkv():
    """q / k / v (5120, 1024, 1024) in one launch: 448 tiles, no split (the partial traffic of a
    split 192-tile tail costs more than it saves); every tile equals the unsplit single-group
    launch bitwise."""
    k, widths, bits = 5120, (5120, 1024, 1024), 4
    assert plan(M4, k, list(widths)) == 0
    x, mats, X, Ts, SUs, SVs = _grouped("qkv", k, widths, bits)
    print(f"config4 qkv: m={M4} widths={widths}", flush=True)
    y = torch.ops.exl3rocm.linear_groups(X, Ts, SUs, SVs, [bits] * 3, False, True)
    rows = [0, 300, 1800, 2047]
    n0 = 0
    for (tr, su, sv), T, SU, SV, n in zip(mats, Ts, SUs, SVs, widths):
        y0 = torch.empty(M4, n, dtype=torch.float16, device=DEV)
        E.exl3_gemm_trellis(X, T, y0, SU, torch.empty_like(X), SV, bits, False, True)
        assert torch.equal(y[:, n0:n0 + n].view(torch.int16), y0.view(torch.int16)), n0
        assert_close(y[rows, n0:n0 + n].cpu().numpy(), cpu.linear(x[rows], tr, bits, su, sv, 2), ("qkv", n0))
        n0 += n


def test_config4_grouped_gate_up():
    """gate / up (2 x 17408) in one launch: 2176 tiles = 8 full waves + 128 tail tiles of `up`
    split into 2 pieces.  Whole tiles equal the unsplit launch bitwise; both kinds match the oracle."""
    k, widths, bits = 5120, (17408, 17408), 4
    assert plan(M4, k, list(widths)) > 0
    x, mats, X, Ts, SUs, SVs = _grouped("gu", k, widths, bits)
    print(f"config4 gate/up: m={M4} widths={widths}", flush=True)
    y = torch.ops.exl3rocm.linear_groups(X, Ts, SUs, SVs, [bits] * 2, False, True)
    n = widths[0]
    tiles_n = n // 128
    y0 = [torch.empty(M4, n, dtype=torch.float16, device=DEV) for _ in range(2)]
    for g in range(2):
        E.exl3_gemm_trellis(X, Ts[g], y0[g], SUs[g], torch.empty_like(X), SVs[g], bits, False, True)
    assert torch.equal(y[:, :n].view(torch.int16), y0[0].view(torch.int16))      # gate: whole tiles only
    # up: tiles 1088 + v; split ones are v >= 2048 - 1088 = 960 -> row tile 7 from column tile 960 - 952
    v0 = 2048 - 1088
    r7, c7 = (v0 // tiles_n) * 256, (v0 % tiles_n) * 128
    up = y[:, n:]
    assert torch.equal(up[:r7].view(torch.int16), y0[1][:r7].view(torch.int16))
    assert torch.equal(up[r7:, :c7].view(torch.int16), y0[1][r7:, :c7].view(torch.int16))
    assert_close(up[r7:, c7:].cpu().numpy(), y0[1][r7:, c7:].cpu().numpy(), "split vs unsplit")
    rows = [3, 1000, r7 + 5, 2047]
    for g, (tr, su, sv) in enumerate(mats):
        assert_close(y[rows, g * n:(g + 1) * n].cpu().numpy(), cpu.linear(x[rows], tr, bits, su, sv, 2), ("gu", g))


@pytest.mark.parametrize("name,m,k,n", [("down", 64, 17408, 5120), ("o", 40, 5120, 5120), ("qkv-k", 200, 5120, 1024),
                                        ("gate", 33, 5120, 17408), ("gate", 100, 5120, 17408)])
def test_small_m_prefill_splits_every_tile(name, m, k, n):
    """M in (32, 256]: one row tile of few column tiles (down: 40) is split along K into pieces
    (down: 6 of ~45 steps) so the launch fills the CUs; gate's 136 tiles (more than half a wave)
    take two unequal pieces each (54 and 26 of 80 steps, the long ones dispatched first).  The
    rows past M of the single row tile are dead (no loads, no MFMAs, no partials; M = 100 leaves
    a consumer wave with 3 of its 4 row tiles live).  Oracle on rows spread over the tile,
    repeatable bitwise, and equal to the unsplit reference entry point to the parity bar."""
    bits = 4
    tr, su, sv = synth.layer("smallm", name, k, n, bits)
    x = synth.activations(synth.key_of("smallm", name, "x"), m, k)
    X, T, SU, SV = to_dev(x, tr.view(np.int16), su, sv)
    assert plan(m, k, [n]) > 0
    print(f"small-M split {name}: m={m} k={k} n={n}", flush=True)
    y = torch.ops.exl3rocm.linear(X, T, SU, SV, bits, False, True)
    y2 = torch.ops.exl3rocm.linear(X, T, SU, SV, bits, False, True)
    y0 = torch.empty_like(y)
    E.exl3_gemm_trellis(X, T, y0, SU, torch.empty_like(X), SV, bits, False, True)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    assert_close(y.cpu().numpy(), y0.cpu().numpy(), "split vs unsplit")
    rows = sorted({0, 1, m // 2, m - 1})
    assert_close(y[rows].cpu().numpy(), cpu.linear(x[rows], tr, bits, su, sv, 2), f"{name} vs oracle")


# ---------------------------------------------------------------------------------- config 3
@pytest.mark.parametrize("k,n", [(5120, 17408), (17408, 5120)])
def test_config3_heavy_tail_m16_m32(k, n, monkeypatch):
    """M = 16 and 32 (pre-rotated input) with heavy-tail x at 4 bpw on the GEMV route: oracle, and
    every row == its M = 1 call bitwise."""
    monkeypatch.setattr(ops, "MR_MAX", 32)
    bits = 4
    tr, su, sv = synth.layer("cfg3", f"{k}x{n}", k, n, bits)
    x = synth.activations(synth.key_of("cfg3", f"{k}x{n}", "x"), 32, k, heavy_tail=True)
    X, T, SU, SV = to_dev(x, tr.view(np.int16), su, sv)
    print(f"config3 heavy tail k={k} n={n}", flush=True)
    rows1 = torch.cat([torch.ops.exl3rocm.linear(X[r:r + 1], T, SU, SV, bits, False, True) for r in range(32)])
    ref = cpu.linear(x, tr, bits, su, sv, 2)
    for m in (4, 16, 32):
        ym = torch.ops.exl3rocm.linear(X[:m], T, SU, SV, bits, False, True)
        assert torch.equal(ym.view(torch.int16), rows1[:m].view(torch.int16)), m
        assert_close(ym.cpu().numpy(), ref[:m], (k, n, m))


# ---------------------------------------------------------------------------------- mixed bitrates
def test_mixed_bitrate_qkv_module_vs_oracle():
    """qkv_proj with q at 2 bpw and k / v at 5 bpw (the reference checkpoint's mix), loaded through
    the plugin; M = 1 (runs of equal K: q alone, k / v grouped), M = 4 and M = 64 (prefill, one
    launch per run) against the oracle."""
    from exl3rocm import plugin
    k = 5120
    spec = [("q", 2, 5120), ("k", 5, 1024), ("v", 5, 1024)]
    groups = [(name, K, k, n) for name, K, n in spec]
    method = plugin.Exl3LinearMethod(plugin.Exl3Config("mul1"), groups)
    lay = torch.nn.Module()
    method.create_weights(lay, k, [n for _, _, n in spec], k, sum(n for _, _, n in spec), torch.float16)
    lay.to(DEV)
    mats = [synth.layer("mixqkv", name, k, n, K) for name, K, n in spec]
    for (name, K, n), (tr, su, sv) in zip(spec, mats):
        lay.trellis.weight_loader(lay.trellis, torch.from_numpy(tr.view(np.int16)), name)
        lay.suh.weight_loader(lay.suh, torch.from_numpy(su), name)
        lay.svh.weight_loader(lay.svh, torch.from_numpy(sv), name)
        lay.mul1.weight_loader(lay.mul1, torch.tensor(0x83DCD12D), name)
    method.process_weights_after_loading(lay)
    assert lay.exl3_mgemm_ptrs is None                 # mixed K: no single pointer-table launch
    x = synth.activations(synth.key_of("mixqkv", "x"), 64, k)
    ref = np.concatenate([cpu.linear(x[:8], tr, K, su, sv, 2) for (_, K, _), (tr, su, sv) in zip(spec, mats)], axis=1)
    X = to_dev(x)[0]
    y1 = method.apply(lay, X[:1])
    y4 = method.apply(lay, X[:4])
    y64 = method.apply(lay, X)
    torch.cuda.synchronize()
    assert torch.equal(y4[:1].view(torch.int16), y1.view(torch.int16))
    assert_close(y1.cpu().numpy(), ref[:1], "M=1", strict=True)
    assert_close(y4.cpu().numpy(), ref[:4], "M=4")
    assert_close(y64[:8].cpu().numpy(), ref, "M=64")


# ---------------------------------------------------------------------------------- boundary
def test_exl3_gemm_dispatcher_routes_and_matches_the_ops():
    """The reference's row dispatcher (exl3_gemm -> route tag) through the C ABI: m <= 32 takes the
    fused GEMV (tag 1), larger m the prefill GEMM (tag 2), although the plain GEMV itself takes up
    to 64 rows; outputs equal the op's bitwise (this shape is outside the op's crossover table, so
    the op's boundary is 32 too)."""
    k, n, bits = 2048, 1024, 4
    tr, su, sv = synth.layer("disp", 0, k, n, bits)
    x = synth.activations(synth.key_of("disp", "x"), 40, k)
    X, T, SU, SV = to_dev(x, tr.view(np.int16), su, sv)
    for m, tag in ((1, 1), (8, 1), (32, 1), (40, 2)):
        assert E.exl3_gemv_mr_supported(m, k, n, bits, False, True) == (m <= _lib.GEMV_MAX_ROWS)
        assert ops.gemv_rows(m, k, n) == (m <= 32)
        C = torch.empty(m, n, dtype=torch.float16, device=DEV)
        A_had = torch.empty(m, k, dtype=torch.float16, device=DEV)
        assert E.exl3_gemm(X[:m].contiguous(), T, C, SU, A_had, SV, -1, False, True, 0) == tag
        want = torch.ops.exl3rocm.linear(X[:m], T, SU, SV, bits, False, True)
        if m == 40:
            # the dispatcher's prefill is exl3_gemm_trellis (never split): equal to the unsplit launch
            want = torch.empty_like(C)
            E.exl3_gemm_trellis(X[:m].contiguous(), T, want, SU, torch.empty_like(A_had), SV, bits, False, True)
        assert torch.equal(C.view(torch.int16), want.view(torch.int16)), m
    torch.cuda.synchronize()
    assert_close(C.cpu().numpy(), cpu.linear(x, tr, bits, su, sv, 2), "dispatcher m=40")


def test_recon_prefill_route_through_the_op(monkeypatch):
    """EXL3_PREFILL=recon (the reference's reconstruct + hgemm_recon route, ops.py:86-97) through
    exl3rocm::linear and linear_groups: bitwise equal to the fused route (same MFMA order; the
    layer is small enough that the fused launch has no split tail), and within the bar of the oracle."""
    k, m = 512, 96                      # K too short for a split launch: the same summation order
    widths = (512, 384)
    mats = [synth.layer("recon-op", i, k, n, 4) for i, n in enumerate(widths)]
    x = synth.activations(synth.key_of("recon-op", "x"), m, k)
    X = to_dev(x)[0]
    Ts = [to_dev(t.view(np.int16))[0] for t, _, _ in mats]
    SUs = [to_dev(s)[0] for _, s, _ in mats]
    SVs = [to_dev(s)[0] for _, _, s in mats]
    fused = torch.ops.exl3rocm.linear_groups(X, Ts, SUs, SVs, [4, 4], False, True)
    monkeypatch.setattr(ops, "PREFILL_ROUTE", "recon")
    ops.reserve_weight_buffer(DEV, k * max(widths))
    recon = torch.ops.exl3rocm.linear_groups(X, Ts, SUs, SVs, [4, 4], False, True)
    single = torch.ops.exl3rocm.linear(X, Ts[0], SUs[0], SVs[0], 4, False, True)
    torch.cuda.synchronize()
    assert torch.equal(recon.view(torch.int16), fused.view(torch.int16))
    assert torch.equal(single.view(torch.int16), fused[:, :widths[0]].view(torch.int16))
    ref = np.concatenate([cpu.linear(x[:6], t, 4, s, v, 2) for t, s, v in mats], axis=1)
    assert_close(recon[:6].cpu().numpy(), ref, "recon route")


def test_serving_sequence_captures_without_manual_reserve():
    """Load on the default stream, eager warm-up on a side stream S, then capture on S: no
    reserve_workspace call by hand.  Replays equal the eager output."""
    from exl3rocm import plugin
    k, n, bits = 2048, 1536, 4
    groups = [("gate", bits, k, n), ("up", bits, k, n)]
    method = plugin.Exl3LinearMethod(plugin.Exl3Config("mul1"), groups)
    lay = torch.nn.Module()
    method.create_weights(lay, k, [n, n], k, 2 * n, torch.float16)
    lay.to(DEV)
    for i in range(2):
        tr, su, sv = synth.layer("serve", i, k, n, bits)
        lay.trellis.weight_loader(lay.trellis, torch.from_numpy(tr.view(np.int16)), i)
        lay.suh.weight_loader(lay.suh, torch.from_numpy(su), i)
        lay.svh.weight_loader(lay.svh, torch.from_numpy(sv), i)
        lay.mul1.weight_loader(lay.mul1, torch.tensor(0x83DCD12D), i)
    method.process_weights_after_loading(lay)
    X = to_dev(synth.activations(synth.key_of("serve", "x"), 8, k))[0]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        eager1 = method.apply(lay, X[:1])                 # warm-up: M = 1 only
        eager8 = method.apply(lay, X)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        y1 = method.apply(lay, X[:1])
        y8 = method.apply(lay, X)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y1.view(torch.int16), eager1.view(torch.int16))
        assert torch.equal(y8.view(torch.int16), eager8.view(torch.int16))
        method.apply(lay, X)                              # eager work between replays
        torch.cuda.synchronize()


def test_layer_loaded_from_a_checkpoint_file_vs_oracle(tmp_path):
    """A real safetensors checkpoint (tensor data + quantization_config.json) loaded through
    exl3rocm.checkpoint onto the GPU: the fused q/k/v module (2 / 5 / 5 bpw) at M = 1 and 40
    against the oracle on the same file data."""
    from exl3rocm import checkpoint
    from test_host import QKV, _qconfig, write_exl3_checkpoint
    data = write_exl3_checkpoint(tmp_path, QKV, qconfig=_qconfig(QKV))
    method, lay = checkpoint.load_linear(str(tmp_path), "model.layers.0.self_attn.qkv_proj", device=DEV)
    x = synth.activations(synth.key_of("ckpt", "x"), 40, 256)
    X = to_dev(x)[0]
    ref = np.concatenate([cpu.linear(x, tr.view(np.uint16), K, su, sv, 2)
                          for (K, _, _), (tr, su, sv) in zip(QKV.values(), data.values())], axis=1)
    y1 = method.apply(lay, X[:1])
    y40 = method.apply(lay, X)
    torch.cuda.synchronize()
    assert_close(y1.cpu().numpy(), ref[:1], "file M=1", strict=True)
    assert_close(y40.cpu().numpy(), ref, "file M=40")


# ---------------------------------------------------------------------------------------------- 64 rows
@pytest.mark.parametrize("k,n,bits,cb", [(5120, 17408, 4, 2), (17408, 5120, 3, 2), (2048, 1024, 5, 1)])
def test_gemv_64_rows_bitwise_rows_and_oracle(k, n, bits, cb):
    """The plain GEMV's third and fourth 16-row tiles (33 to 64 rows): every row of an m-row call
    is bitwise equal to its M = 1 call, and the rows match the oracle."""
    tr, su, sv = synth.layer("rows48", f"{k}x{n}x{bits}", k, n, bits)
    x = synth.activations(synth.key_of("rows48", f"{k}x{n}x{bits}", "x"), 64, k, heavy_tail=True)
    X, T, SU, SV = to_dev(x, tr.view(np.int16), su, sv)
    print(f"64-row GEMV k={k} n={n} bits={bits} cb={cb}", flush=True)
    rows1 = torch.empty(64, n, dtype=torch.float16, device=DEV)
    for r in range(64):
        assert E.exl3_gemv_mr(X[r:r + 1], T, rows1[r:r + 1], SU, None, SV, bits, cb == 1, cb == 2) == 0
    for m in (33, 40, 47, 48, 49, 57, 63, 64):
        assert E.exl3_gemv_mr_supported(m, k, n, bits, cb == 1, cb == 2)
        ym = torch.full((m, n), float("nan"), dtype=torch.float16, device=DEV)
        assert E.exl3_gemv_mr(X[:m], T, ym, SU, None, SV, bits, cb == 1, cb == 2) == 0
        assert torch.equal(ym.view(torch.int16), rows1[:m].view(torch.int16)), m
    torch.cuda.synchronize()
    assert_close(rows1.cpu().numpy(), cpu.linear(x, tr, bits, su, sv, cb), (k, n, bits, cb))
    assert not E.exl3_gemv_mr_supported(65, k, n, bits, cb == 1, cb == 2)


@pytest.mark.parametrize("k,n,bits,cb", [(2048, 1024, 2, 0), (2048, 1024, 8, 0), (5120, 5120, 6, 1), (5120, 5120, 2, 2),
                                          (5120, 5120, 8, 2), (1024, 4096, 1, 1)])
def test_gemv_small_rows_every_codebook(k, n, bits, cb):
    """The one-tile forms at 2-16 rows for every codebook and the extreme bitrates: MT 6 (one quad of
    partial loads in flight, in one pass up to 4 rows and several above) up to 8 rows on the
    512-workgroup grid of 5120 x 5120 and up to 16 on the smaller grids of 2048 x 1024 and
    1024 x 4096, MT 5 at 9-16 rows on the full grid: every row bitwise equal to its M = 1 call,
    the rows against the oracle."""
    tr, su, sv = synth.layer("rows16", f"{k}x{n}x{bits}x{cb}", k, n, bits)
    x = synth.activations(synth.key_of("rows16", f"{k}x{n}x{bits}", "x"), 16, k, heavy_tail=True)
    X, T, SU, SV = to_dev(x, tr.view(np.int16), su, sv)
    print(f"small-row GEMV k={k} n={n} bits={bits} cb={cb} grid={_lib.lib().exl3_gemv_grid(k, n, 1)}", flush=True)
    rows1 = torch.empty(16, n, dtype=torch.float16, device=DEV)
    for r in range(16):
        assert E.exl3_gemv_mr(X[r:r + 1], T, rows1[r:r + 1], SU, None, SV, bits, cb == 1, cb == 2) == 0
    for m in (2, 3, 4, 5, 7, 8, 9, 13, 16):
        ym = torch.full((m, n), float("nan"), dtype=torch.float16, device=DEV)
        assert E.exl3_gemv_mr(X[:m], T, ym, SU, None, SV, bits, cb == 1, cb == 2) == 0
        assert torch.equal(ym.view(torch.int16), rows1[:m].view(torch.int16)), m
    torch.cuda.synchronize()
    assert_close(rows1.cpu().numpy(), cpu.linear(x, tr, bits, su, sv, cb), (k, n, bits, cb))


@pytest.mark.parametrize("k,n,bits,cb", [(5120, 17408, 4, 2), (1024, 16384, 5, 1), (2048, 4096, 3, 0)])
def test_gemv_17_32_rows_bitwise_rows_and_oracle(k, n, bits, cb):
    """Two 16-row tiles (17-32 rows): MT 7 (two quads of partial loads in flight) where every block
    has at most 8 contributors (5120 -> 17408: ~5; 1024 -> 16384: 5), MT 2 otherwise (2048 -> 4096:
    17): every row bitwise equal to its M = 1 call, the rows against the oracle."""
    tr, su, sv = synth.layer("rows32", f"{k}x{n}x{bits}x{cb}", k, n, bits)
    x = synth.activations(synth.key_of("rows32", f"{k}x{n}x{bits}", "x"), 32, k, heavy_tail=True)
    X, T, SU, SV = to_dev(x, tr.view(np.int16), su, sv)
    print(f"17-32-row GEMV k={k} n={n} bits={bits} cb={cb} grid={_lib.lib().exl3_gemv_grid(k, n, 1)}", flush=True)
    rows1 = torch.empty(32, n, dtype=torch.float16, device=DEV)
    for r in range(32):
        assert E.exl3_gemv_mr(X[r:r + 1], T, rows1[r:r + 1], SU, None, SV, bits, cb == 1, cb == 2) == 0
    for m in (17, 20, 25, 31, 32):
        ym = torch.full((m, n), float("nan"), dtype=torch.float16, device=DEV)
        assert E.exl3_gemv_mr(X[:m], T, ym, SU, None, SV, bits, cb == 1, cb == 2) == 0
        assert torch.equal(ym.view(torch.int16), rows1[:m].view(torch.int16)), m
    torch.cuda.synchronize()
    assert_close(rows1.cpu().numpy(), cpu.linear(x, tr, bits, su, sv, cb), (k, n, bits, cb))


def test_fused_forms_decline_above_32_rows():
    """The fused-epilogue GEMV forms take at most 32 rows: 33 declines without writing."""
    k, n, bits = 1024, 512, 4
    tr, su, sv = synth.layer("fused33", 0, k, n, bits)
    X, T, SU, SV = to_dev(synth.activations(synth.key_of("fused33", "x"), 33, k), tr.view(np.int16), su, sv)
    y = torch.full((33, n), 7.0, dtype=torch.float16, device=DEV)
    assert E.exl3_gemv_mr_approx(X, T, y, SU, None, SV, bits, "affine") == 1
    gu = torch.randn(33, 2 * k, device=DEV, dtype=torch.float16)
    assert E.exl3_gemv_silu_in(gu[:, :k], gu[:, k:], T, y, SU, None, SV, bits, False, True) == 1
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())


# ---------------------------------------------------------------------------------- route boundary
ROUTE_CASES = [(6144, (5120,), 4), (5120, (17408,), 4), (5120, (17408, 17408), 4), (5120, (5120, 1024, 1024), 4)]


@pytest.mark.parametrize("k,widths,bits", ROUTE_CASES)
def test_routing_follows_the_measured_crossover(k, widths, bits):
    """linear / linear_groups at the measured crossover b of the launch's shape and at b + 1: the
    (grouped) GEMV launch at b rows and the grouped prefill GEMM at b + 1, bitwise; the first and
    last rows of both against the oracle."""
    if ops.PREFILL_ROUTE != "fused":
        pytest.skip("EXL3_PREFILL selects the reconstruct + GEMM route above the boundary")
    b = ops.gemv_max_rows(k, sum(widths))
    assert ops.MR_MAX is None and b == ops.GEMV_CROSSOVER[(k, sum(widths))]
    g = len(widths)
    tag = f"route{k}x{'-'.join(map(str, widths))}"
    mats = [synth.layer(tag, i, k, n, bits) for i, n in enumerate(widths)]
    x = synth.activations(synth.key_of(tag, "x"), b + 1, k)
    X = to_dev(x)[0]
    Ts = [to_dev(t.view(np.int16))[0] for t, _, _ in mats]
    SUs = [to_dev(s)[0] for _, s, _ in mats]
    SVs = [to_dev(s)[0] for _, _, s in mats]
    print(f"route boundary k={k} widths={widths} b={b}", flush=True)
    for m, gemv in ((b, True), (b + 1, False)):
        Xm = X[:m].contiguous()
        got = (torch.ops.exl3rocm.linear(Xm, Ts[0], SUs[0], SVs[0], bits, False, True) if g == 1 else
               torch.ops.exl3rocm.linear_groups(Xm, Ts, SUs, SVs, [bits] * g, False, True))
        want = torch.empty_like(got)
        if not gemv:
            xh = torch.empty(g, m, k, dtype=torch.float16, device=DEV)
            E.exl3_gemm_trellis_grouped(Xm, Ts, want, SUs, xh, SVs, bits, False, True)
        elif g == 1:
            assert E.exl3_gemv_mr(Xm, Ts[0], want, SUs[0], None, SVs[0], bits, False, True) == 0
        elif len(set(widths)) == 1:
            assert E.exl3_gemv_mr_grouped(Xm, Ts, want, SUs, None, SVs, bits, False, True, g) == 0
        else:
            assert E.exl3_gemv_mr_grouped_widths(Xm, Ts, want, SUs, SVs, bits, False, True) == 0
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (m, gemv)
        rows = [0, m - 1]
        ref = np.concatenate([cpu.linear(x[rows], t, bits, s, v, 2) for t, s, v in mats], axis=1)
        assert_close(got[rows].cpu().numpy(), ref, (k, widths, m))
