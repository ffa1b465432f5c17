"""GPU parity of the down-projection GEMV with the SiLU-and-mul input formed as it loads
(exl3_gemv_silu_in, op exl3rocm::silu_mul_linear) -- run with -m gpu on an MI355X.

The fused form must equal the two-launch form (exl3_silu_mul, then exl3_gemv_mr) bitwise at every
row count (in-LDS rotation below the pre-rotation row count, the pre-rotation pass from it), every
row must equal its m == 1 call, and the result must meet the north-star bar against the oracle
(act = fp16(fp16(silu(g)) * u) in float64, then the faithful linear).
"""
import numpy as np
import pytest
import torch

import cpu
import exl3_oracle as O
from exl3rocm import _lib, kernels as E, ops, synth
from test_gpu_parity import DEV, assert_close, to_dev

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]


def down(k, n, bits, m, tag="silu-in", spread=1.0):
    tr, su, sv = synth.layer(tag, f"{k}x{n}x{bits}", k, n, bits)
    gu = synth.activations(synth.key_of(tag, f"{k}x{n}x{bits}", "gu", m), m, 2 * k)
    gu = (gu.astype(np.float32) * spread).astype(np.float16)
    return gu, tr, su, sv


def two_launch(GU, T, SU, SV, k, bits, mcg, mul1):
    act = torch.empty(GU.shape[0], k, dtype=torch.float16, device=DEV)
    E.silu_mul(GU[:, :k], GU[:, k:], act)
    y = torch.empty(GU.shape[0], SV.shape[0], dtype=torch.float16, device=DEV)
    assert E.exl3_gemv_mr(act, T, y, SU, None, SV, bits, mcg, mul1) == 0
    return act, y


def fused(GU, T, SU, SV, k, bits, mcg, mul1, A_had=None):
    y = torch.empty(GU.shape[0], SV.shape[0], dtype=torch.float16, device=DEV)
    assert E.exl3_gemv_silu_in(GU[:, :k], GU[:, k:], T, y, SU, A_had, SV, bits, mcg, mul1) == 0
    return y


def same(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def raw_silu_in(GU, T, SU, SV, k, bits, mcg, mul1):
    """The C-ABI call without A_had: the kernel rotates (and applies the SiLU) in LDS at any m."""
    m, n = GU.shape[0], SV.shape[0]
    y = torch.empty(m, n, dtype=torch.float16, device=DEV)
    ws = E.workspace(GU.device, E.gemv_workspace_bytes(m, k, n, bits))
    rc = _lib.lib().exl3_gemv_silu_in(GU.data_ptr(), GU.data_ptr() + 2 * k, GU.stride(0), T.data_ptr(), y.data_ptr(),
                                      n, SU.data_ptr(), None, SV.data_ptr(), m, k, n, bits, int(mcg), int(mul1),
                                      ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return y


@pytest.mark.parametrize("m,k,n,bits,cb", [(1, 17408, 5120, 4, 2), (2, 17408, 5120, 4, 2), (4, 17408, 5120, 4, 2),
                                           (5, 17408, 5120, 4, 2), (8, 17408, 5120, 4, 2), (12, 17408, 5120, 4, 2),
                                           (16, 17408, 5120, 4, 2), (6, 1024, 768, 4, 2), (9, 1024, 768, 4, 2),
                                           (32, 17408, 5120, 4, 2), (1, 512, 256, 3, 0), (3, 1024, 768, 2, 1),
                                           (16, 2048, 1024, 6, 2), (11, 256, 128, 8, 1)])
def test_silu_in_matches_two_launches(m, k, n, bits, cb):
    gu, tr, su, sv = down(k, n, bits, m)
    print(f"silu_in m={m} k={k} n={n} bits={bits} cb={cb}", flush=True)
    GU, T, SU, SV = to_dev(gu, tr.view(np.int16), su, sv)
    mcg, mul1 = cb == 1, cb == 2
    act, want = two_launch(GU, T, SU, SV, k, bits, mcg, mul1)
    got = fused(GU, T, SU, SV, k, bits, mcg, mul1)
    assert same(got, want), "fused input == silu_mul then exl3_gemv_mr"
    if m > 1:
        # the pre-rotation pass (from the library's SiLU pre-rotation row count, 4 unless
        # EXL3_GEMV_SILU_PREROT_M sets it) leaves the rotated activation in A_had; without A_had
        # the kernel forms and rotates it in LDS
        xr = torch.empty(m * k, dtype=torch.float16, device=DEV)
        assert same(fused(GU, T, SU, SV, k, bits, mcg, mul1, A_had=xr), want)
        assert same(raw_silu_in(GU, T, SU, SV, k, bits, mcg, mul1), want), "in-LDS form"
        if m >= int(_lib.lib().exl3_gemv_silu_prerot_rows()):
            xw = torch.empty(m, k, dtype=torch.float16, device=DEV)
            E.had_r_128(act, xw, SU, None, 1.0)
            assert same(xr.view(m, k), xw), "A_had == the exact rotation of the activation"
        y1 = torch.empty(1, n, dtype=torch.float16, device=DEV)
        for r in (0, m - 1):
            assert E.exl3_gemv_silu_in(GU[r:r + 1, :k], GU[r:r + 1, k:], T, y1, SU, None, SV, bits, mcg, mul1) == 0
            assert same(y1, want[r:r + 1]), ("row == its m == 1 call", r)
    torch.cuda.synchronize()


def test_silu_in_vs_oracle():
    m, k, n, bits = 3, 2048, 1024, 4
    gu, tr, su, sv = down(k, n, bits, m, tag="silu-in-oracle", spread=4.0)
    GU, T, SU, SV = to_dev(gu, tr.view(np.int16), su, sv)
    got = fused(GU, T, SU, SV, k, bits, False, True)
    g, u = gu[:, :k].astype(np.float64), gu[:, k:].astype(np.float64)
    with np.errstate(over="ignore"):                  # exp(-g) = inf for very negative g: silu -> -0
        act = O.to_f16(O.to_f16(g / (1.0 + np.exp(-g))) * u)
    ref = cpu.linear(act.astype(np.float16), tr, bits, su, sv, 2)
    torch.cuda.synchronize()
    assert_close(got.cpu().numpy(), ref, "silu_in vs oracle")


def test_silu_in_saturating_gate():
    """Gate values out to about +-40 (silu underflows to -0 and saturates to g) and large up values."""
    m, k, n, bits = 2, 1024, 512, 4
    gu, tr, su, sv = down(k, n, bits, m, tag="silu-in-sat", spread=8.0)
    GU, T, SU, SV = to_dev(gu, tr.view(np.int16), su, sv)
    _, want = two_launch(GU, T, SU, SV, k, bits, False, True)
    assert same(fused(GU, T, SU, SV, k, bits, False, True), want)
    assert torch.isfinite(want).all()


@pytest.mark.parametrize("m", [1, 5, 40])
def test_silu_mul_linear_op(m):
    """The op: M <= 32 on the fused GEMV, M > 32 on the prefill whose input transform forms the
    activation; == the two-launch form bitwise; rows of a [b, s, 2k] input keep their leading
    shape."""
    k, n, bits = 1024, 768, 4
    gu, tr, su, sv = down(k, n, bits, m, tag="silu-in-op")
    GU, T, SU, SV = to_dev(gu, tr.view(np.int16), su, sv)
    y = torch.ops.exl3rocm.silu_mul_linear(GU.view(1, m, 2 * k), T, SU, SV, bits, False, True)
    assert y.shape == (1, m, n)
    act = torch.empty(m, k, dtype=torch.float16, device=DEV)
    E.silu_mul(GU[:, :k], GU[:, k:], act)
    want = torch.ops.exl3rocm.linear(act, T, SU, SV, bits, False, True)
    assert same(y.view(m, n), want)
    with pytest.raises(RuntimeError):
        torch.ops.exl3rocm.silu_mul_linear(GU[:, :k], T, SU, SV, bits, False, True)


def test_silu_in_graph_replays():
    m, k, n, bits = 4, 17408, 5120, 4
    gu, tr, su, sv = down(k, n, bits, m, tag="silu-in-graph")
    GU, T, SU, SV = to_dev(gu, tr.view(np.int16), su, sv)
    eager = fused(GU, T, SU, SV, k, bits, False, True)
    y = torch.empty_like(eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.reserve_workspace(DEV, k, n, bits)
        E.exl3_gemv_silu_in(GU[:, :k], GU[:, k:], T, y, SU, None, SV, bits, False, True)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        E.exl3_gemv_silu_in(GU[:, :k], GU[:, k:], T, y, SU, None, SV, bits, False, True)
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert same(y, eager)
        eager = fused(GU, T, SU, SV, k, bits, False, True)
        torch.cuda.synchronize()


@pytest.mark.parametrize("m,k,n", [(300, 1024, 768), (2048, 17408, 5120)])
def test_prefill_silu_in_matches_two_launch(m, k, n):
    """exl3_gemm_trellis_silu_in (the prefill's input transform forms act = fp16(fp16(silu(g)) * u)
    as it loads gate and up) == exl3_silu_mul, then the grouped prefill of act: output and rotated
    input bitwise, with ragged rows (300: two row blocks) and at config 4's down shape (2048 x
    17408 -> 5120: a split tail), activations spread x4; and the oracle bar on the first rows."""
    bits = 4
    gu, tr, su, sv = down(k, n, bits, m, tag="silu-in-prefill", spread=4.0)
    GU, T, SU, SV = to_dev(gu, tr.view(np.int16), su, sv)
    act = torch.empty(m, k, dtype=torch.float16, device=DEV)
    E.silu_mul(GU[:, :k], GU[:, k:], act)
    want = torch.empty(m, n, dtype=torch.float16, device=DEV)
    xh0 = torch.empty(m, k, dtype=torch.float16, device=DEV)
    E.exl3_gemm_trellis_grouped(act, [T], want, [SU], xh0, [SV], bits, False, True)
    y = torch.full((m, n), float("nan"), dtype=torch.float16, device=DEV)
    xh = torch.full((m, k), float("nan"), dtype=torch.float16, device=DEV)
    E.exl3_gemm_trellis_silu_in(GU[:, :k], GU[:, k:], T, y, SU, xh, SV, bits, False, True)
    torch.cuda.synchronize()
    assert same(xh, xh0)
    assert same(y, want)
    if m <= 300:
        g = gu[:4, :k].astype(np.float64)
        u = gu[:4, k:].astype(np.float64)
        with np.errstate(over="ignore"):
            a = O.to_f16(O.to_f16(g / (1.0 + np.exp(-g))) * u)
        assert_close(y[:4].cpu().numpy(), cpu.linear(a.astype(np.float16), tr, bits, su, sv, 2), "prefill silu_in")


def test_prefill_silu_in_graph_replays():
    """silu_mul_linear at M = 64 (the prefill route: the input transform forms the activation, the
    tiles split along K) captured in a graph after an eager warm-up on the capture stream (which
    sizes its workspace): every replay, with eager work and synchronisations between them, equals
    the eager result bitwise (the last piece of each split tile resets its counter; no memset node)."""
    m, k, n, bits = 64, 17408, 5120, 4
    gu, tr, su, sv = down(k, n, bits, m, tag="silu-in-prefill-graph")
    GU, T, SU, SV = to_dev(gu, tr.view(np.int16), su, sv)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        eager = torch.ops.exl3rocm.silu_mul_linear(GU, T, SU, SV, bits, False, True)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        y = torch.ops.exl3rocm.silu_mul_linear(GU, T, SU, SV, bits, False, True)
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert same(y, eager)
        with torch.cuda.stream(s):
            again = torch.ops.exl3rocm.silu_mul_linear(GU, T, SU, SV, bits, False, True)
        torch.cuda.synchronize()
        assert same(again, eager)


@pytest.mark.parametrize("m", [1, 5, 40])
def test_plugin_apply_silu_mul(m):
    """The plugin's hook for a model's MLP (in place of act_fn + down_proj): a down layer created
    and loaded through Exl3LinearMethod; apply_silu_mul(layer, gu) == apply(layer, silu_mul(gu))
    bitwise (fused GEMV at 1 and 5 rows, the prefill's input transform at 40), to the bar against
    the oracle, leading shape, dtype and bias kept; a gu of the wrong width is rejected."""
    from exl3rocm import plugin
    k, n, bits = 1024, 768, 4
    method = plugin.Exl3LinearMethod(plugin.Exl3Config("mul1"), [("down", bits, k, n)])
    lay = torch.nn.Module()
    method.create_weights(lay, k, [n], k, n, torch.float16)
    lay.to(DEV)
    gu, tr, su, sv = down(k, n, bits, m, tag="silu-plugin", spread=4.0)
    lay.trellis.weight_loader(lay.trellis, torch.from_numpy(tr.view(np.int16)))
    lay.suh.weight_loader(lay.suh, torch.from_numpy(su))
    lay.svh.weight_loader(lay.svh, torch.from_numpy(sv))
    lay.mul1.weight_loader(lay.mul1, torch.tensor(0x83DCD12D))
    method.process_weights_after_loading(lay)
    GU = to_dev(gu)[0]
    y = method.apply_silu_mul(lay, GU.view(1, m, 2 * k))
    assert y.shape == (1, m, n) and y.dtype == torch.float16
    act = torch.empty(m, k, dtype=torch.float16, device=DEV)
    E.silu_mul(GU[:, :k], GU[:, k:], act)
    want = method.apply(lay, act)
    assert same(y.view(m, n), want)
    g, u = gu[:, :k].astype(np.float64), gu[:, k:].astype(np.float64)
    with np.errstate(over="ignore"):
        a = O.to_f16(O.to_f16(g / (1.0 + np.exp(-g))) * u)
    ref = cpu.linear(a.astype(np.float16), tr, bits, su, sv, 2)
    torch.cuda.synchronize()
    assert_close(y.view(m, n).cpu().numpy(), ref, ("apply_silu_mul", m))
    yb = method.apply_silu_mul(lay, GU.float(), bias=torch.ones(n, device=DEV))
    assert yb.dtype == torch.float32
    assert torch.equal(yb, want.float() + 1)
    with pytest.raises(ValueError):
        method.apply_silu_mul(lay, GU[:, :k])
