"""GPU parity of the opt-in approximate mul1 GEMV routes (exl3_gemv_mr_approx) against the oracle
(run with -m gpu on an MI355X).

* affine (mode 1): C from the unrounded mul1 weights.  Against oracle.linear_approx_rotated("affine")
  to fp32-accumulation noise, and against the faithful output within the rel-L2 1e-3 bar.
* int8 (mode 2): the rotated input quantized per (row, 128-input slice), the reference's int8
  activation path (reference exl3_oracle.py:357-412; gates of the reference's
  tests/test_gpu_int8.py: NRMS < 2e-3 and cosine > 0.999999 against the int8 oracle), plus the
  int8 error family against the faithful output.
Both: every row of an m-row call equals its m == 1 call bitwise, and the op route
(EXL3_GEMV_APPROX) calls them.
"""
import numpy as np
import pytest
import torch

import exl3_oracle as O
from exl3rocm import kernels as E, ops, synth
from test_gpu_parity import DEV, assert_close, stats, to_dev

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

CASES = [(256, 128, 3), (1024, 512, 4), (5120, 1024, 4), (5120, 5120, 2), (17408, 5120, 4), (2048, 1024, 6)]


def run(mode, x, tr, su, sv, bits):
    X, T, SU, SV = to_dev(x, tr.view(np.int16), su, sv)
    y = torch.empty(x.shape[0], sv.shape[0], dtype=torch.float16, device=DEV)
    assert E.exl3_gemv_mr_approx(X, T, y, SU, None, SV, bits, mode) == 0
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("k,n,bits", CASES)
@pytest.mark.parametrize("mode", ["affine", "int8"])
def test_approx_vs_oracle(mode, k, n, bits):
    tr, su, sv = synth.layer("approx", f"{k}x{n}x{bits}", k, n, bits)
    m = 3
    x = synth.activations(synth.key_of("approx", k, n, bits, "x"), m, k, heavy_tail=(k == 5120))
    print(f"approx {mode}: k={k} n={n} bits={bits}", flush=True)
    got = run(mode, x, tr, su, sv, bits).astype(np.float64)
    ref = O.linear_approx(x, tr, bits, su, sv, mode)
    st = stats(got, ref)
    # the same arithmetic up to fp32 accumulation order (and, for int8, a rounding tie of a / q
    # in float32 against float64 now and then)
    assert st["rel_l2"] <= (2e-4 if mode == "affine" else 1e-3), st
    assert st["normalized_rms_err"] < 2e-3 and st["cosine_similarity"] > 0.999999, st
    faithful = O.linear(x, tr, bits, su, sv, 2)
    dev = stats(got, faithful)
    if mode == "affine":
        assert dev["rel_l2"] <= 1e-3, dev
    else:
        assert dev["rel_l2"] <= 2e-2 and dev["cosine_similarity"] > 0.999, dev   # the int8 error family


@pytest.mark.parametrize("k,n", [(5120, 2048), (5120, 1024), (2048, 5120), (17408, 1024)])
@pytest.mark.parametrize("mode", ["affine", "int8"])
def test_approx_rows_equal_m1(mode, k, n):
    """Row sums (affine) and scales (int8) of the single-row layout (2 values a lane) equal the
    multi-row layout's (8 a lane) bitwise, whichever layout a workgroup's unit count selects."""
    bits = 4
    tr, su, sv = synth.layer("approx-rows", f"{mode}{k}x{n}", k, n, bits)
    x = synth.activations(synth.key_of("approx-rows", mode, k, n, "x"), 32, k)
    X, T, SU, SV = to_dev(x, tr.view(np.int16), su, sv)
    rows1 = []
    for r in range(32):
        y1 = torch.empty(1, n, dtype=torch.float16, device=DEV)
        E.exl3_gemv_mr_approx(X[r:r + 1], T, y1, SU, None, SV, bits, mode)
        rows1.append(y1)
    rows1 = torch.cat(rows1)
    for m in (2, 8, 12, 32):
        ym = torch.empty(m, n, dtype=torch.float16, device=DEV)
        E.exl3_gemv_mr_approx(X[:m], T, ym, SU, None, SV, bits, mode)
        assert torch.equal(ym.view(torch.int16), rows1[:m].view(torch.int16)), (mode, m)
    torch.cuda.synchronize()
    assert_close(rows1.cpu().numpy(), O.linear_approx(x, tr, bits, su, sv, mode), mode)


def test_approx_op_route(monkeypatch):
    k, n, bits = 1024, 768, 4
    tr, su, sv = synth.layer("approx-op", 0, k, n, bits)
    x = synth.activations(synth.key_of("approx-op", "x"), 4, k)
    X, T, SU, SV = to_dev(x, tr.view(np.int16), su, sv)
    for mode in ("affine", "int8"):
        monkeypatch.setattr(ops, "GEMV_APPROX", mode)
        y = torch.ops.exl3rocm.linear(X, T, SU, SV, bits, False, True)
        yg = torch.ops.exl3rocm.linear_groups(X, [T, T], [SU, SU], [SV, SV], [bits, bits], False, True)
        want = torch.empty_like(y)
        E.exl3_gemv_mr_approx(X, T, want, SU, None, SV, bits, mode)
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))
        assert torch.equal(yg[:, :n].view(torch.int16), want.view(torch.int16))
        assert torch.equal(yg[:, n:].view(torch.int16), want.view(torch.int16))
    monkeypatch.setattr(ops, "GEMV_APPROX", "")
    faithful = torch.ops.exl3rocm.linear(X, T, SU, SV, bits, False, True)
    assert not torch.equal(faithful.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("mode", ["affine", "int8"])
def test_approx_streams_and_graph_replays_are_deterministic(mode):
    """Four layers on four streams (each its own workspace), 20 rounds, equal their serial
    results bitwise; a captured graph of one call replays to the eager result (the reference's
    int8 contract, tests/test_int8_contract.py: concurrent-stream determinism; here the route is
    also graph-capturable rather than falling back under capture)."""
    k, n, bits = 1024, 512, 4
    layers = []
    for i in range(4):
        tr, su, sv = synth.layer("approx-streams", i, k, n, bits)
        x = synth.activations(synth.key_of("approx-streams", i, "x"), 2, k)
        layers.append(to_dev(x, tr.view(np.int16), su, sv))
    outs = [torch.empty(2, n, dtype=torch.float16, device=DEV) for _ in layers]
    want = []
    for (X, T, SU, SV), y in zip(layers, outs):
        E.exl3_gemv_mr_approx(X, T, y, SU, None, SV, bits, mode)
        want.append(y.clone())
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in layers]
    for _ in range(20):
        for s, (X, T, SU, SV), y in zip(streams, layers, outs):
            with torch.cuda.stream(s):
                E.exl3_gemv_mr_approx(X, T, y, SU, None, SV, bits, mode)
    torch.cuda.synchronize()
    for y, w in zip(outs, want):
        assert torch.equal(y.view(torch.int16), w.view(torch.int16))
    X, T, SU, SV = layers[0]
    y = torch.empty(2, n, dtype=torch.float16, device=DEV)
    s = streams[0]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        E.exl3_gemv_mr_approx(X, T, y, SU, None, SV, bits, mode)
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want[0].view(torch.int16))
