"""GPU parity on the reference checkpoint's own layer shapes (run with -m gpu on an MI355X).

The reference checks and times its kernels on the Qwen3.8-27B checkpoint's shapes
(vllm_plugin/tests/gemv_bench.py:18-28, vllm_plugin/tests/mr_check.py:20-42,
vllm_plugin/tests/prefill_gemm_bench.py:8).  Several lie outside the synthetic configuration-1
layer set:

* attention q (with its gate) 5120 -> 12288, GDN qkv 5120 -> 10240, GDN z 5120 -> 6144;
* attention o / GDN out 6144 -> 5120: k = 6144, 48 Hadamard blocks per column block;
* lm_head 5120 -> 248320: 1,940 column blocks, the largest completion-counter plan the GEMV
  takes (the counter region holds 2,048).

Checks:
* GEMV, every shape and bitrate of the reference's scoreboard: M = 1 against the oracle (the
  parity bar, the reference's normalized-RMS gate, and one last-place step per fp16 rounding on
  any element beyond its max-abs gate: assert_m1); every row of an m-row call bitwise equal to
  its M = 1 call for m in {2, 3, 4, 8, 12, 16, 32} (the reference's mr_check); all 32 rows
  against the oracle.
* lm_head at M = 1 and M = 32: column slices (first, middle and last blocks) against the oracle;
  the 8- and 32-row calls bitwise equal to the M = 1 calls on every column.
* prefill at M = 2048 on 5120 -> 10240, 6144 -> 5120 and 5120 -> 248320: whole tiles bitwise
  equal to exl3_gemm_trellis (the never-splitting entry point), split tiles to the parity bar,
  rows spread over every row tile against the oracle.
* configuration 1's M = 8 legs at 4 bpw through the ops: the grouped gate/up launch, the
  grouped-widths q/k/v launch (5120 / 1024 / 1024) and down, against the oracle.
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

LM_HEAD_N = 248320
PC_CUS, PC_MT = 256, 256            # prefill: tiles per wave (one per CU) and rows per tile

# (k, n, bits): the reference scoreboard's shapes outside GEMV_CASES of test_gpu_parity
CKPT_GEMV = [
    (5120, 12288, 2), (5120, 12288, 4),                   # attention q (+ gate)
    (5120, 10240, 2), (5120, 10240, 4),                   # GDN qkv
    (5120, 6144, 4),                                      # GDN z
    (6144, 5120, 3), (6144, 5120, 4), (6144, 5120, 5),    # attention o, GDN out
    (5120, 17408, 2), (5120, 17408, 1),                   # gate / up at 2 and 1 bpw
]
ROW_COUNTS = (2, 3, 4, 8, 12, 16, 32)


def _linear(X, T, SU, SV, bits):
    return torch.ops.exl3rocm.linear(X, T, SU, SV, bits, False, True)


def ulp16(v):
    """fp16 last-place step at magnitude |v| (normal range; 2^-24 below it)."""
    e = np.floor(np.log2(np.maximum(np.abs(np.asarray(v, dtype=np.float64)), 2.0 ** -14)))
    return 2.0 ** (e - 10)


def assert_m1(got, ref, svh, what):
    """An M = 1 output against the faithful oracle: the parity bar and the reference's
    normalized-RMS gate (2e-4); its normalized max-abs gate (3e-3) becomes a per-element bound for
    the elements beyond it: one last-place step of each fp16 rounding after the sums,
    |got - ref| <= |svh| ulp(h) + ulp(y) with h = y / svh the rotated C before its svh scale.
    The max-abs gate is a sample statistic: fp32 sums that land on the other side of a rounding
    boundary than the exact sum flip single outputs (an output of 84 by 1/16, 3.1e-3 of an RMS
    of 20), and 17,408 outputs at 2 bpw do."""
    st = assert_close(got, ref, what)
    assert st["normalized_rms_err"] <= 2e-4, (what, st)
    g = np.asarray(got, dtype=np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    sv = np.abs(np.asarray(svh, dtype=np.float64).ravel())
    rms = np.sqrt(np.mean(r ** 2))
    d = np.abs(g - r)
    big = d > 3e-3 * rms
    bound = sv[big] * ulp16(r[big] / sv[big]) + ulp16(r[big])
    assert bool(np.all(d[big] <= bound)), (what, int(big.sum()), (d[big] / bound).max())


@pytest.mark.parametrize("k,n,bits", CKPT_GEMV)
def test_checkpoint_gemv_rows_and_oracle(k, n, bits, monkeypatch):
    monkeypatch.setattr(ops, "MR_MAX", 32)             # the GEMV route up to 32 rows on every shape
    tr, su, sv = synth.layer("ckpt", f"{k}x{n}x{bits}", k, n, bits)
    x = synth.activations(synth.key_of("ckpt", f"{k}x{n}x{bits}", "x"), 32, k)
    X, T, SU, SV = to_dev(x, tr.view(np.int16), su, sv)
    print(f"checkpoint GEMV k={k} n={n} bits={bits}", flush=True)
    rows1 = torch.cat([_linear(X[r:r + 1], T, SU, SV, bits) for r in range(32)])
    for m in ROW_COUNTS:
        ym = _linear(X[:m], T, SU, SV, bits)
        assert torch.equal(ym.view(torch.int16), rows1[:m].view(torch.int16)), m
    torch.cuda.synchronize()
    ref = cpu.linear(x, tr, bits, su, sv, 2)
    got = rows1.cpu().numpy()
    assert_m1(got[:1], ref[:1], sv, (k, n, bits, "M=1"))
    assert_close(got, ref, (k, n, bits, "32 rows"))


def _device_trellis(k, n, bits, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randint(0, 65536, (k // 16, n // 16, 16 * bits), device=DEV, dtype=torch.int32,
                         generator=g).to(torch.int16)


def _slice_ref(x, T, bits, su, sv, c0, c1):
    """Oracle output columns [c0, c1) (whole 128-column blocks): the trellis tiles of those
    columns and their svh."""
    tr = T[:, c0 // 16:c1 // 16, :].contiguous().cpu().numpy().view(np.uint16)
    return cpu.linear(x, tr, bits, su, sv[c0:c1], 2)


LM_SLICES = [(0, 1024), (124160 - 512, 124160 + 512), (LM_HEAD_N - 1024, LM_HEAD_N)]


def test_lm_head_gemv_m1_m32():
    """5120 -> 248320 at 4 bpw: 77,600 units over 512 workgroups and 1,940 completion counters."""
    k, n, bits = 5120, LM_HEAD_N, 4
    assert n // 128 <= 2048                             # one completion counter per column block
    T = _device_trellis(k, n, bits, 248320)
    su = synth.scales(synth.key_of("ckpt-lm", "suh"), k)
    sv = synth.scales(synth.key_of("ckpt-lm", "svh"), n)
    x = synth.activations(synth.key_of("ckpt-lm", "x"), 32, k)
    X, SU, SV = to_dev(x, su, sv)
    print(f"lm_head GEMV k={k} n={n}", flush=True)
    rows1 = torch.cat([_linear(X[r:r + 1], T, SU, SV, bits) for r in range(32)])
    for m in (8, 32):
        ym = _linear(X[:m], T, SU, SV, bits)
        assert torch.equal(ym.view(torch.int16), rows1[:m].view(torch.int16)), m
    again = _linear(X[:1], T, SU, SV, bits)            # counters left zero: repeatable
    assert torch.equal(again.view(torch.int16), rows1[:1].view(torch.int16))
    torch.cuda.synchronize()
    for c0, c1 in LM_SLICES:
        ref = _slice_ref(x, T, bits, su, sv, c0, c1)
        got = rows1[:, c0:c1].cpu().numpy()
        assert_m1(got[:1], ref[:1], sv[c0:c1], ("lm_head M=1", c0))
        assert_close(got, ref, ("lm_head 32 rows", c0))


def _prefill_plan(m, k, n):
    wa = (ctypes.c_int * 1)(n)
    ws = int(_lib.lib().exl3_gemm_trellis_workspace_size(m, k, wa, 1))
    tiles_n = n // 128
    tiles = ((m + PC_MT - 1) // PC_MT) * tiles_n
    n_full = (tiles // PC_CUS) * PC_CUS if ws > 0 else tiles
    return ws, tiles_n, n_full


@pytest.mark.parametrize("k,n", [(5120, 10240), (6144, 5120), (5120, LM_HEAD_N)])
def test_checkpoint_prefill_m2048(k, n):
    """M = 2048, 4 bpw: 5120 -> 10240 (640 tiles: the 128-tile tail in 2 pieces), 6144 -> 5120
    (320 tiles: the 64-tile tail in 4 pieces of 24 steps), lm_head (15,520 tiles, no split)."""
    m, bits = 2048, 4
    ws, tiles_n, n_full = _prefill_plan(m, k, n)
    assert (ws > 0) == (n != LM_HEAD_N)
    T = _device_trellis(k, n, bits, k * 7 + n)
    su = synth.scales(synth.key_of("ckpt-pf", k, n, "suh"), k)
    sv = synth.scales(synth.key_of("ckpt-pf", k, n, "svh"), n)
    x = synth.activations(synth.key_of("ckpt-pf", k, n, "x"), m, k)
    X, SU, SV = to_dev(x, su, sv)
    print(f"checkpoint prefill m={m} k={k} n={n} whole tiles {n_full}", flush=True)
    y = _linear(X, T, SU, SV, bits)
    y0 = torch.empty_like(y)
    E.exl3_gemm_trellis(X, T, y0, SU, torch.empty_like(X), SV, bits, False, True)
    # whole tiles: tile u -> row tile u // tiles_n, column tile u % tiles_n
    r_full = (n_full // tiles_n) * PC_MT
    c_full = (n_full % tiles_n) * 128
    assert torch.equal(y[:r_full].view(torch.int16), y0[:r_full].view(torch.int16))
    if r_full < m:
        assert torch.equal(y[r_full:r_full + PC_MT, :c_full].view(torch.int16),
                           y0[r_full:r_full + PC_MT, :c_full].view(torch.int16))
        # the last row tiles (split tiles among them) against the unsplit launch
        assert_close(y[r_full:].cpu().numpy(), y0[r_full:].cpu().numpy(), "split vs unsplit")
    y2 = _linear(X, T, SU, SV, bits)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))            # repeatable
    rows = [0, 1, 255, 256 + 77, 1024, 1791, 1792 + 5, 2046, 2047]
    slices = LM_SLICES if n == LM_HEAD_N else [(0, n)]
    torch.cuda.synchronize()
    for c0, c1 in slices:
        ref = _slice_ref(x[rows], T, bits, su, sv, c0, c1)
        assert_close(y[rows, c0:c1].cpu().numpy(), ref, (k, n, c0))


def test_config1_m8_legs_vs_oracle():
    """Configuration 1 at M = 8, 4 bpw, through the ops as the plugin calls them: q/k/v as one
    grouped-widths launch, gate/up as one grouped launch, down alone; every row against the oracle
    and equal to its M = 1 call."""
    bits, m = 4, 8
    spec = {"q": (5120, 5120), "k": (5120, 1024), "v": (5120, 1024), "gate": (5120, 17408),
            "up": (5120, 17408), "down": (17408, 5120)}
    mats = {nm: synth.layer("cfg1-m8", nm, k, n, bits) for nm, (k, n) in spec.items()}
    dev = {nm: to_dev(tr.view(np.int16), su, sv) for nm, (tr, su, sv) in mats.items()}
    x5 = synth.activations(synth.key_of("cfg1-m8", "x5120"), m, 5120)
    x17 = synth.activations(synth.key_of("cfg1-m8", "x17408"), m, 17408)
    X5, X17 = to_dev(x5, x17)
    ops = torch.ops.exl3rocm

    def grouped(X, names):
        return ops.linear_groups(X, [dev[nm][0] for nm in names], [dev[nm][1] for nm in names],
                                 [dev[nm][2] for nm in names], [bits] * len(names), False, True)

    print("config1 M=8 legs", flush=True)
    legs = {("q", "k", "v"): X5, ("gate", "up"): X5, ("down",): X17}
    for names, X in legs.items():
        y = grouped(X, names) if len(names) > 1 else ops.linear(X, *dev[names[0]], bits, False, True)
        y1 = torch.cat([grouped(X[r:r + 1], names) if len(names) > 1 else
                        ops.linear(X[r:r + 1], *dev[names[0]], bits, False, True) for r in range(m)])
        assert torch.equal(y.view(torch.int16), y1.view(torch.int16)), names
        torch.cuda.synchronize()
        xin = x17 if names == ("down",) else x5
        ref = np.concatenate([cpu.linear(xin, mats[nm][0], bits, mats[nm][1], mats[nm][2], 2) for nm in names],
                             axis=1)
        assert_close(y.cpu().numpy(), ref, names)
