"""Seeded sweep over the supported domain of the routed ops (run with -m gpu on an MI355X).

Each case draws rows (1 to 300; every sixth case one row), k and the group widths (multiples
of 128; one case in eight at the reference checkpoint's sizes), the group count (1 to 4), bits (1 to 8, mixed between groups in some cases) and the
codebook, and runs torch.ops.exl3rocm.linear / linear_groups as a model would.  Checks per case:
  * the first, middle and last rows of every group against the oracle (rel-L2 and the per-element
    bound of test_gpu_parity.assert_close);
  * on the columns of every run of equal-K groups that takes the GEMV (rows <= that run's route
    boundary), those rows bitwise equal to the m == 1 call of the same op;
  * a second call bitwise equal to the first (completion counters and split workspaces reset).
A second sweep runs a gated MLP (hidden k, intermediate n) through linear_silu_mul and
silu_mul_linear: each equal, bitwise, to its unfused composition (linear_groups + silu_mul;
silu_mul + linear) on whatever route the rows take, and both against the oracle.
The draws cover shapes no hand-written case has (k = 128, single-unit blocks, uneven grouped
widths, GEMM launches of a few tiles), at sizes the oracle finishes in well under a second.
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

ROWS = (1, 2, 3, 5, 8, 9, 13, 16, 17, 24, 31, 32, 33, 47, 48, 49, 64, 65, 100, 257, 300)


# checkpoint-sized draws: the reference model's input widths and module output widths
BIG_K = (5120, 6144, 17408)
BIG_N = (1024, 5120, 6144, 10240, 12288, 17408)


def draw(n_cases=144, seed=20261203):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n_cases):
        g = int(rng.choice([1, 1, 2, 2, 3, 4]))
        if i % 8 == 7:                                            # one case in eight: checkpoint-sized
            g = min(g, 2)
            k = int(rng.choice(BIG_K))
            widths = tuple(int(rng.choice(BIG_N)) for _ in range(g))
        else:
            k = 128 * int(rng.integers(1, 33))                    # 128 .. 4096
            widths = tuple(128 * int(rng.integers(1, 25)) for _ in range(g))
        bits = int(rng.integers(1, 9))
        if g > 1 and rng.random() < 0.3:                          # mixed bitrates: runs of equal K
            K = tuple(int(rng.integers(1, 9)) for _ in range(g))
        else:
            K = (bits,) * g
        cb = int(rng.integers(0, 3))
        m = 1 if i % 6 == 0 else int(rng.choice(ROWS))           # every sixth case: one row
        out.append((i, m, k, widths, K, cb))
    return out


CASES = draw()


def gemv_columns(m, k, widths, K):
    """Column ranges of the runs of consecutive equal-K groups (at most the library's group limit
    per run) that take the GEMV at m rows, as the op routes them."""
    cols, i, n0 = [], 0, 0
    while i < len(widths):
        j = i + 1
        while j < len(widths) and j - i < _lib.MAX_GROUPS and K[j] == K[i]:
            j += 1
        w = sum(widths[i:j])
        if ops.gemv_rows(m, k, w):
            cols.append((n0, n0 + w))
        n0 += w
        i = j
    return cols


def run(X, Ts, SUs, SVs, K, cb):
    mcg, mul1 = cb == 1, cb == 2
    if len(Ts) == 1:
        return torch.ops.exl3rocm.linear(X, Ts[0], SUs[0], SVs[0], K[0], mcg, mul1)
    return torch.ops.exl3rocm.linear_groups(X, Ts, SUs, SVs, list(K), mcg, mul1)


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-m{c[1]}-k{c[2]}-n{'+'.join(map(str, c[3]))}-K{''.join(map(str, c[4]))}-cb{c[5]}"
                                             for c in CASES])
def test_sweep_routed_ops_vs_oracle(case):
    i, m, k, widths, K, cb = case
    print(f"sweep case {i}: m={m} k={k} widths={widths} K={K} cb={cb}", flush=True)
    tag = f"sweep{i}"
    mats = [synth.layer(tag, g, k, n, bits) for g, (n, bits) in enumerate(zip(widths, K))]
    x = synth.activations(synth.key_of(tag, "x"), m, k)
    X = to_dev(x)[0]
    Ts = [to_dev(tr.view(np.int16))[0] for tr, _, _ in mats]
    SUs = [to_dev(su)[0] for _, su, _ in mats]
    SVs = [to_dev(sv)[0] for _, _, sv in mats]
    y = run(X, Ts, SUs, SVs, K, cb)
    assert y.shape == (m, sum(widths)) and y.dtype == torch.float16
    rows = sorted({0, m // 2, m - 1})
    n0 = 0
    for (tr, su, sv), n, bits in zip(mats, widths, K):
        ref = cpu.linear(x[rows], tr, bits, su, sv, cb)
        assert_close(y[rows, n0:n0 + n].cpu().numpy(), ref, ("oracle", n0, bits))
        n0 += n
    for c0, c1 in gemv_columns(m, k, widths, K):
        for r in rows:
            y1 = run(X[r:r + 1], Ts, SUs, SVs, K, cb)
            assert torch.equal(y[r, c0:c1].view(torch.int16), y1[0, c0:c1].view(torch.int16)), ("row == m=1", r, c0)
    again = run(X, Ts, SUs, SVs, K, cb)
    assert torch.equal(y.view(torch.int16), again.view(torch.int16)), "repeat call"
    torch.cuda.synchronize()


def draw_mlp(n_cases=48, seed=20261204):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n_cases):
        if i % 8 == 7:                                            # the reference model's MLP
            k, n = 5120, 17408
        else:
            k = 128 * int(rng.integers(1, 33))                    # hidden 128 .. 4096
            n = 128 * int(rng.integers(1, 25))                    # intermediate 128 .. 3072
        bits = int(rng.integers(1, 9))
        cb = int(rng.integers(0, 3))
        m = 1 if i % 6 == 0 else int(rng.choice(ROWS))
        out.append((i, m, k, n, bits, cb))
    return out


MLP_CASES = draw_mlp()


def silu_mul_ref(g, u):
    """fp16(fp16(silu(g)) * u) in float64, one rounding each."""
    g, u = np.asarray(g, np.float64), np.asarray(u, np.float64)
    with np.errstate(over="ignore"):                  # exp(-g) = inf for very negative g: silu -> -0
        return O.to_f16(O.to_f16(g / (1.0 + np.exp(-g))) * u)


@pytest.mark.parametrize("case", MLP_CASES, ids=[f"{c[0]}-m{c[1]}-k{c[2]}-n{c[3]}-K{c[4]}-cb{c[5]}" for c in MLP_CASES])
def test_sweep_mlp_ops_vs_oracle(case):
    i, m, k, n, bits, cb = case
    print(f"mlp sweep case {i}: m={m} k={k} n={n} K={bits} cb={cb}", flush=True)
    mcg, mul1 = cb == 1, cb == 2
    tag = f"mlpsweep{i}"
    gate, up = (synth.layer(tag, g, k, n, bits) for g in range(2))
    down = synth.layer(tag, 2, n, k, bits)
    x = synth.activations(synth.key_of(tag, "x"), m, k)
    rows = sorted({0, m // 2, m - 1})
    # a power-of-two input scale that puts the gate outputs near unit RMS, as a normalised MLP
    # input would (unit-scale random weights give outputs ~ sqrt(k): SiLU(g) * u and then the down
    # projection would overflow fp16)
    g0 = cpu.linear(x[rows], gate[0], bits, gate[1], gate[2], cb).astype(np.float64)
    x = (x.astype(np.float32) * 2.0 ** -np.round(np.log2(np.sqrt(np.mean(g0 ** 2)) + 1e-30))).astype(np.float16)
    X = to_dev(x)[0]
    Tgu = [to_dev(tr.view(np.int16))[0] for tr, _, _ in (gate, up)]
    SUgu = [to_dev(su)[0] for _, su, _ in (gate, up)]
    SVgu = [to_dev(sv)[0] for _, _, sv in (gate, up)]
    Td, SUd, SVd = to_dev(down[0].view(np.int16), down[1], down[2])
    act = torch.ops.exl3rocm.linear_silu_mul(X, Tgu, SUgu, SVgu, [bits, bits], mcg, mul1)
    gu = torch.ops.exl3rocm.linear_groups(X, Tgu, SUgu, SVgu, [bits, bits], mcg, mul1)
    act2 = torch.empty_like(act)
    E.silu_mul(gu[:, :n], gu[:, n:], act2)
    assert torch.equal(act.view(torch.int16), act2.view(torch.int16)), "linear_silu_mul == linear_groups + silu_mul"
    assert torch.isfinite(act).all()
    g_ref, u_ref = (cpu.linear(x[rows], tr, bits, su, sv, cb) for tr, su, sv in (gate, up))
    assert_close(act[rows].cpu().numpy(), silu_mul_ref(g_ref, u_ref), "act vs oracle")
    y = torch.ops.exl3rocm.silu_mul_linear(gu, Td, SUd, SVd, bits, mcg, mul1)
    y2 = torch.ops.exl3rocm.linear(act, Td, SUd, SVd, bits, mcg, mul1)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), "silu_mul_linear == silu_mul + linear"
    assert torch.isfinite(y).all()
    act_rows = act[rows].cpu().numpy()
    assert_close(y[rows].cpu().numpy(), cpu.linear(act_rows, down[0], bits, down[1], down[2], cb), "down vs oracle")
    if ops.gemv_rows(m, n, k):
        for r in rows:
            y1 = torch.ops.exl3rocm.silu_mul_linear(gu[r:r + 1], Td, SUd, SVd, bits, mcg, mul1)
            assert torch.equal(y[r].view(torch.int16), y1[0].view(torch.int16)), ("row == m=1", r)
    again = torch.ops.exl3rocm.silu_mul_linear(gu, Td, SUd, SVd, bits, mcg, mul1)
    assert torch.equal(y.view(torch.int16), again.view(torch.int16)), "repeat call"
    torch.cuda.synchronize()
