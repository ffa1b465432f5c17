"""Seeded sweep over the supported domain of the routed ops (run with -m gpu on an MI355X).

Each case draws rows (1 to 300; every sixth case one row), k and the group widths (multiples
of 128; one case in eight at the reference checkpoint's sizes), the group count (1 to 4), bits (1 to 8, mixed between groups in some cases) and the
codebook, and runs torch.ops.exl3rocm.linear / linear_groups as a model would.  Checks per case:
  * the first, middle and last rows of every group against the oracle (rel-L2 and the per-element
    bound of test_gpu_parity.assert_close);
  * on the columns of every run of equal-K groups that takes the GEMV (rows <= that run's route
    boundary), those rows bitwise equal to the m == 1 call of the same op;
  * a second call bitwise equal to the first (completion counters and split workspaces reset).
The draws cover shapes no hand-written case has (k = 128, single-unit blocks, uneven grouped
widths, GEMM launches of a few tiles), at sizes the oracle finishes in well under a second.
"""
import numpy as np
import pytest
import torch

import cpu
from exl3rocm import _lib, ops, synth
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
