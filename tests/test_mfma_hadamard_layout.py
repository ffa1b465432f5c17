"""CPU checks of the matrix-core Hadamard's operand layout (had128_mfma16 in
qwen38-27b-exl3-rdna4_amd/csrc/exl3_device.h): the 128-point transform of 16 rows as
v_mfma_f32_16x16x32_f16 products D = H^T X^T per 16-column output tile t and 32-input step s.

Restated from the kernel's formulas (lane l: row / column index l & 15, k-chunk g = l >> 4,
element e of the lane's 8-element fragment):
  * output column of tile t, A-row i:  c(t, i) = 32 (t >> 1) + 8 (i >> 2) + 4 (t & 1) + (i & 3)
  * input index of step s:            k = 32 s + 8 g + e
  * A fragment sign:                  (-1)^popcount((t >> 1) & s)  [selects the negated A fragment]
                                      * (-1)^(popcount((j & 3) & (e & 3)) + (t & 1)(e >> 2)
                                               + popcount((j >> 2) & g))
and the result layout D[4 g + e][j] (lane l holds 4 consecutive rows of column j = l & 15).
The checks: the column map is a bijection onto the block, the factorised sign equals the
natural-order Sylvester entry H[c][k] = (-1)^popcount(c & k) for every lane, element, tile and
step, and tiles 2p, 2p + 1 leave the 8 consecutive outputs 32 p + 8 g .. + 7 in each lane.
"""
import numpy as np


def popcount(v):
    return bin(v).count("1")


def col(t, i):
    return 32 * (t >> 1) + 8 * (i >> 2) + 4 * (t & 1) + (i & 3)


def a_sign(j, g, e, tau):
    return -1 if (popcount((j & 3) & (e & 3)) + (tau & (e >> 2)) + popcount((j >> 2) & g)) & 1 else 1


def test_output_columns_cover_the_block_once():
    cols = sorted(col(t, i) for t in range(8) for i in range(16))
    assert cols == list(range(128))


def test_factorised_signs_are_the_sylvester_entries():
    for lane in range(64):
        j, g = lane & 15, lane >> 4
        for t in range(8):
            for s in range(4):
                step = -1 if popcount((t >> 1) & s) & 1 else 1
                for e in range(8):
                    k = 32 * s + 8 * g + e
                    h = -1 if popcount(col(t, j) & k) & 1 else 1
                    assert step * a_sign(j, g, e, t & 1) == h, (lane, t, s, e)


def test_paired_tiles_hold_consecutive_outputs_per_lane():
    for lane in range(64):
        g = lane >> 4
        for p in range(4):
            # result rows 4 g + e' of tiles 2p (e < 4) and 2p + 1 (e >= 4)
            got = [col(2 * p + (e >> 2), 4 * g + (e & 3)) for e in range(8)]
            assert got == list(range(32 * p + 8 * g, 32 * p + 8 * g + 8)), (lane, p, got)


def test_the_products_reproduce_the_transform():
    """The whole sequence with numbers: for random rows, summing A-fragment * B-fragment products
    per (tile, step) in the kernel's order gives x @ H for every output (exact in float64)."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal((16, 128))
    i = np.arange(128)
    H = np.where(np.vectorize(popcount)(i[:, None] & i[None, :]) & 1, -1.0, 1.0)
    want = x @ H
    got = np.zeros((16, 128))
    for t in range(8):
        for lane in range(64):
            j, g = lane & 15, lane >> 4
            for s in range(4):
                step = -1 if popcount((t >> 1) & s) & 1 else 1
                for e in range(8):
                    k = 32 * s + 8 * g + e
                    # A[i = j][k] * B[k][row]: lane l contributes its A row j's products with every row
                    for row in range(16):
                        got[row, col(t, j)] += step * a_sign(j, g, e, t & 1) * x[row, k]
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)
