"""CPU tests pinning the oracle restatement (oracle/exl3_oracle.py, oracle/exl3_cpu.c).

Three kinds of pins, so a plausible mistake (dropped term, wrong shift, transposed index,
wrong rounding) fails at least one of them:
  1. golden vectors written by the reference's own oracle (tests/golden/make_golden.py);
  2. the reference's known-answer and invariant tests (reference tests/test_oracle.py:20-176);
  3. independent restatements (explicit bit ring, Sylvester matrix, closed-form mul1).
The C restatement is pinned against the numpy one and the same golden vectors.
"""
import hashlib

import numpy as np
import pytest

import cpu
import exl3_oracle as O
from exl3rocm import synth

RNG = np.random.default_rng(20260923)


# ------------------------------------------------------------------ golden vectors (reference oracle)
def test_rowcol_golden(golden):
    g, _ = golden
    r, c = O.position_rowcol(np.arange(256))
    np.testing.assert_array_equal(np.stack([r, c]), g["rowcol"])


@pytest.mark.parametrize("bits", range(1, 9))
def test_windows_golden(golden, bits):
    g, _ = golden
    np.testing.assert_array_equal(O.state_windows(g[f"win_tiles_b{bits}"], bits), g[f"win_states_b{bits}"])


@pytest.mark.parametrize("cb", [0, 1, 2])
def test_codebook_tables_golden(golden, cb):
    g, meta = golden
    table = O.codebook_f16(np.arange(65536), cb).view(np.uint16)
    np.testing.assert_array_equal(table[::61], g[f"cb{cb}_sample"])
    assert hashlib.sha256(table.tobytes()).hexdigest() == meta[f"cb{cb}_sha256"]
    # the C restatement decodes the same table
    np.testing.assert_array_equal(cpu.decode_states(np.arange(65536, dtype=np.uint16), cb).view(np.uint16), table)


@pytest.mark.parametrize("bits", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_reconstruct_golden(golden, bits, cb):
    g, _ = golden
    tr = g[f"dt_trellis_b{bits}"]
    want = g[f"dt_W_b{bits}_cb{cb}"]
    np.testing.assert_array_equal(O.reconstruct(tr, bits, cb).view(np.uint16), want)
    np.testing.assert_array_equal(cpu.reconstruct(tr, bits, cb).view(np.uint16), want)


def test_hadamard_stages_golden(golden):
    g, _ = golden
    a, suh, c, svh = g["had_a"], g["had_suh"], g["had_c"], g["had_svh"]
    np.testing.assert_array_equal(O.had_in(a, suh).astype(np.float16).view(np.uint16), g["had_in_faithful"])
    np.testing.assert_array_equal(O.had_out(c, svh).astype(np.float16).view(np.uint16), g["had_out_faithful"])
    np.testing.assert_allclose(O.had_in(a, suh, faithful=False), g["had_in_exact"], rtol=0, atol=1e-12)
    np.testing.assert_allclose(O.had_out(c, svh, faithful=False), g["had_out_exact"], rtol=0, atol=1e-12)
    np.testing.assert_array_equal(cpu.had_in(a, suh)[0].view(np.uint16), g["had_in_faithful"])
    np.testing.assert_array_equal(cpu.had_out(c, svh)[0].view(np.uint16), g["had_out_faithful"])


def test_linear_golden(golden):
    g, meta = golden
    for case in meta["cases"]:
        p = case["name"]
        args = (g[p + "x"], g[p + "trellis"], case["bits"], g[p + "suh"], g[p + "svh"], case["cb"])
        np.testing.assert_array_equal(O.linear(*args).astype(np.float16).view(np.uint16)[0], g[p + "y"], err_msg=p)
        np.testing.assert_array_equal(cpu.linear(*args).view(np.uint16)[0], g[p + "y"], err_msg=p)


def test_headline_config0_golden(golden):
    """K = N = 4096, 4 bpw, mcg, counter-RNG inputs: the C restatement reproduces the reference
    oracle's faithful output bit for bit, and the decoded weights hash identically."""
    g, _ = golden
    tr, su, sv = synth.layer("config0", 0, 4096, 4096, 4)
    x = synth.activations(synth.key_of("config0", 0, "x"), 1, 4096)
    W = cpu.reconstruct(tr, 4, 1)
    assert hashlib.sha256(W.view(np.uint16).tobytes()).digest() == g["config0_W_sha"].tobytes()
    np.testing.assert_array_equal(cpu.linear(x, tr, 4, su, sv, 1).view(np.uint16)[0], g["config0_y"])


# ------------------------------------------------------------------ reference KATs and invariants
@pytest.mark.parametrize("bits", range(1, 9))
def test_state_transition_identity(bits):
    for _ in range(4):
        tile = RNG.integers(0, 65536, size=16 * bits, dtype=np.uint16)
        assert O.transition_ok(O.state_windows(tile, bits), bits)


@pytest.mark.parametrize("bits", [3, 4])
def test_boundary_tiles(bits):
    for tile in (np.zeros(16 * bits, np.uint16), np.full(16 * bits, 0xFFFF, np.uint16),
                 np.arange(16 * bits, dtype=np.uint16), ((np.arange(16 * bits) * 7919) & 0xFFFF).astype(np.uint16)):
        w = O.state_windows(tile, bits)
        assert w.shape == (256,) and O.transition_ok(w, bits)


def test_zero_and_ones_tiles_known_states():
    assert (O.state_windows(np.zeros(48, np.uint16), 3) == 0).all()
    assert (O.state_windows(np.full(48, 0xFFFF, np.uint16), 3) == 0xFFFF).all()


@pytest.mark.parametrize("bits", range(1, 9))
def test_windows_match_explicit_bit_ring(bits):
    """Brute force over an explicit MSB-first bit list, independent of the shift formula."""
    for _ in range(3):
        tile = RNG.integers(0, 65536, size=16 * bits, dtype=np.uint16)
        np.testing.assert_array_equal(O.state_windows(tile, bits), O.state_windows_bruteforce(tile, bits))


def test_position_bijection_and_fragment_table():
    r, c = O.position_rowcol(np.arange(256))
    assert len(set(zip(r.tolist(), c.tolist()))) == 256
    for L in (0, 5, 31):
        rr, cc = O.position_rowcol(np.array([8 * L + i for i in range(8)]))
        r0, cA = 2 * (L % 4), 2 * (L // 8) + ((L >> 2) & 1)
        assert list(zip(rr.tolist(), cc.tolist())) == [(r0, cA), (r0 + 1, cA), (r0 + 8, cA), (r0 + 9, cA),
                                                        (r0, cA + 8), (r0 + 1, cA + 8), (r0 + 8, cA + 8),
                                                        (r0 + 9, cA + 8)]


def test_qblock_layout_used_by_the_kernels():
    """State p of q-block q (tile position 32q + p) sits at column q + 8((p>>2)&1), row
    8((p>>1)&1) + 2(p>>3) + (p&1) -- the decomposition the HIP decoder relies on."""
    t = np.arange(256)
    r, c = O.position_rowcol(t)
    q, p = t >> 5, t & 31
    np.testing.assert_array_equal(c, q + 8 * ((p >> 2) & 1))
    np.testing.assert_array_equal(r, 8 * ((p >> 1) & 1) + 2 * (p >> 3) + (p & 1))


def test_mul1_constants_and_zero_state():
    assert O.K_INV == 0.00676727294921875 and O.K_BIAS == -10.3828125
    v = float(O.codebook_f16(np.array([0]), 2)[0])
    assert v == float(np.float16(O.K_INV * 1024.0 + O.K_BIAS)) == -3.453125


def test_mul1_range_and_affinity():
    vals = O.codebook_f16(np.arange(65536), 2).astype(np.float64)
    assert vals.min() > (0 - 510) / 147.7 - 0.01 and vals.max() < (1020 - 510) / 147.7 + 0.01
    w = np.array([0x1234, 0x5678, 0x9ABC, 0xDEF0])
    s = O.byte_sum(O.codebook_hash(w, 2))
    for si, v in zip(s, O.codebook_f16(w, 2)):
        assert float(v) == float(np.float16(O.K_INV * (1024.0 + float(si)) + O.K_BIAS))


def test_mul1_single_rounding_exact():
    """(1024 + s) * k_inv + k_bias is exact in float64 for every s in [0, 1020] (so rounding it
    once equals a fused fp16 multiply-add), and it differs from a two-rounding evaluation for
    some s -- the test would catch an unfused restatement."""
    s = np.arange(1021, dtype=np.float64)
    exact = (1024.0 + s) * O.K_INV + O.K_BIAS
    scaled = exact * 2.0 ** 18
    assert np.all(scaled == np.round(scaled))          # an integer multiple of 2^-18: exact
    two = (np.float16(1024.0 + s) * np.float16(O.K_INV)).astype(np.float16).astype(np.float64) + O.K_BIAS
    assert np.any(two.astype(np.float16) != exact.astype(np.float16))


def test_known_answers_all_codebooks():
    """Closed-form states 0, 1, 0xFFFF (hand-evaluated from the codebook definitions)."""
    want = {2: (0xC2E8, 0x3921, 0xB936), 1: (0x3F60, 0x304E, 0x3ACD), 0: (0x3A25, 0xBB5B, 0xB110)}
    for cb, bits in want.items():
        got = O.codebook_f16(np.array([0, 1, 0xFFFF]), cb).view(np.uint16)
        assert tuple(int(v) for v in got) == bits, cb


def test_hadamard_matrix_properties():
    H = O.sylvester128()
    assert np.allclose(H @ H.T, 128 * np.eye(128))
    x = RNG.standard_normal((3, 256))
    np.testing.assert_allclose(O.had128(x).reshape(3, 2, 128), (x.reshape(3, 2, 128) @ H.T) * O.R_SCALE, atol=1e-12)
    np.testing.assert_allclose(O.had128(O.had128(x)), x, atol=1e-10)
    imp = np.zeros(128)
    imp[0] = 1.0
    assert np.allclose(np.abs(O.had128(imp)), O.R_SCALE)


def test_pipeline_composition_and_grid():
    tr = RNG.integers(0, 65536, size=(8, 8, 48), dtype=np.uint16)
    a = O.to_f16(RNG.standard_normal(128) * 0.3)
    suh = O.to_f16(np.abs(RNG.standard_normal(128)) + 0.5)
    svh = O.to_f16(np.abs(RNG.standard_normal(128)) + 0.5)
    y = O.linear(a, tr, 3, suh, svh, 2, faithful=False)[0]
    W = O.reconstruct(tr, 3, 2).astype(np.float64)
    np.testing.assert_allclose(y, O.had_out(O.had_in(a, suh, False) @ W, svh, False), atol=1e-12)
    yf = O.linear(a, tr, 3, suh, svh, 2)
    assert (O.to_f16(yf) == yf).all()
    assert np.allclose(O.linear(np.zeros(128), tr, 3, suh, svh, 2), 0.0)
    outl = np.tile([100.0, -100.0], 64)
    outl[0] = 1e4
    assert np.isfinite(O.linear(outl, tr, 3, np.ones(128), np.ones(128), 2)).all()


@pytest.mark.parametrize("bits,cb,m", [(2, 2, 1), (4, 1, 3), (5, 0, 2), (8, 2, 1)])
def test_c_restatement_matches_numpy(bits, cb, m):
    tr = RNG.integers(0, 65536, size=(16, 8, 16 * bits), dtype=np.uint16)
    x = RNG.standard_normal((m, 256)).astype(np.float16)
    su = synth.scales(11, 256)
    sv = synth.scales(12, 128)
    np.testing.assert_array_equal(cpu.reconstruct(tr, bits, cb).view(np.uint16),
                                  O.reconstruct(tr, bits, cb).view(np.uint16))
    np.testing.assert_array_equal(cpu.linear(x, tr, bits, su, sv, cb).view(np.uint16),
                                  O.linear(x, tr, bits, su, sv, cb).astype(np.float16).view(np.uint16))


def test_f16_rounding_of_c_restatement():
    vals = np.concatenate([RNG.standard_normal(5000) * 10.0 ** RNG.uniform(-9, 5, 5000),
                           [0.0, 65504.0, 65519.99, 65520.0, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -24]])
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([cpu.f64_to_f16_bits(v) for v in vals], dtype=np.uint16)
    np.testing.assert_array_equal(got, want)


def test_synth_is_deterministic_and_distributed():
    a = synth.trellis(synth.key_of("c", 1, "trellis"), 256, 128, 4)
    b = synth.trellis(synth.key_of("c", 1, "trellis"), 256, 128, 4)
    assert a.shape == (16, 8, 64) and (a == b).all()
    x = synth.normal(99, 200000)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    s = synth.scales(5, 100000).astype(np.float64)
    assert abs(np.mean(np.log(np.abs(s)))) < 0.01 and abs(np.std(np.log(np.abs(s))) - 0.25) < 0.01
    assert 0.45 < np.mean(s > 0) < 0.55
    h = synth.activations(7, 1, 10000, heavy_tail=True).astype(np.float64)
    assert 0.3 < np.mean(np.abs(h) > 6) * 100 < 3.0      # ~1% of channels scaled x20


# ---------------------------------------------------------------------------------------------
# approximate mul1 forms: unrounded weights, int8 activations (reference exl3_oracle.py:357-412)
# ---------------------------------------------------------------------------------------------
def test_affine_weights_round_to_the_mul1_table(golden):
    """The unrounded mul1 weights, rounded once to fp16, are the reference's whole mul1 table."""
    import hashlib
    g, meta = golden
    w = O.mul1_affine_weights(np.arange(65536)).astype(np.float16).view(np.uint16)
    assert hashlib.sha256(w.tobytes()).hexdigest() == meta["cb2_sha256"]
    assert np.array_equal(w, O.codebook_f16(np.arange(65536), 2).view(np.uint16))


def test_quantize_splats_matches_reference_vectors(golden):
    g, _ = golden
    a = g["qs_a"]
    for res in (0, 1):
        v, v2, s1, s2 = O.quantize_splats(a, 1.0, residual=bool(res))
        assert np.array_equal(v, g[f"qs_v_r{res}"])
        assert [s1, s2] == list(g[f"qs_sums_r{res}"])
        if res:
            assert np.array_equal(v2, g["qs_v2_r1"])
    v, _, _, _ = O.quantize_splats(np.array([0.5, 1.5, 2.5, -2.5, 300.0, -300.0]), 1.0)
    assert list(v) == [0, 2, 2, -2, 127, -127]                 # round half to even, clamp at 127


def test_gemv_int8_reference_matches_reference_vectors(golden):
    g, meta = golden
    for case in meta["int8_cases"]:
        pre, bits = case["name"], case["bits"]
        S = O.states_matrix(g[pre + "trellis"], bits)
        for res in (0, 1):
            y = O.gemv_int8_reference(g[pre + "a_had"], S, case["q"], g[pre + "svh"].astype(np.float64), bool(res))
            np.testing.assert_allclose(y, g[pre + f"y_r{res}"], rtol=1e-12, atol=1e-12)


def test_sliced_int8_equals_global_when_every_slice_holds_the_max(golden):
    """The kernels' per-slice scale form against the reference's global-scale vectors, on the case
    whose every 128-input slice holds the global maximum (so both scales agree): equal up to the
    kernels' fp16 staging of C and y."""
    g, meta = golden
    case = [c for c in meta["int8_cases"] if c["name"] == "int8_2_"][0]
    a = g["int8_2_a_had"]
    assert np.allclose(O.slice_scales(a), case["q"])
    y = O.linear_approx_rotated(a, g["int8_2_trellis"], case["bits"], g["int8_2_svh"], "int8")[0]
    ref = g["int8_2_y_r0"]
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-3


def test_int8_is_lossless_on_exactly_quantized_input():
    """Rotated inputs that are q * integers with |v| <= 127 and 127 q in every slice quantize
    without loss: the int8 form equals the affine form exactly."""
    rng = np.random.default_rng(8)
    k, n, bits = 256, 128, 4
    q = 2.0 ** -5
    v = rng.integers(-120, 121, size=(3, k)).astype(np.float64)
    v[:, ::128] = 127.0
    a = v * q
    tr = rng.integers(0, 65536, size=(k // 16, n // 16, 16 * bits), dtype=np.uint16)
    sv = np.ones(n, dtype=np.float16)
    ya = O.linear_approx_rotated(a, tr, bits, sv, "affine")
    yi = O.linear_approx_rotated(a, tr, bits, sv, "int8")
    assert np.array_equal(ya, yi)


def test_affine_form_is_near_the_faithful_linear():
    rng = np.random.default_rng(9)
    k, n, bits = 512, 256, 4
    tr = rng.integers(0, 65536, size=(k // 16, n // 16, 16 * bits), dtype=np.uint16)
    x = rng.standard_normal((2, k)).astype(np.float16)
    su = np.ones(k, dtype=np.float16)
    sv = np.ones(n, dtype=np.float16)
    yf = O.linear(x, tr, bits, su, sv, 2)
    ya = O.linear_approx(x, tr, bits, su, sv, "affine")
    yi = O.linear_approx(x, tr, bits, su, sv, "int8")
    assert O.rel_l2(ya, yf) < 1e-3 and 0 < O.rel_l2(yi, yf) < 2e-2


def test_int8_slice_sums_are_exact_in_fp32():
    """Arithmetic bound of the GEMV's int8 route (the counterpart of the reference's integer
    overflow proof, tests/test_arithmetic_bounds.py): the decoder hands the MFMA the byte sums s
    (<= 4 * 255 = 1020) and the quantized v (|v| <= 127), so one 128-input slice's sum of v * s is
    an integer below 2^24 and its fp32 accumulation, in any order, is exact.  With 1024 + s it
    would not be; 1024 sum v joins in the fold instead, through 1024 k_inv + k_bias, which is
    itself exact in fp32."""
    worst = 128 * 127 * 1020
    assert worst < 2 ** 24
    assert 128 * 127 * (1024 + 1020) > 2 ** 24
    s = O.byte_sum(O.codebook_hash(np.arange(65536, dtype=np.uint32), 2))
    assert int(s.max()) <= 1020 and int(s.min()) >= 0
    acc = np.float32(0.0)
    for _ in range(128):                                   # the worst case, summed in fp32
        acc = np.float32(acc + np.float32(127 * 1020))
    assert int(acc) == worst
    k_sum = np.float32(1024.0) * np.float32(O.K_INV) + np.float32(O.K_BIAS)
    assert float(k_sum) == 1024.0 * O.K_INV + O.K_BIAS == -3.453125



def _full_range_blocks(rng, rows):
    """fp16 rows of 128 spanning the whole fp16 range: +-65504, the smallest subnormal 2^-24, and
    the rest spread over every binade from 2^-24 to 2^10, random signs (so the scaled outputs stay
    below 65504)."""
    e = rng.integers(-24, 11, size=(rows, 128)).astype(np.float64)
    m = 1.0 + rng.integers(0, 1024, size=(rows, 128)) / 1024.0
    x = (np.where(rng.integers(0, 2, size=(rows, 128)) == 1, -1.0, 1.0) * m * np.exp2(e)).astype(np.float16)
    x[:, 0], x[:, 1], x[:, 2] = np.float16(65504.0), np.float16(-65504.0), np.float16(2.0 ** -24)
    x[:, 3] = -np.float16(2.0 ** -24)
    return x


def test_float64_block_sums_of_fp16_are_exact():
    """The exactness the float64 Hadamards rest on: every fp16 value is an integer multiple of
    2^-24 below 2^16 in magnitude, so any sum of 128 of them (every partial sum of any order) is an
    integer of at most 47 bits in units of 2^-24, inside float64's 53-bit significand.  Checked on
    blocks spanning the full fp16 range: the oracle's float64 butterflies (scale 1) equal the exact
    integer transform in units of 2^-24 for every output."""
    rng = np.random.default_rng(40)
    x = _full_range_blocks(rng, 64)
    units = (x.astype(np.float64) * 2.0 ** 24).astype(np.int64)          # exact: fp16 * 2^24 is an integer
    assert np.array_equal(units.astype(np.float64) / 2.0 ** 24, x.astype(np.float64))
    i = np.arange(128)
    H = np.where(np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :]) & 1, -1, 1).astype(np.int64)
    exact = units @ H                                                    # int64: |sum| < 128 * 2^40
    got = O.had128(x.astype(np.float64), 1.0)
    assert np.array_equal(got * 2.0 ** 24, exact.astype(np.float64))
    assert np.abs(exact).max() < 2 ** 47
