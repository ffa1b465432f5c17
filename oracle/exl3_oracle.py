"""CPU restatement of the EXL3 trellis arithmetic -- TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it; the ``exl3rocm`` package never does, and its kernels fail loudly when the
HIP library is missing instead of falling back here.

It restates, in vectorised numpy of this repository's own structure, the
semantics of the reference oracle ``reference/exl3_oracle.py`` (cited per
function below).  Pins (tests/test_oracle.py):

* golden vectors written by ``tests/golden/make_golden.py`` from the reference
  oracle itself: windows for bits 1..8, full codebook tables for cb 0/1/2
  (SHA-256), decoded trellises, faithful Hadamard stages, faithful GEMVs;
* the reference's own known-answer and invariant tests (``tests/test_oracle.py``
  of the reference): state-transition identity, position bijection and fragment
  table, mul1 zero state / range / byte-sum affinity, Hadamard orthonormality,
  involution and impulse, pipeline composition, fp16 grid;
* independent restatements: a brute-force MSB-first bit ring against the shift
  formula, a butterfly Hadamard against the Sylvester matrix.

Nothing here is "parity unpinned".
"""
from __future__ import annotations

import numpy as np

# fp16 bit patterns and multipliers of the codebooks (reference exl3_oracle.py:40-47)
K_INV_BITS = 0x1EEE
K_BIAS_BITS = 0xC931
MUL1_MULT = 0x83DCD12D
MCG_MULT = 0xCBAC1FED
CB0_MULT = 89226354
CB0_ADD = 64248484
LOP3_MASK = 0x8FFF8FFF
LOP3_XOR = 0x3B603B60
R_SCALE = 0.088388347648   # the Hadamard scale every reference call site passes


def f16_value(bits: int) -> float:
    return float(np.array([bits & 0xFFFF], dtype=np.uint16).view(np.float16)[0])


K_INV = f16_value(K_INV_BITS)     # 0.00676727294921875
K_BIAS = f16_value(K_BIAS_BITS)   # -10.3828125


def to_f16(x) -> np.ndarray:
    """Round to the nearest fp16 (ties to even), returned as float64 values."""
    return np.asarray(x, dtype=np.float64).astype(np.float16).astype(np.float64)


# ---------------------------------------------------------------------------
# Position placement inside a 16x16 tile (reference exl3_oracle.py:129-146)
# ---------------------------------------------------------------------------
def position_rowcol(t):
    """Trellis position t in [0, 256) -> (k-row, n-col) of the tile.

    With L = t // 8 and i = t % 8: row = 2(L%4) + (i&1) + 8((i>>1)&1),
    col = 2(L>>3) + ((L>>2)&1) + 8(i>>2).
    """
    t = np.asarray(t, dtype=np.int64)
    L, i = t >> 3, t & 7
    row = 2 * (L & 3) + (i & 1) + 8 * ((i >> 1) & 1)
    col = 2 * (L >> 3) + ((L >> 2) & 1) + 8 * (i >> 2)
    return row, col


POS_ROW, POS_COL = position_rowcol(np.arange(256))


# ---------------------------------------------------------------------------
# State windows of the tail-biting bit ring (reference exl3_oracle.py:149-188)
# ---------------------------------------------------------------------------
_WIN = {}


def _window_plan(bits: int):
    """Per-position (word_hi, word_lo, right_shift) of the 16-bit window ending at bit (t+1)*bits."""
    if bits not in _WIN:
        t = np.arange(256, dtype=np.int64)
        end = (t + 257) * bits                  # ring end bit, shifted by one lap so it stays positive
        first = end - 16
        nw = 8 * bits
        hi = (first // 32) % nw                 # word holding the window's first (most significant) bit
        lo = ((end - 1) // 32) % nw             # word holding its last bit
        shift = ((end - 1) // 32 + 1) * 32 - end
        _WIN[bits] = (hi, lo, shift.astype(np.uint64))
    return _WIN[bits]


def ring_words(tiles: np.ndarray) -> np.ndarray:
    """uint32 view of packed tiles: word i = u16[2i] | u16[2i+1] << 16 (little endian)."""
    tiles = np.ascontiguousarray(tiles, dtype=np.uint16)
    return tiles.view("<u4")


def state_windows(tiles: np.ndarray, bits: int) -> np.ndarray:
    """(..., 16*bits) uint16 tiles -> (..., 256) uint16 trellis states, in position order."""
    assert tiles.shape[-1] == 16 * bits
    w = ring_words(tiles).astype(np.uint64)
    hi, lo, shift = _window_plan(bits)
    merged = (w[..., hi] << np.uint64(32)) | w[..., lo]
    return ((merged >> shift) & np.uint64(0xFFFF)).astype(np.uint16)


def state_windows_bruteforce(tile: np.ndarray, bits: int) -> np.ndarray:
    """Independent restatement: expand the ring into an explicit MSB-first bit list and read
    the 16 bits ending at (t+1)*bits for each t (used only to pin ``state_windows``)."""
    words = ring_words(np.asarray(tile, dtype=np.uint16))
    ring = [(int(wd) >> (31 - j)) & 1 for wd in words for j in range(32)]
    nbits = len(ring)
    out = np.zeros(256, dtype=np.uint16)
    for t in range(256):
        end = (t + 1) * bits
        v = 0
        for b in range(end - 16, end):
            v = (v << 1) | ring[b % nbits]
        out[t] = v
    return out


def transition_ok(states: np.ndarray, bits: int) -> bool:
    """w_{t+1} == ((w_t << bits) & 0xFFFF) | (w_{t+1} & (2^bits - 1)) around the ring."""
    w = np.asarray(states, dtype=np.uint32)
    nxt = np.roll(w, -1, axis=-1)
    mask = (1 << bits) - 1
    return bool(((((w << bits) & 0xFFFF) | (nxt & mask)) == nxt).all())


# ---------------------------------------------------------------------------
# Codebooks (reference exl3_oracle.py:67-123)
# ---------------------------------------------------------------------------
def byte_sum(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.uint64)
    return ((x & 0xFF) + ((x >> 8) & 0xFF) + ((x >> 16) & 0xFF) + ((x >> 24) & 0xFF)).astype(np.int64)


def codebook_hash(states: np.ndarray, cb: int) -> np.ndarray:
    """32-bit hash of each 16-bit state: w*0x83DCD12D (cb2), w*0xCBAC1FED (cb1), w*89226354+64248484 (cb0)."""
    w = np.asarray(states, dtype=np.uint64) & np.uint64(0xFFFF)
    if cb == 2:
        x = w * np.uint64(MUL1_MULT)
    elif cb == 1:
        x = w * np.uint64(MCG_MULT)
    elif cb == 0:
        x = w * np.uint64(CB0_MULT) + np.uint64(CB0_ADD)
    else:
        raise ValueError(f"codebook must be 0, 1 or 2, got {cb}")
    return x & np.uint64(0xFFFFFFFF)


def codebook_f16(states: np.ndarray, cb: int) -> np.ndarray:
    """16-bit states -> exact fp16 codebook values (numpy float16).

    cb2 (mul1): fp16_rne((1024 + bytesum(x)) * K_INV + K_BIAS); the float64 expression is
    exact, so one rounding reproduces the kernel's fused fp16 multiply-add.
    cb1 (mcg) / cb0 (3inst): x' = (x & 0x8FFF8FFF) ^ 0x3B603B60, value = fp16_rne(fp16(x'.lo) + fp16(x'.hi)).
    """
    x = codebook_hash(states, cb)
    if cb == 2:
        v = (1024.0 + byte_sum(x).astype(np.float64)) * K_INV + K_BIAS
        return v.astype(np.float16)
    x = (x & np.uint64(LOP3_MASK)) ^ np.uint64(LOP3_XOR)
    lo = (x & np.uint64(0xFFFF)).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (x >> np.uint64(16)).astype(np.uint16).view(np.float16).astype(np.float64)
    return (lo + hi).astype(np.float16)


def codebook_flags(mcg: bool, mul1: bool) -> int:
    """Op flags -> codebook id: mul1 -> 2, mcg -> 1, neither -> 0 (3inst)."""
    return 2 if mul1 else (1 if mcg else 0)


# ---------------------------------------------------------------------------
# Whole-trellis decode (reference exl3_oracle.py:191-230)
# ---------------------------------------------------------------------------
def reconstruct(trellis: np.ndarray, bits: int, cb: int) -> np.ndarray:
    """(k/16, n/16, 16*bits) uint16 trellis -> dense fp16 W[k, n]."""
    kt, nt, per = trellis.shape
    assert per == 16 * bits
    vals = codebook_f16(state_windows(trellis, bits), cb)           # (kt, nt, 256)
    tile = np.zeros((kt, nt, 16, 16), dtype=np.float16)
    tile[:, :, POS_ROW, POS_COL] = vals
    return tile.transpose(0, 2, 1, 3).reshape(kt * 16, nt * 16)


def states_matrix(trellis: np.ndarray, bits: int) -> np.ndarray:
    kt, nt, _ = trellis.shape
    st = state_windows(trellis, bits)
    tile = np.zeros((kt, nt, 16, 16), dtype=np.uint16)
    tile[:, :, POS_ROW, POS_COL] = st
    return tile.transpose(0, 2, 1, 3).reshape(kt * 16, nt * 16)


# ---------------------------------------------------------------------------
# 128-point Hadamard (reference exl3_oracle.py:236-304)
# ---------------------------------------------------------------------------
def sylvester128() -> np.ndarray:
    """Natural-order Sylvester matrix H[i, j] = (-1)^popcount(i & j) (unscaled)."""
    i = np.arange(128)
    pc = np.vectorize(lambda v: bin(int(v)).count("1"))(i[:, None] & i[None, :])
    return np.where(pc & 1, -1.0, 1.0)


def had128(x, scale: float = R_SCALE) -> np.ndarray:
    """scale * H128 applied to every 128-block of the last axis, in float64 (butterfly form;
    exact for fp16 inputs since every partial sum fits in float64)."""
    x = np.array(x, dtype=np.float64, copy=True)
    n = x.shape[-1]
    assert n % 128 == 0
    y = x.reshape(-1, n // 128, 128)
    h = 1
    while h < 128:
        y = y.reshape(y.shape[0], y.shape[1], 128 // (2 * h), 2, h)
        a = y[..., 0, :].copy()
        b = y[..., 1, :]
        y[..., 0, :] = a + b
        y[..., 1, :] = a - b
        y = y.reshape(y.shape[0], y.shape[1], 128)
        h *= 2
    return (y * scale).reshape(x.shape)


def had_in(a, suh, faithful: bool = True) -> np.ndarray:
    """A_had = fp16(Had128(fp16(a * suh))) (faithful) or Had128(a * suh) (exact)."""
    p = np.asarray(a, dtype=np.float64) * np.asarray(suh, dtype=np.float64)
    if faithful:
        return to_f16(had128(to_f16(p)))
    return had128(p)


def had_out(c, svh, faithful: bool = True) -> np.ndarray:
    """y = fp16(fp16(Had128(c)) * svh) (faithful) or Had128(c) * svh (exact)."""
    y = had128(c)
    if faithful:
        return to_f16(to_f16(y) * np.asarray(svh, dtype=np.float64))
    return y * np.asarray(svh, dtype=np.float64)


# ---------------------------------------------------------------------------
# The quantized linear (reference exl3_oracle.py:307-351)
# ---------------------------------------------------------------------------
def linear(x, trellis: np.ndarray, bits: int, suh, svh, cb: int = 2, faithful: bool = True) -> np.ndarray:
    """y[m, :] = had_out(had_in(x[m], suh) @ W, svh) for every row of x (float64 result).

    Faithful staging: fp16 x / suh / svh, fp16 pre-scale product, fp16 A_had, float64
    dot, fp16 C, fp16 output Hadamard, fp16 post-scale product.
    """
    x = np.atleast_2d(np.asarray(x, dtype=np.float64))
    if faithful:
        x, suh, svh = to_f16(x), to_f16(suh), to_f16(svh)
    W = reconstruct(trellis, bits, cb).astype(np.float64)
    a = had_in(x, suh, faithful)
    c = a @ W
    if faithful:
        c = to_f16(c)
    return had_out(c, svh, faithful)


# ---------------------------------------------------------------------------
# Approximate mul1 forms: unrounded weights (affine) and int8 activations
# (reference exl3_oracle.py:357-412)
# ---------------------------------------------------------------------------
def mul1_affine_weights(states: np.ndarray) -> np.ndarray:
    """mul1 weights before their fp16 rounding: (1024 + bytesum(w * 0x83DCD12D)) * K_INV + K_BIAS,
    exact in float64 (codebook_f16 is this value rounded once to fp16)."""
    s = byte_sum(codebook_hash(states, 2)).astype(np.float64)
    return (1024.0 + s) * K_INV + K_BIAS


def quantize_splats(a_had, q: float, residual: bool = False):
    """Symmetric int8 quantization with clamp [-127, 127] (reference exl3_oracle.py:357-371):
    v = clip(rint(a / q)); with residual a second int8 v2 of the remainder at scale q / 254.
    Returns (v, v2 or None, sum(v), sum(v2))."""
    a = np.asarray(a_had, dtype=np.float64)
    v = np.clip(np.rint(a / q).astype(np.int64), -127, 127)
    v2, s2 = None, 0
    if residual:
        r = a - q * v.astype(np.float64)
        v2 = np.clip(np.rint(r / (q / 254.0)).astype(np.int64), -127, 127)
        s2 = int(v2.sum())
    return v, v2, int(v.sum()), s2


def gemv_int8_reference(a_had, states: np.ndarray, q: float, svh, residual: bool = False) -> np.ndarray:
    """The reference's int8-activation GEMV with one global scale q (exl3_oracle.py:374-412):
    exact integer accumulation of v . bytesum, then the affine epilogue
    y_rot = K_INV * (q acc1 + q2 acc2) + (1024 K_INV + K_BIAS) (q s1 + q2 s2), and the exact
    output transform (float64, no fp16 rounding).  states: (k, n) 16-bit state matrix."""
    a = np.asarray(a_had, dtype=np.float64)
    v, v2, s1, s2 = quantize_splats(a, q, residual)
    s = byte_sum(codebook_hash(states, 2)).astype(np.int64)
    acc = q * (v @ s).astype(np.float64)
    suma = q * s1
    if residual:
        q2 = q / 254.0
        acc = acc + q2 * (v2 @ s).astype(np.float64)
        suma += q2 * s2
    y_rot = K_INV * acc + (1024.0 * K_INV + K_BIAS) * suma
    return had_out(y_rot, svh, faithful=False)


def slice_scales(a_had, slice_len: int = 128) -> np.ndarray:
    """One int8 scale per (row, slice of slice_len inputs): max(|a| over the slice, 1e-8) / 127
    (the per-slice form of the reference's quantization, exl3_oracle.py:378-384)."""
    a = np.atleast_2d(np.asarray(a_had, dtype=np.float64))
    m, k = a.shape
    amax = np.abs(a.reshape(m, k // slice_len, slice_len)).max(axis=2)
    return np.maximum(amax, 1e-8) / 127.0


def linear_approx(x, trellis: np.ndarray, bits: int, suh, svh, mode: str) -> np.ndarray:
    """The GEMV's approximate mul1 routes, staged as the kernels stage them: faithful fp16 A_had,
    then linear_approx_rotated."""
    x = to_f16(np.atleast_2d(np.asarray(x, dtype=np.float64)))
    return linear_approx_rotated(had_in(x, to_f16(suh), True), trellis, bits, svh, mode)


def linear_approx_rotated(a, trellis: np.ndarray, bits: int, svh, mode: str) -> np.ndarray:
    """From the rotated input a [m, k]: C = sum over k of a_k w_k with the unrounded weights
    w_k = K_INV (1024 + s_k) + K_BIAS (mode "affine"), or with a_k replaced by q v_k, v_k the int8
    quantization of a at one scale q per 128-input slice (mode "int8"); C rounded to fp16;
    faithful output transform."""
    a = np.atleast_2d(np.asarray(a, dtype=np.float64))
    svh = to_f16(svh)
    S = states_matrix(trellis, bits)
    W = mul1_affine_weights(S)
    if mode == "int8":
        q = slice_scales(a)
        m, k = a.shape
        qk = np.repeat(q, 128, axis=1)
        v = np.clip(np.rint(a / qk), -127, 127)
        a = v * qk
    elif mode != "affine":
        raise ValueError(mode)
    c = to_f16(a @ W)
    return had_out(c, svh, True)


# ---------------------------------------------------------------------------
# Error metrics used by the tests
# ---------------------------------------------------------------------------
def rel_l2(got, ref) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))
