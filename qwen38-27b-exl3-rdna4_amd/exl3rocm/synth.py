"""Seeded synthetic EXL3 layers from a language-independent counter RNG.

Every tensor is a pure function of a 64-bit key, so the GPU harness, the CPU
baseline and the tests rebuild identical inputs without shipping data.  The
generator is SplitMix64 in counter mode: value ``i`` of a stream with key ``k``
is ``mix64(k + (i + 1) * 0x9E3779B97F4A7C15)`` (Steele, Lea, Flood, "Fast
splittable pseudorandom number generators", OOPSLA 2014).

Distributions follow the benchmark configurations of the reference layer
benchmarks (``bench/bench_layer.py``, ``vllm_plugin/tests/gemv_bench.py``):

* trellis: uniform 16-bit words (every bitstream is a valid code,
  ``vllm_plugin/tests/xcheck_ext.py:11-12``);
* ``suh`` / ``svh``: random sign times ``exp(N(0, 0.25^2))``, rounded to fp16;
* activations: ``N(0, 1)`` fp16, optionally with 1% of channels scaled x20.
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def mix64(z: np.ndarray) -> np.ndarray:
    """SplitMix64 finaliser on a uint64 array (wrapping arithmetic)."""
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def key_of(*parts) -> int:
    """64-bit stream key from a tuple of names / integers (FNV-1a over the text, then mixed)."""
    h = 0xCBF29CE484222325
    for b in "/".join(str(p) for p in parts).encode():
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return int(mix64(np.array([h], dtype=np.uint64))[0])


def stream_u64(key: int, n: int, start: int = 0) -> np.ndarray:
    """Values ``start .. start+n-1`` of the counter stream ``key``."""
    i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return mix64(np.uint64(key) + i * GOLDEN)


def uniform_u16(key: int, shape) -> np.ndarray:
    n = int(np.prod(shape))
    words = stream_u64(key, (n + 3) // 4)
    return words.view("<u2")[:n].reshape(shape).copy()


def _unit_open(u: np.ndarray) -> np.ndarray:
    """uint64 -> float64 uniform on the open interval (0, 1) (53-bit grid, half-step offset)."""
    return ((u >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)


def normal(key: int, n: int) -> np.ndarray:
    """Box-Muller N(0, 1) float64 samples, one pair of stream values per sample."""
    u = stream_u64(key, 2 * n)
    u1 = _unit_open(u[0::2])
    u2 = _unit_open(u[1::2])
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def trellis(key: int, k: int, n: int, bits: int) -> np.ndarray:
    """Uniform packed trellis ``(k/16, n/16, 16*bits)`` uint16."""
    return uniform_u16(key, (k // 16, n // 16, 16 * bits))


def scales(key: int, n: int) -> np.ndarray:
    """``+-1 * exp(N(0, 0.25^2))`` as fp16 (the suh / svh distribution)."""
    mag = np.exp(0.25 * normal(key, n))
    sign = np.where(stream_u64(key ^ 0x5A5A5A5A5A5A5A5A, n) & np.uint64(1), -1.0, 1.0)
    return (sign * mag).astype(np.float16)


def activations(key: int, m: int, k: int, heavy_tail: bool = False) -> np.ndarray:
    """``N(0, 1)`` fp16 activations ``[m, k]``; heavy_tail scales 1% of channels by 20."""
    x = normal(key, m * k).reshape(m, k)
    if heavy_tail:
        sel = (stream_u64(key ^ 0x0123456789ABCDEF, k) % np.uint64(100)) == np.uint64(0)
        x[:, sel] *= 20.0
    return x.astype(np.float16)


def layer(config: str, layer_id, k: int, n: int, bits: int):
    """(trellis, suh, svh) of one synthetic layer, keyed by (config, layer, tensor)."""
    return (trellis(key_of(config, layer_id, "trellis"), k, n, bits),
            scales(key_of(config, layer_id, "suh"), k),
            scales(key_of(config, layer_id, "svh"), n))
