#!/usr/bin/env python3
"""Write the golden EXL3 vectors in ``tests/golden/exl3_golden.npz``.

This script is the only place that executes the reference's Python oracle
(``reference/exl3_oracle.py``), and only in the build container where the
reference checkout exists.  It stores inputs and outputs as plain arrays
(no pickle); the tests compare this repository's own oracle restatement and
the HIP kernels against them.  The reference itself never travels.

What is pinned (reference function, file:line):

* ``tile_windows`` (exl3_oracle.py:156) for bits 1..8 on boundary and random tiles
* ``t_to_rowcol`` (:129) for t = 0..255
* ``decode_codebook`` (:101) full 65536-entry tables for cb 0/1/2 (SHA-256 of the
  fp16 bit patterns plus a strided sample)
* ``decode_trellis`` (:206) on 32x32 trellises for every (bits, cb)
* ``had_in`` / ``had_out`` (:277, :290), faithful and exact
* ``gemv_mul1`` (:307, faithful=True) on several (k, n, bits, cb), plus the
  K=N=4096 4-bpw mcg layer of the headline CPU configuration, whose inputs are
  regenerated from the counter RNG (``exl3rocm.synth``) rather than stored.
* ``quantize_splats`` (:357) on ties, clamps and random data, plain and residual
* ``gemv_int8_reference`` (:374) on two layers, plain and residual, global q

Usage: python tests/golden/make_golden.py [--reference /root/reference]
"""
from __future__ import annotations

import argparse
import hashlib
import importlib.util
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "qwen38-27b-exl3-rdna4_amd"))
from exl3rocm import synth  # noqa: E402


def load_reference(root: str):
    path = os.path.join(root, "reference", "exl3_oracle.py")
    spec = importlib.util.spec_from_file_location("reference_exl3_oracle", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def f16_bits(v: np.ndarray) -> np.ndarray:
    return np.asarray(v, dtype=np.float64).astype(np.float16).view(np.uint16)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--out", default=os.path.join(HERE, "exl3_golden.npz"))
    args = ap.parse_args()
    O = load_reference(args.reference)
    rng = np.random.default_rng(20260923)
    out: dict[str, np.ndarray] = {}
    meta: dict = {"source": "reference/exl3_oracle.py", "cases": []}

    # --- t -> (row, col) ----------------------------------------------------
    r, c = O.t_to_rowcol(np.arange(256))
    out["rowcol"] = np.stack([r, c]).astype(np.int16)

    # --- state windows ------------------------------------------------------
    for bits in range(1, 9):
        n16 = 16 * bits
        tiles = [
            np.zeros(n16, dtype=np.uint16),
            np.full(n16, 0xFFFF, dtype=np.uint16),
            np.arange(n16, dtype=np.uint16),
            ((np.arange(n16, dtype=np.uint32) * 7919) & 0xFFFF).astype(np.uint16),
            rng.integers(0, 65536, size=n16, dtype=np.uint16),
            rng.integers(0, 65536, size=n16, dtype=np.uint16),
        ]
        tiles = np.stack(tiles)
        out[f"win_tiles_b{bits}"] = tiles
        out[f"win_states_b{bits}"] = np.stack([O.tile_windows(t, bits) for t in tiles])

    # --- codebook tables ----------------------------------------------------
    allw = np.arange(65536, dtype=np.uint16)
    for cb in (0, 1, 2):
        bits16 = f16_bits(O.decode_codebook(allw, cb))
        out[f"cb{cb}_sample"] = bits16[::61].copy()
        meta[f"cb{cb}_sha256"] = hashlib.sha256(bits16.tobytes()).hexdigest()

    # --- decode_trellis -----------------------------------------------------
    for bits in range(1, 9):
        tr = rng.integers(0, 65536, size=(2, 2, 16 * bits), dtype=np.uint16)
        out[f"dt_trellis_b{bits}"] = tr
        for cb in (0, 1, 2):
            out[f"dt_W_b{bits}_cb{cb}"] = f16_bits(O.decode_trellis(tr, bits, cb))

    # --- Hadamard stages ----------------------------------------------------
    a = (rng.standard_normal(256) * 1.5).astype(np.float16)
    suh = (np.sign(rng.standard_normal(256)) * np.exp(0.25 * rng.standard_normal(256))).astype(np.float16)
    cr = (rng.standard_normal(256) * 3.0).astype(np.float16)
    svh = (np.sign(rng.standard_normal(256)) * np.exp(0.25 * rng.standard_normal(256))).astype(np.float16)
    out["had_a"], out["had_suh"], out["had_c"], out["had_svh"] = a, suh, cr, svh
    out["had_in_faithful"] = f16_bits(O.had_in(a.astype(np.float64), suh.astype(np.float64), faithful=True))
    out["had_in_exact"] = O.had_in(a.astype(np.float64), suh.astype(np.float64), faithful=False)
    out["had_out_faithful"] = f16_bits(O.had_out(cr.astype(np.float64), svh.astype(np.float64), faithful=True))
    out["had_out_exact"] = O.had_out(cr.astype(np.float64), svh.astype(np.float64), faithful=False)

    # --- faithful GEMV, stored inputs ----------------------------------------
    cases = [(256, 128, 3, 2), (128, 256, 4, 1), (256, 256, 2, 0), (512, 128, 8, 2),
             (128, 128, 1, 2), (256, 128, 5, 1), (128, 256, 6, 0), (256, 128, 7, 2)]
    for idx, (k, n, bits, cb) in enumerate(cases):
        tr = rng.integers(0, 65536, size=(k // 16, n // 16, 16 * bits), dtype=np.uint16)
        xa = rng.standard_normal(k).astype(np.float16)
        su = (np.sign(rng.standard_normal(k)) * np.exp(0.25 * rng.standard_normal(k))).astype(np.float16)
        sv = (np.sign(rng.standard_normal(n)) * np.exp(0.25 * rng.standard_normal(n))).astype(np.float16)
        y = O.gemv_mul1(xa.astype(np.float64), tr, bits, su.astype(np.float64), sv.astype(np.float64),
                        cb=cb, faithful=True)
        pre = f"gemv{idx}_"
        out[pre + "trellis"], out[pre + "x"], out[pre + "suh"], out[pre + "svh"] = tr, xa, su, sv
        out[pre + "y"] = f16_bits(y)
        meta["cases"].append({"name": pre, "k": k, "n": n, "bits": bits, "cb": cb})

    # --- headline CPU configuration: K=N=4096, 4 bpw, mcg, counter-RNG inputs --
    k = n = 4096
    bits, cb = 4, 1
    tr, su, sv = synth.layer("config0", 0, k, n, bits)
    xa = synth.activations(synth.key_of("config0", 0, "x"), 1, k)[0]
    y = O.gemv_mul1(xa.astype(np.float64), tr, bits, su.astype(np.float64), sv.astype(np.float64),
                    cb=cb, faithful=True)
    out["config0_y"] = f16_bits(y)
    out["config0_W_sha"] = np.frombuffer(
        hashlib.sha256(f16_bits(O.decode_trellis(tr, bits, cb)).tobytes()).digest(), dtype=np.uint8)
    meta["config0"] = {"k": k, "n": n, "bits": bits, "cb": cb, "keys": ["config0", 0, "trellis|suh|svh|x"]}

    # --- int8 activation path (quantize_splats, gemv_int8_reference) ---------------
    qa = np.concatenate([np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, 127.5, 200.0, -200.0, 0.0, 1e-9]),
                         rng.standard_normal(116) * 40.0])
    for res in (False, True):
        v, v2, s1, s2 = O.quantize_splats(qa, 1.0, residual=res)
        out[f"qs_v_r{int(res)}"] = np.asarray(v, dtype=np.int64)
        if res:
            out["qs_v2_r1"] = np.asarray(v2, dtype=np.int64)
        out[f"qs_sums_r{int(res)}"] = np.array([s1, s2], dtype=np.int64)
    out["qs_a"] = qa
    for idx, (k, n, bits) in enumerate([(256, 128, 3), (512, 256, 4), (384, 256, 4)]):
        tr = rng.integers(0, 65536, size=(k // 16, n // 16, 16 * bits), dtype=np.uint16)
        ah = rng.standard_normal(k) * 0.7
        if idx == 2:
            # every 128-input slice holds the global maximum magnitude: a per-slice scale equals q
            ah = np.clip(ah, -2.5, 2.5)
            ah[::128] = 3.0 * np.sign(rng.standard_normal(k // 128))
        sv = (np.sign(rng.standard_normal(n)) * np.exp(0.25 * rng.standard_normal(n))).astype(np.float16)
        S = O.trellis_states(tr, bits)
        q = max(np.abs(ah).max(), 1e-8) / 127.0
        pre = f"int8_{idx}_"
        out[pre + "trellis"], out[pre + "a_had"], out[pre + "svh"] = tr, ah, sv
        for res in (False, True):
            out[pre + f"y_r{int(res)}"] = O.gemv_int8_reference(ah, S, q, sv.astype(np.float64), residual=res)
        meta.setdefault("int8_cases", []).append({"name": pre, "k": k, "n": n, "bits": bits, "q": q})

    np.savez_compressed(args.out, **out)
    with open(os.path.splitext(args.out)[0] + ".json", "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)
    print(f"wrote {args.out} ({os.path.getsize(args.out)} bytes, {len(out)} arrays)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
