"""Build libexl3_mi355x.so (the HIP kernels + C ABI) for gfx950 with hipcc, in-tree.

Usage: python build_ext.py   (or __graft_entry__.build())
       python build_ext.py --timeline   (also the tracing variant, libexl3_mi355x_timeline.so)
The library lands next to the Python host package: exl3rocm/libexl3_mi355x.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
OUT = os.path.join(HERE, "exl3rocm", "libexl3_mi355x.so")
OUT_TIMELINE = os.path.join(HERE, "exl3rocm", "libexl3_mi355x_timeline.so")
SOURCES = ["exl3_gemv.hip", "exl3_gemv_gated.hip", "exl3_gemv_silu.hip", "exl3_gemv_approx.hip", "exl3_gemv_f32.hip",
           "exl3_gemm.hip", "exl3_had.hip", "exl3_noalloc.hip"]
# Per-source extra flags.  The trellis decode (the GEMV's loop and the prefill producers') is long
# chains of packed-math (VOP3P) ops whose results need extra wait states on gfx950; the ILP
# scheduler interleaves the independent chains so the hazards are hidden instead of padded with
# s_nop (prefill producer interval: 38 -> 11 s_nop, config 4 +1.4 %).
EXTRA = {src: ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]
         for src in ("exl3_gemv.hip", "exl3_gemv_gated.hip", "exl3_gemv_silu.hip", "exl3_gemv_approx.hip", "exl3_gemv_f32.hip",
                     "exl3_gemm.hip")}
# The float transform's MFMA results feed VALU conversions directly: with the VGPR form of the MFMA
# they need no accumulator-register reads (32 per group of 16 rows x 128 columns).
EXTRA["exl3_had.hip"] = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument", "-I", INCLUDE,
]


def _compile(src: str, objdir: str, extra=(), suffix: str = "") -> str:
    obj = os.path.join(objdir, os.path.splitext(src)[0] + suffix + ".o")
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src, []), *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed on {src}")
    return obj


def _link(objs, out: str):
    tmp = out + ".tmp"
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp],
                       capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("link failed")
    os.replace(tmp, out)


def build(verbose: bool = False) -> str:
    objdir = os.path.join(HERE, "_objs")
    os.makedirs(objdir, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(lambda s: _compile(s, objdir), SOURCES))
    _link(objs, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


def build_timeline(verbose: bool = False) -> str:
    """The tracing variant (libexl3_mi355x_timeline.so): exl3_gemv.hip with -DEXL3_TIMELINE (the
    GEMV's per-workgroup phase stamps, include/exl3_mi355x_timeline.h), every other unit as built
    by build().  For bench.py --timeline only; the product library never carries the stamps."""
    objdir = os.path.join(HERE, "_objs")
    build()
    tl_obj = _compile("exl3_gemv.hip", objdir, extra=["-DEXL3_TIMELINE"], suffix="_timeline")
    objs = [tl_obj if s == "exl3_gemv.hip" else os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    _link(objs, OUT_TIMELINE)
    if verbose:
        print(f"built {OUT_TIMELINE}")
    return OUT_TIMELINE


if __name__ == "__main__":
    if "--timeline" in sys.argv[1:]:
        build_timeline(verbose=True)
    else:
        build(verbose=True)
