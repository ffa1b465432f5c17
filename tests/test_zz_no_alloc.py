"""The allocation-free GEMV entry point, exl3_gemv_mr_noalloc, through the C ABI.

GPU: it gives exl3_gemv_mr's output bitwise (the same kernels; the workspace is the library's
per-GPU device array), on two calls in a row, the second with a smaller input, and under graph
capture with no workspace reserved anywhere, also when the first call of a fresh process is the
captured one (the set-up's symbol lookup and counter-clearing kernel then land in the graph).
CPU: a shape whose workspace exceeds the array is rejected before any launch.
"""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import cpu
from exl3rocm import _lib, kernels as E, synth


def _fake(addr):
    return ctypes.c_void_p(addr)


def test_noalloc_rejects_oversize_and_ineligible_shapes_without_a_gpu():
    L = _lib.lib()
    a = 1 << 20                                             # 16-byte aligned stand-ins, never dereferenced
    p = [_fake(a * (i + 1)) for i in range(5)]
    assert L.exl3_gemv_workspace_size(32, 256, 21888, 4, 1) > _lib.NOALLOC_SCRATCH_BYTES
    assert L.exl3_gemv_mr_noalloc(p[0], 256, p[1], p[2], 21888, p[3], p[4], 32, 256, 21888, 4, 0, 1, None) \
        == _lib.EWORKSPACE
    assert L.exl3_gemv_mr_noalloc(p[0], 256, p[1], p[2], 128, p[3], p[4], _lib.GEMV_MAX_ROWS + 1, 256, 128, 4, 0, 1,
                                  None) == _lib.DECLINED    # m > 64: the GEMV's own status, before any launch
    assert L.exl3_gemv_mr_noalloc(None, 256, p[1], p[2], 128, p[3], p[4], 1, 256, 128, 4, 0, 1, None) == _lib.EINVAL
    assert L.exl3_gemv_workspace_size(32, 17408, 5120, 4, 1) <= _lib.NOALLOC_SCRATCH_BYTES
    assert L.exl3_gemv_workspace_size(32, 5120, 17408, 8, 1) <= _lib.NOALLOC_SCRATCH_BYTES


DEV = "cuda:0"


def _case(tag, m, k, n, bits):
    tr, su, sv = synth.layer("noalloc", tag, k, n, bits)
    x = synth.activations(synth.key_of("noalloc", tag, "x"), m, k)
    dev = [torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in (x, tr.view(np.int16), su, sv)]
    return (x, tr, su, sv), dev


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
def test_noalloc_equals_gemv_mr_on_two_calls():
    """Two calls in a row on one GPU's array, the second smaller (fewer rows, a narrower layer):
    each equals exl3_gemv_mr bitwise and the oracle to the parity bar."""
    for tag, m, k, n, bits in (("a", 16, 5120, 17408, 4), ("b", 3, 2048, 1024, 3)):
        print(f"noalloc call {tag}: m={m} k={k} n={n} bits={bits}", flush=True)
        (x, tr, su, sv), (X, T, SU, SV) = _case(tag, m, k, n, bits)
        y = torch.full((m, n), float("nan"), dtype=torch.float16, device=DEV)
        assert E.exl3_gemv_mr_noalloc(X, T, y, SU, SV, bits, False, True) == 0
        want = torch.empty_like(y)
        assert E.exl3_gemv_mr(X, T, want, SU, None, SV, bits, False, True) == 0
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16)), tag
        ref = cpu.linear(x, tr, bits, su, sv, 2).astype(np.float64)
        got = y.cpu().numpy().astype(np.float64)
        assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-3, tag


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
def test_noalloc_graph_capture_replays():
    """Captured with no workspace reserved for the capture stream: replays equal the eager call,
    with eager calls of another shape on the same array between replays."""
    (_, _, _, _), (X, T, SU, SV) = _case("g", 4, 4096, 4096, 4)
    (_, _, _, _), (X2, T2, SU2, SV2) = _case("g2", 1, 1024, 512, 2)
    eager = torch.empty(4, 4096, dtype=torch.float16, device=DEV)
    E.exl3_gemv_mr_noalloc(X, T, eager, SU, SV, 4, False, True)
    y = torch.empty_like(eager)
    y2 = torch.empty(1, 512, dtype=torch.float16, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        E.exl3_gemv_mr_noalloc(X, T, y, SU, SV, 4, False, True)
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), eager.view(torch.int16))
        E.exl3_gemv_mr_noalloc(X2, T2, y2, SU2, SV2, 2, False, True)     # other shape, same array
        torch.cuda.synchronize()


# Run in a child process so that the library's first exl3_gemv_mr_noalloc call on the device is the
# captured one, whatever ran before in the test process.
CAPTURE_FIRST = r"""
import sys
sys.path[:0] = PATHS
import numpy as np, torch
from exl3rocm import kernels as E, synth
dev = "cuda:0"
tr, su, sv = synth.layer("noalloc", "first", 5120, 5120, 4)
x = synth.activations(synth.key_of("noalloc", "first", "x"), 4, 5120)
X, T, SU, SV = (torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in (x, tr.view(np.int16), su, sv))
y = torch.full((4, 5120), float("nan"), dtype=torch.float16, device=dev)
s = torch.cuda.Stream()
s.wait_stream(torch.cuda.current_stream())
torch.cuda.synchronize()
print("capturing the first noalloc call", flush=True)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    assert E.exl3_gemv_mr_noalloc(X, T, y, SU, SV, 4, False, True) == 0
replays = []
for _ in range(3):
    y.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    replays.append(y.clone())
eager = torch.empty_like(y)
assert E.exl3_gemv_mr_noalloc(X, T, eager, SU, SV, 4, False, True) == 0
want = torch.empty_like(y)
assert E.exl3_gemv_mr(X, T, want, SU, None, SV, 4, False, True) == 0
torch.cuda.synchronize()
assert torch.equal(eager.view(torch.int16), want.view(torch.int16)), "eager noalloc != exl3_gemv_mr"
for i, r in enumerate(replays):
    assert torch.equal(r.view(torch.int16), eager.view(torch.int16)), f"replay {i} != eager"
print("noalloc capture-first ok", flush=True)
"""


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
def test_noalloc_first_call_captured_in_a_fresh_process():
    """A child process whose first exl3_gemv_mr_noalloc call is inside torch.cuda.graph: three
    replays each equal a later eager call bitwise, and that equals exl3_gemv_mr."""
    here = os.path.dirname(os.path.abspath(__file__))
    paths = [os.path.join(os.path.dirname(here), "qwen38-27b-exl3-rdna4_amd"), here]
    script = CAPTURE_FIRST.replace("PATHS", repr(paths))
    print("child: noalloc first call under capture", flush=True)
    r = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "noalloc capture-first ok" in r.stdout, r.stdout[-2000:]
