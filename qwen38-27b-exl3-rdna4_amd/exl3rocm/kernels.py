"""Tensor-level wrappers of the C ABI (one per reference extension call), on the current stream.

Each function takes torch tensors, validates shapes the way the reference bindings do
(TORCH_CHECK -> RuntimeError) and calls libexl3_mi355x.so.  Names follow the reference
extension (`exllamav3_ext`): decode, reconstruct, reconstruct_slice, had_r_128, exl3_gemv,
exl3_gemv_mr, exl3_gemv_mr_grouped, exl3_gemv_mr_supported, exl3_mgemm, hgemm_recon, exl3_gemm
(plus exl3_gemv_mr_grouped_widths and exl3_gemm_trellis_grouped, which have no reference counterpart).
"""
from __future__ import annotations

from ctypes import c_int as C_int
from typing import Optional, Sequence

import torch

from . import _lib as L


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _cb_flags(mcg: bool, mul1: bool):
    return int(bool(mcg)), int(bool(mul1))


def _need(cond: bool, msg: str):
    if not cond:
        raise RuntimeError(f"exl3rocm: {msg}")


def _cuda(*ts):
    for t in ts:
        _need(t is None or t.is_cuda, "tensors must be on a GPU (no CPU path)")


def _bits_of(trellis: torch.Tensor) -> int:
    return trellis.shape[-1] // 16


# ---------------------------------------------------------------------------------------------
# workspace (GEMV split-K partials + completion counters), one per (device, stream)
# ---------------------------------------------------------------------------------------------
_workspaces: dict = {}
_reserved: dict = {}        # device -> the largest workspace any reservation asked for


def workspace(device: torch.device, nbytes: int, stream: Optional[int] = None, reserve: bool = False) -> torch.Tensor:
    """Grow-only zeroed workspace for the current (or given) stream of `device`.

    Layers reserve at load time (reserve=True, Exl3LinearMethod.process_weights_after_loading),
    which also raises the device's reserved size.  A stream's first eager call then allocates
    that whole reserved size, not just its own call's, so the serving sequence (load, eager
    warm-up on stream S, graph capture on S) never needs an allocation during capture, on any
    stream.  During capture a stream without a large enough workspace raises."""
    device = torch.device(device)
    if stream is None:
        stream = torch.cuda.current_stream(device).cuda_stream
    if reserve:
        _reserved[device] = max(_reserved.get(device, 0), nbytes)
    key = (device, stream)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        _need(not torch.cuda.is_current_stream_capturing(),
              "GEMV workspace: this stream made no eager call of this size before graph capture")
        buf = torch.zeros(max(nbytes, _reserved.get(device, 0), 4096), dtype=torch.uint8, device=device)
        _workspaces[key] = buf
    return buf


_pf_workspaces: dict = {}
_pf_bound = None


def prefill_workspace_bound() -> int:
    """Bytes of a prefill split workspace that serves every shape (the library's bound, ~43 MB)."""
    global _pf_bound
    if _pf_bound is None:
        _pf_bound = int(L.lib().exl3_gemm_trellis_workspace_bound())
    return _pf_bound


def prefill_workspace(device: torch.device, nbytes: int, stream: Optional[int] = None) -> Optional[torch.Tensor]:
    """Zeroed workspace of the prefill GEMM's split tail for the current (or given) stream.  A
    stream's first call outside graph capture allocates the bound every shape fits in
    (exl3_gemm_trellis_workspace_bound), so a later capture on that stream splits exactly as
    eager calls do.  A stream that captures before any eager prefill call has none: its launches
    run unsplit, and the tail tiles' outputs can differ from the eager split's in the last place
    (another fp32 summation order)."""
    if nbytes <= 0:
        return None
    device = torch.device(device)
    if stream is None:
        stream = torch.cuda.current_stream(device).cuda_stream
    key = (device, stream)
    buf = _pf_workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            return buf
        buf = torch.zeros(max(nbytes, prefill_workspace_bound()), dtype=torch.uint8, device=device)
        _pf_workspaces[key] = buf
    return buf


def reserve_prefill_workspace(device: torch.device, stream: Optional[int] = None) -> None:
    """Allocate the current (or given) stream's prefill workspace now (load time)."""
    prefill_workspace(device, prefill_workspace_bound(), stream)


def gemv_workspace_bytes(m: int, k: int, n: int, K: int, groups: int = 1) -> int:
    return int(L.lib().exl3_gemv_workspace_size(m, k, n, K, groups))


# ---------------------------------------------------------------------------------------------
def decode(codes: torch.Tensor, out: torch.Tensor, mcg: bool, mul1: bool) -> None:
    _cuda(codes, out)
    _need(codes.dtype == torch.int16 and out.dtype == torch.float32 and codes.numel() == out.numel(),
          "decode: int16 codes and a float32 output of the same size")
    _need(codes.is_contiguous() and out.is_contiguous(), "decode: contiguous tensors")
    L.check(L.lib().exl3_decode(codes.data_ptr(), out.data_ptr(), codes.numel(), *_cb_flags(mcg, mul1),
                                _stream(codes)), "decode")


def reconstruct(W: torch.Tensor, trellis: torch.Tensor, K: int, mcg: bool, mul1: bool) -> None:
    _cuda(W, trellis)
    k, n = trellis.shape[0] * 16, trellis.shape[1] * 16
    _need(trellis.shape[2] == 16 * K, "reconstruct: trellis last dim must be 16*K")
    _need(W.dtype == torch.float16 and tuple(W.shape) == (k, n) and W.is_contiguous(), "reconstruct: W [k, n] fp16")
    L.check(L.lib().exl3_reconstruct(W.data_ptr(), trellis.data_ptr(), k, n, K, *_cb_flags(mcg, mul1),
                                     _stream(W)), "reconstruct")


def reconstruct_slice(W: torch.Tensor, trellis: torch.Tensor, K: int, mcg: bool, mul1: bool, n0: int) -> None:
    _cuda(W, trellis)
    k, n = trellis.shape[0] * 16, trellis.shape[1] * 16
    _need(trellis.shape[2] == 16 * K, "reconstruct_slice: trellis last dim must be 16*K")
    _need(W.dtype == torch.float16 and W.dim() == 2 and W.shape[0] == k and W.stride(1) == 1,
          "reconstruct_slice: W [k, w] fp16 with unit column stride")
    L.check(L.lib().exl3_reconstruct_slice(W.data_ptr(), W.stride(0), trellis.data_ptr(), k, n, K,
                                           *_cb_flags(mcg, mul1), n0, W.shape[1], _stream(W)), "reconstruct_slice")


def had_r_128(inp: torch.Tensor, out: torch.Tensor, pre: Optional[torch.Tensor], post: Optional[torch.Tensor],
              scale: float, exact: bool = True) -> None:
    """Blockwise Hadamard over the last dim (multiple of 128); 2-D operands may have any row stride.
    exact: float64 butterflies (exl3_had_r_128, also the fused GEMV's values); otherwise the
    float32 values the prefill GEMM uses (exl3_had_r_128_f32)."""
    _cuda(inp, out, pre, post)
    _need(inp.dtype == torch.float16 and out.dtype == torch.float16 and inp.shape == out.shape,
          "had_r_128: fp16 tensors of equal shape")
    _need(inp.stride(-1) == 1 and out.stride(-1) == 1, "had_r_128: unit stride rows")
    cols = inp.shape[-1]

    def as2d(t):
        if t.dim() == 2:
            return t
        _need(t.is_contiguous(), "had_r_128: tensors above 2-D must be contiguous")
        return t.view(-1, cols)

    i2, o2 = as2d(inp), as2d(out)
    rows = i2.shape[0]
    fn = L.lib().exl3_had_r_128 if exact else L.lib().exl3_had_r_128_f32
    L.check(fn(i2.data_ptr(), i2.stride(0) if rows > 1 else cols, o2.data_ptr(),
                                   o2.stride(0) if rows > 1 else cols, rows, cols,
                                   pre.data_ptr() if pre is not None else None,
                                   post.data_ptr() if post is not None else None, float(scale), _stream(inp)),
            "had_r_128")


def _rows(x: torch.Tensor):
    k = x.shape[-1]
    x2 = x.reshape(-1, k)
    _need(x2.dtype == torch.float16 and x2.stride(-1) == 1, "x must be fp16 with unit stride")
    return x2, x2.shape[0], k


def _ldy(y: torch.Tensor, n: int, fp32: bool = False) -> int:
    want = torch.float32 if fp32 else torch.float16
    _need(y.dtype == want and y.stride(-1) == 1, f"output must be {'fp32' if fp32 else 'fp16'} with unit column stride")
    return y.stride(-2) if y.dim() >= 2 and y.shape[-2] > 1 else max(n, y.shape[-1])


def exl3_gemv_mr_supported(m: int, k: int, n: int, K: int, mcg: bool, mul1: bool) -> bool:
    return bool(L.lib().exl3_gemv_mr_supported(m, k, n, K, *_cb_flags(mcg, mul1)))


def exl3_gemv(A, B, C, suh, A_had, svh, mcg: bool, mul1: bool) -> int:
    """M == 1 linear; returns 0 (done) or 1 (declined, C untouched).  A float32 C takes the fp32
    output (C = H(x suh) . W kept in fp32, y = H(C) r svh; reference tests/test_fused_had.py:153-158)."""
    _cuda(A, B, C, suh, svh)
    _need(C.dtype in (torch.float16, torch.float32), "exl3_gemv: fp16 or fp32 output")
    x2, m, k = _rows(A)
    n = svh.shape[0]
    K = _bits_of(B)
    ws = workspace(A.device, gemv_workspace_bytes(max(m, 1), k, n, K))
    f32 = C.dtype == torch.float32
    fn = L.lib().exl3_gemv_f32 if f32 else L.lib().exl3_gemv
    return L.check(fn(x2.data_ptr(), x2.stride(0) if m > 1 else k, B.data_ptr(), C.data_ptr(),
                      _ldy(C, n, f32), suh.data_ptr(), A_had.data_ptr() if A_had is not None else None,
                      svh.data_ptr(), m, k, n, K, *_cb_flags(mcg, mul1), ws.data_ptr(), ws.numel(),
                      _stream(A)), "exl3_gemv")


_prerot = None


def _rot_scratch(A_had, device, groups: int, m: int, k: int, silu: bool = False):
    """The A_had scratch for the multi-row GEMV (groups * m * k fp16): the caller's when it is large
    enough, else a fresh one; none below the library's pre-rotation row count (the kernel rotates
    in LDS there: exl3_gemv_prerot_rows, or exl3_gemv_silu_prerot_rows for the SiLU-input form)."""
    global _prerot
    if _prerot is None:
        _prerot = (int(L.lib().exl3_gemv_prerot_rows()), int(L.lib().exl3_gemv_silu_prerot_rows()))
    if m <= 1 or m < _prerot[1 if silu else 0]:
        return None
    if A_had is not None and A_had.dtype == torch.float16 and A_had.is_contiguous() and A_had.numel() >= groups * m * k:
        return A_had
    return torch.empty(groups * m * k, dtype=torch.float16, device=device)


def exl3_gemv_mr(A, B, C, suh, A_had, svh, K: int, mcg: bool, mul1: bool) -> int:
    _cuda(A, B, C, suh, svh)
    x2, m, k = _rows(A)
    n = svh.shape[0]
    _need(B.shape[-1] == 16 * K, "exl3_gemv_mr: trellis last dim must be 16*K")
    ws = workspace(A.device, gemv_workspace_bytes(m, k, n, K))
    xr = _rot_scratch(A_had, A.device, 1, m, k)
    return L.check(L.lib().exl3_gemv_mr(x2.data_ptr(), x2.stride(0) if m > 1 else k, B.data_ptr(), C.data_ptr(),
                                        _ldy(C, n), suh.data_ptr(), xr.data_ptr() if xr is not None else None,
                                        svh.data_ptr(), m, k, n, K,
                                        *_cb_flags(mcg, mul1), ws.data_ptr(), ws.numel(), _stream(A)),
                   "exl3_gemv_mr")


APPROX_MODES = {"affine": 1, "int8": 2}


def exl3_gemv_mr_approx(A, B, C, suh, A_had, svh, K: int, mode: str) -> int:
    """The opt-in approximate mul1 GEMV: mode "affine" (unrounded weights) or "int8" (int8
    activations, one scale per 128-input slice); see include/exl3_mi355x.h."""
    _cuda(A, B, C, suh, svh)
    _need(mode in APPROX_MODES, f"exl3_gemv_mr_approx: mode must be one of {sorted(APPROX_MODES)}")
    x2, m, k = _rows(A)
    n = svh.shape[0]
    _need(B.shape[-1] == 16 * K, "exl3_gemv_mr_approx: trellis last dim must be 16*K")
    ws = workspace(A.device, gemv_workspace_bytes(m, k, n, K))
    xr = _rot_scratch(A_had, A.device, 1, m, k)
    return L.check(L.lib().exl3_gemv_mr_approx(x2.data_ptr(), x2.stride(0) if m > 1 else k, B.data_ptr(), C.data_ptr(),
                                               _ldy(C, n), suh.data_ptr(), xr.data_ptr() if xr is not None else None,
                                               svh.data_ptr(), m, k, n, K, APPROX_MODES[mode], ws.data_ptr(),
                                               ws.numel(), _stream(A)), "exl3_gemv_mr_approx")


def exl3_gemv_mr_noalloc(A, B, C, suh, svh, K: int, mcg: bool, mul1: bool) -> int:
    """exl3_gemv_mr with its workspace in the library's per-GPU device array: no allocation here
    or in the library.  Calls that overlap on one GPU race (one stream at a time)."""
    _cuda(A, B, C, suh, svh)
    x2, m, k = _rows(A)
    n = svh.shape[0]
    _need(B.shape[-1] == 16 * K, "exl3_gemv_mr_noalloc: trellis last dim must be 16*K")
    rc = L.lib().exl3_gemv_mr_noalloc(x2.data_ptr(), x2.stride(0) if m > 1 else k, B.data_ptr(), C.data_ptr(),
                                      _ldy(C, n), suh.data_ptr(), svh.data_ptr(), m, k, n, K, *_cb_flags(mcg, mul1),
                                      _stream(A))
    if rc == L.EWORKSPACE:
        raise L.Exl3Error(f"exl3rocm: exl3_gemv_mr_noalloc: m={m} k={k} n={n} needs more than the "
                          f"{L.NOALLOC_SCRATCH_BYTES}-byte scratch array")
    return L.check(rc, "exl3_gemv_mr_noalloc")


def exl3_gemv_mr_grouped(A, B: Sequence[torch.Tensor], C, suh: Sequence[torch.Tensor], A_had,
                         svh: Sequence[torch.Tensor], K: int, mcg: bool, mul1: bool, bszm_for_warps: int = 1) -> int:
    _cuda(A, C, *B, *suh, *svh)
    x2, m, k = _rows(A)
    g = len(B)
    n = svh[0].shape[0]
    _need(1 <= g <= L.MAX_GROUPS and len(suh) == g and len(svh) == g, "grouped: 1..4 groups with suh/svh each")
    _need(all(s.shape[0] == n for s in svh), "grouped: groups must share n")
    _need(C.shape[-1] >= g * n, "grouped: output narrower than groups * n")
    ws = workspace(A.device, gemv_workspace_bytes(m, k, n, K, g))
    xr = _rot_scratch(A_had, A.device, g, m, k)
    pt, _a = L.ptr_array([b.data_ptr() for b in B])
    ps, _b = L.ptr_array([s.data_ptr() for s in suh])
    pv, _c = L.ptr_array([s.data_ptr() for s in svh])
    return L.check(L.lib().exl3_gemv_mr_grouped(x2.data_ptr(), x2.stride(0) if m > 1 else k, pt, C.data_ptr(),
                                                _ldy(C, g * n), ps, xr.data_ptr() if xr is not None else None, pv,
                                                g, m, k, n, K, *_cb_flags(mcg, mul1),
                                                bszm_for_warps, ws.data_ptr(), ws.numel(), _stream(A)),
                   "exl3_gemv_mr_grouped")


def exl3_gemv_mr_grouped_widths(A, B: Sequence[torch.Tensor], C, suh: Sequence[torch.Tensor],
                                svh: Sequence[torch.Tensor], K: int, mcg: bool, mul1: bool, A_had=None) -> int:
    """Groups of any widths sharing x and K (q/k/v) in one launch; group i writes the columns after
    groups 0..i-1 of C.  No counterpart in the reference extension (it launches these one by one)."""
    _cuda(A, C, *B, *suh, *svh)
    x2, m, k = _rows(A)
    g = len(B)
    widths = [int(s.shape[0]) for s in svh]
    _need(1 <= g <= L.MAX_GROUPS and len(suh) == g and len(svh) == g, "grouped: 1..4 groups with suh/svh each")
    _need(C.shape[-1] >= sum(widths), "grouped: output narrower than the groups")
    wa = (C_int * g)(*widths)
    ws = workspace(A.device, int(L.lib().exl3_gemv_workspace_size_widths(m, k, wa, g)))
    xr = _rot_scratch(A_had, A.device, g, m, k)
    pt, _a = L.ptr_array([b.data_ptr() for b in B])
    ps, _b = L.ptr_array([s.data_ptr() for s in suh])
    pv, _c = L.ptr_array([s.data_ptr() for s in svh])
    return L.check(L.lib().exl3_gemv_mr_grouped_widths(x2.data_ptr(), x2.stride(0) if m > 1 else k, pt, C.data_ptr(),
                                                       _ldy(C, sum(widths)), ps,
                                                       xr.data_ptr() if xr is not None else None, pv, wa, g, m, k, K,
                                                       *_cb_flags(mcg, mul1), ws.data_ptr(), ws.numel(), _stream(A)),
                   "exl3_gemv_mr_grouped_widths")


def exl3_gemv_silu_mul(A, B: Sequence[torch.Tensor], C, suh: Sequence[torch.Tensor], svh: Sequence[torch.Tensor],
                       K: int, mcg: bool, mul1: bool) -> int:
    """Gate (group 0) and up (group 1) of equal width n in one GEMV launch (m <= 32); C[m, n] gets
    fp16(fp16(silu(gate)) * up).  No counterpart in the reference extension."""
    _cuda(A, C, *B, *suh, *svh)
    x2, m, k = _rows(A)
    n = svh[0].shape[0]
    _need(len(B) == 2 and len(suh) == 2 and len(svh) == 2 and svh[1].shape[0] == n,
          "silu_mul: gate and up of equal width")
    _need(C.shape[-1] >= n, "silu_mul: output narrower than n")
    ws = workspace(A.device, gemv_workspace_bytes(m, k, n, K, 2))
    xr = _rot_scratch(None, A.device, 2, m, k)
    pt, _a = L.ptr_array([b.data_ptr() for b in B])
    ps, _b = L.ptr_array([s.data_ptr() for s in suh])
    pv, _c = L.ptr_array([s.data_ptr() for s in svh])
    return L.check(L.lib().exl3_gemv_silu_mul(x2.data_ptr(), x2.stride(0) if m > 1 else k, pt, C.data_ptr(),
                                              _ldy(C, n), ps, xr.data_ptr() if xr is not None else None, pv, m, k, n,
                                              K, *_cb_flags(mcg, mul1), ws.data_ptr(),
                                              ws.numel(), _stream(A)), "exl3_gemv_silu_mul")


def exl3_gemv_silu_in(gate, up, B, C, suh, A_had, svh, K: int, mcg: bool, mul1: bool) -> int:
    """exl3_gemv_mr over the input fp16(fp16(silu(gate)) * up) (m <= 32), formed as the rows load:
    gate and up are [m, k] views with equal row spacing (typically the two halves of a gated
    module's grouped output).  Bitwise equal to silu_mul followed by exl3_gemv_mr.  No counterpart
    in the reference extension."""
    _cuda(gate, up, B, C, suh, svh)
    k = gate.shape[-1]
    g2, u2 = gate.reshape(-1, k), up.reshape(-1, k)
    m = g2.shape[0]
    n = svh.shape[0]
    _need(u2.shape == g2.shape, "silu_in: gate and up of one shape")
    _need(all(t.dtype == torch.float16 and t.stride(-1) == 1 for t in (g2, u2)), "silu_in: fp16, unit stride")
    _need(m <= 1 or g2.stride(0) == u2.stride(0), "silu_in: gate and up rows equally spaced")
    _need(B.shape[-1] == 16 * K, "exl3_gemv_silu_in: trellis last dim must be 16*K")
    ld_in = g2.stride(0) if m > 1 else k
    ws = workspace(gate.device, gemv_workspace_bytes(m, k, n, K))
    xr = _rot_scratch(A_had, gate.device, 1, m, k, silu=True)
    return L.check(L.lib().exl3_gemv_silu_in(g2.data_ptr(), u2.data_ptr(), ld_in, B.data_ptr(), C.data_ptr(),
                                             _ldy(C, n), suh.data_ptr(), xr.data_ptr() if xr is not None else None,
                                             svh.data_ptr(), m, k, n, K, *_cb_flags(mcg, mul1), ws.data_ptr(),
                                             ws.numel(), _stream(gate)), "exl3_gemv_silu_in")



def exl3_gemm_trellis_silu_in(gate, up, B, C, suh, xh, svh, K: int, mcg: bool, mul1: bool) -> None:
    """The prefill GEMM (any m) over the input fp16(fp16(silu(gate)) * up), formed by the input
    transform as it loads the rows: gate and up are [m, k] views with equal row spacing (the two
    halves of a gated module's grouped output).  xh: [m, k] fp16 scratch.  Bitwise equal to
    silu_mul followed by exl3_gemm_trellis_grouped.  No counterpart in the reference extension."""
    _cuda(gate, up, B, C, suh, svh, xh)
    k = gate.shape[-1]
    g2, u2 = gate.reshape(-1, k), up.reshape(-1, k)
    m = g2.shape[0]
    n = svh.shape[0]
    _need(u2.shape == g2.shape, "silu_in: gate and up of one shape")
    _need(all(t.dtype == torch.float16 and t.stride(-1) == 1 for t in (g2, u2)), "silu_in: fp16, unit stride")
    _need(m <= 1 or g2.stride(0) == u2.stride(0), "silu_in: gate and up rows equally spaced")
    _need(B.shape[-1] == 16 * K, "exl3_gemm_trellis_silu_in: trellis last dim must be 16*K")
    _need(xh.numel() >= m * k and xh.dtype == torch.float16 and xh.is_contiguous(), "gemm silu_in: xh scratch [m, k] fp16")
    ldx = g2.stride(0) if m > 1 else k
    wa = (C_int * 1)(n)
    ws = prefill_workspace(gate.device, int(L.lib().exl3_gemm_trellis_workspace_size(m, k, wa, 1)))
    L.check(L.lib().exl3_gemm_trellis_silu_in(g2.data_ptr(), u2.data_ptr(), ldx, B.data_ptr(), C.data_ptr(), _ldy(C, n),
                                              suh.data_ptr(), xh.data_ptr(), svh.data_ptr(), m, k, n, K,
                                              *_cb_flags(mcg, mul1), ws.data_ptr() if ws is not None else None,
                                              ws.numel() if ws is not None else 0, _stream(gate)),
            "exl3_gemm_trellis_silu_in")

def silu_mul(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor) -> None:
    """out = fp16(fp16(silu(gate)) * up) over rows of n columns (gate / up may be column slices of
    one [rows, 2n] tensor)."""
    _cuda(gate, up, out)
    n = gate.shape[-1]
    g2, u2, o2 = gate.reshape(-1, n), up.reshape(-1, n), out.reshape(-1, n)
    rows = g2.shape[0]
    _need(u2.shape == g2.shape and o2.shape == g2.shape, "silu_mul: gate, up and out of one shape")
    _need(all(t.dtype == torch.float16 and t.stride(-1) == 1 for t in (g2, u2, o2)), "silu_mul: fp16, unit stride")
    _need(rows <= 1 or g2.stride(0) == u2.stride(0), "silu_mul: gate and up rows equally spaced")
    ld_in = g2.stride(0) if rows > 1 else n
    ld_out = o2.stride(0) if rows > 1 else n
    L.check(L.lib().exl3_silu_mul(g2.data_ptr(), u2.data_ptr(), ld_in, o2.data_ptr(), ld_out, rows, n,
                                  _stream(gate)), "exl3_silu_mul")


def exl3_mgemm(x, ptrs_trellis, y, ptrs_suh, xh, ptrs_svh, K: int, mcg: bool, mul1: bool) -> int:
    """Grouped M == 1 over int64 device pointer tables; y is (groups, 1, n)."""
    _cuda(x, ptrs_trellis, y, ptrs_suh, ptrs_svh)
    g = ptrs_trellis.numel()
    k = x.shape[-1]
    n = y.shape[-1]
    _need(x.numel() == k and x.dtype == torch.float16 and x.is_contiguous(), "mgemm: x is one fp16 row")
    _need(y.is_contiguous() and y.numel() == g * n, "mgemm: y (groups, 1, n) contiguous")
    for t in (ptrs_trellis, ptrs_suh, ptrs_svh):
        _need(t.dtype == torch.int64 and t.numel() == g and t.is_contiguous(), "mgemm: int64 pointer tables")
    ws = workspace(x.device, gemv_workspace_bytes(1, k, n, K, g))
    return L.check(L.lib().exl3_mgemm(x.data_ptr(), ptrs_trellis.data_ptr(), y.data_ptr(), ptrs_suh.data_ptr(),
                                      xh.data_ptr() if xh is not None else None, ptrs_svh.data_ptr(), g, k, n, K,
                                      *_cb_flags(mcg, mul1), ws.data_ptr(), ws.numel(), _stream(x)), "exl3_mgemm")


def hgemm_recon(xh: torch.Tensor, W: torch.Tensor, y: torch.Tensor) -> None:
    _cuda(xh, W, y)
    x2, m, k = _rows(xh)
    _need(W.dtype == torch.float16 and W.dim() == 2 and W.shape[0] == k and W.stride(1) == 1, "hgemm_recon: W [k, n]")
    n = W.shape[1]
    L.check(L.lib().exl3_hgemm_recon(x2.data_ptr(), x2.stride(0) if m > 1 else k, W.data_ptr(), W.stride(0),
                                     y.data_ptr(), _ldy(y, n), m, k, n, _stream(xh)), "hgemm_recon")


def exl3_gemm_trellis(A, B, C, suh, xh, svh, K: int, mcg: bool, mul1: bool) -> None:
    _cuda(A, B, C, suh, xh, svh)
    x2, m, k = _rows(A)
    n = svh.shape[0]
    _need(xh.numel() >= m * k and xh.dtype == torch.float16 and xh.is_contiguous(), "gemm: xh scratch [m, k] fp16")
    L.check(L.lib().exl3_gemm_trellis(x2.data_ptr(), x2.stride(0) if m > 1 else k, B.data_ptr(), C.data_ptr(),
                                      _ldy(C, n), suh.data_ptr(), xh.data_ptr(), svh.data_ptr(), m, k, n, K,
                                      *_cb_flags(mcg, mul1), _stream(A)), "exl3_gemm_trellis")


def exl3_gemm_trellis_grouped(A, B: Sequence[torch.Tensor], C, suh: Sequence[torch.Tensor], xh,
                              svh: Sequence[torch.Tensor], K: int, mcg: bool, mul1: bool) -> None:
    """Prefill of groups of any widths sharing x and K (q/k/v, gate/up) with one GEMM launch; group i
    writes the columns after groups 0..i-1 of C.  xh: fp16 scratch of groups * m * k elements.
    No counterpart in the reference extension (its linear_groups runs one prefill per group)."""
    _cuda(A, C, xh, *B, *suh, *svh)
    x2, m, k = _rows(A)
    g = len(B)
    widths = [int(s.shape[0]) for s in svh]
    _need(1 <= g <= L.MAX_GROUPS and len(suh) == g and len(svh) == g, "grouped: 1..4 groups with suh/svh each")
    _need(C.shape[-1] >= sum(widths), "grouped: output narrower than the groups")
    _need(xh.numel() >= g * m * k and xh.dtype == torch.float16 and xh.is_contiguous(),
          "grouped gemm: xh scratch [groups, m, k] fp16")
    wa = (C_int * g)(*widths)
    pt, _a = L.ptr_array([b.data_ptr() for b in B])
    ps, _b = L.ptr_array([s.data_ptr() for s in suh])
    pv, _c = L.ptr_array([s.data_ptr() for s in svh])
    ws = prefill_workspace(A.device, int(L.lib().exl3_gemm_trellis_workspace_size(m, k, wa, g)))
    L.check(L.lib().exl3_gemm_trellis_grouped(x2.data_ptr(), x2.stride(0) if m > 1 else k, pt, C.data_ptr(),
                                              _ldy(C, sum(widths)), ps, xh.data_ptr(), pv, wa, g, m, k, K,
                                              *_cb_flags(mcg, mul1), ws.data_ptr() if ws is not None else None,
                                              ws.numel() if ws is not None else 0, _stream(A)),
            "exl3_gemm_trellis_grouped")


def exl3_gemm(A, B, C, suh, A_had, svh, force_shape_idx: int = -1, mcg: bool = False, mul1: bool = True,
              force_kernel: int = 0) -> int:
    """Row-count dispatcher; returns the route tag (1 = fused GEMV, 2 = prefill GEMM)."""
    _cuda(A, B, C, suh, A_had, svh)
    x2, m, k = _rows(A)
    n = svh.shape[0]
    K = _bits_of(B)
    ws = workspace(A.device, gemv_workspace_bytes(min(max(m, 1), L.GEMV_FUSED_MAX_ROWS), k, n, K)) \
        if m <= L.GEMV_FUSED_MAX_ROWS else None
    return L.check(L.lib().exl3_gemm(x2.data_ptr(), x2.stride(0) if m > 1 else k, B.data_ptr(), C.data_ptr(),
                                     _ldy(C, n), suh.data_ptr(), A_had.data_ptr(), svh.data_ptr(), m, k, n, K,
                                     *_cb_flags(mcg, mul1), ws.data_ptr() if ws is not None else None,
                                     ws.numel() if ws is not None else 0, _stream(A)), "exl3_gemm")
