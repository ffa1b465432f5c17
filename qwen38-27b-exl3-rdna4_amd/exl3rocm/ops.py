"""
EXL3 linear on MI355X as opaque torch custom ops, so torch.compile and HIP-graph capture treat
each call as one node.  Same op names, schemas and routing contract as the reference plugin's
ops (vllm_plugin/exl3rocm/ops.py:65-180); kernels come from libexl3_mi355x.so.

One call computes one checkpoint tensor ("group"): y = had(had(x * suh) @ W_inner) * svh.
Routing by rows M, per launch (gemv_rows: the measured GEMV / GEMM crossover of the launch's shape,
or EXL3_MR_MAX rows for every shape when set):
  M <= the crossover     -> fused GEMV (input Hadamard, trellis decode + MFMA dot, split-K
                            reduction and output Hadamard in one launch); every row is bitwise
                            equal to the M == 1 call of that row; EXL3_GEMV_APPROX=affine|int8
                            selects the opt-in approximate mul1 forms (unrounded weights, or
                            int8 activations as the reference's EXL3_ROCM_GFX1201_INT8 path)
  otherwise              -> input Hadamard pass, then the prefill GEMM (trellis decoded into LDS,
                            fp16 MFMA, fp32 accumulate, output Hadamard and svh in its epilogue);
                            a fused module's groups share one GEMM launch; EXL3_PREFILL=recon takes
                            the reference's reconstruct + hgemm route instead
"""
from __future__ import annotations

import os
from typing import Optional

import torch

from . import _lib
from . import kernels as E

def _env_rows(name: str) -> Optional[int]:
    v = os.environ.get(name)
    return None if v is None or not v.strip() else min(int(v), _lib.GEMV_MAX_ROWS)


# EXL3_MR_MAX (the reference's knob) fixes the GEMV / prefill boundary for every launch; unset, each
# launch takes the measured crossover of its shape from GEMV_CROSSOVER (shapes outside it: DEFAULT_MR)
MR_MAX: Optional[int] = _env_rows("EXL3_MR_MAX")
DEFAULT_MR = 32
# Largest row count at which the fused GEMV beats the prefill GEMM, by (k, output columns of the
# launch: all its groups).  Measured on MI355X for the launches a Qwen3.5-27B checkpoint makes (q/k/v
# and gate/up grouped as linear_groups groups them, and lm_head): both routes at every M from 2 to
# 64, graphs of 24 launches over 8 weight copies, 4 bpw, and 2 / 3 bpw where a checkpoint holds them
# (the boundary moved by <= 4 rows).  Each entry is a boundary b within 1 % of the least summed time
# over M with no step above 5 % from the GEMV at b rows to the GEMM at b + 1, for every bitrate
# measured (re-checked for every entry after each change to the GEMV's input rotation; moved only
# where the old b failed it: 5120 x 5120 15 -> 17, q/k/v 15 -> 19, the k/v pair 33 -> 58; after the
# one-block-per-wave pre-rotation pass, the 14336-column q/k/v 17 -> 25, 6144 x 5120 32 -> 30 and
# 17408 x 5120 35 -> 39).  The
# GEMM's cost is flat within each 16-row MFMA tile; the GEMV's grows with every row and 16-row tile,
# so the GEMM wins early where its 128-column tiles fill the chip (5120 - 7168 columns: b = 17 - 19)
# and late where they do not (the k/v launches, 2 x 17408 columns and lm_head: 58 to the GEMV's
# 64-row limit).
GEMV_CROSSOVER = {
    (5120, 1024): 64, (5120, 2048): 58, (5120, 5120): 17, (5120, 6144): 17, (5120, 7168): 19,
    (5120, 10240): 31, (5120, 12288): 33, (5120, 14336): 25, (5120, 16384): 33, (5120, 17408): 46,
    (5120, 34816): 64, (5120, 248320): 64, (6144, 5120): 30, (17408, 5120): 39,
}


def gemv_max_rows(k: int, width: int) -> int:
    """Most rows a launch of k inputs and `width` output columns takes on the fused GEMV."""
    if MR_MAX is not None:
        return MR_MAX
    return min(GEMV_CROSSOVER.get((k, width), DEFAULT_MR), _lib.GEMV_MAX_ROWS)


def gemv_rows(m: int, k: int, width: int) -> bool:
    """Route of an m-row launch: the fused GEMV (True; every row bitwise equal to its m = 1 call)
    or the prefill GEMM."""
    return m <= gemv_max_rows(k, width)


def fused_rows(m: int, k: int, width: int) -> bool:
    """The GEMV route for the fused-epilogue forms (SiLU input, gated, approximate): <= 32 rows."""
    return m <= min(gemv_max_rows(k, width), _lib.GEMV_FUSED_MAX_ROWS)


# widest non-lm_head layer (17408): the shared reconstruction buffer of the `recon` prefill route
RECON_SLICE_N = int(os.environ.get("EXL3_RECON_SLICE_N", "17408"))
PREFILL_ROUTE = os.environ.get("EXL3_PREFILL", "fused")
# linear_silu_mul on the GEMV route: "unfused" (grouped GEMV + elementwise kernel) or "fused" (one
# gated GEMV launch)
GATED_ROUTE = os.environ.get("EXL3_GATED", "unfused")
def approx_mode(value: Optional[str]) -> str:
    """EXL3_GEMV_APPROX -> the GEMV's approximate mul1 route: "" (faithful, the default; also for
    "0", "off", "none", "faithful"), "affine" (unrounded weights) or "int8" (int8 activations, the
    reference's EXL3_ROCM_GFX1201_INT8 path).  Any other value raises: a misspelt opt-in must not
    silently run (or silently skip) a route with a different numerical budget."""
    v = (value or "").strip().lower()
    if v in ("", "0", "off", "none", "faithful"):
        return ""
    if v not in E.APPROX_MODES:
        raise ValueError(f"exl3rocm: EXL3_GEMV_APPROX={value!r}: expected one of "
                         f"{sorted(E.APPROX_MODES)} or off")
    return v


# opt-in approximate mul1 GEMV, in place of the faithful one where fused_rows holds
GEMV_APPROX = approx_mode(os.environ.get("EXL3_GEMV_APPROX"))

_wbuf: dict = {}


def ext():
    """The loaded HIP library (raises if it is not built)."""
    return _lib.lib()


def reserve_weight_buffer(device, numel):
    """Grow the shared reconstruction buffer (used by the `recon` prefill route) at load time,
    so graph capture never allocates it (reference ops.py:52-57)."""
    device = torch.device(device)
    buf = _wbuf.get(device)
    if buf is None or buf.numel() < numel:
        _wbuf[device] = torch.empty(numel, dtype=torch.float16, device=device)


def _weight_buffer(device, numel):
    reserve_weight_buffer(device, numel)
    return _wbuf[torch.device(device)][:numel]


def reserve_workspace(device, k: int, n: int, K: int, groups: int = 1, m: Optional[int] = None):
    """Reserve the GEMV workspace for up to m rows (load time; default: the most rows gemv_rows
    sends to the GEMV for a module of groups x n columns): the current stream gets it now, and
    every other stream gets at least this much on its first eager call (so a later graph capture on
    that stream never allocates)."""
    if m is None:
        m = gemv_max_rows(k, n * groups)
    if m < 1:
        return
    E.workspace(torch.device(device), E.gemv_workspace_bytes(min(m, _lib.GEMV_MAX_ROWS), k, n, K, groups),
                reserve=True)


def _prep(x: torch.Tensor):
    k = x.shape[-1]
    x2 = x.reshape(-1, k)
    if x2.dtype != torch.float16:
        x2 = x2.to(torch.float16)
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    return x2, k


def _linear_into(x2, trellis, suh, svh, K, mcg, mul1, y, gemv: Optional[bool] = None):
    """One group into y ([M, n] view, unit column stride, any row stride); gemv: the route chosen
    by the caller for the launch this group belongs to (None: by this group's own shape)."""
    M, k = x2.shape
    n = svh.shape[0]
    if gemv is None:
        gemv = gemv_rows(M, k, n)
    if gemv and GEMV_APPROX and mul1 and M <= _lib.GEMV_FUSED_MAX_ROWS:
        rc = E.exl3_gemv_mr_approx(x2, trellis, y, suh, None, svh, K, GEMV_APPROX)
        if rc != 0:
            raise RuntimeError(f"exl3rocm: approximate GEMV declined shape m={M} k={k} n={n} K={K}")
    elif gemv:
        rc = E.exl3_gemv_mr(x2, trellis, y, suh, None, svh, K, mcg, mul1)
        if rc != 0:
            raise RuntimeError(f"exl3rocm: GEMV declined shape m={M} k={k} n={n} K={K}")
    elif PREFILL_ROUTE == "recon":
        # the fused prefill's float32 transforms (exact=False): this route stays bitwise equal to it
        xh = torch.empty_like(x2)
        E.had_r_128(x2, xh, suh, None, 1.0, exact=False)
        for n0 in range(0, n, RECON_SLICE_N):
            n1 = min(n0 + RECON_SLICE_N, n)
            w = _weight_buffer(x2.device, k * (n1 - n0)).view(k, n1 - n0)
            if n0 == 0 and n1 == n:
                E.reconstruct(w, trellis, K, mcg, mul1)
            else:
                E.reconstruct_slice(w, trellis, K, mcg, mul1, n0)
            E.hgemm_recon(xh, w, y[:, n0:n1])
        E.had_r_128(y, y, None, svh, 1.0, exact=False)
    else:
        # the grouped entry point with one group: its launch balances the last wave of tiles
        xh = torch.empty_like(x2)
        E.exl3_gemm_trellis_grouped(x2, [trellis], y, [suh], xh, [svh], K, mcg, mul1)


@torch.library.custom_op("exl3rocm::linear", mutates_args=())
def exl3_linear(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
                K: int, mcg: bool, mul1: bool) -> torch.Tensor:
    x2, k = _prep(x)
    n = svh.shape[0]
    M = x2.shape[0]
    y = torch.empty((M, n), dtype=torch.float16, device=x.device)
    if M == 0:
        return y.view(*x.shape[:-1], n)
    _linear_into(x2, trellis, suh, svh, K, mcg, mul1, y)
    return y.view(*x.shape[:-1], n)


@exl3_linear.register_fake
def _(x, trellis, suh, svh, K, mcg, mul1):
    return x.new_empty((*x.shape[:-1], svh.shape[0]), dtype=torch.float16)


@torch.library.custom_op("exl3rocm::linear_groups", mutates_args=())
def exl3_linear_groups(x: torch.Tensor, trellis: list[torch.Tensor], suh: list[torch.Tensor],
                       svh: list[torch.Tensor], K: list[int], mcg: bool, mul1: bool,
                       ptrs_trellis: Optional[torch.Tensor] = None, ptrs_suh: Optional[torch.Tensor] = None,
                       ptrs_svh: Optional[torch.Tensor] = None) -> torch.Tensor:
    """A fused module made of several checkpoint tensors (e.g. gate_proj + up_proj), each with its
    own K / suh / svh; the concatenation happens inside this opaque op (reference ops.py:106-175).

    ptrs_* = int64 device tensors of per-group data pointers, given when all groups share K and
    width (the reference's M == 1 exl3_mgemm route).  They are accepted and not read: the grouped
    launch takes the same pointers as kernel arguments instead (exl3_gemv_mr_grouped, the same
    kernel, split and output bitwise as exl3_mgemm over the tables), which saves every workgroup a
    dependent load of its table entries before its first trellis request (~1.3 us of a 5120 ->
    2 x 17408 launch)."""
    widths = [s.shape[0] for s in svh]
    if len(trellis) == 1:
        return exl3_linear(x, trellis[0], suh[0], svh[0], K[0], mcg, mul1)
    x2, k = _prep(x)
    M = x2.shape[0]
    ng = len(trellis)
    if M == 0:                                        # every route: an empty batch launches nothing
        return x2.new_empty((*x.shape[:-1], sum(widths)), dtype=torch.float16)
    y = torch.empty((M, sum(widths)), dtype=torch.float16, device=x.device)
    # runs of consecutive groups with equal K share one launch, each group written straight into
    # its row-strided column slice; each run takes the route of its own shape
    i, n0 = 0, 0
    while i < ng:
        j = i + 1
        while j < ng and j - i < _lib.MAX_GROUPS and K[j] == K[i]:
            j += 1
        w = sum(widths[i:j])
        gemv = gemv_rows(M, k, w)
        if j == i + 1 or (gemv and GEMV_APPROX and mul1 and M <= _lib.GEMV_FUSED_MAX_ROWS) or \
                (not gemv and PREFILL_ROUTE == "recon"):
            # one group, the approximate GEMV or the recon prefill: each group its own launch
            c = n0
            for g in range(i, j):
                _linear_into(x2, trellis[g], suh[g], svh[g], K[g], mcg, mul1, y[:, c:c + widths[g]], gemv)
                c += widths[g]
        elif gemv and all(wd == widths[i] for wd in widths[i:j]):
            # equal widths (gate/up, k/v): the reference's grouped entry point
            E.exl3_gemv_mr_grouped(x2, list(trellis[i:j]), y[:, n0:], list(suh[i:j]), None, list(svh[i:j]),
                                   K[i], mcg, mul1, j - i)
        elif gemv:
            # mixed widths (q/k/v)
            E.exl3_gemv_mr_grouped_widths(x2, list(trellis[i:j]), y[:, n0:], list(suh[i:j]), list(svh[i:j]),
                                          K[i], mcg, mul1)
        else:
            # one grouped prefill GEMM launch, each group its own rotated input
            xh = torch.empty((j - i, M, k), dtype=torch.float16, device=x.device)
            E.exl3_gemm_trellis_grouped(x2, list(trellis[i:j]), y[:, n0:], list(suh[i:j]), xh, list(svh[i:j]),
                                        K[i], mcg, mul1)
        n0 += w
        i = j
    return y.view(*x.shape[:-1], n0)


@exl3_linear_groups.register_fake
def _(x, trellis, suh, svh, K, mcg, mul1, ptrs_trellis=None, ptrs_suh=None, ptrs_svh=None):
    return x.new_empty((*x.shape[:-1], sum(s.shape[0] for s in svh)), dtype=torch.float16)


@torch.library.custom_op("exl3rocm::linear_silu_mul", mutates_args=())
def exl3_linear_silu_mul(x: torch.Tensor, trellis: list[torch.Tensor], suh: list[torch.Tensor],
                         svh: list[torch.Tensor], K: list[int], mcg: bool, mul1: bool) -> torch.Tensor:
    """A gated MLP's input: the gate (group 0) and up (group 1) linears of one module followed by
    SiLU-and-mul, act = fp16(fp16(silu(gate)) * up) with gate / up exactly as linear_groups
    computes them.  No counterpart in the reference plugin, whose MLP runs linear_groups and then
    a separate SiluAndMul (the fusion is proposed in reference docs/EFFICIENCY_INVESTIGATION.md:36-66).

    Routes: linear_groups, then an elementwise SiLU-and-mul kernel (the default: measured faster
    on MI355X); or, with EXL3_GATED=fused on the GEMV route (<= 32 rows), equal K and width, one GEMV launch
    whose workgroup completing a 128-column block of both groups applies the activation.  Both
    routes give bitwise the same result."""
    if not (len(trellis) == 2 and len(suh) == 2 and len(svh) == 2 and len(K) == 2):
        raise RuntimeError("exl3rocm: linear_silu_mul takes exactly two groups (gate, up)")
    n = svh[0].shape[0]
    if svh[1].shape[0] != n:
        raise RuntimeError("exl3rocm: linear_silu_mul needs gate and up of equal width")
    x2, k = _prep(x)
    M = x2.shape[0]
    act = torch.empty((M, n), dtype=torch.float16, device=x.device)
    if M == 0:
        return act.view(*x.shape[:-1], n)
    if GATED_ROUTE == "fused" and K[0] == K[1] and fused_rows(M, k, 2 * n):
        E.exl3_gemv_silu_mul(x2, list(trellis), act, list(suh), list(svh), K[0], mcg, mul1)
    else:
        gu = exl3_linear_groups(x2, trellis, suh, svh, K, mcg, mul1)
        E.silu_mul(gu[:, :n], gu[:, n:], act)
    return act.view(*x.shape[:-1], n)


@exl3_linear_silu_mul.register_fake
def _(x, trellis, suh, svh, K, mcg, mul1):
    return x.new_empty((*x.shape[:-1], svh[0].shape[0]), dtype=torch.float16)


@torch.library.custom_op("exl3rocm::silu_mul_linear", mutates_args=())
def exl3_silu_mul_linear(gu: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
                         K: int, mcg: bool, mul1: bool) -> torch.Tensor:
    """A gated MLP's output: SiLU-and-mul of gu = [gate | up] (the [.., 2k] output of the gate/up
    linear_groups), act = fp16(fp16(silu(gate)) * up), then the down linear of act.  No
    counterpart in the reference plugin, whose MLP runs a separate SiluAndMul before the down
    linear (the fusion is proposed in reference docs/EFFICIENCY_INVESTIGATION.md:36-66).

    On the GEMV route (<= 32 rows) one GEMV launch forms act from gate and up as its input rows
    load; on the prefill route the prefill's input transform forms act as it loads the rows (one transform launch and one
    GEMM launch, no act in memory); on the approximate GEMV routes and the recon prefill route the
    elementwise kernel writes act and linear runs on it.  Every route equals silu_mul followed by
    linear, bitwise."""
    k2 = gu.shape[-1]
    k = suh.shape[0]
    if k2 != 2 * k:
        raise RuntimeError(f"exl3rocm: silu_mul_linear takes [gate | up] of 2 * {k} columns, got {k2}")
    g2, _ = _prep(gu)
    M = g2.shape[0]
    n = svh.shape[0]
    y = torch.empty((M, n), dtype=torch.float16, device=gu.device)
    if M == 0:
        return y.view(*gu.shape[:-1], n)
    if fused_rows(M, k, n) and not (GEMV_APPROX and mul1):
        rc = E.exl3_gemv_silu_in(g2[:, :k], g2[:, k:], trellis, y, suh, None, svh, K, mcg, mul1)
        if rc != 0:
            raise RuntimeError(f"exl3rocm: GEMV declined shape m={M} k={k} n={n} K={K}")
    elif not gemv_rows(M, k, n) and PREFILL_ROUTE != "recon":
        xh = torch.empty((M, k), dtype=torch.float16, device=gu.device)
        E.exl3_gemm_trellis_silu_in(g2[:, :k], g2[:, k:], trellis, y, suh, xh, svh, K, mcg, mul1)
    else:
        act = torch.empty((M, k), dtype=torch.float16, device=gu.device)
        E.silu_mul(g2[:, :k], g2[:, k:], act)
        _linear_into(act, trellis, suh, svh, K, mcg, mul1, y)
    return y.view(*gu.shape[:-1], n)


@exl3_silu_mul_linear.register_fake
def _(gu, trellis, suh, svh, K, mcg, mul1):
    return gu.new_empty((*gu.shape[:-1], svh.shape[0]), dtype=torch.float16)
