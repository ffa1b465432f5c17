#!/usr/bin/env python3
"""Benchmark of the MI355X EXL3 quantized-linear engine (one GPU).

Headline (BASELINE.json metric, configuration 1): M = 1 decode through the 7 EXL3 linears of a
Qwen-27B-shaped decoder layer (q, k, v, o 5120-wide attention projections and the
5120 -> 17408 -> 5120 MLP) at 4 bpw, mul1 codebook, with the plugin's own routing (q/k/v as one
fused module, gate/up through the grouped pointer-table launch).  One *step* = one layer's
linears on one token.  Steps cycle over 8 distinct copies of the layer's weights (1.3 GB, ~5x the
256 MB Infinity Cache) and are replayed from one HIP graph holding a step per copy (an 8-layer
stack), so weights stream from HBM as in decode.

  value        = whole-job trellis + x + suh + svh + y bytes / elapsed time  (GB/s)
  roofline     = the dominant kernel (the M=1 4-bpw GEMV): algorithmic bytes per launch / mean
                 launch duration from HIP events on its stream, vs 8 TB/s
  cpu_baseline = the C oracle restatement (faithful GEMV) on a bounded sample, host cores

Extras: configuration 4 prefill (M = 2048 through a 64-layer stack, TFLOPS vs 2.5 PF fp16 MFMA),
configuration 3 small-batch crossover, configuration 2 bitrate sweep.

  python bench.py [--steps K] [--warmup W] [--no-prefill] [--no-sweep] [--no-cpu]
  python bench.py --traffic-probe      (what the PMC traffic passes profile)
  python bench.py --prefill-only       (configuration 4 alone, for the prefill PMC passes)
  python bench.py --config3-only       (configuration 3 alone, for its kernel trace)
  python bench.py --checkpoint-only    (the reference checkpoint's shapes alone, for their kernel trace)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "qwen38-27b-exl3-rdna4_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
MFMA_FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, published
HIDDEN, INTER, KV = 5120, 17408, 1024
# VALU decode budget (diagnostic): vector lane-ops per second of the whole chip (256 CUs x 4 SIMDs x
# 16 lanes x 2.4 GHz, one full-rate op per lane per clock) and the lane-ops per weight of the 4-bpw
# mul1 GEMV loop (ISA count of the built loop: 129 VALU instructions per lane per 32 weights)
VALU_LANE_OPS_PER_S = 256 * 4 * 16 * 2.4e9
VALU_OPS_PER_WEIGHT_4BPW = 129 / 32
LAYER = [("q", HIDDEN, HIDDEN), ("k", HIDDEN, KV), ("v", HIDDEN, KV), ("o", HIDDEN, HIDDEN),
         ("gate", HIDDEN, INTER), ("up", HIDDEN, INTER), ("down", INTER, HIDDEN)]


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algo_bytes(m, k, n, bits):
    return k * n * bits // 8 + 2 * m * k + 2 * k + 2 * n + 2 * m * n


class LayerSet:
    """One decoder layer's EXL3 weights (device), with the plugin's module grouping."""

    def __init__(self, torch, base, copy_id, bits, mul1=True):
        self.t = torch
        self.bits = bits
        dev = "cuda"
        self.w = {}
        for name, k, n in LAYER:
            tr, su, sv = base[name]
            T = torch.from_numpy(tr.view(np.int16)).to(dev) if copy_id == 0 else base["_dev"][name][0].clone()
            self.w[name] = (T, torch.from_numpy(su).to(dev), torch.from_numpy(sv).to(dev))
        self.mcg, self.mul1 = (not mul1), mul1
        g = [self.w["gate"], self.w["up"]]
        self.gu_ptrs = [torch.tensor([x[i].data_ptr() for x in g], dtype=torch.int64, device=dev) for i in range(3)]

    def launch(self, name, x5120, x17408):
        """One of the step's four GEMV launches, as the plugin makes it: "qkv" (one grouped-widths
        launch), "o", "gate_up" (the grouped pointer-table launch) or "down"."""
        ops = self.t.ops.exl3rocm
        w, b, mc, m1 = self.w, self.bits, self.mcg, self.mul1
        if name == "qkv":
            return ops.linear_groups(x5120, [w["q"][0], w["k"][0], w["v"][0]], [w["q"][1], w["k"][1], w["v"][1]],
                                     [w["q"][2], w["k"][2], w["v"][2]], [b, b, b], mc, m1)
        if name == "gate_up":
            return ops.linear_groups(x5120, [w["gate"][0], w["up"][0]], [w["gate"][1], w["up"][1]],
                                     [w["gate"][2], w["up"][2]], [b, b], mc, m1, *self.gu_ptrs)
        return ops.linear(x17408 if name == "down" else x5120, *w[name], b, mc, m1)

    def step(self, x5120, x17408):
        return tuple(self.launch(name, x5120, x17408) for name in STEP_LAUNCHES)


# the step's GEMV launches: q/k/v grouped (mixed widths), o, gate/up grouped (pointer tables), down
STEP_LAUNCHES = ("qkv", "o", "gate_up", "down")


def launches_per_step():
    return len(STEP_LAUNCHES)


def build_layers(torch, bits, copies, mul1=True, tag="config1"):
    from exl3rocm import synth
    base = {name: synth.layer(tag, f"{name}-b{bits}", k, n, bits) for name, k, n in LAYER}
    sets = [LayerSet(torch, base, 0, bits, mul1)]
    base["_dev"] = sets[0].w
    for c in range(1, copies):
        sets.append(LayerSet(torch, base, c, bits, mul1))
    return base, sets


def capture_steps(torch, sets, x5120, x17408, steps):
    """Graphs of the timed region: one graph of `block` consecutive steps cycling over the weight
    copies (a layer stack, as a captured decode step replays it), replayed steps // block times,
    plus one of the remaining steps % block; and one single-step graph per copy for the warmup."""
    from exl3rocm import ops as exl3_ops
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for name, k, n in LAYER:
            exl3_ops.reserve_workspace("cuda", k, n, sets[0].bits, groups=2)
        for ls in sets:                      # warm every path on the capture stream
            ls.step(x5120, x17408)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    def graph_of(first, count):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in range(first, first + count):
                sets[i % len(sets)].step(x5120, x17408)
        return g

    singles = [graph_of(i, 1) for i in range(len(sets))]
    block = min(steps, 256)
    full = graph_of(0, block) if steps >= block > 0 else None
    rest = graph_of(0, steps % block) if steps % block else None
    torch.cuda.synchronize()
    return {"singles": singles, "block": block, "full": full, "rest": rest}


def device_copy_gbs(torch, nbytes=1 << 30, reps=30):
    """What HBM delivers: a 1 GiB torch copy_ (read + write bytes counted, 4x the 256 MB cache),
    median of `reps` HIP-event-timed copies after 5 untimed (the reference's roofline probe,
    bench/bench_layer.py:43-60, at a size past this GPU's cache); and a read-only sweep (a sum over
    the same 1 GiB, median of `reps`).  Returns (copy GB/s, read GB/s)."""
    src = torch.ones(nbytes // 2, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        dst.copy_(src)
        e1.record()
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e3)
    # read only (the GEMV's traffic is almost all reads): a sum over the same 1 GiB
    tr = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        src.sum(dtype=torch.float32)
        e1.record()
        e1.synchronize()
        tr.append(e0.elapsed_time(e1) * 1e3)
    del src, dst
    torch.cuda.empty_cache()
    return round(2.0 * nbytes / float(np.median(ts)) / 1e3, 1), round(nbytes / float(np.median(tr)) / 1e3, 1)


def time_graphs(torch, graphs, steps, warmup):
    """Exactly `steps` steps after `warmup` untimed single steps: the block graph steps // block
    times, then the remainder graph; HIP events on the replay stream, plus host wall time."""
    per = graphs["singles"]
    for i in range(warmup):
        per[i % len(per)].replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps // graphs["block"]):
        graphs["full"].replay()
    if graphs["rest"] is not None:
        graphs["rest"].replay()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return e0.elapsed_time(e1) / 1e3, wall


def per_shape_gemv(torch, sets, x5120, x17408, reps=64):
    """Mean launch duration of each layer GEMV alone (graph of `reps` launches over the weight
    copies, HIP events on the replay stream)."""
    from exl3rocm import kernels as E
    out = {}
    s = torch.cuda.Stream()
    for name, k, n in LAYER:
        x = x17408 if k == INTER else x5120
        y = torch.empty(1, n, dtype=torch.float16, device="cuda")
        with torch.cuda.stream(s):
            for ls in sets:
                T, SU, SV = ls.w[name]
                E.exl3_gemv(x, T, y, SU, None, SV, ls.mcg, ls.mul1)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for r in range(reps):
                T, SU, SV = sets[r % len(sets)].w[name]
                E.exl3_gemv(x, T, y, SU, None, SV, sets[0].mcg, sets[0].mul1)
        with torch.cuda.stream(s):
            g.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(3):
                g.replay()
            e1.record(s)
        s.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (3 * reps)
        b = algo_bytes(1, k, n, sets[0].bits)
        out[name] = {"k": k, "n": n, "us": round(us, 3), "gbs": round(b / us / 1e3, 1),
                     "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
    return out


# The reference checkpoint's GEMV shapes with their calls per decode token (the reference's
# scoreboard, vllm_plugin/tests/gemv_bench.py:18-28): (name, k, n, bits, calls per token)
CKPT_CASES = [
    ("gate|up K3", 5120, 17408, 3, 70), ("gate|up K2", 5120, 17408, 2, 56), ("gate|up K1", 5120, 17408, 1, 2),
    ("down K3", 17408, 5120, 3, 64),
    ("gdn qkv K4", 5120, 10240, 4, 12), ("gdn qkv K2", 5120, 10240, 2, 35),
    ("gdn z K4", 5120, 6144, 4, 48), ("gdn out K4", 6144, 5120, 4, 48),
    ("attn q K2", 5120, 12288, 2, 11), ("attn q K4", 5120, 12288, 4, 4),
    ("attn kv K5", 5120, 1024, 5, 18), ("attn kv K6", 5120, 1024, 6, 8), ("attn kv K4", 5120, 1024, 4, 6),
    ("attn o K3", 6144, 5120, 3, 4), ("attn o K5", 6144, 5120, 5, 4),
    ("lm_head K4", 5120, 248320, 4, 1),
]
CKPT_PREFILL = [("gdn qkv", 5120, 10240, 4), ("gdn out / attn o", 6144, 5120, 4), ("lm_head", 5120, 248320, 4)]


def _device_layer(torch, k, n, bits, g):
    T = torch.randint(0, 65536, (k // 16, n // 16, 16 * bits), device="cuda", dtype=torch.int32, generator=g).to(torch.int16)
    su = (torch.randn(k, device="cuda", generator=g).sign() * torch.exp(0.25 * torch.randn(k, device="cuda", generator=g))).half()
    sv = (torch.randn(n, device="cuda", generator=g).sign() * torch.exp(0.25 * torch.randn(n, device="cuda", generator=g))).half()
    return T, su, sv


def _warm(torch, fn, seconds, stream=None):
    """Call fn in batches of 4 until `seconds` of wall time have passed (clocks up to speed)."""
    t0 = time.perf_counter()
    while True:
        for _ in range(4):
            fn()
        (stream or torch.cuda).synchronize()
        if time.perf_counter() - t0 >= seconds:
            return


def checkpoint_shapes(torch, reps=32, m_prefill=2048):
    """The reference checkpoint's own shapes: every M = 1 case of the reference's GEMV scoreboard
    (device-generated weights, enough copies for >= 1 GiB so they stream from HBM; mean of a graph
    of `reps` launches over the copies, HIP events), its per-token total weighted by calls per
    decode token, and the prefill at M = 2048 on its three shapes outside configuration 1."""
    g = torch.Generator(device="cuda").manual_seed(20261202)
    s = torch.cuda.Stream()
    gemv, total_us = {}, 0.0
    for name, k, n, bits, calls in CKPT_CASES:
        copies = max(2, (1 << 30) // (k * n * bits // 8) + 1)
        ws = [_device_layer(torch, k, n, bits, g) for _ in range(copies)]
        x = torch.randn(1, k, device="cuda", dtype=torch.float16, generator=g)
        y = torch.empty(1, n, dtype=torch.float16, device="cuda")
        with torch.cuda.stream(s):
            for w in ws:
                torch.ops.exl3rocm.linear(x, *w, bits, False, True)
        s.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            for r in range(reps):
                y = torch.ops.exl3rocm.linear(x, *ws[r % copies], bits, False, True)
        with torch.cuda.stream(s):
            _warm(torch, graph.replay, 0.1, s)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(3):
                graph.replay()
            e1.record(s)
        s.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (3 * reps)
        b = algo_bytes(1, k, n, bits)
        gemv[name] = {"k": k, "n": n, "bits": bits, "calls_per_token": calls, "us": round(us, 2),
                      "gbs": round(b / us / 1e3, 1), "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
        total_us += us * calls
        del graph, ws
        torch.cuda.empty_cache()
    prefill = {}
    for name, k, n, bits in CKPT_PREFILL:
        w = _device_layer(torch, k, n, bits, g)
        x = torch.randn(m_prefill, k, device="cuda", dtype=torch.float16, generator=g)
        # 0.3 s of warm calls first (the first milliseconds of GEMM work after a host pause ran up to
        # 30 % slow, the clocks still rising), then the median of three blocks of 4 calls
        _warm(torch, lambda: torch.ops.exl3rocm.linear(x, *w, bits, False, True), 0.3)
        blocks = []
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(4):
                torch.ops.exl3rocm.linear(x, *w, bits, False, True)
            e1.record()
            torch.cuda.synchronize()
            blocks.append(e0.elapsed_time(e1) * 1e3 / 4)
        us = sorted(blocks)[1]
        prefill[name] = {"m": m_prefill, "k": k, "n": n, "bits": bits, "us": round(us, 1),
                         "tflops": round(2 * m_prefill * k * n / us / 1e6, 1)}
        del w, x
        torch.cuda.empty_cache()
    return {"gemv_m1": gemv, "gemv_us_per_token_weighted": round(total_us, 1), "prefill": prefill}


def approx_m1(torch, sets, x5120, x17408, reps=64):
    """The opt-in approximate mul1 GEMV (exl3_gemv_mr_approx) at M = 1 on the configuration-1
    shapes: mean launch duration per mode, as per_shape_gemv times the faithful one, and each
    mode's rel-L2 deviation from the faithful output of the same launch."""
    from exl3rocm import kernels as E
    out = {}
    s = torch.cuda.Stream()
    for mode in ("affine", "int8"):
        row = {}
        for name, k, n in LAYER:
            x = x17408 if k == INTER else x5120
            y = torch.empty(1, n, dtype=torch.float16, device="cuda")
            yf = torch.empty_like(y)
            with torch.cuda.stream(s):
                for ls in sets:
                    T, SU, SV = ls.w[name]
                    E.exl3_gemv_mr_approx(x, T, y, SU, None, SV, ls.bits, mode)
                T, SU, SV = sets[0].w[name]
                E.exl3_gemv_mr_approx(x, T, y, SU, None, SV, sets[0].bits, mode)
                E.exl3_gemv(x, T, yf, SU, None, SV, False, True)
            s.synchronize()
            dev = ((y.float() - yf.float()).norm() / yf.float().norm()).item()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for r in range(reps):
                    T, SU, SV = sets[r % len(sets)].w[name]
                    E.exl3_gemv_mr_approx(x, T, y, SU, None, SV, sets[0].bits, mode)
            with torch.cuda.stream(s):
                g.replay()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(s)
                for _ in range(3):
                    g.replay()
                e1.record(s)
            s.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (3 * reps)
            b = algo_bytes(1, k, n, sets[0].bits)
            row[name] = {"us": round(us, 3), "gbs": round(b / us / 1e3, 1), "rel_l2_vs_faithful": round(dev, 6)}
            del g
        out[mode] = row
    return out


def gated_mlp(torch, sets, x5120, ms=(1, 8), reps=32):
    """The MLP of config 1 (gate/up, SiLU-and-mul, down) three ways, duration per MLP from a graph
    of `reps` MLPs over the weight copies (median of 7 interleaved rounds of 3 replays):
      unfused_us: linear_groups(gate, up), the elementwise SiLU-and-mul kernel, linear(down);
      silu_in_us: linear_groups(gate, up), then silu_mul_linear (the down GEMV forms the
                  activation as its input loads: exl3_gemv_silu_in), two launches;
      gated_us:   exl3_gemv_silu_mul (gate/up and the activation in one launch), linear(down)."""
    from exl3rocm import kernels as E
    ops = torch.ops.exl3rocm
    n = INTER
    out = {}
    s = torch.cuda.Stream()
    for m in ms:
        x = x5120.expand(m, HIDDEN).contiguous()
        act = torch.empty(m, n, dtype=torch.float16, device="cuda")

        def gate_up(ls):
            w = ls.w
            ptrs = ls.gu_ptrs if m == 1 else [None] * 3
            return ops.linear_groups(x, [w["gate"][0], w["up"][0]], [w["gate"][1], w["up"][1]],
                                     [w["gate"][2], w["up"][2]], [ls.bits, ls.bits], ls.mcg, ls.mul1, *ptrs)

        def unfused(ls):
            gu = gate_up(ls)
            E.silu_mul(gu[:, :n], gu[:, n:], act)
            ops.linear(act, *ls.w["down"], ls.bits, ls.mcg, ls.mul1)

        def silu_in(ls):
            ops.silu_mul_linear(gate_up(ls), *ls.w["down"], ls.bits, ls.mcg, ls.mul1)

        def gated(ls):
            w = ls.w
            E.exl3_gemv_silu_mul(x, [w["gate"][0], w["up"][0]], act, [w["gate"][1], w["up"][1]],
                                 [w["gate"][2], w["up"][2]], ls.bits, ls.mcg, ls.mul1)
            ops.linear(act, *w["down"], ls.bits, ls.mcg, ls.mul1)

        forms = (("unfused_us", unfused), ("silu_in_us", silu_in), ("gated_us", gated))
        graphs = {}
        for tag, fn in forms:
            with torch.cuda.stream(s):
                for ls in sets:
                    fn(ls)
            s.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for r in range(reps):
                    fn(sets[r % len(sets)])
            graphs[tag] = g
        # the forms' graphs replayed in turn, 7 rounds: the median per form (boxes drift by a few
        # percent over seconds, more than the forms differ)
        times = {tag: [] for tag, _ in forms}
        with torch.cuda.stream(s):
            for tag, _ in forms:
                graphs[tag].replay()
            for _ in range(7):
                for tag, _ in forms:
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record(s)
                    for _ in range(3):
                        graphs[tag].replay()
                    e1.record(s)
                    times[tag].append((e0, e1))
        s.synchronize()
        row = {tag: round(float(np.median([a.elapsed_time(b) for a, b in ev])) * 1e3 / (3 * reps), 2)
               for tag, ev in times.items()}
        del graphs
        out[f"m{m}"] = row
    return out


def cpu_baseline(base, bits, budget_s=8.0, reps=5):
    """The C oracle restatement on the host cores: the configuration-1 layer's 7 faithful GEMVs at
    M = 1 on every thread of this process's CPU share (the affinity mask, or OMP_NUM_THREADS where
    set), repeated until `budget_s` and at least `reps` times (the headline baseline), plus bounded
    side samples: one thread (q shape), decode only (reconstruct), configuration 0 (4096 x 4096
    mcg), configuration 2 (gate shape at 2 / 3 / 5 / 6 / 8 bpw) and a configuration-4 subsample (q
    at M = 64).  Every figure is the median over at least `reps` timed repetitions (after one
    untimed), in GB/s of the same algorithmic bytes as the GPU's."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import cpu  # noqa: E402  (oracle: test infrastructure, used here only as the baseline)
    from exl3rocm import synth
    affinity = len(os.sched_getaffinity(0))
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or affinity
    x = {k: synth.activations(synth.key_of("cpu", k), 1, k) for k in (HIDDEN, INTER)}
    layer_bytes = sum(algo_bytes(1, k, n, bits) for _, k, n in LAYER)

    def timed(fn, nbytes, budget=0.0):
        fn()                                           # untimed: first touch, thread pool start
        times = []
        t_end = time.perf_counter() + budget
        while len(times) < reps or time.perf_counter() < t_end:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        return {"gbs": round(nbytes / med / 1e9, 4), "us_per_call": round(med * 1e6, 1), "reps": len(times),
                "stat": "median"}

    def layer(th):
        for name, k, n in LAYER:
            tr, su, sv = base[name]
            cpu.linear(x[k], tr, bits, su, sv, 2, threads=th)

    head = timed(lambda: layer(threads), layer_bytes, budget_s)
    side = {"threads": threads, "affinity_cores": affinity}
    q_tr, q_su, q_sv = base["q"]
    side["config1_q_1thread"] = timed(lambda: cpu.linear(x[HIDDEN], q_tr, bits, q_su, q_sv, 2, threads=1),
                                      algo_bytes(1, HIDDEN, HIDDEN, bits))
    gate_tr = base["gate"][0]
    side["decode_only_gate"] = timed(lambda: cpu.reconstruct(gate_tr, bits, 2, threads=threads),
                                     HIDDEN * INTER * bits // 8)
    tr0, su0, sv0 = synth.layer("cpu-config0", 0, 4096, 4096, 4)
    x0 = synth.activations(synth.key_of("cpu-config0", "x"), 1, 4096)
    side["config0_mcg_4096"] = timed(lambda: cpu.linear(x0, tr0, 4, su0, sv0, 1, threads=threads),
                                     algo_bytes(1, 4096, 4096, 4))
    sweep = {}
    for b in (2, 3, 5, 6, 8):
        trb, sub, svb = synth.layer("cpu-config2", b, HIDDEN, INTER, b)
        sweep[f"{b}bpw"] = timed(lambda: cpu.linear(x[HIDDEN], trb, b, sub, svb, 2, threads=threads),
                                 algo_bytes(1, HIDDEN, INTER, b))
    side["config2_gate_sweep"] = sweep
    x64 = synth.activations(synth.key_of("cpu-config4", "x"), 64, HIDDEN)
    trq, suq, svq = base["q"]
    side["config4_q_m64"] = timed(lambda: cpu.linear(x64, trq, bits, suq, svq, 2, threads=threads),
                                  algo_bytes(64, HIDDEN, HIDDEN, bits))
    side["config4_q_m64"]["tflops"] = round(2 * 64 * HIDDEN * HIDDEN / (side["config4_q_m64"]["us_per_call"] * 1e6), 6)
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    side["cpu_model"] = model
    layer_weights = sum(k * n for _, k, n in LAYER)
    return {"value": head["gbs"], "unit": "GB/s", "cores": threads, "kind": "port",
            "us_per_layer": head["us_per_call"], "weights_per_s": round(layer_weights / (head["us_per_call"] * 1e-6), 1),
            "sample": f"median of {head['reps']} repetitions of the 7 linears of one configuration-1 layer at M=1, "
                      f"4 bpw mul1 (C oracle restatement, OpenMP {threads} threads of {affinity} in the affinity "
                      f"mask, {head['reps'] * head['us_per_call'] / 1e6:.1f} s); cpu: {model}",
            "side": side}



def prefill_mlp(torch, sets, x5120, m=2048, reps=4, rounds=5):
    """The MLP of config 1 at M = 2048 (the prefill routes), two ways, eager, mean duration per MLP
    over the weight copies (median of `rounds` interleaved rounds):
      unfused_us: linear_groups(gate, up), the elementwise SiLU-and-mul kernel, linear(down);
      silu_in_us: linear_groups(gate, up), then silu_mul_linear (the down prefill's input
                  transform forms the activation as it loads gate and up:
                  exl3_gemm_trellis_silu_in), no activation in memory."""
    from exl3rocm import kernels as E
    ops = torch.ops.exl3rocm
    n = INTER
    x = x5120.expand(m, HIDDEN).contiguous()
    act = torch.empty(m, n, dtype=torch.float16, device="cuda")

    def gate_up(ls):
        w = ls.w
        return ops.linear_groups(x, [w["gate"][0], w["up"][0]], [w["gate"][1], w["up"][1]],
                                 [w["gate"][2], w["up"][2]], [ls.bits, ls.bits], ls.mcg, ls.mul1)

    def unfused(ls):
        gu = gate_up(ls)
        E.silu_mul(gu[:, :n], gu[:, n:], act)
        ops.linear(act, *ls.w["down"], ls.bits, ls.mcg, ls.mul1)

    def silu_in(ls):
        ops.silu_mul_linear(gate_up(ls), *ls.w["down"], ls.bits, ls.mcg, ls.mul1)

    forms = (("unfused_us", unfused), ("silu_in_us", silu_in))
    for _, fn in forms:
        fn(sets[0])
    torch.cuda.synchronize()
    times = {tag: [] for tag, _ in forms}
    for _ in range(rounds):
        for tag, fn in forms:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for r in range(reps):
                fn(sets[r % len(sets)])
            e1.record()
            torch.cuda.synchronize()
            times[tag].append(e0.elapsed_time(e1) * 1e3 / reps)
    return {"m": m, **{tag: round(sorted(v)[len(v) // 2], 1) for tag, v in times.items()}}

def prefill_chunk(torch, layers=64, m=2048, bits=4, iters=2):
    """Configuration 4: M = 2048 through a 64-layer stack of the 7 linears (independent weights per
    layer, generated on the device), fp16 activations."""
    from exl3rocm import ops as exl3_ops  # noqa: F401
    g = torch.Generator(device="cuda").manual_seed(20260923)
    stack = []
    for _ in range(layers):
        lw = {}
        for name, k, n in LAYER:
            T = torch.randint(0, 65536, (k // 16, n // 16, 16 * bits), device="cuda", dtype=torch.int32,
                              generator=g).to(torch.int16)
            su = (torch.randn(k, device="cuda", generator=g).sign() * torch.exp(
                0.25 * torch.randn(k, device="cuda", generator=g))).half()
            sv = (torch.randn(n, device="cuda", generator=g).sign() * torch.exp(
                0.25 * torch.randn(n, device="cuda", generator=g))).half()
            lw[name] = (T, su, sv)
        stack.append(lw)
    xa = torch.randn(m, HIDDEN, device="cuda", dtype=torch.float16, generator=g)
    xb = torch.randn(m, INTER, device="cuda", dtype=torch.float16, generator=g)
    ops = torch.ops.exl3rocm

    # the plugin's module grouping: q/k/v and gate/up are fused modules (one linear_groups call,
    # one GEMM launch each), o and down single linears
    def chunk():
        for lw in stack:
            for names in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
                x = xb if names[0] == "down" else xa
                if len(names) == 1:
                    ops.linear(x, *lw[names[0]], bits, False, True)
                else:
                    ops.linear_groups(x, [lw[nm][0] for nm in names], [lw[nm][1] for nm in names],
                                      [lw[nm][2] for nm in names], [bits] * len(names), False, True)

    chunk()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        chunk()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / iters
    flops = 2.0 * m * sum(k * n for _, k, n in LAYER) * layers
    tf = flops / us / 1e6
    del stack
    torch.cuda.empty_cache()
    return {"m": m, "layers": layers, "bits": bits, "us_per_chunk": round(us, 1), "tflops": round(tf, 1),
            "frac_mfma_fp16": round(tf / MFMA_FP16_PEAK_TFLOPS, 4), "flops_per_chunk": flops}


def small_batch(torch, sets, ms=(1, 2, 4, 8, 12, 16, 17, 20, 24, 28, 32, 33, 36, 40, 44, 48, 49, 56, 64, 65, 128, 256),
                reps=32):
    """Configuration 3: gate (5120 -> 17408), down (17408 -> 5120) and the grouped gate/up launch
    (5120 -> 2 x 17408) at M from 1 to 256, heavy-tail activations.  Per M: the op (its route: the
    fused GEMV up to the measured crossover b of the launch's shape, the prefill GEMM above), the
    GEMV (<= 64 rows) and the prefill GEMM called directly, and the GEMM without a workspace (its
    tiles unsplit, the plan's comparison) at M in {4, ..., 256}.  Also b, the step at the route
    boundary op(b + 1) / op(b) - 1, the op's worst ratio to the faster route over M <= 64, and the
    smallest M at which the GEMM beats the GEMV.  Mean duration per call from a graph of `reps`
    calls over the weight copies (HIP events on the replay stream): the median of three blocks of
    two replays, each graph after 8 warm replays (~10 ms) and the whole section after ~0.3 s of
    M = 1 launches: the first graph timed after a host-side pause (capture, new inputs) ran 5-12 %
    slower than the same graph timed again, the order of the forms deciding which looked faster."""
    from exl3rocm import kernels as E, ops, synth, _lib
    res = {}
    s = torch.cuda.Stream()

    def graph_us(fn, blocks=3):
        with torch.cuda.stream(s):
            for ls in sets:
                fn(ls)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for r in range(reps):
                fn(sets[r % len(sets)])
        ts = []
        with torch.cuda.stream(s):
            for _ in range(8):
                g.replay()
            for _ in range(blocks):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(s)
                g.replay()
                g.replay()
                e1.record(s)
                s.synchronize()
                ts.append(e0.elapsed_time(e1) * 1e3 / (2 * reps))
        del g
        return round(sorted(ts)[len(ts) // 2], 2)

    x1 = torch.from_numpy(synth.activations(synth.key_of("cfg3", HIDDEN, 1), 1, HIDDEN)).cuda()
    graph_us(lambda ls: torch.ops.exl3rocm.linear(x1, *ls.w["gate"], ls.bits, ls.mcg, ls.mul1), blocks=240)

    for name, k, names in (("gate", HIDDEN, ("gate",)), ("down", INTER, ("down",)), ("gate_up", HIDDEN, ("gate", "up"))):
        n = HIDDEN if name == "down" else INTER
        ng = len(names)
        b = ops.gemv_max_rows(k, ng * n)
        m_all = sorted(set(ms) | {b, b + 1})
        xs = {m: torch.from_numpy(synth.activations(synth.key_of("cfg3", k, m), m, k, heavy_tail=True)).cuda()
              for m in m_all}
        W = lambda ls, i: [ls.w[nm][i] for nm in names]
        op_us, gemv_us, gemm_us, unsplit = {}, {}, {}, {}
        for m in m_all:
            x = xs[m]
            y = torch.empty(m, ng * n, dtype=torch.float16, device="cuda")
            xh = torch.empty(ng, m, k, dtype=torch.float16, device="cuda")
            ah = torch.empty(ng * m * k, dtype=torch.float16, device="cuda")
            if ng == 1:
                op_us[m] = graph_us(lambda ls, x=x: torch.ops.exl3rocm.linear(x, *ls.w[name], ls.bits, ls.mcg, ls.mul1))
            else:
                op_us[m] = graph_us(lambda ls, x=x: torch.ops.exl3rocm.linear_groups(
                    x, W(ls, 0), W(ls, 1), W(ls, 2), [ls.bits] * ng, ls.mcg, ls.mul1))
            if 1 < m <= _lib.GEMV_MAX_ROWS and ng == 1:
                gemv_us[m] = graph_us(lambda ls, x=x, y=y, ah=ah: E.exl3_gemv_mr(
                    x, ls.w[name][0], y, ls.w[name][1], ah, ls.w[name][2], ls.bits, ls.mcg, ls.mul1))
            elif 1 < m <= _lib.GEMV_MAX_ROWS:
                gemv_us[m] = graph_us(lambda ls, x=x, y=y, ah=ah: E.exl3_gemv_mr_grouped(
                    x, W(ls, 0), y, W(ls, 1), ah, W(ls, 2), ls.bits, ls.mcg, ls.mul1, ng))
            if m > 1:
                gemm_us[m] = graph_us(lambda ls, x=x, y=y, xh=xh: E.exl3_gemm_trellis_grouped(
                    x, W(ls, 0), y, W(ls, 1), xh, W(ls, 2), ls.bits, ls.mcg, ls.mul1))
            if ng == 1 and m in (4, 8, 16, 32, 64, 128, 256):
                unsplit[m] = graph_us(lambda ls, x=x, y=y, xh=xh: E.exl3_gemm_trellis(
                    x, ls.w[name][0], y, ls.w[name][1], xh[0], ls.w[name][2], ls.bits, ls.mcg, ls.mul1))
        cross = [m for m in gemv_us if gemm_us[m] < gemv_us[m]]
        worst = max(op_us[m] / min(gemv_us[m], gemm_us[m]) for m in gemv_us)
        row = {"launch": f"{k} -> {' + '.join([str(n)] * ng)}", "route_boundary": b,
               "boundary_step": round(op_us[b + 1] / op_us[b] - 1, 4),
               "boundary_note": "GEMV at b rows, GEMM at b + 1" if b < _lib.GEMV_MAX_ROWS else
                                f"b = the GEMV's {_lib.GEMV_MAX_ROWS}-row maximum: the GEMM at b + 1 is the only route",
               "op_over_faster_route_max": round(worst, 4),
               "gemm_faster_from_m": min(cross) if cross else f"none up to {max(gemv_us)}",
               "op_us": {f"m{m}": v for m, v in op_us.items()},
               "gemv_us": {f"m{m}": v for m, v in gemv_us.items()},
               "prefill_gemm_us": {f"m{m}": v for m, v in gemm_us.items()}}
        if unsplit:
            row["prefill_gemm_unsplit_us"] = {f"m{m}": v for m, v in unsplit.items()}
        res[name] = row
    return res


def traffic_probe(torch, bits=4, copies=8):
    """--traffic-probe: the dispatches two rocprofv3 --pmc passes (FETCH_SIZE, then WRITE_SIZE)
    read for roofline.traffic: a 256 MiB device copy (calibration: it reads and writes a known
    byte count) and one eager pass of the configuration-1 step over every weight copy."""
    n = 256 << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    from exl3rocm import synth
    _, sets = build_layers(torch, bits, copies)
    x5120 = torch.from_numpy(synth.activations(synth.key_of("config1", "x", HIDDEN), 1, HIDDEN)).cuda()
    x17408 = torch.from_numpy(synth.activations(synth.key_of("config1", "x", INTER), 1, INTER)).cuda()
    for ls in sets:
        ls.step(x5120, x17408)
    torch.cuda.synchronize()
    step_bytes = sum(algo_bytes(1, k, n_, bits) for _, k, n_ in LAYER)
    print(json.dumps({"copy_bytes": n, "copies": copies, "launches_per_step": launches_per_step(),
                      "step_algorithmic_bytes": step_bytes}), flush=True)
    return 0


TL_NAMES = ("entry", "issued", "loop", "loop_end", "stored", "counted", "summed", "end")


def timeline(torch, sets, x5120, x17408, reps=16):
    """--timeline (the tracing library, libexl3_mi355x_timeline.so): per-workgroup phase stamps
    (include/exl3_mi355x_timeline.h) of each configuration-1 GEMV launch.  A graph of `reps`
    launches of one kind over the weight copies is replayed twice; the stamps are those of its last
    launch (steady state, weights from HBM).  Times in us from the first workgroup's entry: the
    median and the last workgroup per phase, the critical (last-ending) workgroup's own phases, and
    the launch's mean duration from HIP events on the replay stream."""
    import ctypes
    from exl3rocm import _lib
    L = _lib.lib()
    if not hasattr(L, "exl3_timeline_read"):
        raise SystemExit("bench.py --timeline needs the tracing library (build_ext.py --timeline)")
    ip = ctypes.POINTER(ctypes.c_int)
    L.exl3_timeline_shape.argtypes = [ip, ip]
    L.exl3_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    mw, ph = ctypes.c_int(), ctypes.c_int()
    L.exl3_timeline_shape(ctypes.byref(mw), ctypes.byref(ph))
    buf = np.zeros(mw.value * ph.value, dtype=np.uint64)
    s = torch.cuda.Stream()
    out = {}
    for name in STEP_LAUNCHES:
        with torch.cuda.stream(s):
            for ls in sets:
                ls.launch(name, x5120, x17408)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for r in range(reps):
                sets[r % len(sets)].launch(name, x5120, x17408)
        assert L.exl3_timeline_clear() == 0
        with torch.cuda.stream(s):
            g.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            g.replay()
            e1.record(s)
        s.synchronize()
        assert L.exl3_timeline_read(buf.ctypes.data, buf.nbytes) == 0
        raw = buf.reshape(mw.value, ph.value)
        live = raw[:, 0] != 0                                # workgroups of this launch (all run)
        hw = raw[live, 8]
        t = raw[live, :8].astype(np.int64)
        us = (t - t[:, :1].min()) * 10 / 1e3                 # 100 MHz ticks -> us from the first entry
        reducer = t[:, 6] >= t[:, 0]                         # reduced in this launch (not a stale stamp)
        # per CU (XCC, SE, SH, CU): when its last loop ended; first-dispatched (older) workgroups
        cu = ((hw >> np.uint64(32)) * np.uint64(1 << 16) + ((hw >> np.uint64(8)) & np.uint64(0xFF))).astype(np.int64)
        cu_end = np.array([us[cu == c, 3].max() for c in np.unique(cu)])
        xcc = (hw >> np.uint64(32)).astype(np.int64)
        older = np.arange(len(t)) < min(256, len(t))
        crit = int(np.argmax(us[:, 7]))
        row = {"wgs": int(len(t)), "launch_us": round(e0.elapsed_time(e1) * 1e3 / reps, 2)}
        for i, nm in enumerate(TL_NAMES):
            col = us[reducer, i] if nm == "summed" else us[:, i]
            row[nm] = {"p50": round(float(np.median(col)), 2), "max": round(float(col.max()), 2)}
        row["loop_us"] = {"p50": round(float(np.median(us[:, 3] - us[:, 2])), 2),
                          "max": round(float((us[:, 3] - us[:, 2]).max()), 2)}
        row["critical_wg"] = {nm: round(float(us[crit, i]), 2) for i, nm in enumerate(TL_NAMES)
                              if nm != "summed" or reducer[crit]}
        row["cus"] = int(len(cu_end))
        row["cu_loop_end"] = {q: round(float(np.percentile(cu_end, p)), 2) for q, p in
                              (("min", 0), ("p10", 10), ("p50", 50), ("p90", 90), ("max", 100))}
        row["loop_end_older_younger_p50"] = [round(float(np.median(us[older, 3])), 2),
                                             round(float(np.median(us[~older, 3])), 2)]
        row["xcc_loop_end_p50"] = [round(float(np.median(us[xcc == x, 3])), 2) for x in np.unique(xcc)]
        out[name] = row
        del g
    print("| launch | WGs | launch us | " + " | ".join(f"{nm} p50 / max" for nm in TL_NAMES) + " | loop us p50 / max |")
    print("|---|---|---|" + "---|" * (len(TL_NAMES) + 1))
    for name, r in out.items():
        cells = " | ".join(f"{r[nm]['p50']:.2f} / {r[nm]['max']:.2f}" for nm in TL_NAMES)
        print(f"| {name} | {r['wgs']} | {r['launch_us']} | {cells} | {r['loop_us']['p50']:.2f} / {r['loop_us']['max']:.2f} |")
    for name, r in out.items():
        print(f"critical workgroup of {name}: " + ", ".join(f"{k} {v:.2f}" for k, v in r["critical_wg"].items()))
        print(f"  {name}: loop end per CU ({r['cus']} CUs) {r['cu_loop_end']}; older / younger workgroups "
              f"p50 {r['loop_end_older_younger_p50']}; per XCC p50 {r['xcc_loop_end_p50']}")
    print(json.dumps({"timeline": out}), flush=True)
    return 0


def measured_traffic():
    """HBM bytes per GEMV launch of the configuration-1 step, from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by the same counter on a copy of known size);
    None when that summary is absent."""
    path = os.path.join(REPO, "profiles", "gemv_traffic_config1.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--copies", type=int, default=8)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--traffic-probe", action="store_true", help="only the dispatches the PMC traffic passes read")
    ap.add_argument("--config3-only", action="store_true",
                    help="only the configuration-3 section (the GEMV at small M, the prefill GEMM split and "
                         "unsplit at M = 4-256; what its kernel-trace profile reads); prints its dict")
    ap.add_argument("--timeline", action="store_true",
                    help="only the per-workgroup phase timeline of each configuration-1 GEMV launch (loads the "
                         "tracing library exl3rocm/libexl3_mi355x_timeline.so: build_ext.py --timeline)")
    ap.add_argument("--checkpoint-only", action="store_true",
                    help="only the reference checkpoint's shapes (GEMV at M = 1, prefill at M = 2048; what "
                         "its kernel-trace profile reads); prints its dict")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the configuration-4 prefill chunk (what the prefill PMC passes read); prints its dict")
    args = ap.parse_args()
    if args.steps < 1 or args.warmup < 0:
        print("bench.py: --steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this engine runs on one GPU; multi-GPU runs are not part of this build "
              "(the path would shard q/k/v/gate/up by 128-column blocks and o/down by 128-row "
              "blocks, each GPU running these kernels on its shard)", file=sys.stderr)
        return 2

    if args.timeline:
        os.environ["EXL3_MI355X_LIB"] = os.path.join(REPO, "qwen38-27b-exl3-rdna4_amd", "exl3rocm",
                                                     "libexl3_mi355x_timeline.so")
    import torch
    from exl3rocm import _lib, ops  # noqa: F401
    _lib.lib()
    bits = 4
    if args.traffic_probe:
        return traffic_probe(torch, bits, args.copies)
    if args.prefill_only:
        print(json.dumps(prefill_chunk(torch)), flush=True)
        return 0
    if args.checkpoint_only:
        print(json.dumps(checkpoint_shapes(torch)), flush=True)
        return 0
    if args.timeline:
        _, sets = build_layers(torch, bits, args.copies)
        from exl3rocm import synth
        x5120 = torch.from_numpy(synth.activations(synth.key_of("config1", "x", HIDDEN), 1, HIDDEN)).cuda()
        x17408 = torch.from_numpy(synth.activations(synth.key_of("config1", "x", INTER), 1, INTER)).cuda()
        return timeline(torch, sets, x5120, x17408)
    if args.config3_only:
        _, sets = build_layers(torch, bits, args.copies)
        print(json.dumps(small_batch(torch, sets)), flush=True)
        return 0
    log("building layer set (4 bpw, mul1) x %d copies" % args.copies)
    base, sets = build_layers(torch, bits, args.copies)
    from exl3rocm import synth
    x5120 = torch.from_numpy(synth.activations(synth.key_of("config1", "x", HIDDEN), 1, HIDDEN)).cuda()
    x17408 = torch.from_numpy(synth.activations(synth.key_of("config1", "x", INTER), 1, INTER)).cuda()
    graphs = capture_steps(torch, sets, x5120, x17408, args.steps)
    log("timing %d decode steps" % args.steps)
    elapsed, wall = time_graphs(torch, graphs, args.steps, args.warmup)
    step_bytes = sum(algo_bytes(1, k, n, bits) for _, k, n in LAYER)
    value = args.steps * step_bytes / elapsed / 1e9
    ms_per_step = elapsed * 1e3 / args.steps
    lps = launches_per_step()
    avg_launch_us = ms_per_step * 1e3 / lps
    achieved = step_bytes / lps / avg_launch_us / 1e3
    traffic = measured_traffic()
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": round(traffic) if traffic is not None else None,
                "traffic_source": "profiles/gemv_traffic_config1.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE)",
                "kernel": "gemv_kernel<4,2,0,0> (every M=1 launch of the step)",
                "bytes_per_launch": step_bytes / lps, "mean_launch_us": round(avg_launch_us, 3)}
    copy_gbs, read_gbs = device_copy_gbs(torch)
    roofline["achievable_gbs"] = copy_gbs
    roofline["frac_of_achievable"] = round(achieved / copy_gbs, 4)
    roofline["achievable_source"] = "device copy of 1 GiB (torch copy_, read + write bytes), median of 30, HIP events"
    roofline["achievable_read_gbs"] = read_gbs
    roofline["frac_of_achievable_read"] = round(achieved / read_gbs, 4)
    weights = sum(k * n for _, k, n in LAYER)
    valu_floor_us = weights * VALU_OPS_PER_WEIGHT_4BPW / VALU_LANE_OPS_PER_S * 1e6
    roofline["valu_decode_roof"] = {
        "ops_per_weight": round(VALU_OPS_PER_WEIGHT_4BPW, 3), "weights_per_step": weights,
        "lane_ops_per_s": VALU_LANE_OPS_PER_S, "floor_us_per_step": round(valu_floor_us, 2),
        "max_gbs": round(step_bytes / valu_floor_us / 1e3, 1),
        "frac_of_valu_roof": round(valu_floor_us / (ms_per_step * 1e3), 4)}
    extra = {"launches_per_step": lps, "step_bytes": step_bytes, "wall_s": round(wall, 3),
             "us_per_layer": round(ms_per_step * 1e3, 3), "weights_per_s": round(weights / (ms_per_step * 1e-3), 1)}
    log("per-shape GEMV timing")
    extra["per_shape_m1"] = per_shape_gemv(torch, sets, x5120, x17408)
    # the same step graphs again, now that the GPU has run decode work for a while: 400 steps after
    # 40 warmup steps (a decode loop's clock; the timed region above follows ~1 s of idle set-up)
    n_s = args.steps if graphs["rest"] is not None else max(1, 400 // graphs["block"]) * graphs["block"]
    el_s, _ = time_graphs(torch, graphs, n_s, 40)
    extra["headline_steady"] = {"steps": n_s, "warmup": 40, "gbs": round(n_s * step_bytes / el_s / 1e9, 1),
                                "us_per_step": round(el_s * 1e6 / n_s, 2)}
    log("reference checkpoint shapes (GEMV scoreboard, prefill)")
    extra["checkpoint_shapes"] = checkpoint_shapes(torch)
    log("approximate mul1 GEMV (opt-in affine / int8 routes)")
    extra["approx_m1"] = approx_m1(torch, sets, x5120, x17408)
    log("gated MLP (gate/up, SiLU-and-mul, down) three ways")
    extra["gated_mlp"] = gated_mlp(torch, sets, x5120, ms=(1, 2, 4, 8, 16))
    log("gated MLP at M=2048 (prefill routes) two ways")
    extra["gated_mlp_prefill"] = prefill_mlp(torch, sets, x5120)
    if not args.no_sweep:
        log("small-batch crossover")
        extra["config3_small_batch"] = small_batch(torch, sets)
        del graphs
        sweep = {}
        for b in (2, 3, 5, 6, 8):
            _, ss = build_layers(torch, b, 4, tag="config2")
            sweep[f"{b}bpw"] = per_shape_gemv(torch, ss, x5120, x17408, reps=32)
            del ss
        _, ss = build_layers(torch, 4, 4, mul1=False, tag="config2")
        sweep["4bpw_mcg"] = per_shape_gemv(torch, ss, x5120, x17408, reps=32)
        del ss
        extra["config2_sweep_m1"] = sweep
        torch.cuda.empty_cache()
    if not args.no_prefill:
        log("prefill chunk (M=2048, 64 layers)")
        del sets
        torch.cuda.empty_cache()
        extra["config4_prefill"] = prefill_chunk(torch)
    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline(base, bits)
    line = {
        "metric": "EXL3 GEMV GB/s (% HBM peak) at M=1; prefill TFLOPS (% MFMA) at M=2048",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic (counter-RNG seeded trellis / suh / svh / x)",
        "config": {"workload": "config1: M=1 decode step through the 7 EXL3 linears of a Qwen-27B-shaped layer "
                               "(hidden 5120, 40q/8kv x 128, intermediate 17408), 4 bpw mul1, 8 weight copies",
                   "m": 1, "bits": bits, "codebook": "mul1", "copies": args.copies},
        "frac_hbm": round(value / HBM_PEAK_GBS, 4),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
