"""Checkers of the gfx950 machine code this repository builds (test infrastructure; nothing in the
product imports it): the prefill kernel's explicit LDS-DMA waits, and the cross-workgroup
completion protocols of the GEMV and the prefill's split tiles.

The producer waves of `gemm_pc_kernel` request xh rows straight into LDS (`buffer_load_dwordx4 ...
lds`, 8 per K step) and, before each workgroup barrier, wait with an explicit `s_waitcnt
vmcnt(N)` whose N counts the loads issued after the rows the consumers read next.  That count is
only right if the compiler emits exactly the loads the source counts, in the source's order: a
merge of adjacent trellis-word loads (three `buffer_load_dword` into one `buffer_load_dwordx3`)
or a load hoisted above the row requests leaves rows in flight at the barrier.

This module reads the code object out of the built library (`llvm-objcopy` + `clang-offload-bundler`
+ `llvm-objdump`, all ROCm tools run on this repository's own build), splits each kernel into
basic blocks (fall-through and taken-branch edges; llvm-objdump names a branch's target in its
comment), and checks on every control-flow path into every `s_barrier`:

    all LDS-DMA loads except the most recent batch of 8 are complete,

using the in-order completion of vector-memory operations: a load L is complete after a wait
`vmcnt(N)` when at least N vector-memory operations were issued after L and before the wait.
At barrier B_s the most recent batch holds the rows of step s + 2 (read after B_s+1); every older
batch (the rows of step s + 1, read right after B_s) must have landed.
"""
from __future__ import annotations

import os
import re
import subprocess
import tempfile
from dataclasses import dataclass, field

LLVM = "/opt/rocm/llvm/bin"
LDS_BATCH = 8                      # xh row loads a producer wave issues per K step
VMCNT_MAX = 63                     # gfx9 vmcnt field: 6 bits

_VMEM = re.compile(r"^(buffer|global|flat|scratch)_(load|store|atomic)")
_BRANCH = re.compile(r"^s_(c?branch\w*)$")
_TARGET = re.compile(r"<(?P<sym>[^>+]+)\+0x(?P<off>[0-9a-f]+)>")


@dataclass
class Inst:
    addr: int
    op: str
    text: str


@dataclass
class Block:
    start: int
    insts: list = field(default_factory=list)
    preds: list = field(default_factory=list)


_BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def code_object_disassembly(obj_path: str, workdir: str) -> str:
    """gfx950 disassembly of a host object or shared library built by build_ext.py.  A linked
    library's `.hip_fatbin` section holds one offload bundle per translation unit, back to back:
    each is unbundled and disassembled."""
    fb = os.path.join(workdir, "fatbin")
    subprocess.run([f"{LLVM}/llvm-objcopy", "--dump-section", f".hip_fatbin={fb}", obj_path, os.devnull],
                   check=True, capture_output=True)
    data = open(fb, "rb").read()
    starts = [m.start() for m in re.finditer(re.escape(_BUNDLE_MAGIC), data)]
    out = []
    for i, s in enumerate(starts):
        part = os.path.join(workdir, f"bundle{i}")
        with open(part, "wb") as f:
            f.write(data[s:starts[i + 1] if i + 1 < len(starts) else len(data)])
        co = part + ".co"
        subprocess.run([f"{LLVM}/clang-offload-bundler", "--unbundle", "--type=o",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={part}", f"--output={co}"],
                       check=True, capture_output=True)
        r = subprocess.run([f"{LLVM}/llvm-objdump", "-d", "--mcpu=gfx950", co], check=True, capture_output=True,
                           text=True)
        out.append(r.stdout)
    return "\n".join(out)


def functions(dis: str) -> dict:
    """symbol -> [Inst] from llvm-objdump output."""
    out, cur = {}, None
    for line in dis.splitlines():
        m = re.match(r"^([0-9a-f]+) <(.+)>:$", line)
        if m:
            cur = m.group(2)
            out[cur] = []
            continue
        if cur is None or not line.startswith("\t"):
            continue
        m = re.search(r"//\s*([0-9A-F]+):", line)
        if not m:
            continue
        text = line.split("//")[0].strip()
        if not text:
            continue
        # llvm-objdump names a branch's target in the comment (`// ADDR: WORD <sym+0xoff>`): keep it
        tgt = _TARGET.search(line.split("//", 1)[1])
        if tgt and _BRANCH.match(text.split()[0]):
            text = f"{text} {tgt.group(0)}"
        out[cur].append(Inst(int(m.group(1), 16), text.split()[0], text))
    return out


def blocks(insts: list) -> list:
    """Basic blocks with predecessor lists (branch targets are `<sym+0xoff>` in the listing)."""
    if not insts:
        return []
    base = insts[0].addr
    leaders = {insts[0].addr}
    for i, ins in enumerate(insts):
        if _BRANCH.match(ins.op) or ins.op == "s_endpgm":
            m = _TARGET.search(ins.text)
            if m:
                leaders.add(base + int(m.group("off"), 16))
            if i + 1 < len(insts):
                leaders.add(insts[i + 1].addr)
    bl, index = [], {}
    for ins in insts:
        if ins.addr in leaders:
            index[ins.addr] = len(bl)
            bl.append(Block(ins.addr))
        bl[-1].insts.append(ins)
    for bi, b in enumerate(bl):
        last = b.insts[-1]
        succ = []
        if _BRANCH.match(last.op):
            m = _TARGET.search(last.text)
            if m:
                succ.append(index[base + int(m.group("off"), 16)])
            if last.op != "s_branch" and bi + 1 < len(bl):
                succ.append(bi + 1)
        elif last.op != "s_endpgm" and bi + 1 < len(bl):
            succ.append(bi + 1)
        for s in succ:
            bl[s].preds.append(bi)
    return bl


# ---------------------------------------------------------------------------------------------
# Branch-flag constraints.  The compiler lowers "wait for everything on the last interval, else
# for the older batch" as
#     s_mov_b64 s[a:b], -1 ; s_cbranch_scc0 L ; s_waitcnt vmcnt(0) ; s_mov_b64 s[a:b], 0
#  L: s_andn2_b64 vcc, exec, s[a:b] ; s_cbranch_vccnz TOP ; s_waitcnt vmcnt(N) ; s_branch TOP
# where the taken vccnz edge is only reachable through the vmcnt(0) block (exec is nonzero where such
# a wave-uniform flag is tested, so vcc = exec & ~flag is nonzero exactly when the flag is 0).  A
# backward walk that
# crosses a vcc branch edge carries what the edge implies about vcc ("nz" or "z"), turns it into a
# condition on s[a:b] at the s_andn2_b64 that set vcc, and drops the path at an s_mov_b64 of s[a:b]
# that contradicts it.  Any other write to the registers involved forgets the condition (the path
# is kept: conservative).
# ---------------------------------------------------------------------------------------------
def _regs(tok: str) -> set:
    tok = tok.strip()
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return {f"s{i}" for i in range(int(m.group(1)), int(m.group(2)) + 1)}
    if re.fullmatch(r"s\d+", tok):
        return {tok}
    if tok in ("vcc", "vcc_lo", "vcc_hi"):
        return {"vcc_lo", "vcc_hi"} if tok == "vcc" else {tok}
    return set()


def _dest_regs(ins: Inst) -> set:
    if _VMEM.match(ins.op) and "store" in ins.op or ins.op.startswith(("s_cbranch", "s_branch", "s_waitcnt", "s_barrier",
                                                                      "s_cmp", "s_nop", "s_setprio")):
        return set()
    parts = ins.text.split(None, 1)
    return _regs(parts[1].split(",")[0]) if len(parts) > 1 else set()


def _edge_constraint(bl: list, pred: int, succ: int, cons: frozenset):
    """cons plus what taking the edge pred -> succ implies about vcc at the end of pred; None when
    that contradicts a condition already carried (the path is infeasible)."""
    last = bl[pred].insts[-1]
    if last.op not in ("s_cbranch_vccnz", "s_cbranch_vccz"):
        return cons
    m = _TARGET.search(last.text)
    taken = m is not None and bl[succ].start == bl[0].start + int(m.group("off"), 16)
    nonzero = taken == (last.op == "s_cbranch_vccnz")
    if ("vcc", not nonzero) in cons:
        return None
    return cons | {("vcc", nonzero)}


def _step_constraint(ins: Inst, cons: frozenset):
    """(conditions, feasible) after walking backward over ins: each condition on a register ins
    writes is translated (vcc set by s_andn2_b64 from a flag pair), checked (an s_mov_b64 of the
    flag pair) or forgotten (any other write)."""
    if not cons:
        return cons, True
    written = _dest_regs(ins)
    if not written:
        return cons, True
    out = set()
    for reg, nonzero in cons:
        if not written & _regs(reg):
            out.add((reg, nonzero))
            continue
        if reg == "vcc":
            m = re.fullmatch(r"s_andn2_b64 vcc, exec, (s\[\d+:\d+\])", ins.text)
            # vcc = exec & ~s: nonzero exactly when s does not cover exec (exec is nonzero here)
            if m:
                out.add((m.group(1), nonzero))
            continue
        m = re.fullmatch(rf"s_mov_b64 {re.escape(reg)}, (-?\d+)", ins.text)
        if m:
            v = int(m.group(1))
            if (v == -1 and nonzero) or (v == 0 and not nonzero):
                return frozenset(), False               # exec & ~(-1) == 0, exec & ~0 == exec != 0
    return frozenset(out), True


def _vmcnt(text: str) -> int:
    m = re.search(r"vmcnt\((\d+)\)", text)
    return int(m.group(1)) if m else VMCNT_MAX


def _is_lds_dma(ins: Inst) -> bool:
    return ins.op.startswith("buffer_load") and re.search(r"\blds\b", ins.text) is not None


@dataclass
class Violation:
    barrier_addr: int
    path_note: str


def check_barriers(insts: list) -> tuple:
    """(violations, barriers checked, max lds loads in flight seen) for one kernel.

    Backward walk from each s_barrier over every path.  State: lds loads seen (up to the first
    load of the older batch), vector-memory operations seen c (issued between the point and the
    barrier), and thresh = min over waits passed of (ops between that wait and the barrier) +
    its vmcnt.  A load at backward count c is complete when c >= thresh; the first older-batch
    load is the last one that needs checking (older loads have larger c)."""
    bl = blocks(insts)
    violations, checked = [], 0
    cap = VMCNT_MAX + 1
    for bi, b in enumerate(bl):
        for pos, ins in enumerate(b.insts):
            if ins.op != "s_barrier":
                continue
            checked += 1
            seen = set()
            stack = [(bi, pos - 1, 0, 0, cap, frozenset())]
            bad = None
            while stack and bad is None:
                blk, p, lds, c, thresh, cons = stack.pop()
                feasible = True
                while p >= 0:
                    cur = bl[blk].insts[p]
                    cons, feasible = _step_constraint(cur, cons)
                    if not feasible:
                        break
                    if cur.op == "s_waitcnt":
                        thresh = min(thresh, c + _vmcnt(cur.text))
                    elif _VMEM.match(cur.op):
                        if _is_lds_dma(cur):
                            lds += 1
                            if lds > LDS_BATCH:
                                if c < thresh:
                                    bad = f"lds load at {cur.addr:#x}: {c} later ops, wait allows {thresh}"
                                break
                        c = min(c + 1, cap)
                    p -= 1
                else:
                    key = (blk, lds, c, thresh, cons)
                    if key in seen:
                        continue
                    seen.add(key)
                    for pr in bl[blk].preds:
                        pc = _edge_constraint(bl, pr, blk, cons)
                        if pc is not None:
                            stack.append((pr, len(bl[pr].insts) - 1, lds, c, thresh, pc))
                    continue
            if bad is not None:
                violations.append(Violation(ins.addr, bad))
    return violations, checked


# ---------------------------------------------------------------------------------------------
# Completion protocols (gemv_kernel: split-K partial sums; gemm_pc_kernel: K-split pieces)
#
# A contributor stores its fp32 partial, then increments the block's completion counter (a relaxed
# atomic); the contributor that sees the count complete loads every partial and finishes the block.
# There is no acquire or release: correctness rests on three properties of the machine code,
# checked on every control-flow path:
#   stores    every vector store to global memory (partials, counter resets, outputs) carries sc1:
#             write-through to the device-coherent level, so another CU's device-scope load sees it
#             once it has completed;
#   ordering  every partial store has completed before the counter add that announces it: on every
#             path into every vector atomic, each store issued before the completion phase (not
#             reachable from an atomic) is followed by an s_waitcnt vmcnt(0) before the atomic;
#   loads     every vector load that can run after a counter atomic carries sc1 (device scope: it
#             misses the local L2 for the coherent copy) -- the partials, and the svh the same code
#             reads next to them;
# and on the atomics themselves, whose agent-scope form on gfx950 is the plain atomic (the same
# encoding as workgroup scope; system scope adds sc0 sc1 -- SCOPE_ENCODINGS, pinned against this
# hipcc by tests/test_pc_schedule.py).
# ---------------------------------------------------------------------------------------------
# (scope) -> cache-policy bits the compiler emits on gfx950 for relaxed atomic load / store / rmw
SCOPE_ENCODINGS = {
    "load": {"workgroup": {"sc0"}, "agent": {"sc1"}, "system": {"sc0", "sc1"}},
    "store": {"workgroup": {"sc0"}, "agent": {"sc1"}, "system": {"sc0", "sc1"}},
    "rmw": {"workgroup": set(), "agent": set(), "system": {"sc1"}},      # besides sc0 = return the old value
}
_ATOMIC = re.compile(r"^(buffer|global|flat)_atomic")
_STORE = re.compile(r"^(buffer|global|flat)_store")
_LOAD = re.compile(r"^(buffer|global|flat)_load")


def cache_bits(text: str) -> set:
    return {b for b in ("sc0", "sc1", "nt") if re.search(rf"\b{b}\b", text)}


def _reachable_from(bl: list, starts: list) -> set:
    """(block, index) of every instruction reachable after the given (block, index) points."""
    seen, out = set(), set()
    stack = [(b, i + 1) for b, i in starts]
    while stack:
        b, i = stack.pop()
        if (b, i) in seen:
            continue
        seen.add((b, i))
        if i >= len(bl[b].insts):
            for s, blk in enumerate(bl):
                if b in blk.preds:
                    stack.append((s, 0))
            continue
        out.add((b, i))
        stack.append((b, i + 1))
    return out


@dataclass
class ProtocolReport:
    atomics: int
    stores: int
    loads_after: int
    violations: list


def check_protocol(insts: list) -> ProtocolReport:
    """The three properties above on one kernel's instructions."""
    bl = blocks(insts)
    where = [(b, i) for b, blk in enumerate(bl) for i in range(len(blk.insts))]
    atomics = [(b, i) for b, i in where if _ATOMIC.match(bl[b].insts[i].op)]
    after = _reachable_from(bl, atomics)
    viol, nstore, nload = [], 0, 0
    for b, i in where:
        ins = bl[b].insts[i]
        if _STORE.match(ins.op) and not _is_lds_dma(ins):
            nstore += 1
            if "sc1" not in cache_bits(ins.text):
                viol.append(f"store without sc1 at {ins.addr:#x}: {ins.text}")
        if _LOAD.match(ins.op) and not _is_lds_dma(ins) and (b, i) in after:
            nload += 1
            if "sc1" not in cache_bits(ins.text):
                viol.append(f"load after a counter atomic without sc1 at {ins.addr:#x}: {ins.text}")
        if _ATOMIC.match(ins.op) and "nt" in cache_bits(ins.text):
            viol.append(f"non-temporal counter atomic at {ins.addr:#x}")
    # ordering: backward from each atomic, a pre-completion store must meet a vmcnt(0) first
    for ab, ai in atomics:
        stack, seen = [(ab, ai - 1, frozenset())], set()
        while stack:
            b, i, cons = stack.pop()
            stop = False
            while i >= 0:
                ins = bl[b].insts[i]
                cons, feasible = _step_constraint(ins, cons)
                if not feasible:
                    stop = True
                    break
                if ins.op == "s_waitcnt" and _vmcnt(ins.text) == 0:
                    stop = True
                    break
                if _STORE.match(ins.op) and not _is_lds_dma(ins) and (b, i) not in after:
                    viol.append(f"store at {ins.addr:#x} may be in flight at the counter atomic at "
                                f"{bl[ab].insts[ai].addr:#x}")
                    stop = True
                    break
                i -= 1
            if stop or (b, cons) in seen:
                continue
            seen.add((b, cons))
            for pr in bl[b].preds:
                pc = _edge_constraint(bl, pr, b, cons)
                if pc is not None:
                    stack.append((pr, len(bl[pr].insts) - 1, pc))
    return ProtocolReport(len(atomics), nstore, nload, viol)


def protocol_report(obj_path: str, kinds=("gemv_kernel", "gemm_pc_kernel")) -> dict:
    """{kernel symbol: ProtocolReport} for every instantiation of the given kernels in obj_path."""
    with tempfile.TemporaryDirectory() as d:
        dis = code_object_disassembly(obj_path, d)
    return {name: check_protocol(insts) for name, insts in functions(dis).items()
            if any(k in name for k in kinds)}


def pc_kernel_report(obj_path: str) -> dict:
    """{kernel symbol: (violations, barriers)} for every gemm_pc_kernel instantiation in obj_path."""
    with tempfile.TemporaryDirectory() as d:
        dis = code_object_disassembly(obj_path, d)
    rep = {}
    for name, insts in functions(dis).items():
        if "gemm_pc_kernel" in name:
            rep[name] = check_barriers(insts)
    return rep
