"""Checker of the prefill kernel's explicit memory waits on the gfx950 machine code this repository
builds (test infrastructure; nothing in the product imports it).

The producer waves of `gemm_pc_kernel` request xh rows straight into LDS (`buffer_load_dwordx4 ...
lds`, 8 per K step) and, before each workgroup barrier, wait with an explicit `s_waitcnt
vmcnt(N)` whose N counts the loads issued after the rows the consumers read next.  That count is
only right if the compiler emits exactly the loads the source counts, in the source's order: a
merge of adjacent trellis-word loads (three `buffer_load_dword` into one `buffer_load_dwordx3`)
or a load hoisted above the row requests leaves rows in flight at the barrier.

This module reads the code object out of the built library (`llvm-objcopy` + `clang-offload-bundler`
+ `llvm-objdump`, all ROCm tools run on this repository's own build), splits each kernel into
basic blocks, and checks on every control-flow path into every `s_barrier`:

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
            stack = [(bi, pos - 1, 0, 0, cap)]
            bad = None
            while stack and bad is None:
                blk, p, lds, c, thresh = stack.pop()
                while p >= 0:
                    cur = bl[blk].insts[p]
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
                    key = (blk, lds, c, thresh)
                    if key in seen:
                        continue
                    seen.add(key)
                    for pr in bl[blk].preds:
                        stack.append((pr, len(bl[pr].insts) - 1, lds, c, thresh))
                    continue
            if bad is not None:
                violations.append(Violation(ins.addr, bad))
    return violations, checked


def pc_kernel_report(obj_path: str) -> dict:
    """{kernel symbol: (violations, barriers)} for every gemm_pc_kernel instantiation in obj_path."""
    with tempfile.TemporaryDirectory() as d:
        dis = code_object_disassembly(obj_path, d)
    rep = {}
    for name, insts in functions(dis).items():
        if "gemm_pc_kernel" in name:
            rep[name] = check_barriers(insts)
    return rep
