"""CPU checks of the cross-workgroup completion protocols in the built machine code (no GPU).

The GEMV's split-K partial sums (gemv_kernel) and the prefill's K-split pieces (gemm_pc_kernel)
finish a block the same way: every contributor stores its fp32 partial, waits for the stores to
complete, adds one to the block's completion counter (a relaxed device-scope atomic), and the one
that sees the count complete loads all the partials.  There is no acquire or release; the protocol
holds because of properties of the emitted instructions, which tests/isa_waits.py checks on every
control-flow path of every instantiation:

* every vector store to global memory carries sc1 (device scope: written through to the coherent
  level);
* every partial store has completed (s_waitcnt vmcnt(0)) before the counter atomic that announces it;
* every vector load that can run after a counter atomic carries sc1 (device scope);
* the scope encodings those checks read (sc1 = agent scope on loads and stores; the plain atomic =
  agent scope for read-modify-write) are what this hipcc emits for gfx950.

Each rule is also shown to catch a planted mistake on a hand-built instruction stream.
"""
import os
import re
import shutil
import subprocess

import pytest

import isa_waits as W

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "qwen38-27b-exl3-rdna4_amd", "exl3rocm", "libexl3_mi355x.so")
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.fixture(scope="module")
def report():
    if not os.path.exists(f"{W.LLVM}/llvm-objdump"):
        pytest.skip("ROCm llvm tools not installed")
    assert os.path.exists(LIB), "libexl3_mi355x.so is not built (run __graft_entry__.build())"
    return W.protocol_report(LIB)


def test_every_completion_kernel_is_checked(report):
    gemv = [k for k in report if "gemv_kernel" in k]
    pc = [k for k in report if "gemm_pc_kernel" in k]
    assert len(pc) == 24                                     # bits 1..8 x codebooks 0..2
    assert len(gemv) >= 8 * 3 * 3 * 4                        # bits x codebooks x row forms x plain/gated/SiLU/fp32
    for name, r in report.items():
        assert r.atomics >= 1, name                          # the counter add
        assert r.loads_after >= 1, name                      # the partial loads
        assert r.stores >= 2, name                           # partials and outputs


def test_completion_protocols_hold_on_every_path(report):
    bad = {k: r.violations[:3] for k, r in report.items() if r.violations}
    assert not bad, bad


# ---------------------------------------------------------------------------------------------
# planted mistakes on hand-built streams
# ---------------------------------------------------------------------------------------------
def _stream(lines):
    return [W.Inst(4 * i, t.split()[0], t) for i, t in enumerate(lines)]


PART_ST = "global_store_dword v[2:3], v26, off sc1"
ATOMIC = "global_atomic_add v12, v[12:13], v1, off sc0"
PART_LD = "global_load_dword v15, v[14:15], off sc1"
Y_ST = "buffer_store_dword v5, v30, s[52:55], 0 offen sc1"


def _good():
    return [PART_ST, "s_waitcnt vmcnt(0)", "s_barrier", ATOMIC, "s_waitcnt vmcnt(0)", PART_LD,
            "s_waitcnt vmcnt(0)", Y_ST, "s_endpgm"]


def test_checker_accepts_the_protocol():
    r = W.check_protocol(_stream(_good()))
    assert r.violations == [] and r.atomics == 1 and r.loads_after == 1 and r.stores == 2


def test_checker_catches_a_partial_store_without_device_scope():
    s = _good()
    s[0] = "global_store_dword v[2:3], v26, off"              # workgroup-visible only
    assert any("store without sc1" in v for v in W.check_protocol(_stream(s)).violations)


def test_checker_catches_a_counter_add_before_the_partials_landed():
    s = _good()
    s[1] = "s_waitcnt vmcnt(1)"                                # the partial may still be in flight
    v = W.check_protocol(_stream(s)).violations
    assert any("may be in flight at the counter atomic" in x for x in v), v


def test_checker_catches_a_partial_load_without_device_scope():
    s = _good()
    s[5] = "global_load_dword v15, v[14:15], off"              # could hit a stale local L2 line
    assert any("load after a counter atomic without sc1" in v for v in W.check_protocol(_stream(s)).violations)


def test_checker_follows_branches_to_the_atomic():
    """The store reaches the atomic only around a branch that skips the wait."""
    s = [PART_ST, "s_cbranch_scc0 1 <k+0x10>", "s_waitcnt vmcnt(0)", "s_nop 0", ATOMIC, "s_endpgm"]
    v = W.check_protocol(_stream(s)).violations
    assert any("may be in flight" in x for x in v), v
    s[1] = "s_nop 0"                                           # no path skips the wait
    assert W.check_protocol(_stream(s)).violations == []


def test_branch_targets_are_read_from_the_disassembly_comment():
    """llvm-objdump names a branch target inside the // comment; the parser keeps it, so blocks()
    sees the taken edge."""
    dis = ("0000000000001000 <k>:\n"
           "\ts_cbranch_scc0 1                                       // 000000001000: BF850001 <k+0x8>\n"
           "\ts_nop 0                                                // 000000001004: BF800000\n"
           "\ts_endpgm                                               // 000000001008: BF810000\n")
    insts = W.functions(dis)["k"]
    assert "<k+0x8>" in insts[0].text
    bl = W.blocks(insts)
    assert [b.start for b in bl] == [0x1000, 0x1004, 0x1008]
    assert sorted(bl[2].preds) == [0, 1]


# the flag idiom: "wait for everything on the last pass, else for the older batch"
def _flag_loop(wait_on_skip):
    return [
        "buffer_load_dwordx4 v4, s[8:11], s65 offen lds",     # 0: older batch
        "buffer_load_dwordx4 v4, s[8:11], s65 offen lds",     # 1
        "buffer_load_dwordx4 v4, s[8:11], s65 offen lds",     # 2: newest batch
        "s_cmp_ge_i32 s37, s31",                              # 3
        "s_mov_b64 s[10:11], -1",                             # 4
        "s_cbranch_scc0 2 <k+0x20>",                          # 5 -> 8
        "s_waitcnt vmcnt(0)",                                 # 6
        "s_mov_b64 s[10:11], 0",                              # 7
        "s_andn2_b64 vcc, exec, s[10:11]",                    # 8
        "s_cbranch_vccnz 2 <k+0x34>",                         # 9 -> 13 (taken only after vmcnt(0))
        wait_on_skip,                                         # 10
        "s_branch 0 <k+0x34>",                                # 11 -> 13
        "s_nop 0",                                            # 12
        "s_barrier",                                          # 13
        "s_endpgm",
    ]


def test_flag_idiom_prunes_the_infeasible_path(monkeypatch):
    monkeypatch.setattr(W, "LDS_BATCH", 1)                    # one load per batch in this stream
    viol, checked = W.check_barriers(_stream(_flag_loop("s_waitcnt vmcnt(1)")))
    assert checked == 1 and viol == []


def test_flag_idiom_keeps_a_feasible_violation(monkeypatch):
    monkeypatch.setattr(W, "LDS_BATCH", 1)
    viol, _ = W.check_barriers(_stream(_flag_loop("s_waitcnt vmcnt(2)")))  # the older batch not waited
    assert len(viol) == 1


def test_flag_idiom_with_another_write_keeps_the_path(monkeypatch):
    """A write to the flag pair the idiom does not recognise forgets the condition: the walk keeps
    the path (conservative) and reports what it finds there."""
    monkeypatch.setattr(W, "LDS_BATCH", 1)
    s = _flag_loop("s_waitcnt vmcnt(1)")
    s[4] = "s_and_b64 s[10:11], s[2:3], -1"                   # flag of unknown value
    viol, _ = W.check_barriers(_stream(s))
    assert len(viol) == 1


# ---------------------------------------------------------------------------------------------
# the scope encodings the rules read, against this hipcc
# ---------------------------------------------------------------------------------------------
SCOPE_PROBE = r"""
#include <hip/hip_runtime.h>
__global__ void k(float* p, unsigned* c)
{
    __hip_atomic_store(p + 0, 1.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_store(p + 64, 2.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p + 128, 3.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    unsigned a = __hip_atomic_fetch_add(c + 0, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    unsigned b = __hip_atomic_fetch_add(c + 64, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned d = __hip_atomic_fetch_add(c + 128, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    float x = __hip_atomic_load(p + 256, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    float y = __hip_atomic_load(p + 320, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float z = __hip_atomic_load(p + 384, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    p[600] = x + y + z + a + b + d;
}
"""
# byte offset of each access in the probe -> (kind, scope)
PROBE_ACCESSES = {("store", 0): "workgroup", ("store", 256): "agent", ("store", 512): "system",
                  ("rmw", 0): "workgroup", ("rmw", 256): "agent", ("rmw", 512): "system",
                  ("load", 1024): "workgroup", ("load", 1280): "agent", ("load", 1536): "system"}


def test_scope_encodings_are_this_compilers(tmp_path):
    if not os.path.exists(HIPCC) or shutil.which("llvm-objdump", path=W.LLVM) is None:
        pytest.skip("hipcc / ROCm llvm tools not installed")
    src = tmp_path / "scope.hip"
    src.write_text(SCOPE_PROBE)
    obj = tmp_path / "scope.o"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-c", str(src), "-o", str(obj)], check=True,
                   capture_output=True)
    work = tmp_path / "w"
    work.mkdir()
    insts = next(v for k, v in W.functions(W.code_object_disassembly(str(obj), str(work))).items() if k.startswith("_Z1k"))
    got = {}
    for ins in insts:
        for kind, pat in (("store", W._STORE), ("rmw", W._ATOMIC), ("load", W._LOAD)):
            if pat.match(ins.op):
                m = re.search(r"offset:(\d+)", ins.text)
                key = (kind, int(m.group(1)) if m else 0)
                if key in PROBE_ACCESSES:
                    got[key] = W.cache_bits(ins.text) - ({"sc0"} if kind == "rmw" else set())   # rmw sc0: return value
    assert set(got) == set(PROBE_ACCESSES), sorted(got)
    for (kind, off), scope in PROBE_ACCESSES.items():
        assert got[(kind, off)] == W.SCOPE_ENCODINGS[kind][scope], (kind, scope, got[(kind, off)])
