"""CPU checks of the prefill GEMM's producer / consumer schedule (gemm_pc_kernel in
csrc/exl3_gemm.hip), no GPU needed.

1. The built library's machine code: on every control-flow path into every workgroup barrier of
   every gemm_pc_kernel<BITS, CB>, only the most recent batch of 8 xh-row loads may still be in
   flight (tests/isa_waits.py).  This is what failed before the trellis fetch used fixed-count
   loads: the compiler merged the 3 / 5 / 6 / 7-bit fetches' single-word loads, so the prologue's
   vmcnt(8 + 2 NW) let half of step 0's rows be in flight at the first barrier.
2. The checker itself, on hand-built instruction streams with planted mistakes.
3. A model of the kernel's stage indexing for every step count a tile or K-split piece can have
   (pc_plan): which LDS stage each interval writes and each consumer step reads, per barrier.
"""
import os

import pytest

import isa_waits as W

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "qwen38-27b-exl3-rdna4_amd", "exl3rocm", "libexl3_mi355x.so")


# ---------------------------------------------------------------------------------------------
# 1. the built machine code
# ---------------------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def pc_report():
    if not os.path.exists(f"{W.LLVM}/llvm-objdump"):
        pytest.skip("ROCm llvm tools not installed")
    assert os.path.exists(LIB), "libexl3_mi355x.so is not built (run __graft_entry__.build())"
    return W.pc_kernel_report(LIB)


def test_every_prefill_kernel_is_checked(pc_report):
    import re
    inst = {tuple(int(v) for v in re.search(r"ILi(\d)ELi(\d)E", k).groups()) for k in pc_report}
    assert inst == {(b, cb) for b in range(1, 9) for cb in range(3)}
    for name, (viol, barriers) in pc_report.items():
        # B_-1, the unrolled intervals and their tail, the piece path, the epilogue
        assert barriers >= 8, (name, barriers)


def test_prefill_rows_landed_at_every_barrier(pc_report):
    bad = {k: [v.path_note for v in viol] for k, (viol, _) in pc_report.items() if viol}
    assert not bad, bad


# ---------------------------------------------------------------------------------------------
# 2. the checker on hand-built streams
# ---------------------------------------------------------------------------------------------
def _stream(lines):
    """[text] -> [Inst]; branch targets written as `<k+0xOFF>` with OFF = 4 * index."""
    return [W.Inst(4 * i, t.split()[0], t) for i, t in enumerate(lines)]


DMA = "buffer_load_dwordx4 v2, s[12:15], s7 offen lds"
WORD = "buffer_load_dword v9, v19, s[16:19], s7 offen"
X3 = "buffer_load_dwordx3 v[10:12], v13, s[16:19], s7 offen"


def _prologue(fetch, wait):
    return [*fetch, *[DMA] * 8, *[DMA] * 8, *fetch, *fetch, f"s_waitcnt vmcnt({wait}) lgkmcnt(0)", "s_barrier",
            "s_endpgm"]


def test_checker_accepts_exact_counts():
    # fetch = 3 words + predecessor, 4 loads; 8 + 2 * 4 issued after step 0's rows
    v, n = W.check_barriers(_stream(_prologue([WORD] * 4, 16)))
    assert n == 1 and not v


def test_checker_flags_a_merged_fetch():
    # the 3 words merged into one dwordx3: 2 loads a fetch, the wait still assumes 4
    v, _ = W.check_barriers(_stream(_prologue([X3, WORD], 16)))
    assert len(v) == 1
    v, _ = W.check_barriers(_stream(_prologue([X3, WORD], 12)))
    assert not v


def test_checker_flags_a_missing_wait():
    s = [*[DMA] * 8, *[DMA] * 8, "s_waitcnt lgkmcnt(0)", "s_barrier", "s_endpgm"]
    assert len(W.check_barriers(_stream(s))[0]) == 1


def test_checker_follows_the_loop_back_edge():
    # each trip issues a batch and a 4-load fetch, then waits for all but 8 + 2 * 4: exact on the
    # first trip (after the prologue's batch and fetch) and on every later one
    body = [*[DMA] * 8, *[WORD] * 4, "s_waitcnt vmcnt(16)", "s_barrier", "s_cbranch_scc1 <k+0x{top:x}>",
            "s_endpgm"]
    pro = [*[DMA] * 8, *[WORD] * 4]
    s = _stream(pro + [t.format(top=4 * len(pro)) for t in body])
    assert not W.check_barriers(s)[0]
    # a 3-load fetch under the same wait: the first trip still has 8 + 8 + 3 ops after the
    # prologue's batch, later trips only 3 + 8 + 3: wrong on the back edge alone
    body = [*[DMA] * 8, *[WORD] * 3, "s_waitcnt vmcnt(16)", "s_barrier", "s_cbranch_scc1 <k+0x{top:x}>",
            "s_endpgm"]
    pro = [*[DMA] * 8, *[WORD] * 8]
    s = _stream(pro + [t.format(top=4 * len(pro)) for t in body])
    assert len(W.check_barriers(s)[0]) == 1
    s = _stream(pro + [t.format(top=4 * len(pro)).replace("s_cbranch_scc1", "s_nop 0 ;") for t in body])
    assert not W.check_barriers(s)[0]


# ---------------------------------------------------------------------------------------------
# 3. the stage schedule
# ---------------------------------------------------------------------------------------------
STAGES = 3


def pc_steps_of_plan(M, K, widths):
    """Step counts of every item of a pc_plan launch: whole tiles K / 64, pieces of the split tail
    [q * all / split, (q + 1) * all / split), or the two unequal pieces [0, cut), [cut, all) of a
    launch of more than half and at most two thirds of a wave (exl3_gemm.hip pc_plan /
    gemm_pc_kernel)."""
    tiles = sum(((M + 255) // 256) * (w // 128) for w in widths)
    full, tail = divmod(tiles, 256)
    all_steps = K // 64
    split = min(256 // tail, all_steps // 8) if full >= 1 and tail > 0 else 1
    if full == 0 and 2 * tail <= 256:
        split = min(256 // tail, all_steps // 8)
    if full == 0 and 2 * tail > 256 and 3 * tail <= 512 and all_steps >= 16:
        cut = (2 * all_steps + 2) // 3
        return {all_steps, cut, all_steps - cut}
    if split < 2:
        split = 1
    out = {all_steps}
    if split > 1:
        out |= {(q + 1) * all_steps // split - q * all_steps // split for q in range(split)}
    return out


def simulate(steps):
    """The kernel's LDS traffic for one tile of `steps` K steps.  Epoch e is the time between
    barriers B_e-1 and B_e (epoch -1: before B_-1).  Returns writes [(stage, step, issued in epoch,
    complete by barrier)] and reads [(stage, step, epoch)]."""
    writes = [
        (0, 0, -1, -1),                                 # prologue: rows and B fragments of step 0
        (1, min(1, steps - 1), -1, 0),                  # rows of step 1: waited for in interval 0
    ]
    for s in range(steps):                              # producer interval s runs in epoch s
        last = s + 1 >= steps                           # the last interval waits for vmcnt(0)
        writes.append(((s + 1) % STAGES, min(s + 1, steps - 1), s, s))          # B fragments (lgkmcnt(0))
        writes.append(((s + 2) % STAGES, min(s + 2, steps - 1), s, s if last else s + 1))   # rows
    reads = [(s % STAGES, s, s) for s in range(steps)]  # consumer step s reads stage s % 3 in epoch s
    return writes, reads


@pytest.mark.parametrize("steps", list(range(1, 40)) + [80, 272])
def test_stage_schedule(steps):
    writes, reads = simulate(steps)
    for stage, step, e in reads:
        # the step's rows and fragments are in the stage before the barrier that opens epoch e
        mine = [w for w in writes if w[0] == stage and w[1] == step and w[3] <= e - 1]
        assert len(mine) >= 2 or (step == 0 and mine), (stage, step, e)
        # no write of other data to the stage is in flight during the reads, and the last write of
        # other data completed before the step's own data was written
        for st, data, issued, done in writes:
            if st != stage or data == step:
                continue
            assert not (issued <= e <= done), f"stage {stage}: step {data} written during step {step}'s reads"
            if done <= e - 1:
                assert all(issued < w[2] or done < w[2] for w in mine), (stage, step, data)
    # both roles pass B_-1 and one barrier per step
    assert len(reads) == steps and sum(1 for w in writes if w[2] >= 0) == 2 * steps


def test_schedule_model_flags_a_two_stage_ring():
    # planted mistake: with two stages the rows of step s + 2 land in the stage step s reads
    global STAGES
    saved, STAGES = STAGES, 2
    try:
        with pytest.raises(AssertionError):
            test_stage_schedule(6)
    finally:
        STAGES = saved


def test_plans_produce_only_modelled_step_counts():
    shapes = [(2048, 5120, [5120]), (2048, 17408, [5120]), (2048, 5120, [17408, 17408]),
              (2048, 5120, [5120, 1024, 1024]), (600, 256, [384]), (256, 1024, [128] * 4), (33, 128, [128]),
              (64, 17408, [5120]), (40, 5120, [5120]), (96, 1024, [512, 384]),
              (33, 5120, [17408]), (64, 1024, [17408]), (768, 5120, [5120, 1024, 1024])]
    for M, K, widths in shapes:
        for st in pc_steps_of_plan(M, K, widths):
            assert st >= 2, (M, K, widths, st)
            test_stage_schedule(st)


def test_unequal_pieces_plan_matches_the_library():
    """The two-piece plan modelled above is the library's: its workspace (4 KB of counters plus
    one fp32 partial tile per piece) for launches of 136 and 168 tiles, and none of it for 170 <
    tiles < 256 (no split, no workspace) and equal pieces for at most half a wave."""
    import ctypes
    from exl3rocm import _lib
    L = _lib.lib()

    def ws(M, K, widths):
        return L.exl3_gemm_trellis_workspace_size(M, K, (ctypes.c_int * len(widths))(*widths), len(widths))

    piece = 256 * 128 * 4
    assert ws(33, 5120, [17408]) == 4096 + 136 * 2 * piece
    assert ws(768, 5120, [5120, 1024, 1024]) == 4096 + 168 * 2 * piece
    assert pc_steps_of_plan(33, 5120, [17408]) == {80, 54, 26}
    assert ws(33, 5120, [17408 + 128 * 60]) == 0                 # 196 tiles: unsplit, no workspace
    assert ws(33, 5120, [128 * 100]) == 4096 + 100 * 2 * piece   # 100 tiles: 2 equal pieces (min(256 / 100, 10))
