"""CPU tests of the C-ABI library: it loads without a GPU, exports every symbol the header
declares, and its host-only entry points (sizing, eligibility, argument validation that returns
before any launch) behave as documented.  No kernel runs here."""
import ctypes
import os
import re

import pytest

from exl3rocm import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "exl3_mi355x.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|size_t)\s+(exl3_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_reference_entry_points():
    names = declared_functions()
    for want in ("exl3_decode", "exl3_reconstruct", "exl3_reconstruct_slice", "exl3_had_r_128", "exl3_gemv",
                 "exl3_gemv_mr", "exl3_gemv_mr_grouped", "exl3_gemv_mr_supported", "exl3_mgemm",
                 "exl3_hgemm_recon", "exl3_gemm"):
        assert want in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(declared_functions()) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_loader_and_abi_version():
    L = _lib.lib()
    assert L.exl3_abi_version() == _lib.ABI_VERSION


def test_grid_choice_depends_only_on_shape():
    L = _lib.lib()
    assert L.exl3_gemv_grid(5120, 5120, 1) == 512           # 40 blocks x 40 units, all resident
    assert L.exl3_gemv_grid(5120, 17408, 2) == 256           # two groups share the resident slots
    assert L.exl3_gemv_grid(5120, 1024, 1) == 160            # 320 units, <= 32 workgroups per block
    assert L.exl3_gemv_grid(256, 128, 1) == 2
    assert L.exl3_gemv_grid(5000, 128, 1) == 0


def test_workspace_sizes():
    L = _lib.lib()
    ws1 = L.exl3_gemv_workspace_size(1, 5120, 5120, 4, 1)
    ws16 = L.exl3_gemv_workspace_size(16, 5120, 5120, 4, 1)
    ws2g = L.exl3_gemv_workspace_size(1, 5120, 5120, 4, 2)
    assert ws1 >= 65536 + 512 * 2 * 128 * 4 and ws16 > ws1 and ws2g >= ws1
    assert L.exl3_gemv_workspace_size(64, 5120, 5120, 4, 1) > 0          # the 64-row plain GEMV
    assert L.exl3_gemv_workspace_size(65, 5120, 5120, 4, 1) == 0        # beyond the GEMV row limit
    assert L.exl3_gemv_workspace_size(1, 5000, 5120, 4, 1) == 0         # k not a multiple of 128


def test_widths_workspace_sizes():
    L = _lib.lib()
    eq = (ctypes.c_int * 2)(4096, 4096)
    assert L.exl3_gemv_workspace_size_widths(4, 5120, eq, 2) == L.exl3_gemv_workspace_size(4, 5120, 4096, 4, 2)
    qkv = (ctypes.c_int * 3)(5120, 1024, 1024)
    assert L.exl3_gemv_workspace_size_widths(1, 5120, qkv, 3) > 65536
    bad = (ctypes.c_int * 2)(5120, 1000)
    assert L.exl3_gemv_workspace_size_widths(1, 5120, bad, 2) == 0
    dummy = ctypes.c_void_p(0x1000)
    arr = (ctypes.c_void_p * 3)(0x1000, 0x1000, 0x1000)
    # output row narrower than the groups' total width
    assert L.exl3_gemv_mr_grouped_widths(dummy, 5120, arr, dummy, 5120, arr, None, arr, qkv, 3, 2, 5120, 4, 0, 1,
                                         dummy, 1 << 30, None) == _lib.EINVAL


def test_mr_supported_predicate():
    L = _lib.lib()
    assert L.exl3_gemv_mr_supported(1, 5120, 5120, 4, 0, 1) == 1
    assert L.exl3_gemv_mr_supported(32, 5120, 1024, 8, 1, 0) == 1
    assert L.exl3_gemv_mr_supported(64, 5120, 1024, 8, 1, 0) == 1
    assert L.exl3_gemv_mr_supported(65, 5120, 1024, 8, 1, 0) == 0
    assert L.exl3_gemv_mr_supported(4, 5120, 1000, 4, 0, 1) == 0
    assert L.exl3_gemv_mr_supported(4, 5120, 1024, 9, 0, 1) == 0


def test_invalid_arguments_return_before_any_launch():
    L = _lib.lib()
    dummy = ctypes.c_void_p(0x1000)
    # bad shapes / null pointers are rejected with EINVAL, declines with DECLINED
    assert L.exl3_reconstruct(dummy, dummy, 100, 128, 4, 0, 1, None) == _lib.EINVAL
    assert L.exl3_reconstruct_slice(dummy, 128, dummy, 128, 128, 4, 0, 1, 8, 16, None) == _lib.EINVAL
    assert L.exl3_had_r_128(dummy, 100, dummy, 100, 1, 100, None, None, 1.0, None) == _lib.EINVAL
    assert L.exl3_decode(None, dummy, 16, 0, 1, None) == _lib.EINVAL
    assert L.exl3_gemv(dummy, 128, dummy, dummy, 128, dummy, None, dummy, 2, 128, 128, 4, 0, 1, dummy, 1 << 20,
                       None) == _lib.DECLINED
    assert L.exl3_gemv_f32(dummy, 128, dummy, dummy, 128, dummy, None, dummy, 2, 128, 128, 4, 0, 1, dummy, 1 << 20,
                           None) == _lib.DECLINED
    assert L.exl3_gemv_f32(dummy, 128, dummy, None, 128, dummy, None, dummy, 1, 128, 128, 4, 0, 1, dummy, 1 << 20,
                           None) == _lib.EINVAL
    assert L.exl3_gemv_mr(dummy, 128, dummy, dummy, 128, dummy, None, dummy, 65, 128, 128, 4, 0, 1, dummy, 1 << 20,
                          None) == _lib.DECLINED
    assert L.exl3_gemv_mr(dummy, 128, dummy, dummy, 128, dummy, None, dummy, 1, 128, 128, 4, 0, 1, dummy, 0,
                          None) == _lib.EWORKSPACE
    assert L.exl3_hgemm_recon(dummy, 64, dummy, 100, dummy, 100, 4, 64, 100, None) == _lib.EINVAL
    assert L.exl3_gemm_trellis(dummy, 128, dummy, dummy, 128, dummy, dummy, dummy, 64, 128, 128, 9, 0, 1,
                               None) == _lib.EINVAL
    assert L.exl3_mgemm(dummy, None, dummy, dummy, None, dummy, 2, 128, 128, 4, 0, 1, dummy, 1 << 20,
                        None) == _lib.EINVAL
    # the prefill SiLU-input form: null up, unaligned gate, K out of range
    assert L.exl3_gemm_trellis_silu_in(dummy, None, 256, dummy, dummy, 128, dummy, dummy, dummy, 64, 128, 128, 4, 0, 1,
                                       None, 0, None) == _lib.EINVAL
    assert L.exl3_gemm_trellis_silu_in(ctypes.c_void_p(0x1002), dummy, 256, dummy, dummy, 128, dummy, dummy, dummy, 64,
                                       128, 128, 4, 0, 1, None, 0, None) == _lib.EINVAL
    assert L.exl3_gemm_trellis_silu_in(dummy, dummy, 256, dummy, dummy, 128, dummy, dummy, dummy, 64, 128, 128, 9, 0, 1,
                                       None, 0, None) == _lib.EINVAL


def test_check_raises_on_errors():
    with pytest.raises(_lib.Exl3Error):
        _lib.check(_lib.EINVAL, "x")
    assert _lib.check(_lib.DECLINED, "x") == _lib.DECLINED


def test_gemv_split_fast_division_matches_brute_force():
    """The kernels' unit split (lo / owner with 32-bit multiply-high division) against 64-bit
    arithmetic and brute force, on the launch shapes of config 1 and random splits."""
    import random
    L = _lib.lib()
    cases = [(1600, 512, 256, 3, 2), (5440, 256, 256, 3, 2), (5440, 256, 0, 3, 2), (320, 160, 160, 3, 2),
             (18496, 512, 256, 3, 2), (77600, 512, 256, 3, 2), (2 ** 21, 512, 256, 3, 2), (40, 2, 2, 1, 1),
             (1, 1, 1, 1, 1), (7, 7, 3, 1, 64), (1600, 512, 256, 2, 3), (2240, 512, 256, 2, 3), (5440, 512, 256, 2, 3),
             (10880, 512, 256, 2, 3)]
    rng = random.Random(7)
    for _ in range(150):
        G = rng.randint(1, 600)
        cases.append((rng.randint(G, 150000), G, rng.randint(0, G), rng.randint(1, 8), rng.randint(1, 8)))
    for c in cases:
        assert L.exl3_gemv_split_check(*c) == 0, c
    assert L.exl3_gemv_split_check(0, 1, 0, 1, 1) == -1
    assert L.exl3_gemv_split_check(2 ** 22, 512, 256, 64, 64) == -1      # beyond the 32-bit domain


def test_prefill_workspace_bound_covers_every_plan():
    """exl3_gemm_trellis_workspace_bound >= the workspace of every plan, and some plan needs all of
    it (170 tiles in two unequal pieces each): tile counts 1 .. 3 waves at one and two row tiles."""
    L = _lib.lib()
    bound = L.exl3_gemm_trellis_workspace_bound()
    worst = 0
    for m in (33, 300):
        for k in (1024, 5120):
            for nt in range(1, 3 * 256 + 1):
                w = (ctypes.c_int * 1)(128 * nt)
                worst = max(worst, L.exl3_gemm_trellis_workspace_size(m, k, w, 1))
    assert 0 < worst == bound, (worst, bound)


def test_silu_prerot_rows_query():
    assert _lib.lib().exl3_gemv_silu_prerot_rows() == int(os.environ.get("EXL3_GEMV_SILU_PREROT_M", "4"))
    assert _lib.lib().exl3_gemv_prerot_rows() == int(os.environ.get("EXL3_GEMV_PREROT_M", "2"))


@pytest.mark.parametrize("env,want", [(None, 2), ("5", 5), ("65", 65)])
def test_prerot_override_in_a_fresh_process(env, want):
    """EXL3_GEMV_PREROT_M is read once per process: unset, exl3_gemv_prerot_rows() is 2 (the fewest
    rows at which the per-launch rule may pre-rotate); set, it is that row count (every launch from
    it, none below).  Checked in a fresh interpreter (no GPU call)."""
    import subprocess
    import sys
    e = dict(os.environ)
    e.pop("EXL3_GEMV_PREROT_M", None)
    if env is not None:
        e["EXL3_GEMV_PREROT_M"] = env
    code = ("import sys; sys.path.insert(0, %r); from exl3rocm import _lib; "
            "print(_lib.lib().exl3_gemv_prerot_rows())") % os.path.join(REPO, "qwen38-27b-exl3-rdna4_amd")
    out = subprocess.run([sys.executable, "-c", code], env=e, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert int(out.stdout.strip().splitlines()[-1]) == want


@pytest.mark.parametrize("env", ["0", "-3", "1", "8", "junk"])
def test_gemv_plan_knobs_out_of_range_in_a_fresh_process(env):
    """The measurement knobs of the GEMV grid plan never break sizing: EXL3_GEMV_MAX_CONTRIB of 0,
    a negative value or a non-number plans as the default (no division by zero); EXL3_GEMV_GRID
    and EXL3_GEMV_WEIGHTS with the same values fall back or clamp.  Every workspace size stays
    positive.  Checked in a fresh interpreter (no GPU call)."""
    import subprocess
    import sys
    e = dict(os.environ)
    e.update({"EXL3_GEMV_MAX_CONTRIB": env, "EXL3_GEMV_GRID": env, "EXL3_GEMV_WEIGHTS": env + "," + env})
    code = ("import sys; sys.path.insert(0, %r); from exl3rocm import _lib; L = _lib.lib(); "
            "print(min(L.exl3_gemv_workspace_size(m, k, n, 4, g) for m in (1, 16, 64) "
            "for k, n in ((5120, 5120), (17408, 5120), (5120, 17408), (128, 128)) for g in (1, 2)))"
            ) % os.path.join(REPO, "qwen38-27b-exl3-rdna4_amd")
    out = subprocess.run([sys.executable, "-c", code], env=e, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert int(out.stdout.strip().splitlines()[-1]) > 0
