"""ctypes binding of libexl3_mi355x.so (include/exl3_mi355x.h).

The library is the only compute path: if it is missing or fails to load, every op raises.
There is no CPU or PyTorch fallback.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("EXL3_MI355X_LIB", os.path.join(HERE, "libexl3_mi355x.so"))

OK, DECLINED, EINVAL, ELAUNCH, EWORKSPACE = 0, 1, -1, -2, -3
MAX_GROUPS = 4
GEMV_MAX_ROWS = 64
GEMV_FUSED_MAX_ROWS = 32
NOALLOC_SCRATCH_BYTES = 17039360
ABI_VERSION = 3

_p, _i, _i64, _sz, _f = C.c_void_p, C.c_int, C.c_int64, C.c_size_t, C.c_float
_pp = C.POINTER(C.c_void_p)
_ip = C.POINTER(C.c_int)

# name -> (restype, argtypes); mirrors include/exl3_mi355x.h
SIGNATURES = {
    "exl3_abi_version": (_i, []),
    "exl3_decode": (_i, [_p, _p, _i64, _i, _i, _p]),
    "exl3_reconstruct": (_i, [_p, _p, _i, _i, _i, _i, _i, _p]),
    "exl3_reconstruct_slice": (_i, [_p, _i64, _p, _i, _i, _i, _i, _i, _i, _i, _p]),
    "exl3_had_r_128": (_i, [_p, _i64, _p, _i64, _i, _i, _p, _p, _f, _p]),
    "exl3_had_r_128_f32": (_i, [_p, _i64, _p, _i64, _i, _i, _p, _p, _f, _p]),
    "exl3_gemv_grid": (_i, [_i, _i, _i]),
    "exl3_gemv_workspace_size": (_sz, [_i, _i, _i, _i, _i]),
    "exl3_gemv_mr_supported": (_i, [_i, _i, _i, _i, _i, _i]),
    "exl3_gemv": (_i, [_p, _i64, _p, _p, _i64, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _sz, _p]),
    "exl3_gemv_f32": (_i, [_p, _i64, _p, _p, _i64, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _sz, _p]),
    "exl3_gemv_mr": (_i, [_p, _i64, _p, _p, _i64, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _sz, _p]),
    "exl3_gemv_mr_grouped": (_i, [_p, _i64, _pp, _p, _i64, _pp, _p, _pp, _i, _i, _i, _i, _i, _i, _i, _i, _p, _sz,
                                  _p]),
    "exl3_gemv_mr_grouped_widths": (_i, [_p, _i64, _pp, _p, _i64, _pp, _p, _pp, _ip, _i, _i, _i, _i, _i, _i, _p,
                                         _sz, _p]),
    "exl3_gemv_workspace_size_widths": (_sz, [_i, _i, _ip, _i]),
    "exl3_gemv_split_check": (_i, [_i, _i, _i, _i, _i]),
    "exl3_gemv_prerot_rows": (_i, []),
    "exl3_gemv_silu_prerot_rows": (_i, []),
    "exl3_gemv_silu_mul": (_i, [_p, _i64, _pp, _p, _i64, _pp, _p, _pp, _i, _i, _i, _i, _i, _i, _p, _sz, _p]),
    "exl3_silu_mul": (_i, [_p, _p, _i64, _p, _i64, _i, _i, _p]),
    "exl3_gemv_silu_in": (_i, [_p, _p, _i64, _p, _p, _i64, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _sz, _p]),
    "exl3_gemm_trellis_silu_in": (_i, [_p, _p, _i64, _p, _p, _i64, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _sz, _p]),
    "exl3_mgemm": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _sz, _p]),
    "exl3_hgemm_recon": (_i, [_p, _i64, _p, _i64, _p, _i64, _i, _i, _i, _p]),
    "exl3_gemm_trellis": (_i, [_p, _i64, _p, _p, _i64, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p]),
    "exl3_gemm_trellis_grouped": (_i, [_p, _i64, _pp, _p, _i64, _pp, _p, _pp, _ip, _i, _i, _i, _i, _i, _i, _p, _sz,
                                       _p]),
    "exl3_gemm_trellis_workspace_size": (_sz, [_i, _i, _ip, _i]),
    "exl3_gemm_trellis_workspace_bound": (_sz, []),
    "exl3_gemm": (_i, [_p, _i64, _p, _p, _i64, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _sz, _p]),
    "exl3_gemv_mr_approx": (_i, [_p, _i64, _p, _p, _i64, _p, _p, _p, _i, _i, _i, _i, _i, _p, _sz, _p]),
    "exl3_gemv_mr_noalloc": (_i, [_p, _i64, _p, _p, _i64, _p, _p, _i, _i, _i, _i, _i, _i, _p]),
}

_lib = None


class Exl3Error(RuntimeError):
    pass


def lib():
    """Load the HIP library (once).  Raises if it is absent: build it with build_ext.py."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise Exl3Error(f"exl3rocm: HIP library not built ({LIB_PATH}); run build_ext.py / __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        # the version first: a library older than these bindings lacks some of their symbols
        L.exl3_abi_version.restype, L.exl3_abi_version.argtypes = C.c_int, []
        if L.exl3_abi_version() != ABI_VERSION:
            raise Exl3Error(f"exl3rocm: ABI version {L.exl3_abi_version()} != {ABI_VERSION} (rebuild the library)")
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str) -> int:
    """Raise on a negative status; return the status otherwise (0 done, >0 declined / route tag)."""
    if rc < 0:
        names = {EINVAL: "invalid arguments", ELAUNCH: "kernel launch failed", EWORKSPACE: "workspace too small"}
        raise Exl3Error(f"exl3rocm: {what} failed: {names.get(rc, rc)}")
    return rc


def ptr_array(ptrs):
    arr = (C.c_void_p * len(ptrs))(*ptrs)
    return C.cast(arr, _pp), arr
