"""Loading of libsc and the ctypes signatures of its C ABI (include/sc_api.h,
include/sc_synth.h).  There is no fallback: if the library is missing the
import fails with the command that builds it."""
from __future__ import annotations

import ctypes as C
import os

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_ROOT, "lib", "libsc.so")

try:  # torch ships its own libamdhip64.so.7; load it first so libsc binds to
    import torch  # noqa: F401  the same HIP runtime as the tensors it is given
except ImportError:  # pragma: no cover - torch is part of the image
    torch = None


class LibscError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"libsc error {code}: {msg}")
        self.code = code


_lib = None

i32, i64, u64, f32p, f64p = C.c_int32, C.c_int64, C.c_uint64, C.POINTER(C.c_float), C.POINTER(C.c_double)
i32p, i64p, vp = C.POINTER(C.c_int32), C.POINTER(C.c_int64), C.c_void_p

_SIGS = {
    "sc_last_error": ([], C.c_char_p),
    "sc_abi_version": ([], C.c_int),
    "sc_patterns": ([i32, i32, C.c_char_p, i64, i32p], C.c_int),
    "sc_mtx_read": ([C.c_char_p, i32, C.POINTER(vp)], C.c_int),
    "sc_mtx_write": ([vp, C.c_char_p], C.c_int),
    "sc_csr_create": ([i32, i32, i32p, i32p, f64p, i32, C.POINTER(vp)], C.c_int),
    "sc_csr_info": ([vp, i32p, i32p, i64p, i32p], C.c_int),
    "sc_csr_arrays": ([vp, C.POINTER(i32p), C.POINTER(i32p), C.POINTER(f64p)], C.c_int),
    "sc_csr_free": ([vp], None),
    "sc_cfmtx_build": ([vp, i32, i32, C.c_char_p, C.POINTER(vp)], C.c_int),
    "sc_cfmtx_write": ([vp, C.c_char_p], C.c_int),
    "sc_cfmtx_read": ([C.c_char_p, C.POINTER(vp)], C.c_int),
    "sc_load_cfmtx_matrices": ([C.c_char_p, C.POINTER(vp), C.POINTER(vp)], C.c_int),
    "sc_read_csr_matrix": ([C.c_char_p, C.POINTER(vp)], C.c_int),
    "sc_companion_mtx_path": ([C.c_char_p, C.c_char_p, C.c_size_t], C.c_int),
    "sc_cfmtx_info": ([vp, i32p, i32p, i32p, i32p, i32p, i32p], C.c_int),
    "sc_cfmtx_pattern": ([vp, i32, C.POINTER(C.c_char_p), i32p, i32p, C.POINTER(i32p), i64p,
                          C.POINTER(i32p), i64p, C.POINTER(f32p), i64p], C.c_int),
    "sc_cfmtx_text": ([vp, C.c_char_p, i64, i64p], C.c_int),
    "sc_cfmtx_free": ([vp], None),
    "sc_plan_create": ([vp, i32, C.POINTER(vp)], C.c_int),
    "sc_plan_info": ([vp, i32p, i32p, i32p, i32p, i64p, i64p, i64p], C.c_int),
    "sc_spmm": ([vp, vp, vp, i32, i32, i32, vp], C.c_int),
    "sc_spmm_noalloc": ([vp, vp, vp, i32, i32, i32, vp], C.c_int),
    "sc_spmv": ([vp, vp, vp, i32, vp], C.c_int),
    "sc_spmm_f16": ([vp, vp, vp, i32, i32, i32, vp], C.c_int),
    "sc_plan_destroy": ([vp], None),
    "sc_plan_describe": ([vp, i32, C.c_char_p, C.c_size_t], C.c_int),
    "sc_spmm_generated": ([vp, vp, vp, vp, vp, i32, i32, i32, vp], C.c_int),
    "sc_synth_uniform": ([i32, i32, C.c_double, C.c_double, u64, C.POINTER(vp)], C.c_int),
    "sc_synth_blocks": ([i32, i32, C.c_double, C.c_double, u64, C.POINTER(vp)], C.c_int),
    "sc_synth_dense": ([f32p, i64, u64], C.c_int),
    "sc_synth_raw": ([u64, C.POINTER(C.c_uint64), i64], C.c_int),
}

EXPORTS = tuple(_SIGS)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; "
                               f"g.build()'` or `make -C sparse-computation_amd/csrc`")
        L = C.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise LibscError(rc, lib().sc_last_error().decode(errors="replace"))
