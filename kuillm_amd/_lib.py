"""ctypes binding of ``libkuiops.so`` -- the C ABI declared in include/kuiops.h.

This module is the only place that talks to the native library.  It loads the
in-tree ``kuillm_amd/libkuiops.so`` (built by ``kuillm_amd.compile``), declares
every entry point's argument types, and turns a negative status into a Python
exception.  It never falls back to anything: if the library is missing or a
call fails, the caller sees an error.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("KUIOPS_LIB", Path(__file__).resolve().parent / "libkuiops.so"))

# kuiops_status
OK = 0
E_UNSUPPORTED = -1
E_INVALID = -2
E_HIP = -3
E_WORKSPACE = -4

# kuiops_dtype
F32, F16, BF16, F64, I64, I32, I16, I8, U8, BOOL = range(10)
# kuiops_b_layout
B_ROW, B_COL = 0, 1
# kuiops_c_kind
C_NONE, C_FULL, C_ROW = 0, 1, 2
# kuiops_ew_op
EW_ADD, EW_SUB, EW_MUL, EW_DIV, EW_NEG, EW_SILU, EW_RSQRT, EW_COS, EW_SIN, EW_EXP, EW_SQRT, EW_POW_SCALAR, \
    EW_EQ, EW_NE, EW_LE, EW_LT, EW_GE, EW_GT, EW_WHERE, EW_BITWISE_NOT, EW_BITWISE_AND, EW_BITWISE_OR = range(22)
# kuiops_op
OP_ADDMM, OP_GEMV_SPLITK, OP_SDPA_DECODE, OP_TOPK, OP_SORT, OP_DECODE_ROWS_BATCHED = 1, 2, 3, 4, 5, 6

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p
_dbl = ctypes.c_double
_flt = ctypes.c_float
_sz = ctypes.c_size_t
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); mirrors include/kuiops.h one to one.
X_PLAIN, X_RMSNORM, X_SWIGLU = 1, 2, 3

SIGNATURES = {
    "kuiops_abi_version": (_int, []),
    "kuiops_status_string": (ctypes.c_char_p, [_int]),
    "kuiops_query_workspace": (_sz, [_int, _i64, _i64, _i64]),
    "kuiops_mm": (_int, [_i64, _i64, _i64, _int, _vp, _i64, _vp, _i64, _int, _int, _vp, _i64, _vp]),
    "kuiops_addmm": (_int, [_i64, _i64, _i64, _dbl, _dbl, _int, _vp, _i64, _vp, _i64, _int,
                            _vp, _int, _i64, _int, _vp, _i64, _int, _vp, _sz, _vp]),
    "kuiops_bmm": (_int, [_i64, _i64, _i64, _i64, _int, _vp, _i64, _i64, _vp, _i64, _i64, _int,
                          _int, _vp, _i64, _i64, _vp]),
    "kuiops_gemv_splitk": (_int, [_i64, _i64, _i64, _int, _vp, _i64, _vp, _i64, _int, _vp, _int,
                                  _vp, _i64, _int, _vp, _sz, _vp]),
    "kuiops_gemv_splitk_noalloc": (_int, [_i64, _i64, _i64, _int, _vp, _i64, _vp, _i64, _int, _vp, _int,
                                          _vp, _i64, _int, _vp]),
    "kuiops_gemv_splitk_noalloc_max_bytes": (_sz, []),
    "kuiops_elementwise": (_int, [_int, _int, _i64p, _int, ctypes.POINTER(_int), ctypes.POINTER(_vp), _i64p,
                                  _dbl, _dbl, _int, _int, _vp, _vp]),
    "kuiops_mean_lastdim": (_int, [_i64, _i64, _int, _vp, _i64, _vp, _vp]),
    "kuiops_cat": (_int, [_int, ctypes.POINTER(_vp), _i64p, _i64p, _i64, _int, _vp, _vp]),
    "kuiops_sdpa_fwd": (_int, [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp, _i64p, _vp, _i64p,
                               _vp, _i64p, _vp, _i64p, _vp, _flt, _int, _vp]),
    "kuiops_sdpa_fwd_bias": (_int, [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp, _i64p, _vp, _i64p,
                                    _vp, _i64p, _vp, _i64p, _vp, _flt, _int, _vp, _i64p, _vp]),
    "kuiops_sdpa_general": (_int, [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp, _i64p, _vp, _i64p,
                                   _vp, _i64p, _vp, _i64p, _vp, _dbl, _int, _vp, _i64p, _vp]),
    "kuiops_sdpa_decode": (_int, [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp, _i64p, _vp, _i64p,
                                  _vp, _i64p, _vp, _i64p, _vp, _flt, _int, _vp, _vp, _sz, _vp]),
    "kuiops_softmax_lastdim": (_int, [_i64, _i64, _int, _vp, _vp, _vp]),
    "kuiops_topk_lastdim": (_int, [_i64, _i64, _i64, _int, _vp, _vp, _vp, _int, _int, _vp, _sz, _vp]),
    "kuiops_softmax_top1": (_int, [_i64, _i64, _int, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp]),
    "kuiops_gather": (_int, [_int, _i64p, _i64p, _int, _int, _vp, _vp, _vp, _vp, _vp]),
    "kuiops_scatter": (_int, [_int, _i64p, _i64p, _int, _int, _vp, _vp, _vp, _vp, _vp]),
    "kuiops_sort_lastdim": (_int, [_i64, _i64, _int, _vp, _vp, _vp, _int, _vp, _sz, _vp]),
    "kuiops_cumsum_lastdim": (_int, [_i64, _i64, _int, _vp, _vp, _vp]),
    "kuiops_top_p_mask": (_int, [_i64, _i64, _vp, _vp, _vp, _dbl, _i64, _dbl, _vp, _vp]),
    "kuiops_multinomial": (_int, [_i64, _i64, _int, _vp, _i64, _vp, _vp, _vp, _vp]),
    "kuiops_index": (_int, [_i64, _i64, _i64, _i64, _int, _vp, _vp, _vp, _vp, _vp]),
    "kuiops_index_multi": (_int, [_i64, _int, _i64p, _i64, _i64, ctypes.POINTER(_vp), _int, _vp, _vp, _vp, _vp]),
    "kuiops_decode_rows_batched": (_int, [_i64, _i64, _i64, _int, _int, _int, _vp, _i64, _vp, _i64, _vp, _i64, _vp,
                                          _flt, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _vp,
                                          _vp, _vp, _i64p, _vp, _i64p, _i64, _vp, _sz, _vp]),
    "kuiops_rmsnorm": (_int, [_i64, _i64, _int, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _flt, _vp, _i64, _vp]),
    "kuiops_silu_mul": (_int, [_i64, _i64, _int, _vp, _i64, _vp, _i64, _vp]),
    "kuiops_rope_kv_append": (_int, [_i64, _i64, _i64, _i64, _i64, _int, _vp, _i64, _i64, _vp, _vp,
                                     _vp, _i64p, _vp, _i64p, _vp, _i64p, _i64, _vp]),
    "kuiops_decode_linear": (_int, [_i64, _i64, _int, _int, _vp, _vp, _vp, _flt, _vp, _vp, _i64, _vp, _vp,
                                    _vp]),
    "kuiops_decode_gate_up": (_int, [_i64, _i64, _int, _int, _vp, _vp, _vp, _flt, _vp, _vp, _i64, _vp, _vp]),
    "kuiops_decode_qkv_rope": (_int, [_i64, _i64, _i64, _i64, _int, _int, _vp, _vp, _i64, _i64, _vp, _vp, _flt,
                                      _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _i64, _i64,
                                      _vp]),
    "kuiops_decode_step_sync_bytes": (_sz, [_i64]),
    "kuiops_decode_step_scratch_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "kuiops_decode_step": (_int, [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _flt, _vp, _i64, _i64,
                                  _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp,
                                  _sz, _vp, _sz, _vp]),
    "kuiops_decode_step_error": (_int, [_vp, _i64, _vp]),
    "kuiops_decode_step_supported": (_int, [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int]),
}


class KuiopsError(RuntimeError):
    """A kuiops entry point returned a negative status."""

    def __init__(self, name, status):
        self.status = status
        super().__init__(f"{name} failed: {status_string(status)} ({status})")


class Unsupported(KuiopsError):
    """KUIOPS_E_UNSUPPORTED: the shape / dtype is outside the kernels."""


_lib = None


def load(path: Path | str | None = None):
    """Load (once) and return the ctypes library.  Raises if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"kuiops native library not built: {p} is missing "
                           "(run `python -c 'import __graft_entry__ as g; g.build()'` "
                           "or `make -C kuillm_amd/csrc`)")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.kuiops_abi_version() != 1:
        raise RuntimeError("libkuiops ABI version mismatch")
    if path is None:
        _lib = lib
    return lib


def loaded() -> bool:
    return _lib is not None


def status_string(status: int) -> str:
    try:
        return load().kuiops_status_string(status).decode()
    except Exception:
        return str(status)


def check(name: str, status: int) -> None:
    if status == OK:
        return
    if status == E_UNSUPPORTED:
        raise Unsupported(name, status)
    raise KuiopsError(name, status)


def call(name: str, *args) -> None:
    """Call entry point ``name`` and raise on a negative status."""
    check(name, getattr(load(), name)(*args))


def strides3(*vals) -> ctypes.Array:
    return (ctypes.c_int64 * 3)(*[int(v) for v in vals])


def i64_array(vals) -> ctypes.Array:
    vals = [int(v) for v in vals]
    return (ctypes.c_int64 * max(1, len(vals)))(*vals)
