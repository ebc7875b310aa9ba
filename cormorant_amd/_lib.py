"""ctypes binding of libcormo_hip.so (the C ABI of include/cormorant_hip.h).

The library is built in-tree by ``cormorant_amd._build`` (``__graft_entry__.build()``).  There
is no fallback: if the shared library is missing or fails to load, every unit call raises.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcormo_hip.so")

CM_OK, CM_EINVAL, CM_EALIGN, CM_EHIP, CM_ENOMEM = 0, -1, -2, -3, -4

_U32, _I32, _I64, _P = ctypes.c_uint32, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p


class CmRowopsDesc(ctypes.Structure):
    """cm_rowops_desc: one row-ops job, the argument registers in register order."""
    _fields_ = [("op", _U32), ("n", _U32), ("c1", _U32), ("c2", _U32),
                ("a", ctypes.c_uint64), ("a_s1", _U32), ("a_s2", _U32),
                ("b", ctypes.c_uint64), ("b_s1", _U32), ("b_s2", _U32),
                ("c", ctypes.c_uint64), ("c_s1", _U32), ("c_s2", _U32),
                ("p", ctypes.c_uint64), ("eps", ctypes.c_int64),
                ("aux", _U32), ("bq_sh", _U32), ("win_lo", _U32), ("win_hi", _U32)]


# name -> (restype, argtypes); every symbol include/cormorant_hip.h declares
SIGNATURES = {
    "cm_abi_version": (_I32, []),
    "cm_last_error": (ctypes.c_char_p, []),
    "cm_init": (_I32, []),
    "cm_host_act_table": (_I32, [_I32, _P]),
    "cm_host_rowops_table_image": (_I32, [_P]),
    "cm_act_table_init": (_I32, [_P]),
    "cm_rowops_tables_init": (_I32, [_P]),
    "cm_vectorop": (_I32, [_P, _P, _P] + [_U32] * 10 + [_P]),
    "cm_matmul": (_I32, [_P, _P, _P, _U32, _U32, _U32, _U32, _I64, _I64, _I64, _U32, _U32, _U32, _P]),
    "cm_matmul_noalloc": (_I32, [_P, _P, _P, _U32, _U32, _U32, _U32, _I64, _I64, _I64, _U32, _U32, _U32, _P]),
    "cm_conv": (_I32, [_P, _P, _P, _P] + [_U32] * 21 + [_P]),
    "cm_conv_w_planes_bytes": (ctypes.c_size_t, [_U32] * 4),
    "cm_conv_split_w": (_I32, [_P, _P, _U32, _U32, _U32, _U32, _P]),
    "cm_conv_planes": (_I32, [_P, _P, _P, _P] + [_U32] * 21 + [_P]),
    "cm_conv_act": (_I32, [_P, _P, _P, _P] + [_U32] * 22 + [_P]),
    "cm_conv_planes_act": (_I32, [_P, _P, _P, _P] + [_U32] * 22 + [_P]),
    "cm_pool": (_I32, [_P, _P] + [_U32] * 17 + [_P]),
    "cm_rowops": (_I32, [_P, _P, _P, _P] + [_U32] * 10 + [_I64] + [_U32] * 4 + [_P]),
    "cm_rowops_chain": (_I32, [ctypes.POINTER(CmRowopsDesc), _U32, _P]),
    "cm_rowops_chain_planes": (_I32, [ctypes.POINTER(CmRowopsDesc), _U32, _P, _P]),
    "cm_vectorop_planes": (_I32, [_P, _P, _P] + [_U32] * 7 + [_P, _P]),
    "cm_attention_planes": (_I32, [_P, _P] + [_U32] * 4 + [ctypes.c_uint64] + [_U32] * 5 + [_P, _P]),
    "cm_matmul_a_planes_bytes": (ctypes.c_size_t, [_U32] * 3),
    "cm_matmul_aplanes": (_I32, [_P, _U32, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "cm_softmax": (_I32, [_P, _P] + [_U32] * 9 + [ctypes.c_uint64, ctypes.c_uint64, _P]),
    "cm_permute16": (_I32, [_P, _P] + [_U32] * 4 + [ctypes.c_uint64] * 4 + [_P]),
    "cm_copy16": (_I32, [_P, _P] + [_U32] * 4 + [ctypes.c_uint64] * 8 + [_P]),
    "cm_embed_rows": (_I32, [_P, _U32, _P, _P, _U32, _U32, _U32, _P]),
    "cm_attention": (_I32, [_P, _P] + [_U32] * 4 + [ctypes.c_uint64] + [_U32] * 3 + [ctypes.c_uint64] + [_U32] * 2 + [_P]),
    "cm_decode_attention": (_I32, [_P, _P, _P, _P] + [_U32] * 7 + [_P]),
    "cm_decode_prep": (_I32, [_P] * 6 + [_U32] * 6 + [_P, _P, _U32, _P, _U32, _P]),
    "cm_decode_attention_prep": (_I32, [_P] * 7 + [_U32] * 6 + [_P, _P, _U32, _P, _U32] + [_U32] * 3 + [_P]),
    "cm_matmul_b_planes_bytes": (ctypes.c_size_t, [_U32] * 3),
    "cm_matmul_split_b": (_I32, [_P, _P, _U32, _U32, _U32, ctypes.c_int64, _U32, _U32, _P]),
    "cm_matmul_planes": (_I32, [_P, _P, _P, _U32, _U32, _U32, _U32, ctypes.c_int64, _U32, ctypes.c_int64, _U32, _P]),
    "cm_matmul_strided": (_I32, [_P, _P, _P] + [_U32] * 5 + [ctypes.c_uint64] * 6 + [_U32] + [ctypes.c_uint64] * 3 + [_U32, _P]),
    "cm_matmul_skinny_multi": (_I32, [_P, _U32, _U32, _U32, _P, _P, _P, _U32, _P]),
    "cm_matmul_skinny_planes": (_I32, [_P, _U32, _U32, _U32, _P, _P, _P, _P]),
    "cm_matmul_skinny_planes_sat": (_I32, [_P, _U32, _U32, _U32, _P, _P, _P, _P]),
    "cm_matmul_skinny_planes_addx": (_I32, [_P, _U32, _U32, _P, _P, _U32, _P, _P, _U32, _U32, _P, _P]),
    "cm_matmul_skinny_planes_mulact": (_I32, [_P, _U32, _U32, _P, _P, _P, _P, _U32, _P, _U32, _P, _P]),
    "cm_timing_enable": (_I32, [_I32]),
    "cm_timing_read": (_I32, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                              ctypes.POINTER(ctypes.c_uint64)]),
    "cm_timing_reset": (_I32, []),
    "cm_timing_read_each": (_I32, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.c_uint64,
                                   ctypes.POINTER(ctypes.c_uint64)]),
    "cm_timing_select": (_I32, [ctypes.c_char_p]),
}


def timing_enable(on: bool) -> None:
    check(lib().cm_timing_enable(1 if on else 0), "cm_timing_enable")


def timing_select(kernel: str = "") -> None:
    """Record only launches of ``kernel`` ("" = every kernel)."""
    check(lib().cm_timing_select(kernel.encode()), "cm_timing_select")


def timing_reset() -> None:
    check(lib().cm_timing_reset(), "cm_timing_reset")


def timing_read(kernel: str):
    """(total milliseconds, launches) of the recorded launches of ``kernel``."""
    ms = ctypes.c_double(0.0)
    n = ctypes.c_uint64(0)
    check(lib().cm_timing_read(kernel.encode(), ctypes.byref(ms), ctypes.byref(n)), "cm_timing_read")
    return ms.value, n.value

def timing_read_each(kernel: str):
    """The recorded launches of ``kernel`` one by one, in launch order (milliseconds)."""
    n = ctypes.c_uint64(0)
    check(lib().cm_timing_read_each(kernel.encode(), None, 0, ctypes.byref(n)), "cm_timing_read_each")
    buf = (ctypes.c_double * max(n.value, 1))()
    check(lib().cm_timing_read_each(kernel.encode(), buf, n.value, ctypes.byref(n)), "cm_timing_read_each")
    return list(buf[:n.value])

_lib = None


class HipLibraryMissing(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """The loaded library (loads on first use; raises if it was never built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HipLibraryMissing(
                f"{LIB_PATH} is not built: run __graft_entry__.build() (hipcc, gfx950)")
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def check(rc: int, what: str) -> None:
    """Raise for a failed call: ValueError for contract violations (the error class the
    reference's simulator raises for bad operands), RuntimeError for HIP failures."""
    if rc == CM_OK:
        return
    msg = lib().cm_last_error().decode(errors="replace")
    if rc in (CM_EINVAL, CM_EALIGN):
        raise ValueError(f"{what}: {msg}")
    if rc == CM_ENOMEM:
        raise MemoryError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (status {rc})")
