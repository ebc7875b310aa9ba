"""ctypes wrapper of ``liboracle.so`` (built from ``cm_oracle.c`` by ``oracle/Makefile``).

TEST INFRASTRUCTURE ONLY -- the checker, never the thing measured or shipped.  Arrays are
numpy raw integer lanes (int16 / uint8 byte images); every call writes into an output the
caller provides or a fresh array it returns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def build(force: bool = False) -> str:
    """Compile ``liboracle.so`` with gcc (seconds)."""
    if force or not os.path.exists(LIB_PATH) or (
            os.path.getmtime(LIB_PATH) < os.path.getmtime(os.path.join(HERE, "cm_oracle.c"))):
        subprocess.check_call(["make", "-s", "-C", HERE, "liboracle.so"])
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        U, I, P, L = ctypes.c_uint, ctypes.c_int, ctypes.c_void_p, ctypes.c_long
        _lib.oracle_vectorop.argtypes = [P, P, P] + [U] * 10
        _lib.oracle_matmul.argtypes = [P, P, P, U, U, U, U, L, L, L, U, U, I]
        _lib.oracle_conv.argtypes = [P, P, P, P] + [U] * 20 + [I]
        _lib.oracle_pool.argtypes = [P, P] + [U] * 17
        _lib.oracle_rowops.argtypes = [P, P, P, P] + [U] * 10 + [ctypes.c_longlong] + [U] * 4
        _lib.oracle_act_table.argtypes = [I, P]
        _lib.oracle_smx_table.argtypes = [P]
        _lib.oracle_rowops_table_image.argtypes = [P]
        _lib.oracle_rowops_reset_params.argtypes = []
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _i16(a):
    return np.ascontiguousarray(np.asarray(a), dtype=np.int16)


def vectorop(a, b, c_len, size, op, outer=1, a_inc=0, b_inc=0, act=0, alpha=0,
             smx_cm=0, smx_cfg=0, smx_mask=0, c=None):
    """VectorOPKernel registers (VectorOP.h:319-333); returns the c image (int16)."""
    a = _i16(a)
    b = _i16(b) if b is not None else np.zeros(8, np.int16)
    if c is None:
        c = np.zeros(c_len, np.int16)
    rc = lib().oracle_vectorop(_p(a), _p(b), _p(c), size, op, outer, a_inc, b_inc, act,
                               alpha & 0xFFFFFFFF, smx_cm, smx_cfg, smx_mask)
    if rc:
        raise ValueError(f"oracle_vectorop: status {rc}")
    return c


def matmul(a, b, n, k, m, batch=1, a_bs=0, b_bs=0, c_bs=None, b_packed=0, gemv_kw=0,
           wrap32=False):
    """MatmulKernel registers (MatmulKernel.h:228-242); returns C [batch * c_bs] int16."""
    a, b = _i16(a), _i16(b)
    if c_bs is None:
        c_bs = n * m
    c = np.zeros(max(batch - 1, 0) * c_bs + n * m, np.int16)
    lib().oracle_matmul(_p(a), _p(b), _p(c), n, k, m, batch, a_bs, b_bs, c_bs, b_packed,
                        gemv_kw, int(bool(wrap32)))
    return c


def conv(x, w, bias, y_len, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, sh, sw,
         dh, dw, pt, pl, has_bias, is_dw, y_cs=0, y_cn=0, y_gs=0, wrap32=False, y=None):
    """ConvKernel registers (ConvKernel.h:229-259); returns the y image (int16)."""
    x, w = _i16(x), _i16(w)
    bias = _i16(bias) if bias is not None else np.zeros(8, np.int16)
    if y is None:
        y = np.zeros(y_len, np.int16)
    lib().oracle_conv(_p(x), _p(w), _p(bias), _p(y), batch, in_ch, in_h, in_w, out_ch, out_h,
                      out_w, kh, kw, sh, sw, dh, dw, pt, pl, has_bias, is_dw, y_cs, y_cn, y_gs,
                      int(bool(wrap32)))
    return y


def pool(x, batch, ch, in_h, in_w, out_h, out_w, ph, pw, sh, sw, pt, pl, dh, dw, ptype, lp,
         cip):
    """PoolingKernel registers (PoolingKernel.h:120-140); returns y [N][C][oh][ow]."""
    x = _i16(x)
    y = np.zeros(batch * ch * out_h * out_w, np.int16)
    lib().oracle_pool(_p(x), _p(y), batch, ch, in_h, in_w, out_h, out_w, ph, pw, sh, sw, pt,
                      pl, dh, dw, ptype, lp, cip)
    return y


def rowops(a, b, c, p, op, n, c1, c2, a_s1, a_s2, b_s1, b_s2, c_s1, c_s2, eps=0, aux=0,
           bq_sh=0, win_lo=0, win_hi=0xFFFFFFFF):
    """One RowOpsKernel job (ROWOPS_RTL_KERNEL.md 1.2) on uint8 byte images; ``c`` is
    updated in place and returned."""
    a = np.ascontiguousarray(a, np.uint8)
    b = np.ascontiguousarray(b, np.uint8) if b is not None and len(b) else None
    p = np.ascontiguousarray(p, np.uint8) if p is not None and len(p) else np.zeros(16, np.uint8)
    assert c.dtype == np.uint8 and c.flags.c_contiguous
    lib().oracle_rowops(_p(a), _p(b) if b is not None else None, _p(c), _p(p), op, n, c1, c2,
                        a_s1, a_s2, b_s1, b_s2, c_s1, c_s2, int(eps), aux, bq_sh, win_lo,
                        win_hi & 0xFFFFFFFF)
    return c


def rowops_reset_params():
    lib().oracle_rowops_reset_params()


def act_table(act: int) -> np.ndarray:
    out = np.zeros(65536, np.int16)
    if lib().oracle_act_table(act, _p(out)):
        raise ValueError(f"act {act} is not an activation of the unit")
    return out


def smx_table() -> np.ndarray:
    out = np.zeros(4096, np.int32)
    lib().oracle_smx_table(_p(out))
    return out


def rowops_table_image() -> np.ndarray:
    out = np.zeros(65536, np.uint8)
    lib().oracle_rowops_table_image(_p(out))
    return out
