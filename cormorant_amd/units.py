"""The five units as calls on device tensors: the register contracts of the reference's
kernels (VectorOP.h:319-333, MatmulKernel.h:228-242, ConvKernel.h:229-259,
PoolingKernel.h:120-140, ROWOPS_RTL_KERNEL.md section 1.2), dispatched to libcormo_hip.so.

Every function takes torch tensors on the GPU holding raw lanes (int16; uint8 byte images
for row-ops), checks on the host that each access the kernels will make stays inside the
tensors (so a bad register value raises instead of faulting the GPU), and enqueues the work
on the current torch stream.  Outputs are written into the tensors the caller passes.
"""
from __future__ import annotations

from typing import Iterable, Optional, Sequence

import ctypes

import torch

from . import _lib

OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_RELU, OP_RELU6 = 0, 1, 2, 3, 4, 5
OP_LEAKY_RELU, OP_SILU, OP_GELU, OP_GELU_TANH, OP_SOFTMAX, OP_SOFTMAX_T = 6, 7, 8, 9, 10, 11
ACT_NONE, ACT_RELU, ACT_RELU6, ACT_LEAKY_RELU, ACT_SILU, ACT_GELU, ACT_GELU_TANH = range(7)
POOL_MAX, POOL_AVG, POOL_LP = 0, 1, 2


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require(t: torch.Tensor, name: str, dtype, elems: int) -> None:
    if t is None:
        raise ValueError(f"{name} is required")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.numel() < elems:
        raise ValueError(f"{name} holds {t.numel()} elements; the call touches {elems}")


def init() -> None:
    """Build and upload the unit tables for the current device."""
    _lib.check(_lib.lib().cm_init(), "cm_init")


# ---------------------------------------------------------------- VectorOP
def vectorop_extent(size: int, op: int, outer: int, a_inc: int, b_inc: int):
    """(a, b, c) elements a call touches (whole 8-lane words per run)."""
    padded = (size + 7) & ~7
    if outer == 0 or size == 0:
        return 0, 0, 0
    if op == OP_SOFTMAX:
        return (outer - 1) * a_inc + padded, 0, (outer - 1) * b_inc + padded
    if op == OP_SOFTMAX_T:
        nq = outer & ~15
        if nq == 0:
            return 0, 0, 0
        return (size - 1) * a_inc + nq, 0, (nq - 1) * b_inc + padded
    a = (outer - 1) * a_inc + padded
    b = (outer - 1) * b_inc + padded if op < OP_RELU else 0
    return a, b, (outer - 1) * (a_inc + b_inc) + padded


def vectorop(a: torch.Tensor, b: Optional[torch.Tensor], c: torch.Tensor, size: int, op: int,
             outer: int = 1, a_inc: int = 0, b_inc: int = 0, act: int = 0, alpha: int = 0,
             smx_cm: int = 0, smx_cfg: int = 0, smx_mask: int = 0) -> torch.Tensor:
    """VectorOPKernel (VectorOP.h:319-333): ops 0..9 element-wise with the fused
    activation; 10 / 11 the softmax unit."""
    na, nb, nc = vectorop_extent(size, op, outer, a_inc, b_inc)
    _require(a, "a", torch.int16, na)
    _require(c, "c", torch.int16, nc)
    if nb:
        _require(b, "b", torch.int16, nb)
    rc = _lib.lib().cm_vectorop(_ptr(a), _ptr(b) if nb else None, _ptr(c), size, op, outer, a_inc,
                                b_inc, act, alpha & 0xFFFFFFFF, smx_cm, smx_cfg, smx_mask, _stream())
    _lib.check(rc, "cm_vectorop")
    return c


# ---------------------------------------------------------------- Matmul
def softmax(a: torch.Tensor, c: torch.Tensor, size: int, op: int, outer: int, a_inc: int, c_inc: int,
            smx_cm: int, smx_cfg: int, smx_mask: int, batch: int = 1, a_bs: int = 0,
            c_bs: int = 0) -> torch.Tensor:
    """The softmax unit over ``batch`` matrices (cm_softmax): matrix i at a + i a_bs, c + i c_bs,
    each the VectorOP softmax call (op 10 rows, 11 keys-major)."""
    if batch and size and outer:
        na, _, nc = vectorop_extent(size, op, outer, a_inc, c_inc)
        _require(a, "a", torch.int16, (batch - 1) * a_bs + na)
        _require(c, "c", torch.int16, (batch - 1) * c_bs + nc)
    rc = _lib.lib().cm_softmax(_ptr(a), _ptr(c), size, op, outer, a_inc, c_inc, smx_cm, smx_cfg, smx_mask,
                               batch, a_bs, c_bs, _stream())
    _lib.check(rc, "cm_softmax")
    return c


def permute16(src: torch.Tensor, dst: torch.Tensor, dims, strides) -> torch.Tensor:
    """dst[i0][i1][i2][i3] = src[sum i_k s_k] (cm_permute16): ``dims`` the 4 dst extents,
    ``strides`` the src strides of those dimensions, in elements."""
    d = [int(v) for v in dims]
    st = [int(v) for v in strides]
    if len(d) != 4 or len(st) != 4 or min(d) < 0 or min(st) < 0:
        raise ValueError("permute16: 4 dims and 4 non-negative strides")
    total = d[0] * d[1] * d[2] * d[3]
    if total:
        _require(src, "src", torch.int16, 1 + sum((dk - 1) * sk for dk, sk in zip(d, st)))
        _require(dst, "dst", torch.int16, total)
    rc = _lib.lib().cm_permute16(_ptr(src), _ptr(dst), *d, *st, _stream())
    _lib.check(rc, "cm_permute16")
    return dst


def copy16(src: torch.Tensor, dst: torch.Tensor, dims, src_strides, dst_strides) -> torch.Tensor:
    """dst[sum i_k t_k] = src[sum i_k s_k] over the 4 ``dims`` (cm_copy16), in elements."""
    d = [int(v) for v in dims]
    ss = [int(v) for v in src_strides]
    ts = [int(v) for v in dst_strides]
    if len(d) != 4 or len(ss) != 4 or len(ts) != 4 or min(d) < 0 or min(ss) < 0 or min(ts) < 0:
        raise ValueError("copy16: 4 dims and 4 non-negative strides on each side")
    if d[0] * d[1] * d[2] * d[3]:
        _require(src, "src", torch.int16, 1 + sum((dk - 1) * sk for dk, sk in zip(d, ss)))
        _require(dst, "dst", torch.int16, 1 + sum((dk - 1) * tk for dk, tk in zip(d, ts)))
    rc = _lib.lib().cm_copy16(_ptr(src), _ptr(dst), *d, *ss, *ts, _stream())
    _lib.check(rc, "cm_copy16")
    return dst


def embed_rows(table: torch.Tensor, ids: torch.Tensor, out: torch.Tensor, rows: int, d: int) -> torch.Tensor:
    """cm_embed_rows: out[t] = table[clamp(ids[t], 0, rows - 1)] for every id, the table int16
    (sign-extended) or 32-bit lanes, out 32-bit lanes [n_ids][d]."""
    n = ids.numel()
    if table.dtype not in (torch.int16, torch.int32, torch.float32) or not table.is_cuda or not table.is_contiguous():
        raise ValueError("embed_rows: table must be a contiguous GPU int16 / int32 / float32 tensor")
    if table.numel() < rows * d:
        raise ValueError(f"embed_rows: table holds {table.numel()} lanes; [{rows}][{d}] needed")
    _require(ids, "ids", torch.int32, n)
    if out.dtype not in (torch.int32, torch.float32) or not out.is_cuda or not out.is_contiguous() \
            or out.numel() < n * d:
        raise ValueError(f"embed_rows: out must be a contiguous GPU 32-bit tensor of {n * d} lanes")
    rc = _lib.lib().cm_embed_rows(_ptr(table), int(table.dtype == torch.int16), _ptr(ids), _ptr(out), n, rows, d,
                                  _stream())
    _lib.check(rc, "cm_embed_rows")
    return out


def attention(qkv: torch.Tensor, o: torch.Tensor, batch: int, seq: int, heads: int, head_dim: int, ld: int,
              q_off: int, k_off: int, v_off: int, o_ld: int, smx_cm: int, smx_cfg: int) -> torch.Tensor:
    """An encoder layer's attention in one call (cm_attention): q.K^T, the keys-major softmax and
    P.V per (sequence, head), Q / K / V read from the fused projection's rows, o merged."""
    if batch and heads:
        cols = heads * head_dim
        for off in (q_off, k_off, v_off):
            if off < 0 or off + cols > ld:
                raise ValueError("attention: head columns past the row")
        _require(qkv, "qkv", torch.int16, (batch * seq - 1) * ld + max(q_off, k_off, v_off) + cols)
        _require(o, "o", torch.int16, (batch * seq - 1) * o_ld + cols)
    rc = _lib.lib().cm_attention(_ptr(qkv), _ptr(o), batch, seq, heads, head_dim, ld, q_off, k_off, v_off, o_ld,
                                 smx_cm, smx_cfg, _stream())
    _lib.check(rc, "cm_attention")
    return o


def matmul_b_extent(k: int, m: int, b_packed: int, gemv_kw: int) -> int:
    if gemv_kw or b_packed == 2:
        return k * m
    if b_packed:
        return ((m + 31) // 32) * k * 32
    return k * m


def matmul(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, n: int, k: int, m: int,
           batch: int = 1, a_bs: int = 0, b_bs: int = 0, c_bs: Optional[int] = None,
           b_packed: int = 0, gemv_kw: int = 0, wrap32: bool = False) -> torch.Tensor:
    """MatmulKernel (MatmulKernel.h:228-242); C row-major [n][m] per batch slice."""
    if c_bs is None:
        c_bs = n * m
    if batch and n and m:
        _require(a, "a", torch.int16, (batch - 1) * a_bs + n * k)
        _require(b, "b", torch.int16, (batch - 1) * b_bs + matmul_b_extent(k, m, b_packed, gemv_kw))
        _require(c, "c", torch.int16, (batch - 1) * c_bs + n * m)
    rc = _lib.lib().cm_matmul(_ptr(a), _ptr(b), _ptr(c), n, k, m, batch, a_bs, b_bs, c_bs,
                              int(b_packed), int(gemv_kw), int(bool(wrap32)), _stream())
    _lib.check(rc, "cm_matmul")
    return c


NOALLOC_MAX_BYTES = 64 << 20       # CM_NOALLOC_MAX_BYTES of include/cormorant_hip.h


def matmul_noalloc(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, n: int, k: int, m: int,
                   batch: int = 1, a_bs: int = 0, b_bs: int = 0, c_bs: Optional[int] = None,
                   b_packed: int = 0, gemv_kw: int = 0, wrap32: bool = False) -> torch.Tensor:
    """cm_matmul_noalloc: ``matmul``'s result with no device allocation (the library's fixed
    scratch; ValueError past its CM_NOALLOC_MAX_BYTES, or before ``init`` on this device)."""
    if c_bs is None:
        c_bs = n * m
    if batch and n and m:
        _require(a, "a", torch.int16, (batch - 1) * a_bs + n * k)
        _require(b, "b", torch.int16, (batch - 1) * b_bs + matmul_b_extent(k, m, b_packed, gemv_kw))
        _require(c, "c", torch.int16, (batch - 1) * c_bs + n * m)
    rc = _lib.lib().cm_matmul_noalloc(_ptr(a), _ptr(b), _ptr(c), n, k, m, batch, a_bs, b_bs, c_bs,
                                      int(b_packed), int(gemv_kw), int(bool(wrap32)), _stream())
    _lib.check(rc, "cm_matmul_noalloc")
    return c


def matmul_skinny_multi(a: torch.Tensor, n: int, k: int, bs, cs, ms, b_packed: int = 0) -> None:
    """cm_matmul_skinny_multi: C_i = sat16(wrap32(A . B_i) >> 8) for up to 4 B images of the
    same A [n][k] (n <= 32) in one launch."""
    count = len(bs)
    if not (len(cs) == len(ms) == count):
        raise ValueError("matmul_skinny_multi: one c and one m per b")
    _require(a, "a", torch.int16, n * k)
    for b, c, m in zip(bs, cs, ms):
        _require(b, "b", torch.int16, matmul_b_extent(k, m, b_packed, 0))
        _require(c, "c", torch.int16, n * m)
    P = ctypes.c_void_p * max(count, 1)
    rc = _lib.lib().cm_matmul_skinny_multi(_ptr(a), n, k, count, P(*[_ptr(b) for b in bs]), P(*[_ptr(c) for c in cs]),
                                           (ctypes.c_uint32 * max(count, 1))(*ms), int(b_packed), _stream())
    _lib.check(rc, "cm_matmul_skinny_multi")


def decode_attention(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, o: torch.Tensor, groups: int, g: int,
                     c: int, smx_cm: int, smx_cfg: int, smx_mask: int, head_dim: int = 64) -> torch.Tensor:
    """cm_decode_attention: per KV group the g query rows against c cache rows, q.K^T, the
    row-mode softmax and P.V in one launch (o like q)."""
    _require(q, "q", torch.int16, groups * g * head_dim)
    _require(kc, "kc", torch.int16, groups * c * head_dim)
    _require(vc, "vc", torch.int16, groups * c * head_dim)
    _require(o, "o", torch.int16, groups * g * head_dim)
    rc = _lib.lib().cm_decode_attention(_ptr(q), _ptr(kc), _ptr(vc), _ptr(o), groups, g, c, head_dim,
                                        smx_cm & 0xFFFFFFFF, smx_cfg & 0xFFFFFFFF, smx_mask & 0xFFFFFFFF, _stream())
    _lib.check(rc, "cm_decode_attention")
    return o


def decode_prep(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, qr: torch.Tensor, kc: torch.Tensor,
                kc_rows: int, vc: torch.Tensor, batch: int, heads: int, kv_heads: int, head_dim: int, pos: int,
                rope_row: torch.Tensor, params_q: torch.Tensor, op_q: int, params_k: torch.Tensor, op_k: int) -> None:
    """cm_decode_prep: q / k RoPE'd at ``pos`` (q into qr, k into the K cache rows), v's rows into
    the V cache rows; caches [batch][kv_heads][kc_rows][head_dim]."""
    _require(q, "q", torch.int16, batch * heads * head_dim)
    _require(k, "k", torch.int16, batch * kv_heads * head_dim)
    _require(v, "v", torch.int16, batch * kv_heads * head_dim)
    _require(qr, "qr", torch.int16, batch * heads * head_dim)
    _require(kc, "kc", torch.int16, batch * kv_heads * kc_rows * head_dim)
    _require(vc, "vc", torch.int16, batch * kv_heads * kc_rows * head_dim)
    _require(rope_row, "rope_row", torch.int32, 2 * head_dim)
    rc = _lib.lib().cm_decode_prep(_ptr(q), _ptr(k), _ptr(v), _ptr(qr), _ptr(kc), _ptr(vc), batch, heads, kv_heads,
                                   head_dim, kc_rows, pos, _ptr(rope_row), _ptr(params_q), op_q & 0xFFFFFFFF,
                                   _ptr(params_k), op_k & 0xFFFFFFFF, _stream())
    _lib.check(rc, "cm_decode_prep")


def decode_attention_prep(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, qr: torch.Tensor, kc: torch.Tensor,
                          vc: torch.Tensor, o: torch.Tensor, batch: int, heads: int, kv_heads: int, head_dim: int,
                          kc_rows: int, pos: int, rope_row: torch.Tensor, params_q: torch.Tensor, op_q: int,
                          params_k: torch.Tensor, op_k: int, smx_cm: int, smx_cfg: int, smx_mask: int) -> torch.Tensor:
    """cm_decode_attention_prep: decode_prep and decode_attention over its outputs in one launch."""
    _require(q, "q", torch.int16, batch * heads * head_dim)
    _require(k, "k", torch.int16, batch * kv_heads * head_dim)
    _require(v, "v", torch.int16, batch * kv_heads * head_dim)
    _require(qr, "qr", torch.int16, batch * heads * head_dim)
    _require(o, "o", torch.int16, batch * heads * head_dim)
    _require(kc, "kc", torch.int16, batch * kv_heads * kc_rows * head_dim)
    _require(vc, "vc", torch.int16, batch * kv_heads * kc_rows * head_dim)
    _require(rope_row, "rope_row", torch.int32, 2 * head_dim)
    rc = _lib.lib().cm_decode_attention_prep(_ptr(q), _ptr(k), _ptr(v), _ptr(qr), _ptr(kc), _ptr(vc), _ptr(o), batch,
                                             heads, kv_heads, head_dim, kc_rows, pos, _ptr(rope_row), _ptr(params_q),
                                             op_q & 0xFFFFFFFF, _ptr(params_k), op_k & 0xFFFFFFFF,
                                             smx_cm & 0xFFFFFFFF, smx_cfg & 0xFFFFFFFF, smx_mask & 0xFFFFFFFF,
                                             _stream())
    _lib.check(rc, "cm_decode_attention_prep")
    return o


def matmul_skinny_planes(a: torch.Tensor, n: int, k: int, planes, cs, ms, wrap32: bool = True) -> None:
    """cm_matmul_skinny_planes: C_i = sat16(wrap32(A . B_i) >> 8) for up to 4 weights given as
    their split images (matmul_b_planes of the same k and m_i) and the same A [n][k], n <= 16;
    with wrap32 False, cm_matmul_skinny_planes_sat: C_i = sat16(floor(A . B_i / 2^8)), exact."""
    count = len(planes)
    if not (len(cs) == len(ms) == count):
        raise ValueError("matmul_skinny_planes: one c and one m per weight")
    _require(a, "a", torch.int16, n * k)
    for pl, c, m in zip(planes, cs, ms):
        need = int(_lib.lib().cm_matmul_b_planes_bytes(k, m, 1))
        if pl.dtype != torch.uint8 or pl.numel() < need or pl.data_ptr() % 256:
            raise ValueError("matmul_skinny_planes: the uint8 image of matmul_b_planes for these k, m")
        _require(c, "c", torch.int16, n * m)
    P = ctypes.c_void_p * max(count, 1)
    name = "cm_matmul_skinny_planes" if wrap32 else "cm_matmul_skinny_planes_sat"
    rc = getattr(_lib.lib(), name)(_ptr(a), n, k, count, P(*[_ptr(x) for x in planes]),
                                   P(*[_ptr(c) for c in cs]), (ctypes.c_uint32 * max(count, 1))(*ms), _stream())
    _lib.check(rc, name)


def matmul_skinny_planes_addx(a: torch.Tensor, n: int, k: int, planes: torch.Tensor, c: torch.Tensor, m: int,
                              x: torch.Tensor, params: torch.Tensor, op: int, out: torch.Tensor,
                              bq_sh: int = 0) -> None:
    """cm_matmul_skinny_planes_addx: C = sat16(wrap32(A . B) >> 8) for one weight's split image,
    then the row-ops COPY / ADDX job ``op`` over x [n][m] and C into out [n][m] in the same launch."""
    _require(a, "a", torch.int16, n * k)
    need = int(_lib.lib().cm_matmul_b_planes_bytes(k, m, 1))
    if planes.dtype != torch.uint8 or planes.numel() < need or planes.data_ptr() % 256:
        raise ValueError("matmul_skinny_planes_addx: the uint8 image of matmul_b_planes for these k, m")
    _require(c, "c", torch.int16, n * m)
    if x.numel() * x.element_size() < n * m * (2 if (op >> 4) & 3 == 0 else 4):
        raise ValueError("matmul_skinny_planes_addx: x smaller than [n][m] of the job's A kind")
    if out.numel() * out.element_size() < n * m * (2 if (op >> 8) & 3 == 0 else 4):
        raise ValueError("matmul_skinny_planes_addx: out smaller than [n][m] of the job's output kind")
    rc = _lib.lib().cm_matmul_skinny_planes_addx(_ptr(a), n, k, _ptr(planes), _ptr(c), m, _ptr(x), _ptr(params),
                                                 op & 0xFFFFFFFF, bq_sh, _ptr(out), _stream())
    _lib.check(rc, "cm_matmul_skinny_planes_addx")


def matmul_skinny_planes_mulact(a: torch.Tensor, n: int, k: int, b_gate: torch.Tensor, b_up: torch.Tensor,
                                c_gate: torch.Tensor, c_up: torch.Tensor, m: int, params: torch.Tensor, op: int,
                                out: torch.Tensor) -> None:
    """cm_matmul_skinny_planes_mulact: the gate and up products of A (each as
    matmul_skinny_planes gives it) and the row-ops MULACT job ``op`` over them into out [n][m],
    one launch."""
    _require(a, "a", torch.int16, n * k)
    need = int(_lib.lib().cm_matmul_b_planes_bytes(k, m, 1))
    for name, img in (("b_gate", b_gate), ("b_up", b_up)):
        if img.dtype != torch.uint8 or img.numel() < need or img.data_ptr() % 256:
            raise ValueError(f"matmul_skinny_planes_mulact: {name} is not the uint8 image of matmul_b_planes for k, m")
    for name, t in (("c_gate", c_gate), ("c_up", c_up), ("out", out)):
        _require(t, name, torch.int16, n * m)
    if params.dtype != torch.uint8 or params.numel() < 16 * (1 if op & F_P_BCAST else m) or not params.is_contiguous():
        raise ValueError("matmul_skinny_planes_mulact: params must be the contiguous uint8 block of the job's entries")
    rc = _lib.lib().cm_matmul_skinny_planes_mulact(_ptr(a), n, k, _ptr(b_gate), _ptr(b_up), _ptr(c_gate), _ptr(c_up),
                                                   m, _ptr(params), op & 0xFFFFFFFF, _ptr(out), _stream())
    _lib.check(rc, "cm_matmul_skinny_planes_mulact")


def matmul_strided(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, n: int, k: int, m: int, batch: int,
                   inner: int, a_view, b_view, c_view, b_trans: bool = False, wrap32: bool = False) -> torch.Tensor:
    """cm_matmul_strided: each view is (offset, ld, bs, bs2) in elements of its tensor; slice bt
    starts at offset + (bt // inner) bs + (bt % inner) bs2."""
    def extent(view, r, cols):
        off, ld, bs, bs2 = view
        return off + ((batch - 1) // inner) * bs + (min(batch, inner) - 1) * bs2 + (r - 1) * ld + cols
    if n and m and batch:
        _require(a, "a", torch.int16, extent(a_view, n, k))
        _require(b, "b", torch.int16, extent(b_view, m, k) if b_trans else extent(b_view, k, m))
        _require(c, "c", torch.int16, extent(c_view, n, m))
    (ao, lda, abs1, abs2), (bo, ldb, bbs1, bbs2), (co, ldc, cbs1, cbs2) = a_view, b_view, c_view
    rc = _lib.lib().cm_matmul_strided(_ptr(a) + 2 * ao, _ptr(b) + 2 * bo, _ptr(c) + 2 * co, n, k, m, batch, inner,
                                      lda, abs1, abs2, ldb, bbs1, bbs2, int(bool(b_trans)), ldc, cbs1, cbs2,
                                      int(bool(wrap32)), _stream())
    _lib.check(rc, "cm_matmul_strided")
    return c


def matmul_b_planes(b: torch.Tensor, k: int, m: int, b_slices: int = 1, b_bs: int = 0, b_packed: int = 0,
                    gemv_kw: int = 0) -> torch.Tensor:
    """B's split image (cm_matmul_split_b) in a new uint8 device tensor, for matmul_planes."""
    nbytes = int(_lib.lib().cm_matmul_b_planes_bytes(k, m, b_slices))
    planes = torch.empty(nbytes + 256, dtype=torch.uint8, device=b.device)
    off = (-planes.data_ptr()) % 256
    planes = planes[off:off + nbytes]
    if b_slices and m:
        _require(b, "b", torch.int16, (b_slices - 1) * b_bs + matmul_b_extent(k, m, b_packed, gemv_kw))
    rc = _lib.lib().cm_matmul_split_b(_ptr(b), _ptr(planes), k, m, b_slices, b_bs, int(b_packed), int(gemv_kw),
                                      _stream())
    _lib.check(rc, "cm_matmul_split_b")
    return planes


def matmul_planes(a: torch.Tensor, b_planes: torch.Tensor, c: torch.Tensor, n: int, k: int, m: int,
                  batch: int = 1, a_bs: int = 0, b_slices: int = 1, c_bs: Optional[int] = None,
                  wrap32: bool = False) -> torch.Tensor:
    """cm_matmul with B's split image from matmul_b_planes."""
    if c_bs is None:
        c_bs = n * m
    if batch and n and m:
        _require(a, "a", torch.int16, (batch - 1) * a_bs + n * k)
        _require(c, "c", torch.int16, (batch - 1) * c_bs + n * m)
        need = int(_lib.lib().cm_matmul_b_planes_bytes(k, m, b_slices))
        if b_planes.dtype != torch.uint8 or b_planes.numel() < need or b_planes.data_ptr() % 256:
            raise ValueError("b_planes: the uint8 image of matmul_b_planes for these k, m, b_slices")
    rc = _lib.lib().cm_matmul_planes(_ptr(a), _ptr(b_planes), _ptr(c), n, k, m, batch, a_bs, b_slices, c_bs,
                                     int(bool(wrap32)), _stream())
    _lib.check(rc, "cm_matmul_planes")
    return c


# ---------------------------------------------------------------- Conv
def conv_weight_numel(out_ch: int, in_ch: int, kh: int, kw: int, depthwise: bool) -> int:
    """Elements of the packed weight image (ConvKernel.h:142-150)."""
    if depthwise:
        return out_ch * ((kh * kw + 7) & ~7)
    tiles = (in_ch + 15) // 16
    rem = in_ch - (tiles - 1) * 16
    return out_ch * kh * kw * ((tiles - 1) * 16 + (8 if rem <= 8 else 16))


def conv_y_extent(batch, out_ch, out_h, out_w, y_cs=0, y_cn=0, y_gs=0) -> int:
    plane = out_h * out_w
    cs = y_cs or plane
    if y_cn:
        last = max((c % y_cn) * cs + (c // y_cn) * y_gs for c in range(out_ch))
        return last + plane
    return (batch - 1) * out_ch * plane + (out_ch - 1) * cs + plane


def conv_small(in_ch: int, kh: int, kw: int, out_ch: int, batch: int = 1) -> bool:
    """A standard convolution cm_conv runs straight on the VALU (its packed weights as they are,
    no GEMM operand): at most 80 taps (in_ch kh kw) per output and 12288 taps x output
    channels, batch up to 65535."""
    return in_ch * kh * kw <= 80 and in_ch * kh * kw * out_ch <= 12288 and batch <= 65535


def conv(x: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor], y: torch.Tensor,
         batch: int, in_ch: int, in_h: int, in_w: int, out_ch: int, out_h: int, out_w: int,
         kh: int, kw: int, stride_h: int = 1, stride_w: int = 1, dilation_h: int = 1,
         dilation_w: int = 1, pad_top: int = 0, pad_left: int = 0, has_bias: int = 0,
         is_depthwise: int = 0, y_cs: int = 0, y_cn: int = 0, y_gs: int = 0,
         wrap32: bool = False, act: int = 0) -> torch.Tensor:
    """ConvKernel (ConvKernel.h:229-259) on packed weights; ``act`` 1 / 2 applies RELU / RELU6 to
    the result (cm_conv_act: the VectorOP RELU / RELU6 of the output fused)."""
    if batch and out_ch and out_h and out_w:
        _require(x, "x", torch.int16, batch * in_ch * in_h * in_w)
        _require(w, "w", torch.int16, conv_weight_numel(out_ch, in_ch, kh, kw, bool(is_depthwise)))
        if has_bias:
            _require(bias, "bias", torch.int16, out_ch)
        _require(y, "y", torch.int16, conv_y_extent(batch, out_ch, out_h, out_w, y_cs, y_cn, y_gs))
        for oh_max, in_dim, k, s, d, p, nm in ((out_h, in_h, kh, stride_h, dilation_h, pad_top, "h"),
                                               (out_w, in_w, kw, stride_w, dilation_w, pad_left, "w")):
            if s == 0 or d == 0:
                raise ValueError(f"conv: zero stride / dilation along {nm}")
    args = (_ptr(x), _ptr(w), _ptr(bias) if has_bias else None, _ptr(y), batch, in_ch, in_h, in_w, out_ch, out_h,
            out_w, kh, kw, stride_h, stride_w, dilation_h, dilation_w, pad_top, pad_left, int(has_bias),
            int(is_depthwise), y_cs, y_cn, y_gs, int(bool(wrap32)))
    if act:
        _lib.check(_lib.lib().cm_conv_act(*args, int(act), _stream()), "cm_conv_act")
    else:
        _lib.check(_lib.lib().cm_conv(*args, _stream()), "cm_conv")
    return y


def conv_w_planes(w: torch.Tensor, out_ch: int, in_ch: int, kh: int, kw: int) -> torch.Tensor:
    """The split image of a standard convolution's packed weights (cm_conv_split_w) in a new
    uint8 device tensor, for conv_planes."""
    nbytes = int(_lib.lib().cm_conv_w_planes_bytes(out_ch, in_ch, kh, kw))
    planes = torch.empty(nbytes + 256, dtype=torch.uint8, device=w.device)
    off = (-planes.data_ptr()) % 256
    planes = planes[off:off + nbytes]
    if out_ch:
        _require(w, "w", torch.int16, conv_weight_numel(out_ch, in_ch, kh, kw, False))
    rc = _lib.lib().cm_conv_split_w(_ptr(w), _ptr(planes), out_ch, in_ch, kh, kw, _stream())
    _lib.check(rc, "cm_conv_split_w")
    return planes


def conv_planes(x: torch.Tensor, w_planes: torch.Tensor, bias: Optional[torch.Tensor], y: torch.Tensor,
                batch: int, in_ch: int, in_h: int, in_w: int, out_ch: int, out_h: int, out_w: int,
                kh: int, kw: int, stride_h: int = 1, stride_w: int = 1, dilation_h: int = 1,
                dilation_w: int = 1, pad_top: int = 0, pad_left: int = 0, has_bias: int = 0,
                y_cs: int = 0, y_cn: int = 0, y_gs: int = 0, wrap32: bool = False, act: int = 0) -> torch.Tensor:
    """cm_conv of a standard convolution with the weights' split image from conv_w_planes;
    ``act`` as conv's (cm_conv_planes_act)."""
    if batch and out_ch and out_h and out_w:
        _require(x, "x", torch.int16, batch * in_ch * in_h * in_w)
        if has_bias:
            _require(bias, "bias", torch.int16, out_ch)
        _require(y, "y", torch.int16, conv_y_extent(batch, out_ch, out_h, out_w, y_cs, y_cn, y_gs))
        need = int(_lib.lib().cm_conv_w_planes_bytes(out_ch, in_ch, kh, kw))
        if w_planes.dtype != torch.uint8 or w_planes.numel() < need or w_planes.data_ptr() % 256:
            raise ValueError("w_planes: the uint8 image of conv_w_planes for these out_ch, in_ch, kh, kw")
        if stride_h == 0 or stride_w == 0 or dilation_h == 0 or dilation_w == 0:
            raise ValueError("conv: zero stride / dilation")
    args = (_ptr(x), _ptr(w_planes), _ptr(bias) if has_bias else None, _ptr(y), batch, in_ch, in_h, in_w, out_ch,
            out_h, out_w, kh, kw, stride_h, stride_w, dilation_h, dilation_w, pad_top, pad_left, int(has_bias), 0,
            y_cs, y_cn, y_gs, int(bool(wrap32)))
    if act:
        _lib.check(_lib.lib().cm_conv_planes_act(*args, int(act), _stream()), "cm_conv_planes_act")
    else:
        _lib.check(_lib.lib().cm_conv_planes(*args, _stream()), "cm_conv_planes")
    return y


# ---------------------------------------------------------------- Pool
def pool(x: torch.Tensor, y: torch.Tensor, batch: int, channels: int, in_h: int, in_w: int,
         out_h: int, out_w: int, pool_h: int, pool_w: int, stride_h: int = 1, stride_w: int = 1,
         pad_top: int = 0, pad_left: int = 0, dil_h: int = 1, dil_w: int = 1,
         pool_type: int = POOL_MAX, lp_order: int = 2, count_include_pad: int = 0) -> torch.Tensor:
    """PoolingKernel (PoolingKernel.h:120-140)."""
    _require(x, "x", torch.int16, batch * channels * in_h * in_w)
    _require(y, "y", torch.int16, batch * channels * out_h * out_w)
    rc = _lib.lib().cm_pool(_ptr(x), _ptr(y), batch, channels, in_h, in_w, out_h, out_w, pool_h,
                            pool_w, stride_h, stride_w, pad_top, pad_left, dil_h, dil_w, pool_type,
                            lp_order, count_include_pad, _stream())
    _lib.check(rc, "cm_pool")
    return y


# ---------------------------------------------------------------- RowOps
RO_COPY, RO_ADDX, RO_DEQUANT, RO_MULACT, RO_NORM, RO_ROPE, RO_XPOSE, RO_TLOAD = 1, 2, 3, 4, 5, 6, 7, 8
RO_FOLD, RO_GATE = 9, 10
K_I16, K_I32, K_F32 = 0, 1, 2
F_B_EN, F_P_BCAST, F_P_KEEP, F_RELU, F_NORM_LN, F_SCALE = (1 << 12, 1 << 13, 1 << 14, 1 << 15,
                                                         1 << 16, 1 << 17)


def _kb(kind: int) -> int:
    return 2 if kind == K_I16 else 4


def rowops_extents(op, n, c1, c2, a_s1, a_s2, b_s1, b_s2, c_s1, c_s2, aux=0, win_lo=0,
                   win_hi=0xFFFFFFFF):
    """Byte extents (a, b, c, p) one job touches; None where the job has no work."""
    code = op & 15
    if code == RO_FOLD:
        s, m = aux & 15, (aux >> 4) & 127
        if not (n and c1 and c2 and m):
            return None
        out = c2 * c1 * n * 2
        s0 = b_s2 - (1 << 32) if b_s2 >= 1 << 31 else b_s2
        a_s2s = a_s2 - (1 << 32) if a_s2 >= 1 << 31 else a_s2
        lo = max(s0, win_lo)
        hi = min(s0 + (c1 - 1) * b_s1 + n, win_hi)     # exclusive source column bound
        if hi <= lo:
            a_lo, a_hi = 0, 0
        else:
            ks = [0, (c2 - 1) * a_s2s]
            a_lo = min(ks) + 2 * lo
            a_hi = max(ks) + 2 * hi
        return (a_lo, a_hi), 0, (out + 15) & ~15, 0
    if not (n and c1 and c2) or n > 4096:
        return None
    last = (c2 - 1), (c1 - 1)
    if code == RO_TLOAD:
        return (0, last[0] * a_s2 + last[1] * a_s1 + 4 * n), 0, 0, 0
    if code == RO_XPOSE:
        R = aux & 15
        if not 1 <= R <= 8:
            return None
        a_end = last[0] * a_s2 + last[1] * a_s1 + (R - 1) * b_s1 + 2 * n
        c_end = last[0] * c_s2 + last[1] * c_s1 + (n - 1) * b_s2 + 2 * R
        if b_s2 == 2 * R:
            c_end = last[0] * c_s2 + last[1] * c_s1 + ((2 * R * n + 15) & ~15)
        return (0, a_end), 0, c_end, 0
    ak, bk, ck = (op >> 4) & 3, (op >> 6) & 3, (op >> 8) & 3
    if code == RO_DEQUANT:
        ck = K_F32
    a_row = ((_kb(ak) * n + 15) & ~15)
    a_end = last[0] * a_s2 + last[1] * a_s1 + (2 * n if code == RO_ROPE else _kb(ak) * n)
    b_end = 0
    if code == RO_ROPE:
        HD = aux & 0xFFF
        if HD == 0 or HD & 15 or HD > 128 or n % HD:
            return None
        b_end = last[0] * b_s2 + last[1] * b_s1 + 8 * HD
    elif (op & F_B_EN) and code != RO_DEQUANT:
        b_end = last[0] * b_s2 + last[1] * b_s1 + _kb(bk) * n
    c_end = last[0] * c_s2 + last[1] * c_s1 + ((_kb(ck) * n + 15) & ~15)
    p_end = 16 * (1 if op & F_P_BCAST else n)
    del a_row
    return (0, a_end), b_end, c_end, p_end


def _byte_ptr(t: torch.Tensor, off: int = 0) -> int:
    return t.data_ptr() + off


def rowops(a, b, c, p, op: int, n: int, c1: int, c2: int, a_s1: int, a_s2: int, b_s1: int,
           b_s2: int, c_s1: int, c_s2: int, eps: int = 0, aux: int = 0, bq_sh: int = 0,
           win_lo: int = 0, win_hi: int = 0xFFFFFFFF, a_off: int = 0, b_off: int = 0,
           c_off: int = 0, p_off: int = 0) -> None:
    """One RowOpsKernel job (ROWOPS_RTL_KERNEL.md 1.2) on GPU uint8 byte images; the
    `*_off` arguments are byte offsets into each image (run_rowops' a_off / b_off / c_off,
    rowops_nodes.py:143-151)."""
    ext = rowops_extents(op, n, c1, c2, a_s1, a_s2, b_s1, b_s2, c_s1, c_s2, aux, win_lo, win_hi)
    if ext is not None:
        (a_lo, a_hi), b_end, c_end, p_end = ext
        for t, nm, off, lo, hi in ((a, "a", a_off, a_lo, a_hi), (b, "b", b_off, 0, b_end),
                                   (c, "c", c_off, 0, c_end), (p, "p", p_off, 0, p_end)):
            if hi <= lo:
                continue
            if t is None or not t.is_cuda or t.dtype != torch.uint8 or not t.is_contiguous():
                raise ValueError(f"rowops: {nm} must be a contiguous GPU uint8 tensor")
            if off + lo < 0 or off + hi > t.numel():
                raise ValueError(f"rowops: {nm} accesses bytes [{off + lo}, {off + hi}) of {t.numel()}")
    rc = _lib.lib().cm_rowops(
        _byte_ptr(a, a_off) if a is not None else None, _byte_ptr(b, b_off) if b is not None else None,
        _byte_ptr(c, c_off) if c is not None else None, _byte_ptr(p, p_off) if p is not None else None,
        op, n, c1, c2, a_s1, a_s2, b_s1, b_s2, c_s1, c_s2, int(eps), aux, bq_sh, win_lo, win_hi,
        _stream())
    _lib.check(rc, "cm_rowops")


def a_planes(n: int, k: int, nsum: int, device) -> torch.Tensor:
    """A new 256-byte aligned uint8 device buffer for the byte planes of an n x k matmul A
    (cm_matmul_a_planes_bytes) with nsum partial row-sum arrays."""
    nbytes = int(_lib.lib().cm_matmul_a_planes_bytes(n, k, nsum))
    buf = torch.empty(nbytes + 256, dtype=torch.uint8, device=device)
    off = (-buf.data_ptr()) % 256
    return buf[off:off + nbytes]


def _require_planes(planes: torch.Tensor, n: int, k: int, nsum: int) -> None:
    need = int(_lib.lib().cm_matmul_a_planes_bytes(n, k, nsum))
    if (not planes.is_cuda or planes.dtype != torch.uint8 or not planes.is_contiguous() or planes.numel() < need
            or planes.data_ptr() % 256):
        raise ValueError(f"planes: a 256-byte aligned uint8 GPU buffer of {need} bytes (a_planes)")


def matmul_aplanes(a_planes: torch.Tensor, nsum: int, b_planes: torch.Tensor, c: torch.Tensor, n: int, k: int,
                   m: int, wrap32: bool = False) -> torch.Tensor:
    """cm_matmul_aplanes: C = A . B with A's planes from its producer (a_planes, nsum row-sum
    arrays) and B's from matmul_b_planes."""
    if n and m:
        _require_planes(a_planes, n, k, nsum)
        _require(c, "c", torch.int16, n * m)
        need = int(_lib.lib().cm_matmul_b_planes_bytes(k, m, 1))
        if b_planes.dtype != torch.uint8 or b_planes.numel() < need or b_planes.data_ptr() % 256:
            raise ValueError("b_planes: the uint8 image of matmul_b_planes for these k, m")
    rc = _lib.lib().cm_matmul_aplanes(_ptr(a_planes), nsum, _ptr(b_planes), _ptr(c), n, k, m, int(bool(wrap32)),
                                      _stream())
    _lib.check(rc, "cm_matmul_aplanes")
    return c


def vectorop_planes(a: torch.Tensor, b: Optional[torch.Tensor], c: Optional[torch.Tensor], size: int, op: int,
                    outer: int, a_inc: int, b_inc: int, planes: torch.Tensor, act: int = 0,
                    alpha: int = 0) -> Optional[torch.Tensor]:
    """cm_vectorop_planes: the VectorOP over `outer` runs of `size` (contiguous output rows) and
    the byte planes of its output for matmul_aplanes (n = outer, k = size, nsum = ceil(size /
    1024)); c None: the planes alone."""
    if outer and size:
        _require(a, "a", torch.int16, (outer - 1) * a_inc + size)
        if op < OP_RELU:
            _require(b, "b", torch.int16, (outer - 1) * b_inc + size)
        if c is not None:
            _require(c, "c", torch.int16, outer * size)
        _require_planes(planes, outer, size, (size + 1023) // 1024)
    rc = _lib.lib().cm_vectorop_planes(_ptr(a), _ptr(b), _ptr(c), size, op, outer, a_inc, b_inc, act, alpha,
                                       _ptr(planes), _stream())
    _lib.check(rc, "cm_vectorop_planes")
    return c


def attention_planes(qkv: torch.Tensor, o: Optional[torch.Tensor], batch: int, seq: int, heads: int, head_dim: int,
                     ld: int, q_off: int, k_off: int, v_off: int, smx_cm: int, smx_cfg: int,
                     planes: torch.Tensor) -> Optional[torch.Tensor]:
    """cm_attention_planes: attention() with o's rows heads x head_dim wide, and o's byte planes
    for matmul_aplanes (n = batch seq, k = heads head_dim, nsum = heads); o None: the planes
    alone."""
    if batch and heads:
        cols = heads * head_dim
        for off in (q_off, k_off, v_off):
            if off < 0 or off + cols > ld:
                raise ValueError("attention: head columns past the row")
        _require(qkv, "qkv", torch.int16, (batch * seq - 1) * ld + max(q_off, k_off, v_off) + cols)
        if o is not None:
            _require(o, "o", torch.int16, batch * seq * cols)
        _require_planes(planes, batch * seq, cols, heads)
    rc = _lib.lib().cm_attention_planes(_ptr(qkv), _ptr(o), batch, seq, heads, head_dim, ld, q_off, k_off, v_off,
                                        smx_cm, smx_cfg, _ptr(planes), _stream())
    _lib.check(rc, "cm_attention_planes")
    return o


def rowops_jobs(jobs: Sequence[dict], planes: Optional[torch.Tensor] = None) -> None:
    """Row-ops jobs in order through cm_rowops_chain, each job a dict of rowops()'s arguments
    with its own tensors (a / b / c / p: GPU uint8 images or None); with ``planes``
    (cm_rowops_chain_planes) also the byte planes of the last job's output, whose c may then be
    None (the planes alone)."""
    descs = (_lib.CmRowopsDesc * len(jobs))()
    for idx, (d, j) in enumerate(zip(descs, jobs)):
        ext = rowops_extents(j["op"], j["n"], j["c1"], j["c2"], j["a_s1"], j["a_s2"], j["b_s1"], j["b_s2"],
                             j["c_s1"], j["c_s2"], j.get("aux", 0), j.get("win_lo", 0), j.get("win_hi", 0xFFFFFFFF))
        if ext is not None:
            (a_lo, a_hi), b_end, c_end, p_end = ext
            for key, lo, hi in (("a", a_lo, a_hi), ("b", 0, b_end), ("c", 0, c_end), ("p", 0, p_end)):
                if hi <= lo:
                    continue
                if key == "c" and j.get("c") is None and planes is not None and idx == len(jobs) - 1:
                    continue                   # the planes' NORM writing the planes alone
                if key == "c" and j.get("c") is None:
                    raise ValueError("rowops: a null output (only the planes' last NORM may omit its rows)")
                t = j.get(key)
                if t is None or not t.is_cuda or t.dtype != torch.uint8 or not t.is_contiguous():
                    raise ValueError(f"rowops: {key} must be a contiguous GPU uint8 tensor")
                if lo < 0 or hi > t.numel():
                    raise ValueError(f"rowops: {key} accesses bytes [{lo}, {hi}) of {t.numel()}")
        for f in ("op", "n", "c1", "c2", "a_s1", "a_s2", "b_s1", "b_s2", "c_s1", "c_s2", "aux",
                  "bq_sh", "win_lo", "win_hi"):
            setattr(d, f, int(j.get(f, 0xFFFFFFFF if f == "win_hi" else 0)))
        d.eps = int(j.get("eps", 0))
        for key in ("a", "b", "c", "p"):
            t = j.get(key)
            setattr(d, key, t.data_ptr() if t is not None else 0)
    if planes is not None:
        last = jobs[-1]
        _require_planes(planes, int(last["c1"]) * int(last["c2"]), int(last["n"]), (int(last["n"]) + 1023) // 1024)
        rc = _lib.lib().cm_rowops_chain_planes(descs, len(jobs), _ptr(planes), _stream())
        _lib.check(rc, "cm_rowops_chain_planes")
        return
    rc = _lib.lib().cm_rowops_chain(descs, len(jobs), _stream())
    _lib.check(rc, "cm_rowops_chain")


def rowops_chain(seg: torch.Tensor, jobs: Sequence[dict]) -> None:
    """A descriptor chain over one GPU byte segment: each job's a / b / c / p are byte
    offsets into ``seg`` (the layout of the reference's chain fixtures)."""
    descs = (_lib.CmRowopsDesc * len(jobs))()
    base = seg.data_ptr()
    for d, j in zip(descs, jobs):
        ext = rowops_extents(j["op"], j["n"], j["c1"], j["c2"], j["a_s1"], j["a_s2"], j["b_s1"],
                             j["b_s2"], j["c_s1"], j["c_s2"], j.get("aux", 0), j.get("win_lo", 0),
                             j.get("win_hi", 0xFFFFFFFF))
        if ext is not None:
            (a_lo, a_hi), b_end, c_end, p_end = ext
            for key, lo, hi in (("a", a_lo, a_hi), ("b", 0, b_end), ("c", 0, c_end), ("p", 0, p_end)):
                if hi > lo and (j[key] + lo < 0 or j[key] + hi > seg.numel()):
                    raise ValueError(f"rowops chain: job {j.get('label')} {key} leaves the segment")
        for f in ("op", "n", "c1", "c2", "a_s1", "a_s2", "b_s1", "b_s2", "c_s1", "c_s2", "aux",
                  "bq_sh", "win_lo", "win_hi"):
            setattr(d, f, int(j.get(f, 0xFFFFFFFF if f == "win_hi" else 0)))
        d.eps = int(j.get("eps", 0))
        for key in ("a", "b", "c", "p"):
            setattr(d, key, base + int(j[key]))
    rc = _lib.lib().cm_rowops_chain(descs, len(jobs), _stream())
    _lib.check(rc, "cm_rowops_chain")


def host_act_table(act: int):
    """The library's full activation table (act 4..6) as a numpy int16 array."""
    import numpy as np
    out = np.zeros(65536, np.int16)
    _lib.check(_lib.lib().cm_host_act_table(act, out.ctypes.data), "cm_host_act_table")
    return out


def host_rowops_table_image():
    import numpy as np
    out = np.zeros(65536, np.uint8)
    _lib.check(_lib.lib().cm_host_rowops_table_image(out.ctypes.data), "cm_host_rowops_table_image")
    return out


def act_table_init(tables) -> None:
    """cm_act_table_init: the current device's SiLU / GELU / GELU-tanh tables from int16
    [3][65536] (f(x) at [x + 32768]); ValueError where a table lacks the unit's form."""
    import numpy as np
    t = np.ascontiguousarray(np.asarray(tables, np.int16).reshape(3, 65536))
    _lib.check(_lib.lib().cm_act_table_init(t.ctypes.data), "cm_act_table_init")


def rowops_tables_init(img) -> None:
    """cm_rowops_tables_init: the current device's 64 KiB row-ops table image."""
    import numpy as np
    b = np.ascontiguousarray(np.asarray(img, np.uint8).reshape(65536))
    _lib.check(_lib.lib().cm_rowops_tables_init(b.ctypes.data), "cm_rowops_tables_init")
